"""Seeded sweep of paged-decode argument combinations against the oracle.

Each case draws its own element type, head geometry, block size, pool layout,
batch and lengths (empty, one-token, tile-edge and long contexts), index types,
per-sequence or cumulative lengths, a fused current row (through the table or
explicit slots), a key mask, the TTS read bounds, FP8 pools where the shape
allows them, and the split (exact bound, a graph's 65536 bound, or a fixed
partition size).  The output must meet oracle.paged_decode within the dtype's
tolerance, and with a fused row the pools must equal oracle.write_current_kv's
bit for bit.  The combinations are those the single-feature tests in
test_gpu_decode.py, test_gpu_decode_bounds.py and test_gpu_fp8.py cover one at a
time (qwen_tts_paged_attention.py:181-287 for the semantics).
"""
import math

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops

pytestmark = pytest.mark.gpu

# (head_dim, num_heads, num_kv_heads): matrix-core shapes, the general kernel's,
# and the small-head kernel's (head_dim or group outside the vector kernels).
GEOMETRIES = [(128, 16, 8), (64, 14, 14), (256, 8, 2), (128, 32, 4), (64, 8, 1),
              (96, 12, 4), (32, 6, 2), (128, 6, 2)]
BLOCKS = [1, 2, 16, 16, 16, 32, 32, 64, 256]  # weighted to the matrix-core kernel


def _draw(seed: int, matrix_core: bool = False):
    """One case; matrix_core: only shapes the matrix-core kernel takes."""
    r = torch.Generator().manual_seed(1000 + seed + (100000 if matrix_core else 0))

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=r))]

    def coin(p=0.5):
        return bool(torch.rand(1, generator=r) < p)

    if matrix_core:
        d, hq, hkv = pick(GEOMETRIES[:5])
        dtype = pick([torch.bfloat16, torch.float16])
        bs = pick([16, 32, 64, 256])
    else:
        d, hq, hkv = pick(GEOMETRIES)
        dtype = pick([torch.bfloat16, torch.float16, torch.float32])
        bs = pick(BLOCKS)
    vector = d in (64, 128, 256) and hq // hkv in (1, 2, 4, 8)
    fp8 = vector and dtype != torch.float32 and bs % 16 == 0 and coin(0.4)
    B = int(torch.randint(1, 65 if matrix_core else 41, (1,), generator=r))
    lens = []
    for _ in range(B):
        kind = int(torch.randint(6, (1,), generator=r))
        lens.append([0, 1, 16 * int(torch.randint(1, 8, (1,), generator=r)),
                     int(torch.randint(2, 300, (1,), generator=r)),
                     int(torch.randint(300, 1200, (1,), generator=r)),
                     int(torch.randint(1200, 2600, (1,), generator=r))][kind])
    if max(lens) == 0:
        lens[0] = 5
    fused = coin(0.6)
    if fused:
        lens = [max(n, 1) for n in lens]  # a current row needs a position
    return dict(
        d=d, hq=hq, hkv=hkv, dtype=dtype, bs=bs, fp8=fp8, lens=lens, fused=fused,
        slots=fused and coin(0.3),
        layout=pick([ops.LAYOUT_NHD, ops.LAYOUT_HND]),
        table_i64=coin(0.3), lens_i64=coin(0.3), cumulative=coin(0.3),
        mask=coin(0.3), bound=pick(["exact", "graph", "fixed"]),
        tts_bounds=coin(0.2), seed=seed)


@pytest.mark.parametrize("matrix_core,seed",
                         [(False, s) for s in range(48)] + [(True, s) for s in range(16)])
def test_random_decode_case_matches_oracle(dev, matrix_core, seed):
    c = _draw(seed, matrix_core)
    gen = torch.Generator().manual_seed(seed)
    d, hq, hkv, bs, lens, layout = c["d"], c["hq"], c["hkv"], c["bs"], c["lens"], c["layout"]
    B = len(lens)
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + 5
    perm = torch.randperm(nb, generator=gen).tolist()
    width = max(max(need), 1) + 1
    rows, cur = [], 0
    for n in need:
        rows.append(perm[cur:cur + n] + [-1] * (width - n))
        cur += n
    table = torch.tensor(rows, dtype=torch.int64 if c["table_i64"] else torch.int32)
    shape = (nb, bs, hkv, d) if layout == ops.LAYOUT_NHD else (nb, hkv, bs, d)
    ks, vs = (0.05, 0.08) if c["fp8"] else (1.0, 1.0)
    if c["fp8"]:
        kp = oracle.quantize_fp8(torch.randn(shape, generator=gen), ks)
        vp = oracle.quantize_fp8(torch.randn(shape, generator=gen), vs)  # unit scale
    else:
        kp = (torch.randn(shape, generator=gen) * 0.5).to(c["dtype"])
        vp = torch.randn(shape, generator=gen).to(c["dtype"])
    q = torch.randn(B, hq, d, generator=gen).to(c["dtype"])
    lens_t = torch.tensor(lens, dtype=torch.int64 if c["lens_i64"] else torch.int32)
    if c["cumulative"]:
        lens_arg = torch.zeros(B + 1, dtype=lens_t.dtype)
        lens_arg[1:] = torch.cumsum(lens_t, 0)
    else:
        lens_arg = lens_t
    valid = None
    if c["mask"]:
        valid = torch.rand(B, max(lens) + 7, generator=gen) < 0.8
        valid[:, 0] = True
    nk = nv = slots = None
    if c["fused"]:
        nk = (torch.randn(B, hkv, d, generator=gen) * 0.5).to(c["dtype"])
        nv = torch.randn(B, hkv, d, generator=gen).to(c["dtype"])
        if c["slots"]:
            # The engine's slot_mapping: the table slot of position len - 1.
            slots = torch.tensor([int(table[b, (n - 1) // bs]) * bs + (n - 1) % bs
                                  for b, n in enumerate(lens)], dtype=torch.int32)
    key_limit = read_width = 0
    if c["tts_bounds"]:
        key_limit = max(1, (max(lens) * 3) // 4)
        read_width = max(1, width - 1)
    max_seq = max(lens) if c["bound"] != "graph" else 65536
    split = 64 if c["bound"] == "fixed" else 0
    print(f"case {seed}: {c}", flush=True)
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.paged_decode(
        q.to(dev), kd, vd, table.to(dev), lens_arg.to(dev), max_seq_len=max_seq,
        scale=d ** -0.5, lens_cumulative=c["cumulative"], layout=layout,
        valid_mask=None if valid is None else valid.to(dev),
        new_k=None if nk is None else nk.to(dev), new_v=None if nv is None else nv.to(dev),
        new_slots=None if slots is None else slots.to(dev), split_tokens=split,
        key_limit=key_limit, table_read_width=read_width, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    k0, v0 = kp, vp
    if c["fused"]:
        k0, v0 = oracle.write_current_kv(kp, vp, table, lens_t, nk, nv, layout=layout,
                                         k_scale=ks, v_scale=vs)
    if c["fp8"]:
        assert torch.equal(kd.cpu().view(torch.uint8), k0.view(torch.uint8))
        assert torch.equal(vd.cpu().view(torch.uint8), v0.view(torch.uint8))
    else:
        assert torch.equal(kd.cpu(), k0) and torch.equal(vd.cpu(), v0)
    ref = oracle.paged_decode(q, k0, v0, table, lens_t, d ** -0.5, layout=layout,
                              valid_mask=valid, key_limit=key_limit or None,
                              table_read_width=read_width or None, k_scale=ks, v_scale=vs)
    tol = 1e-5 if c["dtype"] == torch.float32 else 2e-2
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= tol, f"case {seed}: max error {err:.3e}"
    if seed % 4 == 0:
        # The same call captured in a HIP graph: every replay, with eager work
        # between replays, gives the eager output bit for bit (the fused row is
        # written again with the same values).
        args = (q.to(dev), kd, vd, table.to(dev), lens_arg.to(dev))
        kw = dict(max_seq_len=max_seq, scale=d ** -0.5, lens_cumulative=c["cumulative"],
                  layout=layout, valid_mask=None if valid is None else valid.to(dev),
                  new_k=None if nk is None else nk.to(dev),
                  new_v=None if nv is None else nv.to(dev),
                  new_slots=None if slots is None else slots.to(dev), split_tokens=split,
                  key_limit=key_limit, table_read_width=read_width, k_scale=ks, v_scale=vs)
        gout = torch.empty_like(out)
        stream = torch.cuda.Stream(dev)
        with torch.cuda.stream(stream):
            ops.paged_decode(*args, out=gout, **kw)  # allocates the stream's workspace
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.paged_decode(*args, out=gout, **kw)
        for _ in range(2):
            gout.fill_(7.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(gout, out), f"case {seed}: graph replay differs from eager"
        del graph
