"""Seeded sweep of varlen-attention argument combinations against the oracle.

Each case draws its own element type, head geometry, causality, key source
(packed k/v, a paged prefix plus k/v, or every key from the pool), pool block
size, layout and format (16-bit or FP8 codes), index types, sequence count and
(prefix, new-token) lengths (empty sequences, one-token prompts, prefix-cache
hits, tile edges), and whether the new rows are stored into the pool in the
same launch (with some slots -1).  The output must meet oracle.varlen_attention
within 2e-2, and a fused store must leave the pools equal to
oracle.store_kvcache's bit for bit.  The single-feature tests in
test_gpu_varlen.py and test_gpu_fp8.py cover these one at a time
(flash_attn_varlen_func semantics, qwen_asr_vllm/layers/attention.py:96-139).
"""
import math

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops

pytestmark = pytest.mark.gpu

GEOMETRIES = [(16, 8, 128), (14, 14, 64), (32, 4, 128), (16, 2, 64), (8, 1, 128),
              (64, 8, 128)]


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    return cu


def _draw(seed: int):
    r = torch.Generator().manual_seed(2000 + seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=r))]

    def coin(p=0.5):
        return bool(torch.rand(1, generator=r) < p)

    def rint(lo, hi):
        return int(torch.randint(lo, hi, (1,), generator=r))

    hq, hkv, d = pick(GEOMETRIES)
    mode = pick(["packed", "paged", "pool_only"])
    n = rint(1, 25)
    seqs = []
    for _ in range(n):
        q_len = pick([0, 1, 64, rint(2, 200), rint(200, 700)])
        prefix = 0 if mode == "packed" else pick([0, 1, 16, rint(2, 300), rint(300, 900)])
        extra = pick([0, 0, rint(1, 100)]) if mode == "packed" else 0  # k_len > q_len
        seqs.append((prefix, q_len, extra))
    if sum(q for _, q, _ in seqs) == 0:
        seqs[0] = (seqs[0][0], 5, seqs[0][2])
    return dict(
        hq=hq, hkv=hkv, d=d, dtype=pick([torch.bfloat16, torch.float16]), mode=mode,
        causal=coin(0.7), seqs=seqs, bs=pick([1, 16, 16, 32, 64, 256]),
        layout=pick([ops.LAYOUT_NHD, ops.LAYOUT_HND]), fp8=mode != "packed" and coin(0.3),
        store=mode == "paged" and coin(0.6), table_i64=coin(0.3), slot_i64=coin(0.3),
        seed=seed)


@pytest.mark.parametrize("seed", range(40))
def test_random_varlen_case_matches_oracle(dev, seed):
    c = _draw(seed)
    gen = torch.Generator().manual_seed(seed)
    hq, hkv, d, dt, bs, layout = c["hq"], c["hkv"], c["d"], c["dtype"], c["bs"], c["layout"]
    q_lens = [q for _, q, _ in c["seqs"]]
    if c["mode"] == "packed":
        k_lens = [q + e for _, q, e in c["seqs"]]
    else:
        k_lens = [p + q for p, q, _ in c["seqs"]]
    total_q, total_k = sum(q_lens), sum(k_lens)
    q = torch.randn(total_q, hq, d, generator=gen).to(dt)
    scale = d ** -0.5
    kp = vp = table = slots = None
    ks, vs = (0.05, 0.08) if c["fp8"] else (1.0, 1.0)
    if c["mode"] == "packed":
        k = torch.randn(total_k, hkv, d, generator=gen).to(dt)
        v = torch.randn(total_k, hkv, d, generator=gen).to(dt)
    else:
        need = [math.ceil(kl / bs) for kl in k_lens]
        nb = sum(need) + 3
        width = max(max(need), 1)
        perm = torch.randperm(nb, generator=gen).tolist()
        rows, cur = [], 0
        for m in need:
            rows.append(perm[cur:cur + m] + [-1] * (width - m))
            cur += m
        table = torch.tensor(rows, dtype=torch.int64 if c["table_i64"] else torch.int32)
        shape = (nb, bs, hkv, d) if layout == ops.LAYOUT_NHD else (nb, hkv, bs, d)
        if c["fp8"]:
            kp = oracle.quantize_fp8(torch.randn(shape, generator=gen), ks)
            # Unit-scale values, as for 16-bit pools: the 2e-2 bound is for outputs of
            # order one (bf16's ulp is 2^-5 from 4 to 8).
            vp = oracle.quantize_fp8(torch.randn(shape, generator=gen), vs)
        else:
            kp = torch.randn(shape, generator=gen).to(dt)
            vp = torch.randn(shape, generator=gen).to(dt)
        if c["mode"] == "paged":
            k = torch.randn(total_q, hkv, d, generator=gen).to(dt)
            v = torch.randn(total_q, hkv, d, generator=gen).to(dt)
            if c["store"]:
                sl = []
                for s, (p, ql, _) in enumerate(c["seqs"]):
                    for pos in range(p, p + ql):
                        sl.append(int(table[s, pos // bs]) * bs + pos % bs)
                slots = torch.tensor(sl, dtype=torch.int64 if c["slot_i64"] else torch.int32)
                if slots.numel() > 0:
                    slots[::5] = -1  # padding rows: skipped, pool untouched
        else:
            k = v = None
    cu_q, cu_k = _cu(q_lens), _cu(k_lens)
    print(f"case {seed}: {c}", flush=True)
    kd = None if kp is None else kp.to(dev)
    vd = None if vp is None else vp.to(dev)
    out = ops.varlen_attention(
        q.to(dev), None if k is None else k.to(dev), None if v is None else v.to(dev),
        cu_q.to(dev), cu_k.to(dev), max(q_lens), max(k_lens), scale=scale, causal=c["causal"],
        k_cache=kd, v_cache=vd, block_tables=None if table is None else table.to(dev),
        slot_mapping=None if slots is None else slots.to(dev), layout=layout,
        k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    if slots is not None:
        ek, ev = oracle.store_kvcache(k, v, kp, vp, slots, layout=layout, k_scale=ks, v_scale=vs)
        if c["fp8"]:
            assert torch.equal(kd.cpu().view(torch.uint8), ek.view(torch.uint8))
            assert torch.equal(vd.cpu().view(torch.uint8), ev.view(torch.uint8))
        else:
            assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.varlen_attention(q, k, v, cu_q, cu_k, scale, c["causal"], k_cache=kp,
                                  v_cache=vp, block_tables=table, layout=layout,
                                  k_scale=ks, v_scale=vs)
    if total_q:
        diff = (out.float().cpu() - ref.float()).abs()
        at = int(diff.argmax())
        assert diff.max().item() <= 2e-2, (
            f"case {seed}: max error {diff.max().item():.3e} where |ref| = "
            f"{ref.flatten()[at].abs().item():.3f}")
    if seed % 4 == 0 and total_q:
        # The launch captured in a HIP graph (the persistent schedule reads the
        # lengths on the device, and nothing syncs or allocates).  A replay gives
        # the eager output bit for bit (a fused store writes the same rows
        # again); after new query values are written into the captured buffer,
        # a replay gives what an eager call on them gives.
        qd = q.to(dev)
        call = dict(
            k=None if k is None else k.to(dev), v=None if v is None else v.to(dev),
            cu_seqlens_q=cu_q.to(dev), cu_seqlens_k=cu_k.to(dev), max_seqlen_q=max(q_lens),
            max_seqlen_k=max(k_lens), scale=scale, causal=c["causal"], k_cache=kd, v_cache=vd,
            block_tables=None if table is None else table.to(dev),
            slot_mapping=None if slots is None else slots.to(dev), layout=layout,
            k_scale=ks, v_scale=vs)
        gout = torch.empty_like(out)
        stream = torch.cuda.Stream(dev)
        with torch.cuda.stream(stream):
            ops.varlen_attention(qd, out=gout, **call)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.varlen_attention(qd, out=gout, **call)
        gout.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, out), f"case {seed}: graph replay differs from eager"
        q2 = torch.randn(q.shape, generator=gen).to(dt).to(dev)
        want = ops.varlen_attention(q2, **call)
        qd.copy_(q2)
        gout.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, want), f"case {seed}: replay on new queries differs from eager"
        del graph
