"""Paged decode on the GPU: non-finite values in slots that are not attended,
and the TTS kernel's kernel_seq_len / kernel_page_count bounds.

* Slots past a context's end inside its last block, and masked slots, may
  hold anything in a reused pool, including NaN and infinities (an fp16
  overflow, a stale request).  The reference's Triton kernel loads such rows
  as 0 (qwen_tts_paged_attention.py:245-265), so they never reach the output;
  here both decode kernels (matrix-core: 16-bit K/V with 16-aligned blocks;
  general: fp32 or other block sizes), split and unsplit, must give a finite
  output equal to the oracle's.
* paged_attention_decode's kernel_seq_len and kernel_page_count bound the
  attended tokens and table columns as the Triton kernel's MAX_SEQ_LEN and
  num_page_slots do (:223-241), while the current row is written at
  seq_len - 1 through the table's own entry (:182-221).

Tolerances (max-abs against the oracle in fp32): 1e-5 fp32, 2e-2 bf16/fp16;
pools bit-exact.
"""

import math
import zlib

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops
from voiceagent_amd.agent import paged_attention_decode

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
HQ, HKV, D = 16, 8, 128


def _err(out, ref):
    return (out.float().cpu() - ref.float()).abs().max().item()


def _bits(t):
    # raw bit patterns: NaN-holding pools compare exactly
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def _tables(lens, bs, nb, gen):
    need = [math.ceil(n / bs) for n in lens]
    perm = torch.randperm(nb, generator=gen).tolist()
    width = max(need) + 2
    rows, cur = [], 0
    for n in need:
        rows.append(perm[cur:cur + n] + [-1] * (width - n))
        cur += n
    return torch.tensor(rows, dtype=torch.int32)


def _poison(pool, layout, block, off, value):
    if layout == ops.LAYOUT_NHD:
        pool[block, off] = value
    else:
        pool[block, :, off] = value


@pytest.mark.parametrize(
    "dtype,bs,layout,bound,masked,fused",
    [
        (torch.bfloat16, 16, ops.LAYOUT_NHD, "exact", False, False),   # matrix-core, unsplit
        (torch.bfloat16, 16, ops.LAYOUT_NHD, "graph", False, True),    # matrix-core, split
        (torch.bfloat16, 32, ops.LAYOUT_HND, "exact", True, True),     # matrix-core, key mask
        (torch.float16, 16, ops.LAYOUT_HND, "graph", True, False),     # matrix-core, mask, split
        (torch.float32, 16, ops.LAYOUT_NHD, "exact", True, False),     # general kernel
        (torch.bfloat16, 8, ops.LAYOUT_NHD, "graph", True, True),      # general, split
        (torch.float32, 24, ops.LAYOUT_HND, "graph", False, True),     # general, split
    ],
)
def test_nonfinite_stale_and_masked_slots_do_not_leak(dev, dtype, bs, layout, bound, masked,
                                                      fused):
    gen = torch.Generator().manual_seed(zlib.crc32(repr((dtype, bs, layout, bound)).encode()))
    lens = [1, 5, 17, 31, 100, 257, 611, 1000]
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    B = len(lens)
    table = _tables(lens, bs, nb, gen)
    shape = (nb, bs, HKV, D) if layout == ops.LAYOUT_NHD else (nb, HKV, bs, D)
    kp = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    vp = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    bad = [float("nan"), float("inf"), float("-inf")]
    # Slots past each context's end inside its last block.
    for b, n in enumerate(lens):
        last = table[b, (n - 1) // bs].item()
        for off in range((n - 1) % bs + 1, bs):
            _poison(kp, layout, last, off, bad[off % 3])
            _poison(vp, layout, last, off, bad[(off + 1) % 3])
    valid = None
    if masked:
        width = max(lens) + 5
        valid = torch.rand(B, width, generator=gen) < 0.8
        for b, n in enumerate(lens):
            for t in range(n):
                if not valid[b, t]:
                    blk = table[b, t // bs].item()
                    _poison(kp, layout, blk, t % bs, bad[t % 3])
                    _poison(vp, layout, blk, t % bs, bad[(t + 2) % 3])
    q = torch.randn(B, HQ, D, generator=gen).to(dtype)
    nk = (torch.randn(B, HKV, D, generator=gen) * 0.5).to(dtype) if fused else None
    nv = (torch.randn(B, HKV, D, generator=gen) * 0.5).to(dtype) if fused else None
    lens_t = torch.tensor(lens, dtype=torch.int32)
    k0, v0 = kp.clone(), vp.clone()
    kd, vd = kp.to(dev), vp.to(dev)
    max_seq_len = max(lens) if bound == "exact" else 65536
    print(f"nonfinite case {dtype} bs={bs} {layout} {bound} masked={masked} fused={fused}",
          flush=True)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lens_t.to(dev),
                           max_seq_len=max_seq_len, scale=D ** -0.5, layout=layout,
                           valid_mask=None if valid is None else valid.to(dev),
                           new_k=None if nk is None else nk.to(dev),
                           new_v=None if nv is None else nv.to(dev))
    torch.cuda.synchronize()
    if fused:
        k0, v0 = oracle.write_current_kv(k0, v0, table, lens_t, nk, nv, layout=layout)
        assert torch.equal(_bits(kd.cpu()), _bits(k0)) and torch.equal(_bits(vd.cpu()), _bits(v0))
    ref = oracle.paged_decode(q, k0, v0, table, lens_t, D ** -0.5, layout=layout,
                              valid_mask=valid)
    assert torch.isfinite(ref).all()
    assert torch.isfinite(out.float()).all()
    assert _err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float32, 16),
                                        (torch.bfloat16, 8)])
def test_tts_kernel_seq_len_and_page_count_bound_the_attention(dev, dtype, page):
    # Rows longer than kernel_seq_len attend only its first kernel_seq_len
    # tokens; table columns at or past kernel_page_count read page 0; the
    # current row still lands at seq_len - 1 through the table's own entry.
    gen = torch.Generator().manual_seed(71 + page)
    hq, hkv, d = 16, 8, 128
    lens = [40, 97, 150, 160, 33]
    kernel_seq_len = 128 if page == 16 else 96
    kernel_page_count = 6
    pages = sum(math.ceil(n / page) for n in lens) + 4
    need = max(math.ceil(n / page) for n in lens)
    perm = torch.randperm(pages, generator=gen)
    table = torch.full((len(lens), need), -1, dtype=torch.long)
    cur = 0
    for b, n in enumerate(lens):
        m = math.ceil(n / page)
        table[b, :m] = perm[cur:cur + m]
        cur += m
    kp = (torch.randn(pages, hkv, page, d, generator=gen) * 0.5).to(dtype)
    vp = (torch.randn(pages, hkv, page, d, generator=gen) * 0.5).to(dtype)
    q = torch.randn(len(lens), hq, 1, d, generator=gen).to(dtype)
    nk = (torch.randn(len(lens), hkv, 1, d, generator=gen) * 0.5).to(dtype)
    nv = (torch.randn(len(lens), hkv, 1, d, generator=gen) * 0.5).to(dtype)
    valid = torch.rand(len(lens), kernel_seq_len, generator=gen) < 0.9
    seq = torch.tensor(lens, dtype=torch.long)
    kd, vd = kp.to(dev), vp.to(dev)
    print(f"tts bounds {dtype} page={page} kernel_seq_len={kernel_seq_len}", flush=True)
    out = paged_attention_decode(q.to(dev), kd, vd, table.to(dev), seq.to(dev), valid.to(dev),
                                 new_key=nk.to(dev), new_value=nv.to(dev),
                                 kernel_seq_len=kernel_seq_len,
                                 kernel_page_count=kernel_page_count, validate=False)
    torch.cuda.synchronize()
    ek, ev = oracle.write_current_kv(kp, vp, table, seq, nk[:, :, 0], nv[:, :, 0])
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q[:, :, 0], ek, ev, table, seq, d ** -0.5, layout=oracle.HND,
                              valid_mask=valid, key_limit=kernel_seq_len,
                              table_read_width=kernel_page_count)
    assert _err(out[:, :, 0], ref) <= TOL[dtype]
    # the bounds matter for these rows: without them the result differs
    free = oracle.paged_decode(q[:, :, 0], ek, ev, table, seq, d ** -0.5, layout=oracle.HND,
                               valid_mask=valid)
    assert (free - ref).abs().max().item() > 10 * TOL[dtype]
