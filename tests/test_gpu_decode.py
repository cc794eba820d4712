"""Paged decode on the GPU against the CPU oracle.

Tolerances (max-abs): 1e-5 for fp32 inputs, 2e-2 for bf16/fp16 inputs, both
against the oracle evaluated in fp32 on the same inputs.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import _native, ops, workloads
from voiceagent_amd.agent import PagedAttentionKernelError, paged_attention_decode

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _err(out, ref):
    return (out.float().cpu() - ref.float()).abs().max().item()


def _oracle_for(batch, layer=0):
    return oracle.paged_decode(batch.q.cpu(), batch.k_pools[layer].cpu(),
                               batch.v_pools[layer].cpu(), batch.block_tables.cpu(),
                               batch.context_lens.cpu(), batch.scale)


def test_cfg1_fp32_matches_golden_and_oracle(dev):
    lens = workloads.cfg1_lens(0)
    b = workloads.make_decode_batch(lens, num_blocks=128, dtype=torch.float32, device=dev, seed=0)
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                           max_seq_len=b.max_seq_len, scale=b.scale)
    g = np.load(os.path.join(GOLDEN, "cfg1_decode.npz"))
    ref = _oracle_for(b)
    assert _err(out, ref) <= 1e-5
    assert np.abs(out.cpu().double().numpy() - g["expected"]).max() <= 1e-5
    # cu_seqlens_k form (the engine's AttentionContext) gives identical bits
    out2 = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                            lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale)
    assert torch.equal(out, out2)


def test_cfg2_bf16_single_layer(dev):
    lens = workloads.cfg2_lens(0)
    b = workloads.make_decode_batch(lens, num_blocks=4096, dtype=torch.bfloat16, kv_std=0.5,
                                    device=dev, seed=0)
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                           lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale)
    assert _err(out, _oracle_for(b)) <= 2e-2


@pytest.mark.parametrize("split", [64, 128, 320, 1024])
def test_split_size_does_not_change_result(dev, split):
    lens = [1, 15, 16, 17, 63, 64, 65, 700, 1500]
    b = workloads.make_decode_batch(lens, num_blocks=256, dtype=torch.float32, device=dev, seed=4)
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                           max_seq_len=b.max_seq_len, scale=b.scale, split_tokens=split)
    assert _err(out, _oracle_for(b)) <= 1e-5


@pytest.mark.parametrize("variant", ["single", "batch8"])
def test_long_context_split_and_merge(dev, variant):
    lens = workloads.cfg5_lens(variant)
    nb = sum((n + 15) // 16 for n in lens) + 16
    b = workloads.make_decode_batch(lens, num_blocks=nb, dtype=torch.bfloat16, device=dev, seed=5)
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                           max_seq_len=b.max_seq_len, scale=b.scale)
    assert _err(out, _oracle_for(b)) <= 2e-2
    # repeated launches reuse the partial workspace
    out2 = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                            max_seq_len=b.max_seq_len, scale=b.scale)
    assert torch.equal(out, out2)


def test_max_seq_len_underestimate_still_attends_everything(dev):
    lens = [300, 1000]
    b = workloads.make_decode_batch(lens, num_blocks=128, dtype=torch.float32, device=dev, seed=6)
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                           max_seq_len=200, scale=b.scale, split_tokens=64)
    assert _err(out, _oracle_for(b)) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 8, 64), (32, 8, 128), (16, 2, 256),
                                      (14, 14, 64)])
def test_geometries(dev, dtype, hq, hkv, d):
    g = torch.Generator().manual_seed(hq * 1000 + d)
    lens = [5, 77, 300]
    nb, bs = 64, 16
    kp = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    vp = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    q = torch.randn(3, hq, d, generator=g).to(dtype)
    table = torch.stack([torch.randperm(nb, generator=g)[:20] for _ in lens]).to(torch.int32)
    lt = torch.tensor(lens, dtype=torch.int32)
    scale = d ** -0.5
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=300, scale=scale)
    ref = oracle.paged_decode(q, kp, vp, table, lt, scale)
    assert _err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("bs", [1, 2, 8, 32, 48])
def test_block_sizes(dev, bs):
    g = torch.Generator().manual_seed(bs)
    lens = [3, 40, 130]
    nb = 400
    kp = torch.randn(nb, bs, 8, 128, generator=g)
    vp = torch.randn(nb, bs, 8, 128, generator=g)
    q = torch.randn(3, 16, 128, generator=g)
    width = (130 + bs - 1) // bs
    table = torch.stack([torch.randperm(nb, generator=g)[:width] for _ in lens]).to(torch.int64)
    lt = torch.tensor(lens, dtype=torch.int64)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=130, scale=0.1)
    assert _err(out, oracle.paged_decode(q, kp, vp, table, lt, 0.1)) <= 1e-5


def test_zero_length_and_fully_masked_rows_are_zero(dev):
    g = torch.Generator().manual_seed(9)
    kp = torch.randn(16, 16, 8, 128, generator=g)
    vp = torch.randn(16, 16, 8, 128, generator=g)
    q = torch.randn(3, 16, 128, generator=g)
    table = torch.tensor([[0, 1], [2, 3], [4, 5]], dtype=torch.int32)
    lt = torch.tensor([0, 20, 7], dtype=torch.int32)
    valid = torch.ones(3, 32, dtype=torch.bool)
    valid[2, :] = False
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lt.to(dev),
                           max_seq_len=20, scale=0.1, valid_mask=valid.to(dev)).cpu()
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    ref = oracle.paged_decode(q, kp, vp, table, lt, 0.1, valid_mask=valid)
    assert _err(out, ref) <= 1e-5


def test_invalid_block_ids_are_masked_not_dereferenced(dev):
    g = torch.Generator().manual_seed(10)
    kp = torch.randn(8, 16, 8, 128, generator=g)
    vp = torch.randn(8, 16, 8, 128, generator=g)
    q = torch.randn(1, 16, 128, generator=g)
    table = torch.tensor([[1, 999999, 2]], dtype=torch.int32)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                           torch.tensor([40], dtype=torch.int32, device=dev),
                           max_seq_len=40, scale=0.1)
    keep = torch.ones(1, 40, dtype=torch.bool)
    keep[0, 16:32] = False
    ref = oracle.paged_decode(q, kp, vp, torch.tensor([[1, 0, 2]]), torch.tensor([40]), 0.1,
                              valid_mask=keep)
    assert _err(out, ref) <= 1e-5


def test_engine_fused_store_matches_store_then_attend(dev):
    lens = workloads.cfg2_lens(1)
    b = workloads.make_decode_batch(lens, num_blocks=2048, dtype=torch.bfloat16, kv_std=0.5,
                                    device=dev, seed=11)
    k0, v0 = b.k_pools[0].cpu(), b.v_pools[0].cpu()
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                           lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale,
                           new_k=b.new_k, new_v=b.new_v, new_slots=b.slot_mapping)
    ek, ev = oracle.store_kvcache(b.new_k.cpu(), b.new_v.cpu(), k0, v0, b.slot_mapping.cpu())
    torch.cuda.synchronize()
    assert torch.equal(b.k_pools[0].cpu(), ek) and torch.equal(b.v_pools[0].cpu(), ev)
    ref = oracle.paged_decode(b.q.cpu(), ek, ev, b.block_tables.cpu(), b.context_lens.cpu(),
                              b.scale)
    assert _err(out, ref) <= 2e-2
    # padding rows of a graph bucket: slot -1 skips the write, k_len 1 reads block 0
    slots = b.slot_mapping.clone()
    slots[-3:] = -1
    before = b.k_pools[0].clone()
    ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                     lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale,
                     new_k=b.new_k * 2, new_v=b.new_v * 2, new_slots=slots)
    torch.cuda.synchronize()
    changed = (b.k_pools[0] != before).flatten(1).any(1).nonzero().flatten().tolist()
    expected_blocks = sorted({int(s) // 16 for s in slots.tolist() if s >= 0})
    assert changed == expected_blocks


def test_engine_fused_store_with_contiguous_k_and_strided_v(dev):
    # The engine's decode inputs: k comes out of k_norm (contiguous) while v
    # stays a view of the fused qkv row (row stride (Hq + 2 Hkv) D,
    # models/qwen3.py:44-48).
    lens = workloads.cfg2_lens(2)
    b = workloads.make_decode_batch(lens, num_blocks=2048, dtype=torch.bfloat16, kv_std=0.5,
                                    device=dev, seed=12)
    B = len(lens)
    qkv = torch.zeros(B, (16 + 2 * 8) * 128, dtype=torch.bfloat16, device=dev)
    v_view = qkv[:, (16 + 8) * 128:].view(B, 8, 128)
    v_view.copy_(b.new_v)
    k0, v0 = b.k_pools[0].cpu(), b.v_pools[0].cpu()
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                           lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale,
                           new_k=b.new_k.contiguous(), new_v=v_view, new_slots=b.slot_mapping)
    ek, ev = oracle.store_kvcache(b.new_k.cpu(), b.new_v.cpu(), k0, v0, b.slot_mapping.cpu())
    torch.cuda.synchronize()
    assert v_view.stride(0) == 4096 and b.new_k.contiguous().stride(0) == 1024
    assert torch.equal(b.k_pools[0].cpu(), ek) and torch.equal(b.v_pools[0].cpu(), ev)
    ref = oracle.paged_decode(b.q.cpu(), ek, ev, b.block_tables.cpu(), b.context_lens.cpu(),
                              b.scale)
    assert _err(out, ref) <= 2e-2


def _tts_case(dev, d=128, hq=16, hkv=8, page=2, dtype=torch.float32, seed=17):
    # The reference fixture's structure (tests/test_qwen_tts_paged_attention_kernel.py:16-35),
    # scaled to a head_dim the kernel supports: two requests on disjoint pages with
    # different lengths and a left-padded prompt token.
    g = torch.Generator().manual_seed(seed)
    table = torch.tensor([[3, 5, 0], [1, 7, 2]], dtype=torch.long)
    lens = torch.tensor([3, 5], dtype=torch.long)
    valid = torch.tensor([[True, True, True, False, False], [False, True, True, True, True]])
    kp = torch.zeros(8, hkv, page, d)
    vp = torch.zeros(8, hkv, page, d)
    for p in (3, 5, 1, 7, 2):
        kp[p] = torch.randn(hkv, page, d, generator=g)
        vp[p] = torch.randn(hkv, page, d, generator=g)
    q = torch.randn(2, hq, 1, d, generator=g)
    nk = torch.randn(2, hkv, 1, d, generator=g)
    nv = torch.randn(2, hkv, 1, d, generator=g)
    cast = lambda t: t.to(dtype)  # noqa: E731
    return [cast(x) for x in (q, kp, vp)] + [table, lens, valid] + [cast(nk), cast(nv)]


def test_tts_api_matches_oracle_with_mask(dev):
    q, kp, vp, table, lens, valid, _, _ = _tts_case(dev)
    out = paged_attention_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                                 lens.to(dev), valid.to(dev))
    ref = oracle.paged_decode(q[:, :, 0], kp, vp, table, lens, 128 ** -0.5, layout=oracle.HND,
                              valid_mask=valid)
    assert out.shape == q.shape
    assert _err(out[:, :, 0], ref) <= 1e-5


def test_tts_fused_write_matches_reference_order(dev):
    # test_qwen_tts_paged_attention_kernel.py:144-177 and :349-390: pools equal the
    # expected pools, output equals attention over them.
    q, kp, vp, table, lens, valid, nk, nv = _tts_case(dev, dtype=torch.bfloat16)
    ek, ev = oracle.write_current_kv(kp, vp, table, lens, nk[:, :, 0], nv[:, :, 0])
    kd, vd = kp.to(dev), vp.to(dev)
    out = paged_attention_decode(q.to(dev), kd, vd, table.to(dev), lens.to(dev), valid.to(dev),
                                 new_key=nk.to(dev), new_value=nv.to(dev), validate=False,
                                 kernel_seq_len=128, kernel_page_count=64)
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q[:, :, 0], ek, ev, table, lens, 128 ** -0.5, layout=oracle.HND,
                              valid_mask=valid)
    assert _err(out[:, :, 0], ref) <= 2e-2


@pytest.mark.parametrize("B", [6, 40])
def test_tts_api_page16_mask_and_fused_write(dev, B):
    # The TTS caller's shape of a tick (qwen_tts_outer_varlen.py:392-447): HND
    # pool with 16-token pages, int64 page table padded with -1, a key mask
    # padded with True up to kernel_seq_len, and the current rows written in
    # the same launch.  16-token pages take the matrix-core kernel; B=6 splits
    # contexts into partitions, B=40 runs one partition per (request, kv head).
    g = torch.Generator().manual_seed(70 + B)
    page, hq, hkv, d = 16, 16, 8, 128
    lens = torch.randint(1, 520, (B,), generator=g)
    need = [(int(n) + page - 1) // page for n in lens]
    pages = sum(need) + 3
    perm = torch.randperm(pages, generator=g).tolist()
    width = max(need) + 2
    table = torch.full((B, width), -1, dtype=torch.long)
    cur = 0
    for i, m in enumerate(need):
        table[i, :m] = torch.tensor(perm[cur:cur + m])
        cur += m
    kp = (torch.randn(pages, hkv, page, d, generator=g) * 0.5).to(torch.bfloat16)
    vp = torch.randn(pages, hkv, page, d, generator=g).to(torch.bfloat16)
    q = torch.randn(B, hq, 1, d, generator=g).to(torch.bfloat16)
    nk = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)
    nv = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)
    kernel_seq_len = 640
    valid = torch.ones(B, kernel_seq_len, dtype=torch.bool)
    valid[:, :520] = torch.rand(B, 520, generator=g) < 0.85
    ek, ev = oracle.write_current_kv(kp, vp, table, lens, nk[:, :, 0], nv[:, :, 0])
    kd, vd = kp.to(dev), vp.to(dev)
    out = paged_attention_decode(q.to(dev), kd, vd, table.to(dev), lens.to(dev), valid.to(dev),
                                 new_key=nk.to(dev), new_value=nv.to(dev), validate=False,
                                 kernel_seq_len=kernel_seq_len, kernel_page_count=width + 4)
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q[:, :, 0], ek, ev, table, lens, d ** -0.5, layout=oracle.HND,
                              valid_mask=valid)
    assert _err(out[:, :, 0], ref) <= 2e-2


def test_tts_known_answer_integer_values(dev):
    # test_qwen_tts_outer_varlen_attention.py:54-66 at head_dim 64: constant K/V -> exact.
    kp = torch.zeros(8, 1, 2, 64)
    vp = torch.zeros(8, 1, 2, 64)
    kp[0:2], vp[0:2] = 1.0, 1.0
    kp[2:4], vp[2:4] = 9.0, 9.0
    table = torch.tensor([[0, 1], [2, 3]])
    out = paged_attention_decode(torch.ones(2, 1, 1, 64, device=dev), kp.to(dev), vp.to(dev),
                                 table.to(dev), torch.tensor([4, 4], device=dev))
    out = out.cpu()
    assert torch.all(out[0] == 1.0) and torch.all(out[1] == 9.0)


def test_tts_reference_fixture_on_the_small_head_kernel(dev):
    # The reference's own fixture (tests/test_qwen_tts_paged_attention_kernel.py:16-57,
    # and the fused write of :144-177): HND pool of 2-token pages, head_dim 4, fp32,
    # GQA 2, a left-padded row.  Expected values: the committed float64 brute force
    # (tests/golden/brute.py); the fused pools bit-exact.
    g = np.load(os.path.join(GOLDEN, "tts_seed17.npz"))
    t = {k: torch.from_numpy(g[k]) for k in g.files}
    kd, vd = t["k_pool"].to(dev), t["v_pool"].to(dev)
    out = paged_attention_decode(t["q"].to(dev), kd, vd, t["page_table"].to(dev),
                                 t["seq_lens"].to(dev), t["valid"].to(dev))
    torch.cuda.synchronize()
    assert out.shape == (2, 4, 1, 4)
    assert (out[:, :, 0].double().cpu() - t["expected"]).abs().max().item() <= 1e-5
    assert torch.equal(kd.cpu(), t["k_pool"]) and torch.equal(vd.cpu(), t["v_pool"])
    kd, vd = t["k_pool"].to(dev), t["v_pool"].to(dev)
    out = paged_attention_decode(t["q"].to(dev), kd, vd, t["page_table"].to(dev),
                                 t["seq_lens"].to(dev), t["valid"].to(dev),
                                 new_key=t["new_key"].to(dev), new_value=t["new_value"].to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), t["k_pool_fused"]) and torch.equal(vd.cpu(), t["v_pool_fused"])
    assert (out[:, :, 0].double().cpu() - t["expected_fused"]).abs().max().item() <= 1e-5


@pytest.mark.parametrize(
    "dtype,d,hq,hkv,bs,layout,fused,bound",
    [
        (torch.float32, 1, 4, 2, 2, ops.LAYOUT_HND, False, "exact"),
        (torch.float32, 4, 6, 2, 1, ops.LAYOUT_NHD, True, "exact"),     # group 3, 1-token blocks
        (torch.bfloat16, 32, 8, 8, 5, ops.LAYOUT_HND, True, "limit"),   # current row detached
        (torch.float16, 96, 12, 4, 16, ops.LAYOUT_NHD, False, "exact"),  # head_dim 96, group 3
        (torch.bfloat16, 128, 6, 2, 16, ops.LAYOUT_NHD, True, "exact"),  # head_dim 128, group 3
        (torch.float32, 160, 4, 1, 3, ops.LAYOUT_HND, False, "limit"),   # group 4, odd blocks
    ],
)
def test_small_head_kernel_matches_oracle(dev, dtype, d, hq, hkv, bs, layout, fused, bound):
    # Shapes the vector kernels do not take run on the small-head kernel: any
    # head_dim, any group, any block size, contexts past its 1024-key chunk,
    # a key mask, invalid block ids, the fused current row (in place, or
    # detached past key_limit), and the TTS read bounds.
    gen = torch.Generator().manual_seed(d * 131 + hq)
    lens = [1, 3, 17, 1030, 2500, 700]
    B = len(lens)
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + 6
    perm = torch.randperm(nb, generator=gen).tolist()
    width = max(need) + 1
    rows, cur = [], 0
    for n in need:
        rows.append(perm[cur:cur + n] + [-1] * (width - n))
        cur += n
    table = torch.tensor(rows, dtype=torch.int32)
    table[4, 3] = nb + 7  # an invalid block id inside a context: those tokens are masked
    shape = (nb, bs, hkv, d) if layout == ops.LAYOUT_NHD else (nb, hkv, bs, d)
    kp = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    vp = torch.randn(shape, generator=gen).to(dtype)
    q = torch.randn(B, hq, d, generator=gen).to(dtype)
    valid = torch.rand(B, 2600, generator=gen) < 0.85
    valid[:, 0] = True
    nk = (torch.randn(B, hkv, d, generator=gen) * 0.5).to(dtype) if fused else None
    nv = torch.randn(B, hkv, d, generator=gen).to(dtype) if fused else None
    lens_t = torch.tensor(lens, dtype=torch.int64)
    key_limit = 1600 if bound == "limit" else 0
    read_width = (1500 // bs) if bound == "limit" else 0
    kd, vd = kp.to(dev), vp.to(dev)
    scale = d ** -0.5
    print(f"small head {dtype} d={d} hq={hq} hkv={hkv} bs={bs} {layout} fused={fused} {bound}",
          flush=True)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lens_t.to(dev),
                           max_seq_len=max(lens), scale=scale, layout=layout,
                           valid_mask=valid.to(dev),
                           new_k=None if nk is None else nk.to(dev),
                           new_v=None if nv is None else nv.to(dev),
                           key_limit=key_limit, table_read_width=read_width)
    torch.cuda.synchronize()
    k0, v0 = kp, vp
    if fused:
        k0, v0 = oracle.write_current_kv(kp, vp, table, lens_t, nk, nv, layout=layout)
    assert torch.equal(kd.cpu(), k0) and torch.equal(vd.cpu(), v0)
    # The oracle sees the invalid block as a valid one whose tokens are masked.
    table_o, valid_o = table.clone(), valid.clone()
    table_o[4, 3] = 0
    valid_o[4, 3 * bs:4 * bs] = False
    ref = oracle.paged_decode(q, k0, v0, table_o, lens_t, scale, layout=layout,
                              valid_mask=valid_o, key_limit=key_limit or None,
                              table_read_width=read_width or None)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert (out.float().cpu() - ref).abs().max().item() <= tol


def test_constant_values_property_at_cfg2_scale(dev):
    lens = workloads.cfg2_lens(2)
    b = workloads.make_decode_batch(lens, num_blocks=4096, dtype=torch.bfloat16, device=dev,
                                    seed=12)
    vconst = torch.full_like(b.v_pools[0], 0.375)
    out = ops.paged_decode(b.q, b.k_pools[0], vconst, b.block_tables, b.context_lens,
                           max_seq_len=b.max_seq_len, scale=b.scale)
    assert torch.all(out == 0.375)


def test_graph_capture_replays_match_eager(dev):
    lens = workloads.cfg2_lens(3)
    b = workloads.make_decode_batch(lens, num_blocks=4096, dtype=torch.bfloat16, device=dev,
                                    seed=13)
    max_len = 1024
    cu = b.cu_seqlens_k.clone()
    out = torch.empty_like(b.q)

    def step():
        ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, cu,
                         lens_cumulative=True, max_seq_len=max_len, scale=b.scale, out=out)

    step()  # eager warm-up (256 pairs run unsplit: no workspace on either stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(14)
    for rep in range(4):
        new_lens = torch.randint(1, 600, (len(lens),), generator=g)
        new_lens = torch.minimum(new_lens, torch.tensor(b.lens_list))
        cu.copy_(torch.cat([torch.zeros(1, dtype=torch.long), new_lens.cumsum(0)]).to(cu))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, cu,
                                 lens_cumulative=True, max_seq_len=max_len, scale=b.scale)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), rep
        ref = oracle.paged_decode(b.q.cpu(), b.k_pools[0].cpu(), b.v_pools[0].cpu(),
                                  b.block_tables.cpu(), new_lens, b.scale)
        assert _err(got, ref) <= 2e-2


def test_workspace_reuse_across_batch_sizes(dev):
    # Regression: launches with different (num_seqs x num_kv_heads) share the
    # partial workspace, whose layout depends on the batch; leftover partials of
    # an earlier batch must never leak into a later one.
    for it, B in enumerate([3, 17, 32, 9, 32, 24]):
        g = torch.Generator().manual_seed(200 + it)
        lens = torch.randint(20, 700, (B,), generator=g).tolist()
        b = workloads.make_decode_batch(lens, num_blocks=2048, dtype=torch.bfloat16, kv_std=0.5,
                                        device=dev, seed=it)
        out = torch.full_like(b.q, float("nan"))
        ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                         lens_cumulative=True, max_seq_len=b.max_seq_len, scale=b.scale, out=out)
        assert _err(out, _oracle_for(b)) <= 2e-2, (it, B)


def test_split_merge_with_many_pairs(dev):
    # An explicit split over more than 65536 (sequence, kv head) pairs: the
    # merge grid's second dimension runs to 1040 sequences.  The sequences
    # share a small pool through their block tables.
    B, hkv, d, bs, nb = 1040, 64, 64, 16, 64
    g = torch.Generator().manual_seed(33)
    lens = torch.randint(1, 300, (B,), generator=g)
    lens[:4] = torch.tensor([1, 129, 256, 299])
    width = 19
    table = torch.randint(0, nb, (B, width), generator=g, dtype=torch.int32)
    kp = (torch.randn(nb, bs, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    vp = torch.randn(nb, bs, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(B, hkv, d, generator=g).to(torch.bfloat16)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lens.to(dev),
                           max_seq_len=300, scale=d ** -0.5, split_tokens=128)
    ref = oracle.paged_decode(q, kp, vp, table, lens, d ** -0.5)
    assert B * hkv > 65536
    assert _err(out, ref) <= 2e-2


@pytest.mark.parametrize("max_seq_len", [40960, 65536])
def test_longest_context_with_fused_store(dev, max_seq_len):
    # Qwen3's longest position (max_position_embeddings 40960) in one sequence
    # beside short ones, the current rows stored in the same launch; with the
    # exact maximum and with the bound a decode graph captured at 65536 passes.
    lens = [40960, 1, 17, 300]
    nb = sum((n + 15) // 16 for n in lens) + 8
    b = workloads.make_decode_batch(lens, num_blocks=nb, dtype=torch.bfloat16, kv_std=0.5,
                                    device=dev, seed=40)
    k0, v0 = b.k_pools[0].cpu(), b.v_pools[0].cpu()
    out = ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.context_lens,
                           max_seq_len=max_seq_len, scale=b.scale, new_k=b.new_k,
                           new_v=b.new_v, new_slots=b.slot_mapping)
    ek, ev = oracle.store_kvcache(b.new_k.cpu(), b.new_v.cpu(), k0, v0, b.slot_mapping.cpu())
    torch.cuda.synchronize()
    assert torch.equal(b.k_pools[0].cpu(), ek) and torch.equal(b.v_pools[0].cpu(), ev)
    ref = oracle.paged_decode(b.q.cpu(), ek, ev, b.block_tables.cpu(), b.context_lens.cpu(),
                              b.scale)
    assert _err(out, ref) <= 2e-2


def test_concurrent_decodes_on_two_streams_keep_their_partials(dev):
    # Two split-context decodes in flight at once on two streams (an ASR
    # decode beside a TTS decode, say): each stream has its own partials
    # workspace, so neither reads the other's.
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    batches = [workloads.make_decode_batch([900, 1200, 700], num_blocks=512, dtype=torch.bfloat16,
                                           kv_std=0.5, device=dev, seed=60 + i) for i in range(2)]
    refs = [_oracle_for(b) for b in batches]
    outs = [torch.empty_like(b.q) for b in batches]
    torch.cuda.synchronize()
    for rep in range(20):
        for s, b, o in zip(streams, batches, outs):
            with torch.cuda.stream(s):
                ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables,
                                 b.context_lens, max_seq_len=b.max_seq_len, scale=b.scale, out=o)
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert _err(o, r) <= 2e-2, rep
    ws = [ops._WORKSPACES[(dev.index or 0, s.cuda_stream)] for s in streams]
    assert ws[0].data_ptr() != ws[1].data_ptr()
