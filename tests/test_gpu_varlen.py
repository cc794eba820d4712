"""Varlen attention (causal prefill, block-diagonal encoder) on the GPU
against the CPU oracle.  bf16/fp16 inputs: max-abs error <= 2e-2 against the
oracle evaluated in fp32 on the same inputs; stores are bit-exact."""

import math

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops, workloads
from voiceagent_amd.layers import (AttentionContext, PagedAttention, VarlenSelfAttention,
                                   attention_context)

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _err(out, ref):
    return (out.float().cpu() - ref.float()).abs().max().item()


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    return cu


def test_cfg3_causal_packed(dev):
    b = workloads.make_varlen_batch(workloads.cfg3_lens(0), 16, 8, 128, causal=True, seed=0)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=True)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, True)
    assert _err(out, ref) <= TOL


def test_cfg3_full_size_paged_with_fused_store(dev):
    # The launch bench.py times for config 3: 32 prompts U[50, 450], GQA 16/8,
    # head_dim 128, keys from k/v with the store fused into a block-16 pool
    # (varlen_attention_kernel<bf16, 128, 2, causal, paged>), over shuffled
    # block tables padded with -1.
    lens = workloads.cfg3_lens(0)
    b = workloads.make_varlen_batch(lens, 16, 8, 128, causal=True, seed=31)
    bs = 16
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + 8
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(32)).tolist()
    rows, cur, slots = [], 0, []
    for n, m in zip(lens, need):
        rows.append(perm[cur:cur + m] + [-1] * (max(need) - m))
        slots += [perm[cur + p // bs] * bs + p % bs for p in range(n)]
        cur += m
    table = torch.tensor(rows, dtype=torch.int32)
    slots = torch.tensor(slots, dtype=torch.int32)
    gen = torch.Generator().manual_seed(33)
    kp = torch.randn(nb, bs, 8, 128, generator=gen).to(torch.bfloat16)
    vp = torch.randn(nb, bs, 8, 128, generator=gen).to(torch.bfloat16)
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=True, k_cache=kd, v_cache=vd, block_tables=table.to(dev),
                               slot_mapping=slots.to(dev))
    torch.cuda.synchronize()
    ek, ev = oracle.store_kvcache(b.k, b.v, kp, vp, slots)
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, True)
    assert _err(out, ref) <= TOL
    # With the keys read back from the pool (k = None) the result is the same.
    out2 = ops.varlen_attention(b.q.to(dev), None, None, b.cu_seqlens.to(dev),
                                b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                                causal=True, k_cache=kd, v_cache=vd, block_tables=table.to(dev))
    assert torch.equal(out2, out)


def test_cfg4_encoder_block_diagonal(dev):
    wins = workloads.cfg4_windows(0)
    b = workloads.make_varlen_batch(wins, 14, 14, 64, causal=False, seed=1)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=False)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, False)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (14, 14, 64), (16, 4, 64), (32, 4, 128),
                                      (8, 8, 128)])
def test_ragged_lengths_and_geometries(dev, dtype, causal, hq, hkv, d):
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200]
    b = workloads.make_varlen_batch(lens, hq, hkv, d, causal=causal, dtype=dtype,
                                    seed=hq + d + int(causal))
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=causal)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, causal)
    assert _err(out, ref) <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d", [(14, 14, 64), (16, 8, 128), (16, 4, 64), (32, 4, 128)])
def test_one_query_block_per_sequence(dev, dtype, hq, hkv, d):
    # Non-causal launches whose sequences all fit one query block (128 rows /
    # group) take the instantiation that streams K/V non-temporally; ragged
    # lengths up to the block, one empty sequence.
    bq = 128 // (hq // hkv)
    lens = [n for n in (1, 3, bq // 2 - 1, bq // 2, bq // 2 + 1, bq - 1, bq, 7) if n > 0] + [0, bq]
    b = workloads.make_varlen_batch(lens, hq, hkv, d, causal=False, dtype=dtype, seed=hq + d)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=False)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, False)
    assert b.max_seqlen <= bq
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("hq,hkv,d", [(14, 14, 64), (16, 8, 128)])
def test_one_block_launch_many_items_per_workgroup(dev, hq, hkv, d):
    # Thousands of ragged one-block sequences (and empty ones): each
    # workgroup of the one-block launch runs many items, handing its K/V ring
    # from item to item, and most blocks end inside their 128 rows.  A guard
    # region after the output (where rows past the last sequence's end would
    # land) keeps its sentinel.
    bq = 128 // (hq // hkv)
    g = torch.Generator().manual_seed(hq + d)
    lens = torch.randint(0, bq + 1, (1500 if d == 64 else 900,), generator=g).tolist()
    lens[-1] = 1  # the last sequence's block is nearly all past its end
    b = workloads.make_varlen_batch(lens, hq, hkv, d, causal=False, seed=hq + d + 7)
    total = sum(lens)
    full = torch.full((total + bq, hq, d), 7.0, dtype=torch.bfloat16, device=dev)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=False, out=full[:total])
    torch.cuda.synchronize()
    assert bool((full[total:] == 7.0).all())
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, False)
    assert _err(out, ref) <= TOL


def test_one_block_launch_with_an_output_past_2_gib(dev):
    # An output view whose rows lie more than 2^31 bytes apart in total: the
    # row offsets need 64 bits.
    lens = [5, 104, 64, 1, 128]
    b = workloads.make_varlen_batch(lens, 14, 14, 64, causal=False, seed=3)
    total = sum(lens)
    row = 14 * 64
    step = (1 << 31) // (total - 1) // row * row + row  # token stride in elements
    big = torch.zeros(total * step, dtype=torch.bfloat16, device=dev)
    out = big.as_strided((total, 14, 64), (step, 64, 1))
    assert (total - 1) * step * 2 > (1 << 31)
    ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                         b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                         causal=False, out=out)
    torch.cuda.synchronize()
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, False)
    assert _err(out, ref) <= TOL
    del big


def test_persistent_rounds_long_prompts(dev):
    # 8 prompts of ~2000 tokens, 8 kv heads: each XCD lists 8 pairs x 32 blocks,
    # so every workgroup takes several items in snake order and the level walk
    # crosses 32 levels.
    lens = [2000, 1999, 1500, 2048, 1, 700, 1937, 64]
    b = workloads.make_varlen_batch(lens, 16, 8, 128, causal=True, seed=5)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=True)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, True)
    assert _err(out, ref) <= TOL


def test_persistent_many_pairs_item_refill(dev):
    # 400 sequences x 2 kv heads (group 8, 16-position blocks) = 800 pairs, 100
    # per XCD: the list holds every (pair, block), most blocks past their
    # sequence's end, and one 660-token sequence makes it 42 levels deep, so
    # a workgroup walks more than 64 rounds and refills its item ranges.
    g = torch.Generator().manual_seed(9)
    lens = torch.randint(1, 21, (400,), generator=g).tolist()
    lens[137] = 660
    b = workloads.make_varlen_batch(lens, 16, 2, 128, causal=True, seed=6)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=True)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, True)
    assert _err(out, ref) <= TOL


def _paged_prefill_case(seed=3, bs=16, nb=512, hq=16, hkv=8, d=128, slot_dtype=torch.int32,
                        spec=((0, 70), (32, 50), (160, 1), (48, 200), (0, 1), (17, 64))):
    g = torch.Generator().manual_seed(seed)
    # (cached prefix, new tokens) per sequence: prefix-cache hits and plain prompts
    q_lens = [n for _, n in spec]
    k_lens = [p + n for p, n in spec]
    kp = (torch.randn(nb, bs, hkv, d, generator=g)).to(torch.bfloat16)
    vp = (torch.randn(nb, bs, hkv, d, generator=g)).to(torch.bfloat16)
    width = max(math.ceil(k / bs) for k in k_lens)
    perm = torch.randperm(nb, generator=g).tolist()
    rows, cur = [], 0
    for k in k_lens:
        n = math.ceil(k / bs)
        rows.append(perm[cur:cur + n] + [-1] * (width - n))
        cur += n
    table = torch.tensor(rows, dtype=torch.int32)
    total = sum(q_lens)
    q = torch.randn(total, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(total, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(total, hkv, d, generator=g).to(torch.bfloat16)
    slots = []
    for s, (p, n) in enumerate(spec):
        for pos in range(p, p + n):
            slots.append(int(table[s, pos // bs]) * bs + pos % bs)
    return dict(kp=kp, vp=vp, table=table, q=q, k=k, v=v, cu_q=_cu(q_lens), cu_k=_cu(k_lens),
                max_q=max(q_lens), max_k=max(k_lens), slots=torch.tensor(slots, dtype=slot_dtype))


def test_paged_prefix_with_fused_store(dev):
    c = _paged_prefill_case()
    kd, vd = c["kp"].to(dev), c["vp"].to(dev)
    out = ops.varlen_attention(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), c["cu_q"].to(dev),
                               c["cu_k"].to(dev), c["max_q"], c["max_k"], scale=128 ** -0.5,
                               causal=True, k_cache=kd, v_cache=vd, block_tables=c["table"].to(dev),
                               slot_mapping=c["slots"].to(dev))
    ek, ev = oracle.store_kvcache(c["k"], c["v"], c["kp"], c["vp"], c["slots"])
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.varlen_attention(c["q"], c["k"], c["v"], c["cu_q"], c["cu_k"], 128 ** -0.5, True,
                                  k_cache=c["kp"], v_cache=c["vp"], block_tables=c["table"])
    assert _err(out, ref) <= TOL
    # every key from the pool (the reference's store-then-attend order)
    out2 = ops.varlen_attention(c["q"].to(dev), None, None, c["cu_q"].to(dev), c["cu_k"].to(dev),
                                c["max_q"], c["max_k"], scale=128 ** -0.5, causal=True,
                                k_cache=kd, v_cache=vd, block_tables=c["table"].to(dev))
    assert _err(out2, ref) <= TOL


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 8, 128), (32, 4, 128), (64, 8, 128),
                                      (14, 14, 64), (16, 2, 64)])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_fused_store_geometries(dev, hq, hkv, d, slot_dtype):
    # Every (group, head_dim) store split: rows of one block straddle key tiles
    # (unaligned prefixes), blocks shorter than a store step, and -1 slots
    # (padding rows) that must be skipped without touching the pool.
    spec = ((0, 70), (32, 50), (160, 1), (48, 200), (5, 3), (17, 129), (100, 17))
    c = _paged_prefill_case(seed=hq + d, hq=hq, hkv=hkv, d=d, slot_dtype=slot_dtype, spec=spec)
    c["slots"][::7] = -1
    kd, vd = c["kp"].to(dev), c["vp"].to(dev)
    out = ops.varlen_attention(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), c["cu_q"].to(dev),
                               c["cu_k"].to(dev), c["max_q"], c["max_k"], scale=d ** -0.5,
                               causal=True, k_cache=kd, v_cache=vd, block_tables=c["table"].to(dev),
                               slot_mapping=c["slots"].to(dev))
    ek, ev = oracle.store_kvcache(c["k"], c["v"], c["kp"], c["vp"], c["slots"])
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.varlen_attention(c["q"], c["k"], c["v"], c["cu_q"], c["cu_k"], d ** -0.5, True,
                                  k_cache=c["kp"], v_cache=c["vp"], block_tables=c["table"])
    assert _err(out, ref) <= TOL


def test_rows_without_visible_keys_are_zero(dev):
    # q_len > k_len with bottom-right alignment: the first q_len - k_len rows see nothing.
    g = torch.Generator().manual_seed(4)
    q = torch.randn(10, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(4, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(4, 8, 128, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0, 10], dtype=torch.int32)
    cu_k = torch.tensor([0, 4], dtype=torch.int32)
    out = ops.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cu_q.to(dev), cu_k.to(dev), 10, 4,
                               scale=0.1, causal=True).cpu()
    ref = oracle.varlen_attention(q, k, v, cu_q, cu_k, 0.1, True)
    assert torch.count_nonzero(out[:6]) == 0
    assert _err(out, ref) <= TOL


# ------------------------------------------------------------- layer drop-ins
def test_paged_attention_layer_prefill_then_decode(dev):
    """PagedAttention as the engine drives it: prefill writes the cache, then
    decode steps (fused store) read it; each step is checked against the oracle."""
    g = torch.Generator().manual_seed(5)
    bs, nb = 16, 256
    layer = PagedAttention(16, 128, 128 ** -0.5, 8)
    kv = torch.zeros(2, nb, bs, 8, 128, dtype=torch.bfloat16, device=dev)
    layer.k_cache, layer.v_cache = kv[0], kv[1]
    lens = [37, 90, 5]
    width = 12
    perm = torch.randperm(nb, generator=g).tolist()
    tables = [perm[i * width:(i + 1) * width] for i in range(3)]
    table_t = torch.tensor(tables, dtype=torch.int32, device=dev)
    total = sum(lens)
    q = torch.randn(total, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16)
    slots = [tables[s][p // bs] * bs + p % bs for s, n in enumerate(lens) for p in range(n)]
    cu = _cu(lens)
    ctx = AttentionContext(cu.to(dev), cu.to(dev), max(lens), max(lens),
                           torch.tensor(slots, dtype=torch.int32, device=dev), table_t)
    with attention_context(ctx):
        out = layer(q.to(dev), k.to(dev), v.to(dev))
    ref = oracle.varlen_attention(q, k, v, cu, cu, 128 ** -0.5, True)
    assert _err(out, ref) <= TOL
    kc, vc = oracle.store_kvcache(k, v, torch.zeros(nb, bs, 8, 128, dtype=torch.bfloat16),
                                  torch.zeros(nb, bs, 8, 128, dtype=torch.bfloat16),
                                  torch.tensor(slots))
    torch.cuda.synchronize()
    assert torch.equal(kv[0].cpu(), kc) and torch.equal(kv[1].cpu(), vc)
    for step in range(3):
        lens = [n + 1 for n in lens]
        qd = torch.randn(3, 16, 128, generator=g).to(torch.bfloat16)
        # the engine's v is a strided view of the fused qkv projection
        qkv = torch.randn(3, 32 * 128, generator=g).to(torch.bfloat16)
        kd, vd = qkv[:, 2048:3072].view(3, 8, 128), qkv[:, 3072:].view(3, 8, 128)
        dslots = [tables[s][(n - 1) // bs] * bs + (n - 1) % bs for s, n in enumerate(lens)]
        cu_k = _cu(lens)
        ctx = AttentionContext(torch.arange(4, dtype=torch.int32, device=dev), cu_k.to(dev), 1,
                               max(lens), torch.tensor(dslots, dtype=torch.int32, device=dev),
                               table_t)
        qkv_d = qkv.to(dev)
        with attention_context(ctx):
            out = layer(qd.to(dev), qkv_d[:, 2048:3072].view(3, 8, 128),
                        qkv_d[:, 3072:].view(3, 8, 128))
        kc, vc = oracle.store_kvcache(kd, vd, kc, vc, torch.tensor(dslots))
        ref = oracle.paged_decode(qd, kc, vc, torch.tensor(tables), torch.tensor(lens),
                                  128 ** -0.5)
        assert _err(out, ref) <= TOL, step
        torch.cuda.synchronize()
        assert torch.equal(kv[0].cpu(), kc) and torch.equal(kv[1].cpu(), vc), step


@pytest.mark.parametrize("exact", [False, True])
def test_paged_attention_layer_long_decode_exact_bound(dev, exact):
    """A decode step whose context says its max_seqlen_k is exact (an eager
    step's, max_seqlen_k_exact) splits with fixed partitions; one that does
    not, with the automatic split.  Both match the oracle, pools bit for bit."""
    g = torch.Generator().manual_seed(23)
    bs, hq, hkv, d = 16, 16, 8, 128
    lens = [5000, 300]
    need = [(n + bs - 1) // bs for n in lens]
    nb = sum(need) + 4
    perm = torch.randperm(nb, generator=g).tolist()
    width = max(need)
    rows, cur = [], 0
    for m in need:
        rows.append(perm[cur:cur + m] + [-1] * (width - m))
        cur += m
    table = torch.tensor(rows, dtype=torch.int32)
    kp = (torch.randn(nb, bs, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    vp = (torch.randn(nb, bs, hkv, d, generator=g) * 0.5).to(torch.bfloat16)
    q = torch.randn(2, hq, d, generator=g).to(torch.bfloat16)
    nk = torch.randn(2, hkv, d, generator=g).to(torch.bfloat16)
    nv = torch.randn(2, hkv, d, generator=g).to(torch.bfloat16)
    lt = torch.tensor(lens, dtype=torch.int32)
    slots = torch.tensor([rows[s][(n - 1) // bs] * bs + (n - 1) % bs for s, n in enumerate(lens)],
                         dtype=torch.int32)
    layer = PagedAttention(hq, d, d ** -0.5, hkv)
    layer.k_cache, layer.v_cache = kp.to(dev), vp.to(dev)
    ctx = AttentionContext(torch.arange(3, dtype=torch.int32, device=dev), _cu(lens).to(dev), 1,
                           max(lens), slots.to(dev), table.to(dev), max_seqlen_k_exact=exact)
    print(f"layer decode lens={lens} exact={exact}", flush=True)
    with attention_context(ctx):
        out = layer(q.to(dev), nk.to(dev), nv.to(dev))
    torch.cuda.synchronize()
    ek, ev = oracle.write_current_kv(kp, vp, table, lt, nk, nv, layout=oracle.NHD)
    assert torch.equal(layer.k_cache.cpu(), ek) and torch.equal(layer.v_cache.cpu(), ev)
    ref = oracle.paged_decode(q, ek, ev, table, lt, d ** -0.5)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("fuse", [True, False])
def test_paged_attention_layer_hnd_pool_matches_nhd(dev, fuse):
    """The same engine sequence (prefix-cached prefill, then decode steps) on an
    NHD pool and on an HND pool [nb, Hkv, bs, D]: outputs are bit-identical and
    the pools hold the same rows."""
    g = torch.Generator().manual_seed(15)
    bs, nb = 16, 256
    lens = [37, 90, 5, 130]
    width = 12
    perm = torch.randperm(nb, generator=g).tolist()
    tables = [perm[i * width:(i + 1) * width] for i in range(len(lens))]
    table_t = torch.tensor(tables, dtype=torch.int32, device=dev)
    total = sum(lens)
    q = torch.randn(total, 16, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16).to(dev)
    slots = [tables[s][p // bs] * bs + p % bs for s, n in enumerate(lens) for p in range(n)]
    cu = _cu(lens).to(dev)
    steps = [(torch.randn(len(lens), 16, 128, generator=g).to(torch.bfloat16).to(dev),
              torch.randn(len(lens), 8, 128, generator=g).to(torch.bfloat16).to(dev),
              torch.randn(len(lens), 8, 128, generator=g).to(torch.bfloat16).to(dev))
             for _ in range(3)]
    results = {}
    for layout in (ops.LAYOUT_NHD, ops.LAYOUT_HND):
        layer = PagedAttention(16, 128, 128 ** -0.5, 8)
        layer.fuse_store = fuse
        layer.kv_layout = layout
        shape = (2, nb, bs, 8, 128) if layout == ops.LAYOUT_NHD else (2, nb, 8, bs, 128)
        kv = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
        layer.k_cache, layer.v_cache = kv[0], kv[1]
        outs = []
        ctx = AttentionContext(cu, cu, max(lens), max(lens),
                               torch.tensor(slots, dtype=torch.int32, device=dev), table_t)
        with attention_context(ctx):
            outs.append(layer(q, k, v).clone())
        cur = list(lens)
        for qd, kd, vd in steps:
            cur = [n + 1 for n in cur]
            dslots = [tables[s][(n - 1) // bs] * bs + (n - 1) % bs for s, n in enumerate(cur)]
            ctx = AttentionContext(torch.arange(len(cur) + 1, dtype=torch.int32, device=dev),
                                   _cu(cur).to(dev), 1, max(cur),
                                   torch.tensor(dslots, dtype=torch.int32, device=dev), table_t)
            with attention_context(ctx):
                outs.append(layer(qd, kd, vd).clone())
        torch.cuda.synchronize()
        pool = kv.cpu() if layout == ops.LAYOUT_NHD else kv.cpu().permute(0, 1, 3, 2, 4)
        results[layout] = (outs, pool)
    (o_n, p_n), (o_h, p_h) = results[ops.LAYOUT_NHD], results[ops.LAYOUT_HND]
    assert torch.equal(p_n, p_h)
    for a, b in zip(o_n, o_h):
        assert torch.equal(a, b)


def test_paged_attention_layer_with_qwen3_prologue(dev):
    """forward(q, k, v, prologue=...) takes the raw projections and applies
    Qwen3's q/k RMSNorm + RoPE itself (qk_norm_rope before a prefill, inside
    the launch for a decode step).  Outputs and pools equal, bit for bit, a
    layer fed the normalised and rotated q and k, and match the oracle."""
    g = torch.Generator().manual_seed(25)
    bs, nb = 16, 256
    lens = [37, 90, 5]
    width = 12
    perm = torch.randperm(nb, generator=g).tolist()
    tables = [perm[i * width:(i + 1) * width] for i in range(len(lens))]
    table_t = torch.tensor(tables, dtype=torch.int32, device=dev)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    cs = oracle.rope_cache(128, 1024, 1_000_000.0)
    layers, pools = [], []
    for _ in range(2):
        layer = PagedAttention(16, 128, 128 ** -0.5, 8)
        kv = torch.zeros(2, nb, bs, 8, 128, dtype=torch.bfloat16, device=dev)
        layer.k_cache, layer.v_cache = kv[0], kv[1]
        layers.append(layer)
        pools.append(kv)

    def run(q, k, v, pos, ctx):
        pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
        qn, kn = ops.qk_norm_rope(q.to(dev), k.to(dev), pro)
        with attention_context(ctx):
            fused = layers[0](q.to(dev), k.to(dev), v.to(dev), prologue=pro)
            plain = layers[1](qn, kn, v.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(fused, plain)
        assert torch.equal(pools[0], pools[1])
        return fused, oracle.qk_norm_rope(q, k, pos, wq, wk, 1e-6, cs)

    total = sum(lens)
    q = torch.randn(total, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(total, 8, 128, generator=g).to(torch.bfloat16)
    pos = torch.cat([torch.arange(n) for n in lens])
    slots = [tables[s][p // bs] * bs + p % bs for s, n in enumerate(lens) for p in range(n)]
    cu = _cu(lens)
    ctx = AttentionContext(cu.to(dev), cu.to(dev), max(lens), max(lens),
                           torch.tensor(slots, dtype=torch.int32, device=dev), table_t)
    out, (rq, rk) = run(q, k, v, pos, ctx)
    assert _err(out, oracle.varlen_attention(rq, rk, v, cu, cu, 128 ** -0.5, True)) <= TOL
    kc, vc = oracle.store_kvcache(rk, v, torch.zeros(nb, bs, 8, 128, dtype=torch.bfloat16),
                                  torch.zeros(nb, bs, 8, 128, dtype=torch.bfloat16),
                                  torch.tensor(slots))
    for step in range(2):
        lens = [n + 1 for n in lens]
        qd = torch.randn(3, 16, 128, generator=g).to(torch.bfloat16)
        kd = torch.randn(3, 8, 128, generator=g).to(torch.bfloat16)
        vd = torch.randn(3, 8, 128, generator=g).to(torch.bfloat16)
        dpos = torch.tensor(lens) - 1
        dslots = [tables[s][(n - 1) // bs] * bs + (n - 1) % bs for s, n in enumerate(lens)]
        ctx = AttentionContext(torch.arange(4, dtype=torch.int32, device=dev),
                               _cu(lens).to(dev), 1, max(lens),
                               torch.tensor(dslots, dtype=torch.int32, device=dev), table_t)
        out, (rq, rk) = run(qd, kd, vd, dpos, ctx)
        kc, vc = oracle.store_kvcache(rk, vd, kc, vc, torch.tensor(dslots))
        ref = oracle.paged_decode(rq, kc, vc, torch.tensor(tables), torch.tensor(lens),
                                  128 ** -0.5)
        assert _err(out, ref) <= TOL, step


def test_paged_attention_layer_profiling_pass_without_cache(dev):
    g = torch.Generator().manual_seed(6)
    layer = PagedAttention(16, 128, 128 ** -0.5, 8)
    lens = [64, 64, 64]
    cu = _cu(lens)
    q = torch.randn(192, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(192, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(192, 8, 128, generator=g).to(torch.bfloat16)
    ctx = AttentionContext(cu.to(dev), cu.to(dev), 64, 64, None, None)
    with attention_context(ctx):
        out = layer(q.to(dev), k.to(dev), v.to(dev))
    assert _err(out, oracle.varlen_attention(q, k, v, cu, cu, 128 ** -0.5, True)) <= TOL


def test_varlen_self_attention_layer(dev):
    from voiceagent_amd.audio import batcher

    g = torch.Generator().manual_seed(7)
    cu, widest = batcher.window_cu_seqlens([46, 26, 95, 250], 104)
    total = int(cu[-1])
    q = torch.randn(total, 14, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(total, 14, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(total, 14, 64, generator=g).to(torch.bfloat16)
    layer = VarlenSelfAttention(14, 64, 64 ** -0.5)
    out = layer(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), widest)
    assert _err(out, oracle.varlen_attention(q, k, v, cu, cu, 0.125, False)) <= TOL


def test_causal_prompt_of_4096_tokens(dev):
    # The reference's default max_model_len (config.py:138) as one causal
    # prompt, packed with a short one and a single token: 64 query blocks.
    lens = [4096, 333, 1]
    b = workloads.make_varlen_batch(lens, 16, 8, 128, causal=True, seed=44)
    out = ops.varlen_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.cu_seqlens.to(dev),
                               b.cu_seqlens.to(dev), b.max_seqlen, b.max_seqlen, scale=b.scale,
                               causal=True)
    ref = oracle.varlen_attention(b.q, b.k, b.v, b.cu_seqlens, b.cu_seqlens, b.scale, True)
    assert _err(out, ref) <= TOL
