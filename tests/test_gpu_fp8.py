"""FP8 (OCP e4m3) KV pools on the GPU against the oracle.

* Stores (standalone, fused into decode, fused into prefill) write the codes
  oracle.quantize_fp8 gives, bit for bit: x * (1/scale) in fp32, saturated
  to +-448, rounded to nearest even.
* Decode and prefill over FP8 pools meet oracle.paged_decode /
  oracle.varlen_attention evaluated on the dequantised pools (code * scale)
  at max-abs 2e-2 (bf16 / f16 inputs).
"""

import math

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops, workloads
from voiceagent_amd.layers.attention import PagedAttention
from voiceagent_amd.layers.attention import store_kvcache as layer_store_kvcache
from voiceagent_amd.layers.context import AttentionContext, attention_context

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


def _codes(t):
    return t.view(torch.uint8)


def _err(out, ref):
    return (out.float().cpu() - ref.float()).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [1.0, 0.37, 0.0625])
def test_store_quantises_bit_exactly(dev, dtype, scale):
    gen = torch.Generator().manual_seed(3)
    n, hkv, d, nb, bs = 40, 8, 128, 8, 16
    key = (torch.randn(n, hkv, d, generator=gen) * 3).to(dtype)
    value = (torch.randn(n, hkv, d, generator=gen) * 100).to(dtype)
    # the format's corners: ties, subnormals, saturation, zeros of both signs
    special = torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 448.0, 464.0, 500.0,
                            -1e4, 0.0, -0.0, 2.0 ** -9, 240.0, 7 * 2.0 ** -9, 0.001])
    key[0, 0, :special.numel()] = (special * scale).to(dtype)
    value[1, 3, :special.numel()] = (-special * scale).to(dtype)
    slots = torch.randperm(nb * bs, generator=gen)[:n].to(torch.int32)
    slots[5] = -1
    kp = torch.zeros(nb, bs, hkv, d, dtype=torch.uint8).view(F8)
    vp = torch.zeros_like(kp)
    kd, vd = kp.to(dev), vp.to(dev)
    ops.store_kvcache(key.to(dev), value.to(dev), kd, vd, slots.to(dev), k_scale=scale,
                      v_scale=scale * 2)
    torch.cuda.synchronize()
    ek, ev = oracle.store_kvcache(key, value, kp, vp, slots, k_scale=scale, v_scale=scale * 2)
    assert torch.equal(_codes(kd.cpu()), _codes(ek))
    assert torch.equal(_codes(vd.cpu()), _codes(ev))
    # The reference-signature layer function passes the scales through.
    kl, vl = kp.to(dev), vp.to(dev)
    layer_store_kvcache(key.to(dev), value.to(dev), kl, vl, slots.to(dev), k_scale=scale,
                        v_scale=scale * 2)
    torch.cuda.synchronize()
    assert torch.equal(_codes(kl.cpu()), _codes(ek)) and torch.equal(_codes(vl.cpu()), _codes(ev))


def _fp8_batch(lens, dev, seed, dtype=torch.bfloat16, hq=16, hkv=8, d=128, bs=16,
               layout=ops.LAYOUT_NHD, k_scale=0.05, v_scale=0.08):
    gen = torch.Generator().manual_seed(seed)
    need = [math.ceil(n / bs) for n in lens]
    nb = sum(need) + 8
    perm = torch.randperm(nb, generator=gen).tolist()
    width = max(need) + 1
    rows, cur = [], 0
    for n in need:
        rows.append(perm[cur:cur + n] + [-1] * (width - n))
        cur += n
    table = torch.tensor(rows, dtype=torch.int32)
    shape = (nb, bs, hkv, d) if layout == ops.LAYOUT_NHD else (nb, hkv, bs, d)
    kp = oracle.quantize_fp8(torch.randn(shape, generator=gen), k_scale)
    vp = oracle.quantize_fp8(torch.randn(shape, generator=gen) * 2, v_scale)
    q = torch.randn(len(lens), hq, d, generator=gen).to(dtype)
    nk = torch.randn(len(lens), hkv, d, generator=gen).to(dtype)
    nv = (torch.randn(len(lens), hkv, d, generator=gen) * 2).to(dtype)
    return table, kp, vp, q, nk, nv


@pytest.mark.parametrize(
    "dtype,hq,hkv,d,bs,layout,bound,masked,fused",
    [
        (torch.bfloat16, 16, 8, 128, 16, ops.LAYOUT_NHD, "exact", False, True),   # config 2 shape
        (torch.bfloat16, 16, 8, 128, 16, ops.LAYOUT_HND, "graph", False, True),   # split + merge
        (torch.float16, 16, 8, 128, 32, ops.LAYOUT_NHD, "exact", True, False),    # key mask
        (torch.bfloat16, 8, 1, 64, 16, ops.LAYOUT_HND, "graph", True, True),      # G = 8, D = 64
        (torch.float16, 4, 4, 256, 16, ops.LAYOUT_NHD, "exact", False, True),     # G = 1, D = 256
        (torch.bfloat16, 16, 8, 128, 16, ops.LAYOUT_NHD, "exact_split", True, True),  # fixed, 5000
    ],
)
def test_decode_over_fp8_pool(dev, dtype, hq, hkv, d, bs, layout, bound, masked, fused):
    # exact_split: SPLIT_EXACT over a bound above the automatic fixed-partition range
    lens = [1, 17, 600, 5000] if bound == "exact_split" else [1, 9, 16, 17, 100, 257, 600, 2100]
    ks, vs = 0.05, 0.08
    table, kp, vp, q, nk, nv = _fp8_batch(lens, dev, seed=d + bs, dtype=dtype, hq=hq, hkv=hkv,
                                          d=d, bs=bs, layout=layout, k_scale=ks, v_scale=vs)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    valid = (torch.rand(len(lens), max(lens) + 3, generator=torch.Generator().manual_seed(5))
             < 0.85) if masked else None
    kd, vd = kp.to(dev), vp.to(dev)
    print(f"fp8 decode {dtype} G={hq // hkv} D={d} bs={bs} {layout} {bound} masked={masked}",
          flush=True)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lens_t.to(dev),
                           max_seq_len=65536 if bound == "graph" else max(lens),
                           split_tokens=ops.SPLIT_EXACT if bound == "exact_split" else 0,
                           scale=d ** -0.5, layout=layout,
                           valid_mask=None if valid is None else valid.to(dev),
                           new_k=nk.to(dev) if fused else None,
                           new_v=nv.to(dev) if fused else None, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    ek, ev = kp, vp
    if fused:
        ek, ev = oracle.write_current_kv(kp, vp, table, lens_t, nk, nv, layout=layout,
                                         k_scale=ks, v_scale=vs)
        assert torch.equal(_codes(kd.cpu()), _codes(ek)) and torch.equal(_codes(vd.cpu()),
                                                                         _codes(ev))
    ref = oracle.paged_decode(q, ek, ev, table, lens_t, d ** -0.5, layout=layout,
                              valid_mask=valid, k_scale=ks, v_scale=vs)
    assert _err(out, ref) <= 2e-2


def test_decode_fp8_cfg2_and_constant_values(dev):
    # Config 2's shape and lengths; and a size-independent property: a pool
    # whose value codes are all one code returns that code's value exactly.
    lens = workloads.cfg2_lens(4)
    table, kp, vp, q, nk, nv = _fp8_batch(lens, dev, seed=11)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    out = ops.paged_decode(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lens_t.to(dev),
                           max_seq_len=max(lens), scale=128 ** -0.5, k_scale=0.05, v_scale=0.08)
    ref = oracle.paged_decode(q, kp, vp, table, lens_t, 128 ** -0.5, k_scale=0.05, v_scale=0.08)
    assert _err(out, ref) <= 2e-2
    vconst = torch.full(vp.shape, 0x3C, dtype=torch.uint8).view(F8)  # code 1.5
    out = ops.paged_decode(q.to(dev), kp.to(dev), vconst.to(dev), table.to(dev), lens_t.to(dev),
                           max_seq_len=max(lens), scale=128 ** -0.5, k_scale=0.05, v_scale=0.5)
    assert torch.all(out == 0.75)


def test_fp8_pool_rejects_shapes_without_a_matrix_core_path(dev):
    pool = torch.zeros(4, 8, 2, 128, dtype=torch.uint8, device=dev).view(F8)  # block size 8
    q = torch.zeros(1, 4, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(Exception, match="FP8"):
        ops.paged_decode(q, pool, pool.clone(), torch.zeros(1, 2, dtype=torch.int32, device=dev),
                         torch.ones(1, dtype=torch.int32, device=dev), max_seq_len=8, scale=0.1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_over_fp8_prefix_with_fused_store(dev, dtype):
    # Causal prefill continuing paged prefixes (prefix-cache hits and chunked
    # prompts): prefix keys come from the FP8 pool, new keys from k/v, and
    # the new rows are stored quantised.
    gen = torch.Generator().manual_seed(8)
    hq, hkv, d, bs = 16, 8, 128, 16
    prefix = [0, 16, 37, 300, 5]
    qlens = [50, 1, 64, 129, 200]
    klens = [p + q for p, q in zip(prefix, qlens)]
    need = [math.ceil(k / bs) for k in klens]
    nb = sum(need) + 4
    perm = torch.randperm(nb, generator=gen).tolist()
    rows, cur, slots = [], 0, []
    for pfx, kl, n in zip(prefix, klens, need):
        row = perm[cur:cur + n]
        cur += n
        rows.append(row + [-1] * (max(need) - n))
        slots += [row[p // bs] * bs + p % bs for p in range(pfx, kl)]
    table = torch.tensor(rows, dtype=torch.int32)
    slots = torch.tensor(slots, dtype=torch.int32)
    ks, vs = 0.04, 0.1
    kp = oracle.quantize_fp8(torch.randn(nb, bs, hkv, d, generator=gen), ks)
    vp = oracle.quantize_fp8(torch.randn(nb, bs, hkv, d, generator=gen), vs)
    total = sum(qlens)
    q = torch.randn(total, hq, d, generator=gen).to(dtype)
    k = torch.randn(total, hkv, d, generator=gen).to(dtype)
    v = torch.randn(total, hkv, d, generator=gen).to(dtype)
    cu_q = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32)
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cu_q.to(dev), cu_k.to(dev),
                               max(qlens), max(klens), scale=d ** -0.5, causal=True, k_cache=kd,
                               v_cache=vd, block_tables=table.to(dev), slot_mapping=slots.to(dev),
                               k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    ek, ev = oracle.store_kvcache(k, v, kp, vp, slots, k_scale=ks, v_scale=vs)
    assert torch.equal(_codes(kd.cpu()), _codes(ek)) and torch.equal(_codes(vd.cpu()), _codes(ev))
    ref = oracle.varlen_attention(q, k, v, cu_q, cu_k, d ** -0.5, True, k_cache=kp, v_cache=vp,
                                  block_tables=table, k_scale=ks, v_scale=vs)
    assert _err(out, ref) <= 2e-2
    # Every key from the pool (k = None), after the store.
    out2 = ops.varlen_attention(q.to(dev), None, None, cu_q.to(dev), cu_k.to(dev), max(qlens),
                                max(klens), scale=d ** -0.5, causal=True, k_cache=kd, v_cache=vd,
                                block_tables=table.to(dev), k_scale=ks, v_scale=vs)
    ref2 = oracle.varlen_attention(q, None, None, cu_q, cu_k, d ** -0.5, True, k_cache=ek,
                                   v_cache=ev, block_tables=table, k_scale=ks, v_scale=vs)
    assert _err(out2, ref2) <= 2e-2


def _fp8_prefix_case(gen, table_cols=None):
    """Prompts continuing paged prefixes, with the pool as FP8 codes and as a
    bf16 pool holding the same values rounded once (bf16(code * scale))."""
    hq, hkv, d, bs = 16, 8, 128, 16
    prefix = [0, 16, 37, 300, 5, 129]
    qlens = [50, 1, 64, 129, 200, 3]
    klens = [p + q for p, q in zip(prefix, qlens)]
    need = [math.ceil(k / bs) for k in klens]
    nb = sum(need) + 4
    perm = torch.randperm(nb, generator=gen).tolist()
    rows, cur = [], 0
    for n in need:
        rows.append(perm[cur:cur + n] + [-1] * (max(need) - n))
        cur += n
    table = torch.tensor(rows, dtype=torch.int32)
    if table_cols is not None:
        table = table[:, :table_cols].contiguous()
    ks, vs = 0.04, 0.1
    kp = oracle.quantize_fp8(torch.randn(nb, bs, hkv, d, generator=gen), ks)
    vp = oracle.quantize_fp8(torch.randn(nb, bs, hkv, d, generator=gen), vs)
    kb = oracle.dequantize_fp8(kp, ks).to(torch.bfloat16)
    vb = oracle.dequantize_fp8(vp, vs).to(torch.bfloat16)
    total = sum(qlens)
    q = torch.randn(total, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(total, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(total, hkv, d, generator=gen).to(torch.bfloat16)
    cu_q = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32)
    return dict(q=q, k=k, v=v, cu_q=cu_q, cu_k=cu_k, qlens=qlens, klens=klens, table=table,
                kp=kp, vp=vp, kb=kb, vb=vb, ks=ks, vs=vs, d=d)


def _prefill(c, dev, fp8, new_rows=True, max_k=None):
    kc, vc = (c["kp"], c["vp"]) if fp8 else (c["kb"], c["vb"])
    return ops.varlen_attention(
        c["q"].to(dev), c["k"].to(dev) if new_rows else None, c["v"].to(dev) if new_rows else None,
        c["cu_q"].to(dev), c["cu_k"].to(dev), max(c["qlens"]),
        max(c["klens"]) if max_k is None else max_k, scale=c["d"] ** -0.5, causal=True,
        k_cache=kc.to(dev), v_cache=vc.to(dev), block_tables=c["table"].to(dev),
        k_scale=c["ks"] if fp8 else 1.0, v_scale=c["vs"] if fp8 else 1.0)


@pytest.mark.parametrize("new_rows", [True, False])
def test_fp8_prefix_prefill_equals_bf16_pool_of_its_values(dev, new_rows):
    # The kernel converts each staged code to code * scale rounded once to
    # bf16: the launch must give the bits of the same launch over a bf16 pool
    # holding those values.
    c = _fp8_prefix_case(torch.Generator().manual_seed(31))
    got = _prefill(c, dev, True, new_rows)
    want = _prefill(c, dev, False, new_rows)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = oracle.varlen_attention(c["q"], c["k"] if new_rows else None,
                                  c["v"] if new_rows else None, c["cu_q"], c["cu_k"],
                                  c["d"] ** -0.5, True, k_cache=c["kp"], v_cache=c["vp"],
                                  block_tables=c["table"], k_scale=c["ks"], v_scale=c["vs"])
    assert _err(got, ref) <= 2e-2


def test_fp8_prefix_reads_columns_past_the_table_width_as_bf16_does(dev):
    # Three table columns for prefixes of up to 19 blocks: keys whose column
    # is at or past the width read block 0 on both pool dtypes alike (the
    # TTS padding semantics, qwen_tts_paged_attention.py:458-465).
    c = _fp8_prefix_case(torch.Generator().manual_seed(32), table_cols=3)
    got = _prefill(c, dev, True)
    want = _prefill(c, dev, False)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_fp8_prefix_ignores_max_seqlen_k(dev):
    # Key ranges come from cu_seqlens_k only: an underestimated max_seqlen_k
    # changes nothing (the former prefix copy dropped keys past it).
    c = _fp8_prefix_case(torch.Generator().manual_seed(33))
    got = _prefill(c, dev, True, max_k=1)
    want = _prefill(c, dev, True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_paged_attention_layer_prefill_then_decode_on_fp8_pool(dev):
    # The engine's sequence through the drop-in layer: a prefill that fills
    # the FP8 cache, then decode steps that attend it and append to it.
    gen = torch.Generator().manual_seed(12)
    hq, hkv, d, bs, nb = 16, 8, 128, 16, 64
    layer = PagedAttention(hq, d, d ** -0.5, hkv)
    layer.k_scale, layer.v_scale = 0.03, 0.06
    kc = torch.zeros(nb, bs, hkv, d, dtype=torch.uint8, device=dev).view(F8)
    vc = torch.zeros_like(kc)
    layer.k_cache, layer.v_cache = kc, vc
    lens = [33, 100, 7]
    tables = [[3, 9, 11], [4, 5, 6, 7, 8, 12, 13, 14], [20]]
    width = max(len(t) for t in tables)
    table = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)
    slots = torch.tensor([t[p // bs] * bs + p % bs for t, n in zip(tables, lens)
                          for p in range(n)], dtype=torch.int32)
    total = sum(lens)
    q = torch.randn(total, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(total, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(total, hkv, d, generator=gen).to(torch.bfloat16)
    cu = torch.tensor([0, 33, 133, 140], dtype=torch.int32)
    ctx = AttentionContext(cu_seqlens_q=cu.to(dev), cu_seqlens_k=cu.to(dev), max_seqlen_q=100,
                           max_seqlen_k=100, slot_mapping=slots.to(dev),
                           block_tables=table.to(dev))
    with attention_context(ctx):
        out = layer(q.to(dev), k.to(dev), v.to(dev))
    torch.cuda.synchronize()
    k0 = torch.zeros(nb, bs, hkv, d, dtype=torch.uint8).view(F8)
    ek, ev = oracle.store_kvcache(k, v, k0, k0.clone(), slots, k_scale=0.03, v_scale=0.06)
    assert torch.equal(_codes(kc.cpu()), _codes(ek)) and torch.equal(_codes(vc.cpu()), _codes(ev))
    ref = oracle.varlen_attention(q, k, v, cu, cu, d ** -0.5, True)
    # The prefill attends the new rows as given (16-bit), as it would over a
    # 16-bit cache; the cache holds their codes, which the decode steps read.
    assert _err(out, ref) <= 2e-2
    for step in range(3):
        lens = [n + 1 for n in lens]
        qd = torch.randn(3, hq, d, generator=gen).to(torch.bfloat16)
        kd_ = torch.randn(3, hkv, d, generator=gen).to(torch.bfloat16)
        vd_ = torch.randn(3, hkv, d, generator=gen).to(torch.bfloat16)
        dslots = torch.tensor([t[(n - 1) // bs] * bs + (n - 1) % bs for t, n in zip(tables, lens)],
                              dtype=torch.int32)
        cu_k = torch.tensor([0, lens[0], lens[0] + lens[1], sum(lens)], dtype=torch.int32)
        ctx = AttentionContext(cu_seqlens_q=torch.arange(4, dtype=torch.int32, device=dev),
                               cu_seqlens_k=cu_k.to(dev), max_seqlen_q=1, max_seqlen_k=max(lens),
                               slot_mapping=dslots.to(dev), block_tables=table.to(dev))
        with attention_context(ctx):
            out = layer(qd.to(dev), kd_.to(dev), vd_.to(dev))
        torch.cuda.synchronize()
        ek, ev = oracle.store_kvcache(kd_, vd_, ek, ev, dslots, k_scale=0.03, v_scale=0.06)
        assert torch.equal(_codes(kc.cpu()), _codes(ek)), step
        ref = oracle.paged_decode(qd, ek, ev, table, torch.tensor(lens), d ** -0.5,
                                  k_scale=0.03, v_scale=0.06)
        assert _err(out, ref) <= 2e-2, step


@pytest.mark.parametrize("B", [8, 40])
def test_fused_prologue_over_fp8_pool(dev, B):
    # The Qwen3 q/k prologue fused into a decode over an FP8 pool: q and the
    # current key are normalised and rotated inside the launch, the current
    # row is stored as codes and attended as their values.  B=8 splits the
    # contexts into partitions, B=40 does not.  The fused launch equals the
    # two-launch path (va_qk_norm_rope, then the FP8 decode) bit for bit,
    # output and pool, and the oracle on the dequantised pool within 2e-2.
    lens = torch.randint(20, 300, (B,), generator=torch.Generator().manual_seed(B)).tolist()
    ks, vs = 0.05, 0.08
    table, kp, vp, q, nk, nv = _fp8_batch(lens, dev, seed=B + 3, k_scale=ks, v_scale=vs)
    g = torch.Generator().manual_seed(B + 4)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    cs = oracle.rope_cache(128, 1024, 1_000_000.0)
    pos = torch.tensor(lens) - 1
    lens_t = torch.tensor(lens, dtype=torch.int32)
    print(f"fp8 decode with the fused prologue B={B}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    common = dict(max_seq_len=max(lens), scale=128 ** -0.5, new_v=nv.to(dev), k_scale=ks,
                  v_scale=vs)
    kd1, vd1 = kp.to(dev), vp.to(dev)
    kd2, vd2 = kd1.clone(), vd1.clone()
    td, ld = table.to(dev), lens_t.to(dev)
    out1 = ops.paged_decode(q.to(dev), kd1, vd1, td, ld, new_k=nk.to(dev), prologue=pro,
                            **common)
    qn, kn = ops.qk_norm_rope(q.to(dev), nk.to(dev), pro)
    out2 = ops.paged_decode(qn, kd2, vd2, td, ld, new_k=kn, **common)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(_codes(kd1), _codes(kd2)) and torch.equal(_codes(vd1), _codes(vd2))
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    ek, ev = oracle.write_current_kv(kp, vp, table, lens_t, rk, nv, layout=ops.LAYOUT_NHD,
                                     k_scale=ks, v_scale=vs)
    ref = oracle.paged_decode(rq, ek, ev, table, lens_t, 128 ** -0.5, k_scale=ks, v_scale=vs)
    assert _err(out1, ref) <= 2e-2


@pytest.mark.parametrize("split", [1024, 4096])
def test_fp8_decode_either_side_of_the_twelve_wave_bound(dev, split):
    # Over FP8 pools at head_dim 128 a workgroup that attends at most 2048
    # tokens runs twelve waves, a longer one eight.  One batch, partitions of
    # 1024 and of 4096 tokens, with the fused prologue, the key mask and the
    # fused store: both match the oracle on the dequantised pool.
    lens = [1, 17, 700, 2500, 5000]
    ks, vs = 0.05, 0.08
    table, kp, vp, q, nk, nv = _fp8_batch(lens, dev, seed=split, k_scale=ks, v_scale=vs)
    g = torch.Generator().manual_seed(split + 1)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    cs = oracle.rope_cache(128, 8192, 1_000_000.0)
    pos = torch.tensor(lens) - 1
    lens_t = torch.tensor(lens, dtype=torch.int32)
    valid = torch.rand(len(lens), max(lens) + 3, generator=g) < 0.85
    print(f"fp8 decode, partitions of {split} tokens", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lens_t.to(dev),
                           max_seq_len=max(lens), split_tokens=split, scale=128 ** -0.5,
                           valid_mask=valid.to(dev), new_k=nk.to(dev), new_v=nv.to(dev),
                           prologue=pro, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    ek, ev = oracle.write_current_kv(kp, vp, table, lens_t, rk, nv, layout=ops.LAYOUT_NHD,
                                     k_scale=ks, v_scale=vs)
    assert torch.equal(_codes(kd.cpu()), _codes(ek)) and torch.equal(_codes(vd.cpu()), _codes(ev))
    ref = oracle.paged_decode(rq, ek, ev, table, lens_t, 128 ** -0.5, valid_mask=valid,
                              k_scale=ks, v_scale=vs)
    assert _err(out, ref) <= 2e-2


@pytest.mark.parametrize("hq,hkv,B", [(16, 8, 32), (16, 8, 48), (8, 1, 300)])
def test_fp8_four_wave_workgroups(dev, hq, hkv, B):
    # A launch with more workgroups than CUs takes four-wave workgroups over
    # FP8 pools too (48 x 8 kv heads, 300 sequences of one kv head); 32 x 8
    # takes twelve waves.  With the fused prologue, the key mask and the fused
    # store: bit for bit the two-launch path (va_qk_norm_rope, then the
    # decode), output and pools, and the oracle on the dequantised pool within
    # 2e-2.
    g = torch.Generator().manual_seed(B + hq + 1)
    lens = torch.randint(1, 700, (B,), generator=g).tolist()
    ks, vs = 0.05, 0.08
    table, kp, vp, q, nk, nv = _fp8_batch(lens, dev, seed=B, hq=hq, hkv=hkv, k_scale=ks,
                                          v_scale=vs)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    cs = oracle.rope_cache(128, 1024, 1_000_000.0)
    pos = torch.tensor(lens) - 1
    lens_t = torch.tensor(lens, dtype=torch.int32)
    valid = torch.rand(B, max(lens) + 5, generator=g) < 0.85
    print(f"fp8 four-wave case hq={hq} hkv={hkv} B={B}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    common = dict(max_seq_len=max(lens), scale=128 ** -0.5, valid_mask=valid.to(dev),
                  new_v=nv.to(dev), k_scale=ks, v_scale=vs)
    td, ld = table.to(dev), lens_t.to(dev)
    kd1, vd1 = kp.to(dev), vp.to(dev)
    kd2, vd2 = kd1.clone(), vd1.clone()
    out1 = ops.paged_decode(q.to(dev), kd1, vd1, td, ld, new_k=nk.to(dev), prologue=pro,
                            **common)
    qn, kn = ops.qk_norm_rope(q.to(dev), nk.to(dev), pro)
    out2 = ops.paged_decode(qn, kd2, vd2, td, ld, new_k=kn, **common)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(_codes(kd1), _codes(kd2)) and torch.equal(_codes(vd1), _codes(vd2))
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    ek, ev = oracle.write_current_kv(kp, vp, table, lens_t, rk, nv, layout=ops.LAYOUT_NHD,
                                     k_scale=ks, v_scale=vs)
    assert torch.equal(_codes(vd1.cpu()), _codes(ev))
    ref = oracle.paged_decode(rq, ek, ev, table, lens_t, 128 ** -0.5, valid_mask=valid,
                              k_scale=ks, v_scale=vs)
    assert _err(out1, ref) <= 2e-2
