"""Qwen3 q/k prologue on the GPU: the standalone kernel (va_qk_norm_rope) and
the prologue fused into the paged decode kernel, against the oracle's
restatement of RMSNorm._norm + apply_rotary_emb
(qwen_asr_vllm/layers/layernorm.py:19-25, rotary_embedding.py:9-32).

16-bit results may differ from the oracle on a few elements: the sum of
squares is reduced in a different order, so the fp32 inverse RMS can differ
in its last bit and a normalised element by one unit in the last place (ulp).
The rotation mixes each element with its partner i +- D/2 and preserves the
pair's magnitude r, so such a difference can reach about sqrt(2) ulp(r) plus
the final rounding; the bound is 2 ulp(r) per element (a constant multiple
of the pair's scale, not of a possibly cancelled output).  Attention outputs
keep the 2e-2 (bf16/f16) and 1e-5 (fp32) tolerances."""

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops, workloads

pytestmark = pytest.mark.gpu

MANT = {torch.bfloat16: 7, torch.float16: 10}


def _close_16bit(got, want, dtype):
    """Elements further than 2 ulp of their rotary pair's magnitude from `want`,
    and the bit-exact fraction."""
    g, w = got.float().cpu(), want.float().cpu()
    h = w.shape[-1] // 2
    r = torch.sqrt(w[..., :h] ** 2 + w[..., h:] ** 2)
    r = torch.cat((r, r), dim=-1).clamp_min(2.0 ** -14)
    ulp = torch.exp2(torch.floor(torch.log2(r)) - MANT[dtype])
    bad = (g - w).abs() > 2 * ulp
    exact = (g == w).float().mean().item()
    return int(bad.sum()), exact


def _prologue_inputs(T, hq, hkv, d, dtype, seed, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, hq, d, generator=g).to(dtype)
    k = torch.randn(T, hkv, d, generator=g).to(dtype)
    wq = (torch.rand(d, generator=g) + 0.5).to(dtype)
    wk = (torch.rand(d, generator=g) + 0.5).to(dtype)
    pos = torch.randint(0, max_pos, (T,), generator=g)
    cs = oracle.rope_cache(d, max_pos, 1_000_000.0)
    return q, k, wq, wk, pos, cs


# T = 257 spreads each token's rows over several waves; T = 4096 takes one
# wave per token, with 72 rows in three chunks of loads (Hq 64) or a row group
# holding both query and key rows (Hq 10), or, with at most 8 rows per token
# (Hq 6 + Hkv 2), several tokens per wave.
@pytest.mark.parametrize("dtype,hq,hkv,d,T", [
    (torch.bfloat16, 16, 8, 128, 257), (torch.float16, 16, 8, 128, 257),
    (torch.float32, 16, 8, 128, 257), (torch.bfloat16, 14, 14, 64, 257),
    (torch.bfloat16, 4, 1, 256, 257), (torch.bfloat16, 16, 8, 128, 4096),
    (torch.bfloat16, 64, 8, 128, 4096), (torch.bfloat16, 10, 2, 128, 4096),
    (torch.bfloat16, 6, 2, 128, 4096), (torch.float32, 6, 2, 64, 4096)])
def test_qk_norm_rope_matches_oracle(dev, dtype, hq, hkv, d, T):
    q, k, wq, wk, pos, cs = _prologue_inputs(T, hq, hkv, d, dtype, seed=d + hq)
    print(f"qk_norm_rope {dtype} T={T} Hq={hq} Hkv={hkv} D={d}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    qo, ko = ops.qk_norm_rope(q.to(dev), k.to(dev), pro)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(q, k, pos, wq, wk, 1e-6, cs)
    for got, want, name in ((qo, rq, "q"), (ko, rk, "k")):
        if dtype == torch.float32:
            assert (got.cpu() - want).abs().max().item() <= 1e-5, name
        else:
            nbad, exact = _close_16bit(got, want, dtype)
            print(f"  {name}: {exact:.4%} bit-exact, {nbad} beyond 1 ulp", flush=True)
            assert nbad == 0, name
            assert exact > 0.95, name


@pytest.mark.parametrize("dtype,wdtype", [
    (torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16),
    (torch.float16, torch.bfloat16), (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("T", [257, 4096])
def test_qk_norm_rope_weights_of_another_dtype(dev, dtype, wdtype, T):
    # The norm weights' dtype is independent of the rows' (layernorm.py:19-25
    # multiplies the rounded rows by the weight in place): the kernel unpacks
    # 16-bit weights row by row and takes fp32 weights as they are.
    q, k, wq, wk, pos, cs = _prologue_inputs(T, 16, 8, 128, dtype, seed=T + 3)
    wq, wk = wq.float().mul(1.0 + 2.0 ** -9).to(wdtype), wk.float().to(wdtype)
    print(f"qk_norm_rope rows {dtype} weights {wdtype} T={T}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    qo, ko = ops.qk_norm_rope(q.to(dev), k.to(dev), pro)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(q, k, pos, wq, wk, 1e-6, cs)
    for got, want, name in ((qo, rq, "q"), (ko, rk, "k")):
        if dtype == torch.float32:
            assert (got.cpu() - want).abs().max().item() <= 1e-5, name
        else:
            nbad, exact = _close_16bit(got, want, dtype)
            assert nbad == 0 and exact > 0.95, (name, nbad, exact)


@pytest.mark.parametrize("dtype,d,T", [
    (torch.bfloat16, 128, 4099), (torch.float16, 64, 4097), (torch.float32, 128, 8561),
    (torch.bfloat16, 256, 4097)])
def test_keys_alone_take_several_tokens_per_wave(dev, dtype, d, T):
    # 8 key heads and no query heads, at prompt size: each lane group of a
    # wave takes its own token (T leaves the last wave lanes past the end,
    # which store nothing).  The keys must be the bits that the kernel taking
    # one token per wave gives beside 16 query heads, and meet the oracle.
    q, k, wq, wk, pos, cs = _prologue_inputs(T, 16, 8, d, dtype, seed=T + d)
    print(f"keys alone {dtype} T={T} D={d}", flush=True)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    qd, kd = q.to(dev), k.to(dev)
    alone = torch.full_like(kd, float("nan"))
    assert ops.qk_norm_rope(None, kd, pro, k_out=alone)[0] is None
    _, both = ops.qk_norm_rope(qd, kd, pro)
    torch.cuda.synchronize()
    assert torch.equal(alone, both)
    _, rk = oracle.qk_norm_rope(q, k, pos, wq, wk, 1e-6, cs)
    if dtype == torch.float32:
        assert (alone.cpu() - rk).abs().max().item() <= 1e-5
    else:
        assert _close_16bit(alone, rk, dtype)[0] == 0


def test_qk_norm_rope_in_place_and_strided(dev):
    # q and k as views of one fused qkv row, as the engine produces them
    T, hq, hkv, d = 64, 16, 8, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    q = qkv[:, : hq * d].view(T, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].view(T, hkv, d)
    _, _, wq, wk, pos, cs = _prologue_inputs(T, hq, hkv, d, torch.bfloat16, seed=6)
    rq, rk = oracle.qk_norm_rope(q, k, pos, wq, wk, 1e-6, cs)
    dq = qkv.to(dev)
    qd = dq[:, : hq * d].view(T, hq, d)
    kd = dq[:, hq * d: (hq + hkv) * d].view(T, hkv, d)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    ops.qk_norm_rope(qd, kd, pro, q_out=qd, k_out=kd)
    torch.cuda.synchronize()
    assert _close_16bit(qd, rq, torch.bfloat16)[0] == 0
    assert _close_16bit(kd, rk, torch.bfloat16)[0] == 0
    # v untouched
    assert torch.equal(dq[:, (hq + hkv) * d:].cpu(), qkv[:, (hq + hkv) * d:])


def _decode_case(dtype, seed, B=8, nb=256):
    lens = torch.randint(20, 300, (B,), generator=torch.Generator().manual_seed(seed)).tolist()
    b = workloads.make_decode_batch(lens, num_blocks=nb, dtype=dtype, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(B, 16, 128, generator=g).to(dtype)
    nk = torch.randn(B, 8, 128, generator=g).to(dtype)
    nv = torch.randn(B, 8, 128, generator=g).to(dtype)
    wq = (torch.rand(128, generator=g) + 0.5).to(dtype)
    wk = (torch.rand(128, generator=g) + 0.5).to(dtype)
    cs = oracle.rope_cache(128, 1024, 1_000_000.0)
    pos = torch.tensor(lens) - 1
    return b, lens, q, nk, nv, wq, wk, cs, pos


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("engine_slots", [True, False])
@pytest.mark.parametrize("B", [8, 40])
def test_fused_decode_prologue_matches_oracle(dev, dtype, engine_slots, B):
    # B=8: 64 (sequence, kv head) pairs, split into partitions; B=40: 320 pairs,
    # one partition each, so the first tiles are requested before the length
    # and the position-dependent rotary rows arrive.
    b, lens, q, nk, nv, wq, wk, cs, pos = _decode_case(dtype, seed=11, B=B, nb=1024)
    print(f"fused decode prologue {dtype} engine_slots={engine_slots} B={B}", flush=True)
    kp, vp = b.k_pools[0].to(dev), b.v_pools[0].to(dev)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    out = ops.paged_decode(q.to(dev), kp, vp, b.block_tables.to(dev), b.cu_seqlens_k.to(dev),
                           lens_cumulative=True, max_seq_len=max(lens), scale=128 ** -0.5,
                           new_k=nk.to(dev), new_v=nv.to(dev),
                           new_slots=b.slot_mapping.to(dev) if engine_slots else None,
                           prologue=pro)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    rkp, rvp = oracle.store_kvcache(rk, nv, b.k_pools[0], b.v_pools[0], b.slot_mapping)
    ref = oracle.paged_decode(rq, rkp, rvp, b.block_tables, torch.tensor(lens), 128 ** -0.5)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    err = (out.float().cpu() - ref.float()).abs().max().item()
    print(f"  max abs err {err:.3e}", flush=True)
    assert err <= tol
    slots = b.slot_mapping.tolist()
    got_k = torch.stack([kp.view(-1, 8, 128)[s] for s in slots]).cpu()
    got_v = torch.stack([vp.view(-1, 8, 128)[s] for s in slots]).cpu()
    assert torch.equal(got_v, nv)
    if dtype == torch.float32:
        assert (got_k - rk).abs().max().item() <= 1e-5
    else:
        assert _close_16bit(got_k, rk, dtype)[0] == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B", [8, 40])
def test_fused_decode_prologue_with_key_mask(dev, dtype, B):
    # The prologue together with a key_valid_mask (bf16 takes the matrix-core
    # kernel, fp32 the general one), split into partitions (B=8) or not (B=40).
    b, lens, q, nk, nv, wq, wk, cs, pos = _decode_case(dtype, seed=31, B=B, nb=1024)
    g = torch.Generator().manual_seed(32)
    width = max(lens) - 17
    valid = torch.rand(B, width, generator=g) < 0.75
    kp, vp = b.k_pools[0].to(dev), b.v_pools[0].to(dev)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    out = ops.paged_decode(q.to(dev), kp, vp, b.block_tables.to(dev), b.cu_seqlens_k.to(dev),
                           lens_cumulative=True, max_seq_len=max(lens), scale=128 ** -0.5,
                           new_k=nk.to(dev), new_v=nv.to(dev), new_slots=b.slot_mapping.to(dev),
                           prologue=pro, valid_mask=valid.to(dev))
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(q, nk, pos, wq, wk, 1e-6, cs)
    rkp, rvp = oracle.store_kvcache(rk, nv, b.k_pools[0], b.v_pools[0], b.slot_mapping)
    ref = oracle.paged_decode(rq, rkp, rvp, b.block_tables, torch.tensor(lens), 128 ** -0.5,
                              valid_mask=valid)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert (out.float().cpu() - ref.float()).abs().max().item() <= tol


@pytest.mark.parametrize("B", [16, 40])
def test_fused_prologue_equals_two_launch_path_bitwise(dev, B):
    """The fused prologue runs the same per-row code as va_qk_norm_rope, so
    fused and two-launch decodes agree bit for bit (output and pool)."""
    b, lens, q, nk, nv, wq, wk, cs, pos = _decode_case(torch.bfloat16, seed=21, B=B, nb=1024)
    pro = ops.QKPrologue(wq.to(dev), wk.to(dev), 1e-6, cs.to(dev), pos.to(dev))
    common = dict(lens_cumulative=True, max_seq_len=max(lens), scale=128 ** -0.5,
                  new_v=nv.to(dev), new_slots=b.slot_mapping.to(dev))
    kp1, vp1 = b.k_pools[0].to(dev), b.v_pools[0].to(dev)
    kp2, vp2 = kp1.clone(), vp1.clone()
    tables, cu = b.block_tables.to(dev), b.cu_seqlens_k.to(dev)
    out1 = ops.paged_decode(q.to(dev), kp1, vp1, tables, cu, new_k=nk.to(dev), prologue=pro,
                            **common)
    qn, kn = ops.qk_norm_rope(q.to(dev), nk.to(dev), pro)
    out2 = ops.paged_decode(qn, kp2, vp2, tables, cu, new_k=kn, **common)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(kp1, kp2) and torch.equal(vp1, vp2)


def _prefill_case(seed, paged):
    """Prompts (some continuing a paged prefix), raw q/k projections, random
    per-token positions (not the key index: the launch must read them)."""
    g = torch.Generator().manual_seed(seed)
    hq, hkv, d, bs = 16, 8, 128, 16
    qlens = [50, 1, 130, 257, 64, 3]
    prefix = [0, 16, 37, 0, 200, 5] if paged else [0] * len(qlens)
    klens = [p + n for p, n in zip(prefix, qlens)]
    T = sum(qlens)
    q, k, wq, wk, pos, cs = _prologue_inputs(T, hq, hkv, d, torch.bfloat16, seed=seed)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32)
    case = dict(q=q, k=k, v=v, wq=wq, wk=wk, pos=pos, cs=cs, cu_q=cu_q, cu_k=cu_k, qlens=qlens,
                klens=klens, d=d)
    if paged:
        need = [-(-n // bs) for n in klens]
        nb = sum(need) + 4
        perm = torch.randperm(nb, generator=g).tolist()
        rows, cur, slots = [], 0, []
        for pfx, kl, n in zip(prefix, klens, need):
            row = perm[cur:cur + n]
            cur += n
            rows.append(row + [-1] * (max(need) - n))
            slots += [row[p // bs] * bs + p % bs for p in range(pfx, kl)]
        case.update(table=torch.tensor(rows, dtype=torch.int32),
                    slots=torch.tensor(slots, dtype=torch.int32),
                    kp=torch.randn(nb, bs, hkv, d, generator=g).to(torch.bfloat16),
                    vp=torch.randn(nb, bs, hkv, d, generator=g).to(torch.bfloat16))
    return case


def _run_prefill(c, dev, q, k, prologue=None):
    kw = dict(scale=c["d"] ** -0.5, causal=True, prologue=prologue)
    if "kp" in c:
        kp, vp = c["kp"].to(dev), c["vp"].to(dev)
        out = ops.varlen_attention(q, k, c["v"].to(dev), c["cu_q"].to(dev), c["cu_k"].to(dev),
                                   max(c["qlens"]), max(c["klens"]), k_cache=kp, v_cache=vp,
                                   block_tables=c["table"].to(dev),
                                   slot_mapping=c["slots"].to(dev), **kw)
        return out, kp, vp
    out = ops.varlen_attention(q, k, c["v"].to(dev), c["cu_q"].to(dev), c["cu_k"].to(dev),
                               max(c["qlens"]), max(c["klens"]), **kw)
    return out, None, None


@pytest.mark.parametrize("paged", [True, False])
def test_fused_prefill_query_prologue_matches_oracle(dev, paged):
    # The launch normalises and rotates q itself; the keys go through the
    # standalone kernel alone (num_heads = 0).
    c = _prefill_case(40 + paged, paged)
    pro = ops.QKPrologue(c["wq"].to(dev), c["wk"].to(dev), 1e-6, c["cs"].to(dev),
                         c["pos"].to(dev))
    _, kn = ops.qk_norm_rope(None, c["k"].to(dev), pro)
    q2, k2 = ops.qk_norm_rope(c["q"].to(dev), c["k"].to(dev), pro)
    torch.cuda.synchronize()
    assert torch.equal(kn, k2)  # the same per-row code for the keys
    print(f"fused prefill prologue, paged={paged}", flush=True)
    out, kp, vp = _run_prefill(c, dev, c["q"].to(dev), kn, prologue=pro)
    ref_two, kp2, vp2 = _run_prefill(c, dev, q2, k2)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_norm_rope(c["q"], c["k"], c["pos"], c["wq"], c["wk"], 1e-6, c["cs"])
    if paged:
        # The fused store wrote the processed keys (identical in both paths).
        assert torch.equal(kp, kp2) and torch.equal(vp, vp2)
        ek, ev = oracle.store_kvcache(rk, c["v"], c["kp"], c["vp"], c["slots"])
        ref = oracle.varlen_attention(rq, rk, c["v"], c["cu_q"], c["cu_k"], c["d"] ** -0.5, True,
                                      k_cache=c["kp"], v_cache=c["vp"], block_tables=c["table"])
        assert (kp.cpu() - ek).abs().max().item() <= 2 * 2.0 ** -7 * ek.abs().max().item()
    else:
        ref = oracle.varlen_attention(rq, rk, c["v"], c["cu_q"], c["cu_k"], c["d"] ** -0.5, True)
    err = (out.float().cpu() - ref).abs().max().item()
    two = (out.float() - ref_two.float()).abs().max().item()
    print(f"  max-abs vs oracle {err:.3e}, vs two-launch path {two:.3e}", flush=True)
    assert err <= 2e-2
    assert two <= 2e-2


def test_qwen3_core_prefill_with_the_query_prologue_fused(dev):
    # With varlen_fuse_prologue set, the layer routes a prefill batch through
    # the fused launch: same result as the layer with the prologue unfused
    # (the default: standalone kernel over q and k).
    from voiceagent_amd.layers.context import AttentionContext, attention_context
    from voiceagent_amd.layers.qwen3 import Qwen3AttentionCore

    c = _prefill_case(44, True)
    layers = []
    for fuse in (True, False):
        layer = Qwen3AttentionCore(16, 128, 8, max_position=4096).to(dev)
        with torch.no_grad():
            layer.q_norm_weight.copy_(c["wq"].float())
            layer.k_norm_weight.copy_(c["wk"].float())
        layer.q_norm_weight.data = layer.q_norm_weight.data.to(torch.bfloat16)
        layer.k_norm_weight.data = layer.k_norm_weight.data.to(torch.bfloat16)
        layer.cos_sin_cache = c["cs"].to(dev)
        layer.k_cache, layer.v_cache = c["kp"].to(dev), c["vp"].to(dev)
        layer.varlen_fuse_prologue = fuse
        layers.append(layer)
    ctx = AttentionContext(cu_seqlens_q=c["cu_q"].to(dev), cu_seqlens_k=c["cu_k"].to(dev),
                           max_seqlen_q=max(c["qlens"]), max_seqlen_k=max(c["klens"]),
                           slot_mapping=c["slots"].to(dev), block_tables=c["table"].to(dev))
    outs = []
    with attention_context(ctx):
        for layer in layers:
            outs.append(layer(c["pos"].to(dev), c["q"].to(dev), c["k"].to(dev), c["v"].to(dev)))
    torch.cuda.synchronize()
    assert (outs[0].float() - outs[1].float()).abs().max().item() <= 2e-2
    assert torch.equal(layers[0].k_cache, layers[1].k_cache)
