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
# holding both query and key rows (Hq 6).
@pytest.mark.parametrize("dtype,hq,hkv,d,T", [
    (torch.bfloat16, 16, 8, 128, 257), (torch.float16, 16, 8, 128, 257),
    (torch.float32, 16, 8, 128, 257), (torch.bfloat16, 14, 14, 64, 257),
    (torch.bfloat16, 4, 1, 256, 257), (torch.bfloat16, 16, 8, 128, 4096),
    (torch.bfloat16, 64, 8, 128, 4096), (torch.bfloat16, 6, 2, 128, 4096),
    (torch.float32, 6, 2, 64, 4096)])
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
