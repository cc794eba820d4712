"""Seeded random combinations of the decode and varlen options, against the
oracle: dtype, head_dim, group size, kv heads, block size (including block
sizes that take the general decode kernel), pool layout, index dtypes,
cumulative lengths, key mask, fused current-row write, and an exact
max_seq_len (automatic or exact-bound split) or an upper bound of 4096 or
65536; causal and bidirectional varlen; and causal prefill
over a paged prefix with the store fused.  Each case is small enough for the
CPU oracle.

Tolerances as elsewhere: 1e-5 for fp32 inputs, 2e-2 for 16-bit inputs.
"""

import random

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _decode_case(seed):
    r = random.Random(seed)
    dtype = r.choice([torch.bfloat16, torch.float16, torch.float32])
    d = r.choice([64, 128, 256])
    g = r.choice([1, 2, 4, 8])
    hkv = r.choice([1, 2, 8])
    bs = r.choice([16, 16, 32, 8])
    layout = r.choice([ops.LAYOUT_NHD, ops.LAYOUT_HND])
    B = r.choice([1, 3, 8, 40])
    lens = [r.randint(1, 900) for _ in range(B)]
    return dict(dtype=dtype, d=d, g=g, hkv=hkv, bs=bs, layout=layout, lens=lens,
                table_i64=r.random() < 0.5, cumulative=r.random() < 0.5,
                mask=r.random() < 0.4, fused=r.random() < 0.5, bound=r.random() < 0.3,
                width_extra=r.choice([-50, 0, 7]),
                # drawn last, so the earlier draws of a seed stay as they were
                bound_len=r.choice([4096, 65536]), exact=r.random() < 0.5)


@pytest.mark.parametrize("seed", range(60))
def test_random_decode_options(dev, seed):
    c = _decode_case(seed)
    print(f"decode case {seed}: {c}", flush=True)
    gen = torch.Generator().manual_seed(1000 + seed)
    dtype, d, hkv, bs, lens = c["dtype"], c["d"], c["hkv"], c["bs"], c["lens"]
    hq, B = hkv * c["g"], len(lens)
    need = [(n + bs - 1) // bs for n in lens]
    nb = sum(need) + 5
    perm = torch.randperm(nb, generator=gen).tolist()
    width = max(need) + 1
    table = torch.full((B, width), -1, dtype=torch.int64 if c["table_i64"] else torch.int32)
    cur = 0
    for i, m in enumerate(need):
        table[i, :m] = torch.tensor(perm[cur:cur + m])
        cur += m
    shape = (nb, bs, hkv, d) if c["layout"] == ops.LAYOUT_NHD else (nb, hkv, bs, d)
    kp = (torch.randn(shape, generator=gen) * 0.5).to(dtype)
    vp = torch.randn(shape, generator=gen).to(dtype)
    q = torch.randn(B, hq, d, generator=gen).to(dtype)
    lens_t = torch.tensor(lens, dtype=torch.int64 if c["table_i64"] else torch.int32)
    lens_arg = lens_t
    if c["cumulative"]:
        lens_arg = torch.zeros(B + 1, dtype=lens_t.dtype)
        lens_arg[1:] = torch.cumsum(lens_t, 0)
    valid = None
    if c["mask"]:
        w = max(1, max(lens) + c["width_extra"])
        valid = torch.rand(B, w, generator=gen) < 0.8
    nk = nv = None
    ek, ev = kp, vp
    if c["fused"]:
        nk = (torch.randn(B, hkv, d, generator=gen) * 0.5).to(dtype)
        nv = torch.randn(B, hkv, d, generator=gen).to(dtype)
        ek, ev = oracle.write_current_kv(kp, vp, table, lens_t, nk, nv, layout=c["layout"])
    kd, vd = kp.to(dev), vp.to(dev)
    out = ops.paged_decode(q.to(dev), kd, vd, table.to(dev), lens_arg.to(dev),
                           lens_cumulative=c["cumulative"],
                           max_seq_len=c["bound_len"] if c["bound"] else max(lens),
                           split_tokens=ops.SPLIT_EXACT if c["exact"] and not c["bound"] else 0,
                           scale=d ** -0.5,
                           layout=c["layout"], valid_mask=None if valid is None else valid.to(dev),
                           new_k=None if nk is None else nk.to(dev),
                           new_v=None if nv is None else nv.to(dev))
    torch.cuda.synchronize()
    if c["fused"]:
        assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.paged_decode(q, ek, ev, table, lens_t, d ** -0.5, layout=c["layout"],
                              valid_mask=valid)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= TOL[dtype], (seed, err)


@pytest.mark.parametrize("seed", range(20))
def test_random_varlen_options(dev, seed):
    r = random.Random(5000 + seed)
    dtype = r.choice([torch.bfloat16, torch.float16])
    d = r.choice([64, 128])
    g = r.choice([1, 2, 4, 8])
    hkv = r.choice([1, 2, 8])
    causal = r.random() < 0.6
    n = r.choice([1, 4, 17])
    lens = [r.randint(1, 700) for _ in range(n)]
    print(f"varlen case {seed}: dtype={dtype} d={d} g={g} hkv={hkv} causal={causal} "
          f"lens={lens}", flush=True)
    gen = torch.Generator().manual_seed(6000 + seed)
    total = sum(lens)
    q = torch.randn(total, hkv * g, d, generator=gen).to(dtype)
    k = torch.randn(total, hkv, d, generator=gen).to(dtype)
    v = torch.randn(total, hkv, d, generator=gen).to(dtype)
    cu = torch.zeros(n + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    out = ops.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), cu.to(dev),
                               max(lens), max(lens), scale=d ** -0.5, causal=causal)
    ref = oracle.varlen_attention(q, k, v, cu, cu, d ** -0.5, causal)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= TOL[dtype], (seed, err)


@pytest.mark.parametrize("seed", range(12))
def test_random_paged_prefix_with_fused_store(dev, seed):
    # Prefix-cache hits (keys from the pool) and new tokens (from k/v, stored
    # to their slots in the same launch), random geometry and block size.
    from tests.test_gpu_varlen import _paged_prefill_case

    r = random.Random(7000 + seed)
    hkv = r.choice([1, 2, 8])
    hq = hkv * r.choice([1, 2, 4, 8])
    d = r.choice([64, 128])
    bs = r.choice([16, 32])
    spec = tuple((r.choice([0, 0, r.randint(1, 300)]), r.randint(1, 260))
                 for _ in range(r.choice([1, 3, 9])))
    slot_dtype = r.choice([torch.int32, torch.int64])
    print(f"paged prefix case {seed}: hq={hq} hkv={hkv} d={d} bs={bs} spec={spec}", flush=True)
    nb = sum(-(-(p + n) // bs) for p, n in spec) + 4
    c = _paged_prefill_case(seed=8000 + seed, bs=bs, nb=nb, hq=hq, hkv=hkv, d=d,
                            slot_dtype=slot_dtype, spec=spec)
    kd, vd = c["kp"].to(dev), c["vp"].to(dev)
    out = ops.varlen_attention(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), c["cu_q"].to(dev),
                               c["cu_k"].to(dev), c["max_q"], c["max_k"], scale=d ** -0.5,
                               causal=True, k_cache=kd, v_cache=vd,
                               block_tables=c["table"].to(dev), slot_mapping=c["slots"].to(dev))
    ek, ev = oracle.store_kvcache(c["k"], c["v"], c["kp"], c["vp"], c["slots"])
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    ref = oracle.varlen_attention(c["q"], c["k"], c["v"], c["cu_q"], c["cu_k"], d ** -0.5, True,
                                  k_cache=c["kp"], v_cache=c["vp"], block_tables=c["table"])
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= 2e-2, (seed, err)
