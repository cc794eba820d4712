"""Seeded sweep of store_kvcache argument combinations against the oracle.

Each case draws the element type (bf16, f16, fp32, or 16-bit rows into an FP8
pool), the kv-head count and head_dim, the block size, the pool layout (NHD or
HND), key and value as strided views of wider rows or contiguous, int32 or
int64 slots with -1 and out-of-range entries (both skipped), and the token
count on both sides of the launch's switch from one to four 16-byte words per
lane (about 262144 words).  The pools after the store must equal
oracle.store_kvcache's bit for bit (qwen_asr_vllm/layers/attention.py:31-67).
"""
import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops

pytestmark = pytest.mark.gpu

GEOMETRIES = [(8, 128), (1, 128), (2, 64), (14, 64), (4, 256), (3, 96), (8, 32)]


def _draw(seed: int):
    r = torch.Generator().manual_seed(3000 + seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=r))]

    hkv, d = GEOMETRIES[seed % len(GEOMETRIES)]  # every geometry, in turn
    kind = pick(["bf16", "bf16", "f16", "f32", "fp8"])
    words_per_tok = 2 * hkv * d * (4 if kind == "f32" else 2) // 16
    # Token counts below and above the four-words switch.
    big = int(torch.randint(300000 // words_per_tok + 1, 600000 // words_per_tok + 2, (1,),
                            generator=r))
    n = pick([1, 31, 257, int(torch.randint(3, 900, (1,), generator=r)), big, big])
    return dict(hkv=hkv, d=d, kind=kind, n=n, bs=pick([1, 16, 16, 32, 256]),
                layout=pick([ops.LAYOUT_NHD, ops.LAYOUT_HND]),
                strided=bool(torch.rand(1, generator=r) < 0.4),
                slot_i64=bool(torch.rand(1, generator=r) < 0.4), seed=seed)


@pytest.mark.parametrize("seed", range(32))
def test_random_store_case_matches_oracle(dev, seed):
    c = _draw(seed)
    hkv, d, n, bs, layout = c["hkv"], c["d"], c["n"], c["bs"], c["layout"]
    g = torch.Generator().manual_seed(seed)
    dtype = torch.float32 if c["kind"] == "f32" else (
        torch.float16 if c["kind"] == "f16" else torch.bfloat16)
    nb = (n + 40) // bs + 3
    shape = (nb, bs, hkv, d) if layout == ops.LAYOUT_NHD else (nb, hkv, bs, d)
    ks, vs = (0.05, 0.08) if c["kind"] == "fp8" else (1.0, 1.0)
    if c["kind"] == "fp8":
        kc = oracle.quantize_fp8(torch.randn(shape, generator=g), ks)
        vc = oracle.quantize_fp8(torch.randn(shape, generator=g), vs)
    else:
        kc = torch.randn(shape, generator=g).to(dtype)
        vc = torch.randn(shape, generator=g).to(dtype)
    if c["strided"]:
        # k and v as views of one wider row, as the engine's fused qkv output is.
        rows = torch.randn(n, 3 * hkv * d + 8, generator=g).to(dtype)
        key = rows[:, 8:8 + hkv * d].view(n, hkv, d)
        val = rows[:, 8 + 2 * hkv * d:8 + 3 * hkv * d].view(n, hkv, d)
    else:
        key = torch.randn(n, hkv, d, generator=g).to(dtype)
        val = torch.randn(n, hkv, d, generator=g).to(dtype)
    cap = nb * bs
    slots = torch.randperm(cap, generator=g)[:n].to(torch.int64 if c["slot_i64"] else torch.int32)
    if n > 3:
        slots[1::4] = -1
        slots[2::53] = cap + 5
    ref_slots = torch.where(slots >= cap, torch.full_like(slots, -1), slots)
    print(f"case {seed}: {c}", flush=True)
    ek, ev = oracle.store_kvcache(key, val, kc, vc, ref_slots, layout=layout, k_scale=ks,
                                  v_scale=vs)
    kd, vd = kc.to(dev), vc.to(dev)
    if c["strided"]:
        rd = rows.to(dev)
        kdev = rd[:, 8:8 + hkv * d].view(n, hkv, d)
        vdev = rd[:, 8 + 2 * hkv * d:8 + 3 * hkv * d].view(n, hkv, d)
    else:
        kdev, vdev = key.to(dev), val.to(dev)
    ops.store_kvcache(kdev, vdev, kd, vd, slots.to(dev), layout=layout, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    if c["kind"] == "fp8":
        assert torch.equal(kd.cpu().view(torch.uint8), ek.view(torch.uint8)), f"case {seed}: K"
        assert torch.equal(vd.cpu().view(torch.uint8), ev.view(torch.uint8)), f"case {seed}: V"
    else:
        assert torch.equal(kd.cpu(), ek), f"case {seed}: K"
        assert torch.equal(vd.cpu(), ev), f"case {seed}: V"
