"""store_kvcache on the GPU: bit-exact against the oracle's scatter."""

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops
from voiceagent_amd.layers import store_kvcache

pytestmark = pytest.mark.gpu


def _pools(nb, bs, hkv, d, dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(nb, bs, hkv, d, generator=g).to(dtype).to(dev),
            torch.randn(nb, bs, hkv, d, generator=g).to(dtype).to(dev))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_bit_exact_with_skips(dev, dtype):
    kc, vc = _pools(64, 16, 8, 128, dtype, dev, 1)
    g = torch.Generator().manual_seed(2)
    n = 48
    slots = torch.randperm(64 * 16, generator=g)[:n].to(torch.int32)
    slots[::7] = -1
    key = torch.randn(n, 8, 128, generator=g).to(dtype)
    val = torch.randn(n, 8, 128, generator=g).to(dtype)
    ek, ev = oracle.store_kvcache(key, val, kc.cpu(), vc.cpu(), slots)
    store_kvcache(key.to(dev), val.to(dev), kc, vc, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu().view(torch.int8), ek.view(torch.int8))
    assert torch.equal(vc.cpu().view(torch.int8), ev.view(torch.int8))


def test_store_strided_value_view(dev):
    # The engine's v is a view of the fused qkv output with row stride (Hq + 2 Hkv) * D
    # (qwen_asr_vllm/models/qwen3.py:42-47).
    kc, vc = _pools(128, 16, 8, 128, torch.bfloat16, dev, 3)
    g = torch.Generator().manual_seed(4)
    n = 32
    qkv = torch.randn(n, (16 + 16) * 128, generator=g).to(torch.bfloat16)
    k = qkv[:, 2048:3072].view(n, 8, 128)
    v = qkv[:, 3072:4096].view(n, 8, 128)
    assert v.stride(0) == 4096
    slots = (torch.randperm(128, generator=g)[:n] * 16 + 5).to(torch.int32)
    ek, ev = oracle.store_kvcache(k, v, kc.cpu(), vc.cpu(), slots)
    qkv_d = qkv.to(dev)
    store_kvcache(qkv_d[:, 2048:3072].view(n, 8, 128), qkv_d[:, 3072:4096].view(n, 8, 128),
                  kc, vc, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)


def test_store_hnd_layout_and_out_of_range_slots(dev):
    g = torch.Generator().manual_seed(5)
    kc = torch.randn(16, 4, 32, 64, generator=g).to(torch.bfloat16)  # [pages, Hkv, page, D]
    vc = torch.randn(16, 4, 32, 64, generator=g).to(torch.bfloat16)
    key = torch.randn(6, 4, 64, generator=g).to(torch.bfloat16)
    val = torch.randn(6, 4, 64, generator=g).to(torch.bfloat16)
    slots = torch.tensor([0, 511, 37, -1, 512, 100000], dtype=torch.int64)
    ek, ev = oracle.store_kvcache(key[:4], val[:4], kc, vc, slots[:4], layout=oracle.HND)
    kd, vd = kc.to(dev), vc.to(dev)
    ops.store_kvcache(key.to(dev), val.to(dev), kd, vd, slots.to(dev), layout=ops.LAYOUT_HND)
    torch.cuda.synchronize()
    # slots >= capacity are skipped (never written out of bounds)
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)


def test_store_prefill_sized(dev):
    kc, vc = _pools(1024, 16, 8, 128, torch.bfloat16, dev, 6)
    g = torch.Generator().manual_seed(7)
    n = 8000
    slots = torch.randperm(1024 * 16, generator=g)[:n].to(torch.int32)
    key = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16)
    val = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16)
    ek, ev = oracle.store_kvcache(key, val, kc.cpu(), vc.cpu(), slots)
    store_kvcache(key.to(dev), val.to(dev), kc, vc, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)


@pytest.mark.parametrize("kind,slot_dtype", [
    ("bf16", torch.int32), ("bf16", torch.int64), ("f32", torch.int64), ("fp8", torch.int32),
    ("fp8", torch.int64)])
def test_store_four_words_per_lane(dev, kind, slot_dtype):
    # Launches of at least 256 workgroups' worth of words move four 16-byte words
    # per lane per pass (all loads before the stores); 2051 tokens end on a partial
    # pass, and every fifth slot is -1 and a few are past the pool (both skipped).
    n, nb, bs = 2051, 160, 16
    dtype = torch.float32 if kind == "f32" else torch.bfloat16
    g = torch.Generator().manual_seed(40)
    key = torch.randn(n, 8, 128, generator=g).to(dtype)
    val = torch.randn(n, 8, 128, generator=g).to(dtype)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(slot_dtype)
    slots[::5] = -1
    slots[3::97] = nb * bs + 7
    ref_slots = torch.where(slots >= nb * bs, torch.full_like(slots, -1), slots)
    ks, vs = (0.05, 0.08) if kind == "fp8" else (1.0, 1.0)
    if kind == "fp8":
        kc = oracle.quantize_fp8(torch.randn(nb, bs, 8, 128, generator=g), ks)
        vc = oracle.quantize_fp8(torch.randn(nb, bs, 8, 128, generator=g), vs)
    else:
        kc = torch.randn(nb, bs, 8, 128, generator=g).to(dtype)
        vc = torch.randn(nb, bs, 8, 128, generator=g).to(dtype)
    ek, ev = oracle.store_kvcache(key, val, kc, vc, ref_slots, k_scale=ks, v_scale=vs)
    kd, vd = kc.to(dev), vc.to(dev)
    print(f"store {kind} slots {slot_dtype} n={n}", flush=True)
    ops.store_kvcache(key.to(dev), val.to(dev), kd, vd, slots.to(dev), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    if kind == "fp8":
        assert torch.equal(kd.cpu().view(torch.uint8), ek.view(torch.uint8))
        assert torch.equal(vd.cpu().view(torch.uint8), ev.view(torch.uint8))
    else:
        assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
