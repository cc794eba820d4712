"""The wrappers' host fast path (csrc/host/fast_calls.cpp) on the GPU.

ops.paged_decode and ops.varlen_attention hand common calls to the C++
module, which makes the wrappers' checks and the same C-ABI call; anything it
does not take (no_alloc, an FP8 prefill pool, a bad argument) runs the
Python path.  Both paths launch the same kernels with the same
arguments, so their outputs and pools agree bit for bit; the oracle check of
every other GPU test runs through the fast path.
"""

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import ops, workloads

pytestmark = pytest.mark.gpu


@pytest.fixture
def python_path(monkeypatch):
    """Run the wrappers without the fast path for the duration of a call."""
    def off():
        monkeypatch.setattr(ops, "_FAST", None)
        monkeypatch.setattr(ops, "_FAST_LOADED", True)
    return off


def test_fast_module_is_loaded(dev):
    fast = ops._fast_calls()
    assert fast is not None, "the _fast_calls module was not built or did not load"
    assert fast.NOT_TAKEN == ops._FAST_NOT_TAKEN


@pytest.mark.parametrize("fused,cumulative,layout,masked", [
    (True, True, ops.LAYOUT_NHD, False), (False, False, ops.LAYOUT_NHD, True),
    (True, False, ops.LAYOUT_HND, True)])
@pytest.mark.parametrize("B", [4, 40])
def test_decode_fast_and_python_paths_agree(dev, python_path, fused, cumulative, layout, masked,
                                            B):
    # B=4 splits the contexts (the workspace is allocated by the Python path
    # on the first call, then reused by the fast path); B=40 does not.
    lens = torch.randint(1, 700, (B,), generator=torch.Generator().manual_seed(B)).tolist()
    b = workloads.make_decode_batch(lens, num_blocks=2048, device=dev, seed=B + 1)
    kp, vp = b.k_pools[0], b.v_pools[0]
    if layout == ops.LAYOUT_HND:
        kp, vp = kp.transpose(1, 2).contiguous(), vp.transpose(1, 2).contiguous()
    g = torch.Generator(device=dev).manual_seed(7)
    nk = torch.randn(B, 8, 128, device=dev, generator=g).to(torch.bfloat16)
    nv = torch.randn(B, 8, 128, device=dev, generator=g).to(torch.bfloat16)
    lens_arg = b.cu_seqlens_k if cumulative else b.context_lens
    valid = (torch.rand(B, max(lens) + 5, device=dev, generator=g) < 0.8) if masked else None
    pools = [(kp.clone(), vp.clone()) for _ in range(3)]
    outs = []
    for i, (k, v) in enumerate(pools):
        if i == 2:
            python_path()
        outs.append(ops.paged_decode(b.q, k, v, b.block_tables, lens_arg,
                                     lens_cumulative=cumulative, max_seq_len=b.max_seq_len,
                                     scale=b.scale, layout=layout, valid_mask=valid,
                                     new_k=nk if fused else None, new_v=nv if fused else None))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    for k, v in pools[1:]:
        assert torch.equal(k, pools[0][0]) and torch.equal(v, pools[0][1])
    if not fused:
        ref = oracle.paged_decode(b.q.cpu(), kp.cpu(), vp.cpu(), b.block_tables.cpu(),
                                  b.context_lens.cpu(), b.scale, layout=layout,
                                  valid_mask=None if valid is None else valid.cpu())
        assert (outs[0].float().cpu() - ref.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_fast_and_python_paths_agree(dev, python_path, causal):
    lens = [1, 17, 64, 65, 200, 333]
    vb = workloads.make_varlen_batch(lens, 16, 8, 128, causal=causal, seed=3)
    args = (vb.q.to(dev), vb.k.to(dev), vb.v.to(dev), vb.cu_seqlens.to(dev),
            vb.cu_seqlens.to(dev), vb.max_seqlen, vb.max_seqlen)
    fast = ops.varlen_attention(*args, scale=vb.scale, causal=causal)
    python_path()
    slow = ops.varlen_attention(*args, scale=vb.scale, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(fast, slow)


def test_bad_arguments_raise_the_python_paths_errors(dev):
    # The fast path takes no call with a bad argument; the Python path raises.
    lens = [5, 9]
    b = workloads.make_decode_batch(lens, num_blocks=64, device=dev, seed=2)
    with pytest.raises(ops.AttentionArgumentError, match="head_dim mismatch"):
        ops.paged_decode(b.q[:, :, :64].contiguous(), b.k_pools[0], b.v_pools[0],
                         b.block_tables, b.context_lens, max_seq_len=16, scale=0.1)
    with pytest.raises(ops.AttentionArgumentError, match="contiguous"):
        ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables,
                         b.context_lens.repeat_interleave(2)[::2], max_seq_len=16, scale=0.1)
    fast = ops._fast_calls()
    cpu_q = b.q.cpu()
    # A tensor on another device than the one named: not taken, nothing launched.
    assert fast.paged_decode(cpu_q, b.k_pools[0], b.v_pools[0], b.block_tables,
                             b.context_lens, b.q, None, None, None, None, None, None, 0.0, None,
                             None, None, False, False, 16, 0.1, 0, 0, 0, 1.0, 1.0,
                             b.q.get_device(), 0) == ops._FAST_NOT_TAKEN


def test_store_rope_and_prologue_decode_agree_on_both_paths(dev, python_path):
    g = torch.Generator(device=dev).manual_seed(9)
    n, hkv, d = 300, 8, 128
    key = torch.randn(n, hkv, d, device=dev, generator=g).to(torch.bfloat16)
    value = torch.randn(n, 2 * hkv, d, device=dev, generator=g).to(torch.bfloat16)[:, :hkv]
    slots = torch.randperm(64 * 16, device=dev, generator=g)[:n].to(torch.int32)
    slots[::7] = -1
    q = torch.randn(n, 16, d, device=dev, generator=g).to(torch.bfloat16)
    wq = (torch.rand(d, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(d, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    cs = oracle.rope_cache(d, 4096, 1_000_000.0).to(dev)
    pos = torch.randint(0, 4096, (n,), device=dev, generator=g)
    pro = ops.QKPrologue(wq, wk, 1e-6, cs, pos)
    # decode with the fused prologue: 8 sequences over the stored pool
    lens = torch.tensor([1, 30, 77, 100, 160, 200, 250, 299], dtype=torch.int32, device=dev)
    table = torch.arange(8 * 19, dtype=torch.int32, device=dev).view(8, 19)
    dpro = ops.QKPrologue(wq, wk, 1e-6, cs, (lens - 1).long())
    res = []
    for i in range(2):
        if i == 1:
            python_path()
        kp = torch.zeros(256, 16, hkv, d, dtype=torch.bfloat16, device=dev)
        vp = torch.zeros_like(kp)
        ops.store_kvcache(key, value, kp, vp, slots)
        qo, ko = ops.qk_norm_rope(q, key, pro)
        out = ops.paged_decode(q[:8], kp, vp, table, lens, max_seq_len=300, scale=d ** -0.5,
                               new_k=key[:8], new_v=value[:8], prologue=dpro)
        res.append((kp, vp, qo, ko, out))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)
