"""va_paged_decode_noalloc: the decode without a caller workspace, its split
partials in the library's own scratch buffer.  Called through the C ABI, it
must give the bits of va_paged_decode (same kernels, same split) with a
torch-allocated workspace, on two calls in a row (the second smaller, so it
reads the buffer after the first left partials in it), and both must meet
the oracle at 2e-2 (bf16) with bit-exact pools after the fused store."""

import pytest
import torch

from oracle import attention as oracle
from voiceagent_amd import _native, ops, workloads

pytestmark = pytest.mark.gpu


def _run(batch, no_alloc, max_seq_len, split_tokens=0):
    k, v = batch.k_pools[0].clone(), batch.v_pools[0].clone()
    out = torch.empty_like(batch.q)
    ops.paged_decode(batch.q, k, v, batch.block_tables, batch.cu_seqlens_k, lens_cumulative=True,
                     max_seq_len=max_seq_len, scale=batch.scale, new_k=batch.new_k,
                     new_v=batch.new_v, new_slots=batch.slot_mapping, out=out,
                     split_tokens=split_tokens, no_alloc=no_alloc)
    torch.cuda.synchronize()
    return out, k, v


@pytest.mark.parametrize("first,second,max_seq_len", [
    ([3000, 2500, 4100], [700, 90], 65536),   # split at a graph's bound
    ([16384], [5000], 16384),                 # one long context, exact bound
    ([2000] * 12, [33, 1, 257], 2000),        # 96 pairs split in two, then fewer
])
def test_noalloc_matches_workspace_entry_point_twice(dev, first, second, max_seq_len):
    for step, lens in enumerate((first, second)):
        nb = sum((n + 15) // 16 for n in lens) + 8
        b = workloads.make_decode_batch(lens, num_blocks=nb, dtype=torch.bfloat16, kv_std=0.5,
                                        device=dev, seed=90 + step)
        print(f"noalloc step {step}: lens {lens} bound {max_seq_len}", flush=True)
        got, gk, gv = _run(b, True, max_seq_len)
        ref, rk, rv = _run(b, False, max_seq_len)
        assert torch.equal(got, ref), step
        assert torch.equal(gk, rk) and torch.equal(gv, rv), step
        ek, ev = oracle.store_kvcache(b.new_k.cpu(), b.new_v.cpu(), b.k_pools[0].cpu(),
                                      b.v_pools[0].cpu(), b.slot_mapping.cpu())
        assert torch.equal(gk.cpu(), ek) and torch.equal(gv.cpu(), ev), step
        want = oracle.paged_decode(b.q.cpu(), ek, ev, b.block_tables.cpu(),
                                   b.context_lens.cpu(), b.scale)
        assert (got.float().cpu() - want).abs().max().item() <= 2e-2, step


def test_noalloc_rejects_a_split_beyond_its_scratch(dev):
    # An explicit split of 64 x 4096-token contexts (64 tokens asked, rounded
    # up to the kernel's 256-token unit: 16 partitions) needs
    # 512 pairs x 16 partitions x 2 heads x 130 floats = 8.5 MB: above 4 MiB.
    # The check runs on the host before any launch, so a small pool serves.
    B = 64
    q = torch.zeros(B, 16, 128, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(8, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    table = torch.zeros(B, 256, dtype=torch.int32, device=dev)
    lens = torch.full((B,), 4096, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    with pytest.raises(_native.NativeError, match="scratch"):
        ops.paged_decode(q, pool, pool.clone(), table, lens, max_seq_len=4096, scale=0.1,
                         out=out, split_tokens=64, no_alloc=True)
    with pytest.raises(ops.AttentionArgumentError, match="out"):
        ops.paged_decode(q, pool, pool.clone(), table, lens, max_seq_len=4096, scale=0.1,
                         no_alloc=True)


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    # Both calls split their contexts, so both use the one scratch buffer of
    # the GPU; the second, on another stream and issued without a host sync,
    # must wait for the first (ops orders them on the GPU).
    def batch(lens, seed):
        nb = sum((n + 15) // 16 for n in lens) + 8
        return workloads.make_decode_batch(lens, num_blocks=nb, dtype=torch.bfloat16,
                                           kv_std=0.5, device=dev, seed=seed)

    def call(b, out, no_alloc, max_seq_len):
        ops.paged_decode(b.q, b.k_pools[0], b.v_pools[0], b.block_tables, b.cu_seqlens_k,
                         lens_cumulative=True, max_seq_len=max_seq_len, scale=b.scale, out=out,
                         no_alloc=no_alloc)

    b1, b2 = batch([16384], 95), batch([3000, 2500, 4100], 96)
    ref1, ref2 = torch.empty_like(b1.q), torch.empty_like(b2.q)
    call(b1, ref1, False, 16384)
    call(b2, ref2, False, 65536)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    for rep in range(3):
        out1, out2 = torch.full_like(ref1, float("nan")), torch.full_like(ref2, float("nan"))
        torch.cuda.synchronize()
        print(f"two-stream no_alloc rep {rep}", flush=True)
        with torch.cuda.stream(s1):
            call(b1, out1, True, 16384)
        with torch.cuda.stream(s2):
            call(b2, out2, True, 65536)
        torch.cuda.synchronize()
        assert torch.equal(out1, ref1) and torch.equal(out2, ref2), rep
