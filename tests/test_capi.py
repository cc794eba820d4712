"""CPU checks of the C-ABI library: it loads, exports every function the
header declares, agrees with the ctypes struct layouts, and rejects bad
arguments on the host (no GPU needed: only zero-work or invalid calls)."""

import ctypes
import os
import re

import pytest
import torch

from voiceagent_amd import _native as N
from voiceagent_amd import ops

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "voiceagent_attn.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(va_\w+)\s*\(", text, flags=re.M))


def test_header_functions_are_exported():
    lib = N.lib()
    declared = _declared_functions()
    assert declared == set(N.SIGNATURES), declared ^ set(N.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.va_abi_version() == N.ABI_VERSION == 6


@pytest.mark.parametrize(
    "fn, cls, count_field",
    [("va_store_kvcache", N.StoreArgs, "num_tokens"),
     ("va_paged_decode", N.DecodeArgs, "num_seqs"),
     ("va_varlen_attention", N.VarlenArgs, "num_seqs"),
     ("va_qk_norm_rope", N.QkNormRopeArgs, "num_tokens")],
)
def test_struct_size_contract(fn, cls, count_field):
    lib = N.lib()
    args = N.new_args(cls)
    setattr(args, count_field, 0)
    # matching layout, zero work: succeeds without touching a device
    assert getattr(lib, fn)(ctypes.byref(args), None) == 0
    args.struct_size = ctypes.sizeof(cls) - 8
    assert getattr(lib, fn)(ctypes.byref(args), None) == -1
    assert "struct_size" in N.last_error()


def test_decode_rejects_bad_geometry():
    lib = N.lib()
    args = N.new_args(N.DecodeArgs)
    args.num_seqs = 2
    args.q = args.out = args.block_tables = args.lens = 16
    args.pool.k = args.pool.v = 16
    args.pool.block_size, args.pool.num_blocks = 16, 4
    args.num_heads, args.num_kv_heads, args.head_dim = 6, 4, 128
    assert lib.va_paged_decode(ctypes.byref(args), None) == -1
    assert "multiple" in N.last_error()
    args.num_heads = 8
    args.valid_mask, args.valid_len, args.valid_stride_seq = 16, 64, -64
    assert lib.va_paged_decode(ctypes.byref(args), None) == -1
    assert "valid_stride_seq" in N.last_error()
    args.valid_mask = None
    args.q_stride_seq = 1  # not a 16-byte multiple
    assert lib.va_paged_decode(ctypes.byref(args), None) == -1
    assert "16-byte" in N.last_error()
    # Other head dims take the small-head kernel, which needs element
    # alignment only; the checks still run before any launch.
    args.head_dim, args.dtype = 4, 2  # fp32
    args.q_stride_seq = 1  # 4 bytes: fine for fp32 elements
    args.q = 18  # not 4-byte aligned
    assert lib.va_paged_decode(ctypes.byref(args), None) == -1
    assert "4-byte aligned" in N.last_error()
    args.head_dim = 2000
    assert lib.va_paged_decode(ctypes.byref(args), None) == -1
    assert "head_dim 2000 outside" in N.last_error()


def test_decode_workspace_sizing():
    lib = N.lib()
    args = N.new_args(N.DecodeArgs)
    args.num_seqs, args.num_heads, args.num_kv_heads, args.head_dim = 32, 16, 8, 128
    args.max_seq_len = 48
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) == 0  # one partition
    # 256 (sequence, kv head) pairs fill the CUs: one partition per pair.
    args.max_seq_len = 600
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) == 0
    # Few pairs: contexts are split to occupy the CUs -> partials.
    args.num_seqs = 2
    n = lib.va_paged_decode_workspace_bytes(ctypes.byref(args))
    assert n > 0
    # ...unless no context can hold more than 192 KiB of one kv head's K/V
    # (384 tokens at head_dim 128 in bf16): those stream whole, unmerged.
    args.max_seq_len = 384
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) == 0
    args.max_seq_len = 385
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) > 0
    # With 128 pairs a split would make 2 partitions per pair: the bound
    # scales to 8 / 2 times that, 1536 tokens.
    args.num_seqs = 16
    args.max_seq_len = 1536
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) == 0
    args.max_seq_len = 1537
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) > 0
    # The bound is in bytes: fp32 rows halve it in tokens (192 at 8 partitions).
    args.num_seqs, args.dtype = 2, N.DTYPE_CODES[torch.float32]
    args.max_seq_len = 192
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) == 0
    args.max_seq_len = 193
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) > 0
    args.dtype = N.DTYPE_CODES[torch.bfloat16]
    args.num_seqs, args.max_seq_len = 2, 600
    args.max_seq_len = 16384
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) >= n
    args.split_tokens = 1  # an explicit split is honoured (rounded up to a workgroup round)
    args.num_seqs, args.max_seq_len = 32, 600
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) > 0
    # a tiny explicit split on a long context is capped at 256 partitions
    args.num_seqs, args.split_tokens, args.max_seq_len = 2, 16, 1 << 20
    per_part = 2 * 8 * 2 * (2 * 4 + 128 * 4)  # pairs * G * (m, l + o) bytes
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(args)) <= 256 * per_part + 256
    bad = N.DecodeArgs()
    assert lib.va_paged_decode_workspace_bytes(ctypes.byref(bad)) == 0


def test_varlen_needs_no_workspace_even_for_long_fp8_prefixes():
    # An FP8 pool's prefix is converted inside the kernel: no workspace, at
    # any max_seqlen_k (the former prefix copy took num_seqs x
    # ceil(max_seqlen_k / block_size) blocks: ~4.3 GB at 16 x 65536 tokens).
    lib = N.lib()
    args = N.new_args(N.VarlenArgs)
    args.num_seqs, args.num_heads, args.num_kv_heads, args.head_dim = 16, 16, 8, 128
    args.max_seqlen_q, args.max_seqlen_k = 512, 65536
    args.pool.k = args.pool.v = 1 << 20  # a pool is described; nothing is dereferenced
    args.pool.block_size, args.pool.num_blocks = 16, 1 << 16
    args.pool.kv_format = N.VA_KV_FP8_E4M3
    args.pool.k_scale = args.pool.v_scale = 1.0
    args.block_tables = 1 << 20
    assert lib.va_varlen_workspace_bytes(ctypes.byref(args)) == 0


def test_ops_refuse_cpu_tensors():
    q = torch.zeros(2, 16, 128)
    pool = torch.zeros(4, 16, 8, 128)
    with pytest.raises(ops.AttentionArgumentError, match="GPU"):
        ops.paged_decode(q, pool, pool, torch.zeros(2, 1, dtype=torch.int32),
                         torch.ones(2, dtype=torch.int32), max_seq_len=1, scale=1.0)
    with pytest.raises(ops.AttentionArgumentError, match="GPU"):
        ops.store_kvcache(torch.zeros(2, 8, 128), torch.zeros(2, 8, 128), pool, pool,
                          torch.zeros(2, dtype=torch.int32))


def test_tts_api_contract_errors_on_cpu():
    from voiceagent_amd.agent import PagedAttentionKernelError, paged_attention_decode

    page_table = torch.tensor([[3, 5, 0], [1, 7, 2]], dtype=torch.long)
    seq_lens = torch.tensor([3, 5], dtype=torch.long)
    kp = torch.zeros(8, 2, 2, 4)
    q = torch.ones(2, 4, 1, 4)
    bad = page_table.clone()
    bad[0, 0] = 99
    # test_qwen_tts_paged_attention_kernel.py:60-74: invalid page ids are rejected.
    with pytest.raises(PagedAttentionKernelError, match="page table"):
        paged_attention_decode(q, kp, kp, bad, seq_lens)
    with pytest.raises(PagedAttentionKernelError, match="torch.long"):
        paged_attention_decode(q, kp, kp, page_table, seq_lens.int())
    with pytest.raises(PagedAttentionKernelError, match="together"):
        paged_attention_decode(q, kp, kp, page_table, seq_lens, new_key=torch.zeros(2, 2, 1, 4))
    with pytest.raises(PagedAttentionKernelError, match="GPU"):
        paged_attention_decode(q, kp, kp, page_table, seq_lens)


def test_tts_value_checks_raise_in_the_reference_order():
    # qwen_tts_paged_attention.py:333-341 checks positive lengths, then table
    # capacity, then row by row an invalid used page before a short key mask.
    # Each expected message below follows from that order for the case built.
    from voiceagent_amd.agent import PagedAttentionKernelError
    from voiceagent_amd.agent.paged_attention import _validate_inputs

    kp = torch.zeros(8, 2, 2, 4)  # 8 pages of 2 tokens
    q = torch.ones(2, 4, 1, 4)
    table = torch.tensor([[3, 5, 99], [1, 7, 2]], dtype=torch.long)  # [0, 2] unused below

    def check(lens, tbl=table, mask_width=None):
        mask = None if mask_width is None else torch.ones(2, mask_width, dtype=torch.bool)
        return _validate_inputs(q, kp, kp, tbl, torch.tensor(lens, dtype=torch.long), mask)

    assert check([3, 5]) == (2, 4, 2, 2)  # entries past a row's used pages are not checked
    assert check([3, 5], mask_width=5) == (2, 4, 2, 2)
    with pytest.raises(PagedAttentionKernelError, match="positive"):
        check([0, 7])  # 7 also exceeds the capacity of 6: the length check comes first
    with pytest.raises(PagedAttentionKernelError, match="capacity"):
        check([5, 7], mask_width=1)
    with pytest.raises(PagedAttentionKernelError, match="invalid page"):
        check([5, 5])  # row 0 now uses page 99
    neg = table.clone()
    neg[0, 2] = 0
    neg[1, 1] = -1
    with pytest.raises(PagedAttentionKernelError, match="invalid page"):
        check([3, 3], tbl=neg)
    with pytest.raises(PagedAttentionKernelError, match="shorter"):
        check([3, 5], mask_width=4)
    with pytest.raises(PagedAttentionKernelError, match="shorter"):
        check([5, 3], tbl=neg, mask_width=4)  # row 0's short mask before row 1's page
    with pytest.raises(PagedAttentionKernelError, match="invalid page"):
        check([5, 3], mask_width=4)  # row 0's bad page before its own short mask


def test_bench_library_is_apart_from_the_drop_in_library():
    # The read-floor probe lives in libvoiceagent_bench.so, declared in
    # include/voiceagent_bench.h; the drop-in library exports no diagnostics.
    import bench

    lib = N.lib()
    assert not hasattr(lib, "va_hbm_read_probe") and not hasattr(lib, "va_bench_hbm_read")
    blib = bench.bench_lib()
    assert hasattr(blib, "va_bench_hbm_read") and hasattr(blib, "va_bench_last_error")
    rc = blib.va_bench_hbm_read(16, 15, 1, 0, 16, None)  # unaligned size: host-side reject
    assert rc == -1 and b"aligned" in blib.va_bench_last_error()
    rc = blib.va_bench_hbm_read(16, 16, 1, 7, 16, None)
    assert rc == -1 and b"mode" in blib.va_bench_last_error()
    rc = blib.va_bench_empty(0, None)  # no workgroups: rejected before any launch
    assert rc == -1 and b"workgroups" in blib.va_bench_last_error()
    # The per-CU depth probe checks its depths, alignment and buffer on the host.
    mib = 1 << 20
    rc = blib.va_bench_hbm_depth(1024, 8 * mib, mib, 1, 12, 0, 16, 16, None)
    assert rc == -1 and b"depths" in blib.va_bench_last_error()
    rc = blib.va_bench_hbm_depth(1024, 8 * mib, mib, 1, 0, 0, 16, 16, None)
    assert rc == -1 and b"depths" in blib.va_bench_last_error()
    rc = blib.va_bench_hbm_depth(1024, 8 * mib, mib + 16, 1, 8, 0, 16, 16, None)
    assert rc == -1 and b"aligned" in blib.va_bench_last_error()
    rc = blib.va_bench_hbm_depth(1024, 8 * mib, 4 * mib, 4, 8, 4, 16, 16, None)
    assert rc == -1 and b"exceed" in blib.va_bench_last_error()
    rc = blib.va_bench_hbm_depth(1024, 8 * mib, 64 * 1024, 1, 16, 8, 16, 16, None)
    assert rc == -1 and b"two rounds" in blib.va_bench_last_error()


def test_host_fast_path_module_loads_and_declines_cpu_tensors():
    # csrc/host/fast_calls.cpp: built beside the library, handed its entry
    # points, and it takes no call whose tensors are not on the named GPU.
    fast = ops._fast_calls()
    assert fast is not None
    assert fast.NOT_TAKEN == ops._FAST_NOT_TAKEN
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16)
    pool = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16)
    tables = torch.zeros(2, 1, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    assert fast.paged_decode(q, pool, pool, tables, lens, q, None, None, None, None, None, None,
                             0.0, None, None, None, False, False, 16, 0.1, 0, 0, 0, 1.0, 1.0, 0,
                             0) == ops._FAST_NOT_TAKEN
    cu = torch.tensor([0, 1, 2], dtype=torch.int32)
    assert fast.varlen_attention(q, q, q, cu, cu, 1, 1, 0.1, True, None, None, None, None, q,
                                 False, 0, 0) == ops._FAST_NOT_TAKEN
