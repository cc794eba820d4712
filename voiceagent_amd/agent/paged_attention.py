"""TTS-talker paged decode attention on the HIP kernel.

Drop-in for ``paged_attention_decode`` of
qwen_asr_vllm/agent/qwen_tts_paged_attention.py:383-516: same arguments,
same defaults, same :class:`PagedAttentionKernelError` contract checks
(:290-350, :416-446).  The pool layout is HND ``[pages, kv_heads, page_size,
head_dim]`` and tables/lengths are int64, as the talker's paged cache hands
them over (qwen_tts_outer_varlen.py:392-447).

Differences that callers can observe:

* ``use_triton`` is accepted for signature compatibility; both values run the
  HIP kernel (there is no torch fallback in this build).
* ``block_n``/``num_warps`` are checked as the reference checks them and
  otherwise ignored (the kernel picks its own split).
* ``kernel_seq_len``/``kernel_page_count`` bound the attended keys as the
  Triton kernel's ``MAX_SEQ_LEN``/``num_page_slots`` do (:223-241): tokens at
  or past ``kernel_seq_len`` are not attended and table columns at or past
  ``kernel_page_count`` read as page 0, while the current row is still
  written at ``seq_len - 1`` through the table's own entry (:182-221).  The
  page table is not copied to a padded tensor: columns past its width read as
  page 0 inside the kernel, which is what the reference's zero padding
  (:458-465) produces.
* The fused current-row write uses the row's register copy for position
  ``seq_len - 1`` instead of re-reading the pool, so there is no
  write-then-read hazard between lanes.
"""

from __future__ import annotations

import math

import torch

from voiceagent_amd import ops


class PagedAttentionKernelError(RuntimeError):
    """Raised when the paged decode attention contract is invalid."""


def _validate_inputs(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    key_valid_mask: torch.Tensor | None,
) -> tuple[int, int, int, int]:
    """Contract checks of qwen_tts_paged_attention.py:290-350 (synchronising)."""
    tensors = {
        "query": query,
        "key_pool": key_pool,
        "value_pool": value_pool,
        "page_table": page_table,
        "seq_lens": seq_lens,
    }
    if any(not torch.is_tensor(value) for value in tensors.values()):
        raise PagedAttentionKernelError("paged attention inputs must be tensors")
    if query.ndim != 4 or query.shape[2] != 1:
        raise PagedAttentionKernelError("query must have shape [batch, heads, 1, head_dim]")
    if key_pool.ndim != 4 or value_pool.shape != key_pool.shape:
        raise PagedAttentionKernelError(
            "KV pool must have shape [pages, kv_heads, page_size, head_dim]"
        )
    if page_table.ndim != 2 or seq_lens.ndim != 1 or page_table.shape[0] != query.shape[0]:
        raise PagedAttentionKernelError("page table and sequence lengths must match query batch")
    if seq_lens.shape[0] != query.shape[0] or seq_lens.dtype != torch.long:
        raise PagedAttentionKernelError("seq_lens must be a torch.long vector")
    if page_table.dtype != torch.long:
        raise PagedAttentionKernelError("page_table must be a torch.long matrix")
    device = query.device
    if any(value.device != device for value in tensors.values()):
        raise PagedAttentionKernelError("paged attention inputs must share a device")
    if key_pool.dtype != query.dtype or value_pool.dtype != query.dtype:
        raise PagedAttentionKernelError("query and KV pool must share a dtype")
    if key_pool.shape[3] != query.shape[3]:
        raise PagedAttentionKernelError("query and KV pool head dimensions must match")
    if query.shape[1] % key_pool.shape[1] != 0:
        raise PagedAttentionKernelError("query heads must be divisible by KV heads")
    if key_valid_mask is not None:
        if (
            key_valid_mask.ndim != 2
            or key_valid_mask.shape[0] != query.shape[0]
            or key_valid_mask.dtype != torch.bool
            or key_valid_mask.device != device
        ):
            raise PagedAttentionKernelError(
                "key_valid_mask must be [batch, max_seq] bool on device"
            )
    # The reference checks row by row with one host sync per check; here every
    # flag is computed on the device and read back in one transfer, and the
    # first failing check raises in the reference's order: positive lengths,
    # table capacity, then per row an invalid used entry before a short mask.
    page_size = key_pool.shape[2]
    width = page_table.shape[1]
    page_counts = (seq_lens + page_size - 1) // page_size
    used = torch.arange(width, device=device) < page_counts[:, None]
    bad_entry = (((page_table < 0) | (page_table >= key_pool.shape[0])) & used).any(dim=1)
    row_code = bad_entry.to(torch.int64)
    if key_valid_mask is not None:
        short_mask = seq_lens > key_valid_mask.shape[1]
        row_code = torch.where(bad_entry, row_code, 2 * short_mask.to(torch.int64))
    flags = torch.cat([
        (seq_lens <= 0).any().view(1).to(torch.int64),
        (seq_lens > width * page_size).any().view(1).to(torch.int64),
        row_code,
    ]).tolist()
    if flags[0]:
        raise PagedAttentionKernelError("sequence lengths must be positive")
    if flags[1]:
        raise PagedAttentionKernelError("sequence length exceeds page table capacity")
    for code in flags[2:]:
        if code == 1:
            raise PagedAttentionKernelError("page table contains an invalid page table entry")
        if code == 2:
            raise PagedAttentionKernelError("key_valid_mask is shorter than sequence length")
    return (
        int(query.shape[0]),
        int(query.shape[1]),
        int(key_pool.shape[1]),
        int(key_pool.shape[2]),
    )


def paged_attention_decode(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    key_valid_mask: torch.Tensor | None = None,
    *,
    new_key: torch.Tensor | None = None,
    new_value: torch.Tensor | None = None,
    kernel_seq_len: int | None = None,
    kernel_page_count: int | None = None,
    block_n: int = 128,
    num_warps: int = 4,
    scale: float | None = None,
    use_triton: bool = True,
    validate: bool = True,
) -> torch.Tensor:
    """One-token GQA attention read directly from a physical page pool.

    ``page_table`` maps each request's logical page to a physical page;
    ``key_valid_mask`` supports left-padded prompts.  Returns [B, H, 1, D].
    """
    del use_triton  # always the HIP kernel
    if validate:
        _, num_heads, num_kv_heads, page_size = _validate_inputs(
            query, key_pool, value_pool, page_table, seq_lens, key_valid_mask
        )
    else:
        num_heads = int(query.shape[1])
        num_kv_heads = int(key_pool.shape[1])
        page_size = int(key_pool.shape[2])
    scale = float(scale if scale is not None else 1.0 / math.sqrt(query.shape[-1]))
    if (new_key is None) != (new_value is None):
        raise PagedAttentionKernelError("new_key and new_value must be provided together")
    if new_key is not None:
        expected_shape = (query.shape[0], num_kv_heads, 1, query.shape[-1])
        if (
            tuple(new_key.shape) != expected_shape
            or tuple(new_value.shape) != expected_shape
            or new_key.dtype != query.dtype
            or new_value.dtype != query.dtype
            or new_key.device != query.device
            or new_value.device != query.device
        ):
            raise PagedAttentionKernelError(
                "new KV must have shape [batch, kv_heads, 1, head_dim] and match query"
            )
    if query.device.type != "cuda":
        raise PagedAttentionKernelError("paged attention requires a GPU (HIP) device")
    block_n = int(block_n)
    if block_n <= 0 or block_n & (block_n - 1):
        raise PagedAttentionKernelError("block_n must be a positive power of two")
    if int(num_warps) <= 0:
        raise PagedAttentionKernelError("num_warps must be positive")
    if kernel_seq_len is None:
        max_seq_len = int(seq_lens.max().item())
        kernel_seq_len = int(math.ceil(max_seq_len / block_n) * block_n)
    else:
        kernel_seq_len = int(kernel_seq_len)
    if kernel_page_count is None:
        kernel_page_count = int(math.ceil(kernel_seq_len / page_size))
    else:
        kernel_page_count = int(kernel_page_count)
    if kernel_seq_len <= 0 or kernel_page_count <= 0:
        raise PagedAttentionKernelError("kernel metadata dimensions must be positive")
    del num_heads
    try:
        out = ops.paged_decode(
            query[:, :, 0, :],
            key_pool,
            value_pool,
            page_table,
            seq_lens,
            max_seq_len=kernel_seq_len,
            scale=scale,
            layout=ops.LAYOUT_HND,
            valid_mask=key_valid_mask,
            new_k=None if new_key is None else new_key[:, :, 0, :],
            new_v=None if new_value is None else new_value[:, :, 0, :],
            out=torch.empty_like(query)[:, :, 0, :],
            key_limit=kernel_seq_len,
            table_read_width=kernel_page_count,
        )
    except ops.AttentionArgumentError as exc:
        raise PagedAttentionKernelError(str(exc)) from exc
    return out.unsqueeze(2)
