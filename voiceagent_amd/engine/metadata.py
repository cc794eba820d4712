"""Producers of the attention metadata (mirror of the engine's two builders).

The attention layers only read an :class:`AttentionContext`; the engine
builds it in two ways, and both are restated here so the kernels can be
driven exactly as the engine drives them:

* :func:`prepare_batch` is the eager builder,
  qwen_asr_vllm/engine/model_runner.py:183-233.  Every sequence contributes
  its uncomputed tokens ``[num_computed_tokens, len)``.  The slot of position
  p is ``block_table[p // block_size] * block_size + p % block_size``
  (:202-204).  ``cu_seqlens_k`` accumulates full lengths (:211), and the
  block tables are padded with -1 to the widest (:216-217).
* :class:`DecodeGraphMetadata` is the graph-mode builder,
  qwen_asr_vllm/engine/graph_runner.py:60-191.  It keeps static device
  buffers sized for the largest bucket, plus pinned host mirrors.  Each step
  stages one decode token per sequence into the buffers.  Rows between the
  batch size and the captured bucket are padding: slot -1, block-table row 0
  and key length 1, so their reads stay inside block 0 and their writes are
  skipped (:150-191).  ``max_seqlen_k`` is baked in at ``max_model_len``
  (:81-94).

A sequence is any object with ``num_computed_tokens``, ``block_table`` (a list
of block ids) and ``len()``, the three attributes the reference builders read.
"""

from __future__ import annotations

from typing import Protocol, Sequence

import torch

from voiceagent_amd.layers.context import AttentionContext


class SequenceState(Protocol):
    num_computed_tokens: int
    block_table: list[int]

    def __len__(self) -> int: ...


def slot_of(block_table: Sequence[int], position: int, block_size: int) -> int:
    """Pool slot of ``position`` (model_runner.py:202-204, graph_runner.py:165-168)."""
    return int(block_table[position // block_size]) * block_size + position % block_size


def prepare_batch(
    sequences: Sequence[SequenceState], block_size: int, device: torch.device | str
) -> tuple[torch.Tensor, AttentionContext]:
    """Positions (int64) and the attention context of one eager forward.

    Mirrors ModelRunner._prepare (model_runner.py:183-233) without the token
    ids and audio spans, which do not reach the attention layers.
    """
    positions: list[int] = []
    slot_mapping: list[int] = []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    tables: list[list[int]] = []
    for seq in sequences:
        start, end = int(seq.num_computed_tokens), len(seq)
        if not 0 <= start <= end:
            raise ValueError(f"num_computed_tokens {start} outside [0, {end}]")
        positions.extend(range(start, end))
        slot_mapping.extend(slot_of(seq.block_table, p, block_size) for p in range(start, end))
        cu_q.append(cu_q[-1] + end - start)
        cu_k.append(cu_k[-1] + end)
        max_q = max(max_q, end - start)
        max_k = max(max_k, end)
        tables.append(list(seq.block_table))
    width = max((len(t) for t in tables), default=0)
    padded = [t + [-1] * (width - len(t)) for t in tables]
    i32 = {"dtype": torch.int32, "device": device}
    context = AttentionContext(
        cu_seqlens_q=torch.tensor(cu_q, **i32),
        cu_seqlens_k=torch.tensor(cu_k, **i32),
        max_seqlen_q=max_q,
        max_seqlen_k=max_k,
        slot_mapping=torch.tensor(slot_mapping, **i32),
        block_tables=torch.tensor(padded, **i32).reshape(len(tables), width),
        max_seqlen_k_exact=True,
    )
    return torch.tensor(positions, dtype=torch.int64, device=device), context


class DecodeGraphMetadata:
    """Static decode metadata for captured graphs (graph_runner.py:60-191)."""

    def __init__(
        self,
        max_batch_size: int,
        max_blocks: int,
        block_size: int,
        max_model_len: int,
        device: torch.device | str,
        buckets: Sequence[int] | None = None,
    ) -> None:
        self.max_batch_size = max_batch_size
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.max_model_len = max_model_len
        self.device = torch.device(device)
        self.buckets = sorted(buckets) if buckets else [max_batch_size]
        if self.buckets[-1] > max_batch_size:
            raise ValueError("a bucket exceeds max_batch_size")
        size = max_batch_size
        i32 = {"dtype": torch.int32, "device": self.device}
        self.positions = torch.zeros(size, dtype=torch.int64, device=self.device)
        self.slot_mapping = torch.full((size,), -1, **i32)
        self.cu_seqlens_q = torch.arange(size + 1, **i32)
        self.cu_seqlens_k = torch.zeros(size + 1, **i32)
        self.block_tables = torch.zeros(size, max_blocks, **i32)
        # Pinned host mirrors: the staging copies are asynchronous (graph_runner.py:72-79).
        pinned = {"pin_memory": self.device.type == "cuda"}
        self.host_positions = torch.zeros(size, dtype=torch.int64, **pinned)
        self.host_slot_mapping = torch.full((size,), -1, dtype=torch.int32, **pinned)
        self.host_cu_seqlens_k = torch.zeros(size + 1, dtype=torch.int32, **pinned)
        self.host_block_tables = torch.zeros(size, max_blocks, dtype=torch.int32, **pinned)

    def context(self, batch_size: int) -> AttentionContext:
        """The context a graph of ``batch_size`` rows captures (graph_runner.py:81-94)."""
        return AttentionContext(
            cu_seqlens_q=self.cu_seqlens_q[: batch_size + 1],
            cu_seqlens_k=self.cu_seqlens_k[: batch_size + 1],
            max_seqlen_q=1,
            max_seqlen_k=self.max_model_len,
            slot_mapping=self.slot_mapping[:batch_size],
            block_tables=self.block_tables[:batch_size],
        )

    def warmup_state(self) -> None:
        """Plausible decode state for warm-up and capture (graph_runner.py:103-114)."""
        n = self.max_batch_size
        ctx = min(self.block_size + 1, self.max_model_len)
        self.cu_seqlens_k.copy_(torch.arange(n + 1, dtype=torch.int32) * ctx)
        self.slot_mapping.fill_(-1)
        self.block_tables.zero_()
        self.positions.zero_()

    def bucket_for(self, batch_size: int) -> int | None:
        """Smallest bucket that holds ``batch_size`` rows (graph_runner.py:142-147)."""
        for size in self.buckets:
            if size >= batch_size:
                return size
        return None

    def stage(self, sequences: Sequence[SequenceState]) -> int:
        """Write one decode step's metadata into the static buffers; returns the bucket.

        Each sequence contributes its last position ``len - 1``
        (graph_runner.py:163-176); padding rows up to the bucket get slot -1,
        block-table row 0 and key length 1 (:157-160, :178-180).
        """
        batch = len(sequences)
        bucket = self.bucket_for(batch)
        if bucket is None:
            raise ValueError(f"no bucket for a batch of {batch}")
        self.host_slot_mapping[:bucket].fill_(-1)
        self.host_block_tables[:bucket].zero_()
        self.host_positions[:bucket].zero_()
        running = 0
        for i, seq in enumerate(sequences):
            pos = len(seq) - 1
            table = list(seq.block_table)
            if len(table) > self.max_blocks:
                raise ValueError(f"block table of {len(table)} exceeds max_blocks")
            self.host_positions[i] = pos
            self.host_slot_mapping[i] = slot_of(table, pos, self.block_size)
            self.host_block_tables[i, : len(table)] = torch.tensor(table, dtype=torch.int32)
            running += len(seq)
            self.host_cu_seqlens_k[i + 1] = running
        for i in range(batch, bucket):
            running += 1
            self.host_cu_seqlens_k[i + 1] = running
        nb = {"non_blocking": True}
        self.positions[:bucket].copy_(self.host_positions[:bucket], **nb)
        self.slot_mapping[:bucket].copy_(self.host_slot_mapping[:bucket], **nb)
        self.cu_seqlens_k[: bucket + 1].copy_(self.host_cu_seqlens_k[: bucket + 1], **nb)
        self.block_tables[:bucket].copy_(self.host_block_tables[:bucket], **nb)
        return bucket
