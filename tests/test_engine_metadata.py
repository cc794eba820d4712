"""Engine metadata producers (eager and graph mode) against the formulas of
qwen_asr_vllm/engine/model_runner.py:183-233 and graph_runner.py:81-191,
checked by brute force on small batches (CPU only)."""

from dataclasses import dataclass, field

import pytest
import torch

from voiceagent_amd.engine import DecodeGraphMetadata, prepare_batch, slot_of


@dataclass
class Seq:
    length: int
    num_computed_tokens: int
    block_table: list[int] = field(default_factory=list)

    def __len__(self):
        return self.length


def _blocks(n_tokens, bs, start):
    return list(range(start, start + (n_tokens + bs - 1) // bs))


def test_slot_of_matches_brute_force():
    table = [7, 3, 9]
    bs = 4
    flat = [b * bs + o for b in table for o in range(bs)]
    for pos in range(len(table) * bs):
        assert slot_of(table, pos, bs) == flat[pos]


def test_prepare_batch_mixed_prefill_prefix_and_decode():
    bs = 16
    seqs = [
        Seq(37, 0, [5, 2, 11]),           # fresh prefill
        Seq(40, 32, [1, 4, 6]),           # prefix hit: 8 new tokens at 32..39
        Seq(17, 16, [8, 9]),              # decode: one token at position 16
    ]
    positions, ctx = prepare_batch(seqs, bs, "cpu")
    assert positions.tolist() == list(range(0, 37)) + list(range(32, 40)) + [16]
    assert ctx.cu_seqlens_q.tolist() == [0, 37, 45, 46]
    assert ctx.cu_seqlens_k.tolist() == [0, 37, 77, 94]
    assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (37, 40)
    slots = ctx.slot_mapping.tolist()
    want = [s.block_table[p // bs] * bs + p % bs
            for s in seqs for p in range(s.num_computed_tokens, len(s))]
    assert slots == want
    assert ctx.block_tables.tolist() == [[5, 2, 11], [1, 4, 6], [8, 9, -1]]
    for t in (ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.slot_mapping, ctx.block_tables):
        assert t.dtype == torch.int32
    # an eager step's max_seqlen_k is the exact longest context
    assert ctx.max_seqlen_k_exact


def test_prepare_batch_rejects_bad_progress():
    with pytest.raises(ValueError):
        prepare_batch([Seq(4, 5, [0])], 16, "cpu")


def test_graph_metadata_stage_pads_rows():
    bs = 16
    meta = DecodeGraphMetadata(max_batch_size=8, max_blocks=4, block_size=bs,
                               max_model_len=64, device="cpu", buckets=[2, 4, 8])
    seqs = [Seq(20, 19, [3, 7]), Seq(1, 0, [9]), Seq(33, 32, [0, 1, 2])]
    bucket = meta.stage(seqs)
    assert bucket == 4
    ctx = meta.context(bucket)
    assert ctx.max_seqlen_q == 1 and ctx.max_seqlen_k == 64
    assert not ctx.max_seqlen_k_exact  # max_model_len is only a bound
    assert ctx.cu_seqlens_q.tolist() == [0, 1, 2, 3, 4]
    # real rows accumulate full lengths; the padding row adds a key length of 1
    assert ctx.cu_seqlens_k.tolist() == [0, 20, 21, 54, 55]
    assert ctx.slot_mapping.tolist() == [7 * bs + 3, 9 * bs + 0, 2 * bs + 0, -1]
    assert ctx.block_tables.tolist() == [[3, 7, 0, 0], [9, 0, 0, 0], [0, 1, 2, 0], [0, 0, 0, 0]]
    assert meta.positions[:bucket].tolist() == [19, 0, 32, 0]
    # a smaller batch afterwards re-pads the rows it no longer uses
    bucket = meta.stage(seqs[:1])
    assert bucket == 2
    assert meta.slot_mapping[:2].tolist() == [7 * bs + 3, -1]
    assert meta.cu_seqlens_k[:3].tolist() == [0, 20, 21]
    with pytest.raises(ValueError):
        meta.stage([Seq(1, 0, [0])] * 9)


def test_graph_metadata_warmup_state():
    meta = DecodeGraphMetadata(max_batch_size=4, max_blocks=2, block_size=16,
                               max_model_len=100, device="cpu")
    meta.warmup_state()
    assert meta.cu_seqlens_k.tolist() == [0, 17, 34, 51, 68]
    assert meta.slot_mapping.tolist() == [-1] * 4
    assert int(meta.block_tables.abs().sum()) == 0
