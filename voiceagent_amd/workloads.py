"""Synthetic inputs of the benchmark configurations (shapes and distributions
of the headline workloads), shared by bench.py, the smoke test and the tests.

Geometry is the Qwen3-0.6B decoder (16 query heads, 8 KV heads, head_dim 128,
28 layers; qwen_asr_vllm/config.py:61-71) and the audio encoder (14 heads of
64; config.py:33-47).  Block tables are random permutations of free block
ids, one disjoint run per sequence, as the block manager hands them out.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from voiceagent_amd.audio import batcher

HQ, HKV, HEAD_DIM, LAYERS, BLOCK = 16, 8, 128, 28, 16
ENC_HEADS, ENC_DIM, ENC_WINDOW = 14, 64, 104


@dataclass
class DecodeBatch:
    """One decode step's inputs over ``num_layers`` layer pools (NHD)."""

    q: torch.Tensor                  # [B, Hq, D]
    k_pools: list[torch.Tensor]      # per layer [num_blocks, BLOCK, Hkv, D]
    v_pools: list[torch.Tensor]
    block_tables: torch.Tensor       # [B, width] int32, -1 padded
    context_lens: torch.Tensor       # [B] int32
    cu_seqlens_k: torch.Tensor       # [B + 1] int32
    slot_mapping: torch.Tensor       # [B] int32: slot of position len-1
    new_k: torch.Tensor              # [B, Hkv, D] rows stored this step
    new_v: torch.Tensor
    scale: float
    max_seq_len: int
    lens_list: list[int] = field(default_factory=list)

    @property
    def num_seqs(self) -> int:
        return int(self.q.shape[0])


def _tables(lens: list[int], num_blocks: int, block: int, gen: torch.Generator):
    need = [math.ceil(n / block) for n in lens]
    if sum(need) > num_blocks:
        raise ValueError("pool too small for the requested contexts")
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    width = max(need)
    rows, cursor = [], 0
    for n in need:
        rows.append(perm[cursor:cursor + n] + [-1] * (width - n))
        cursor += n
    return torch.tensor(rows, dtype=torch.int32)


def make_decode_batch(
    lens: list[int],
    *,
    num_blocks: int,
    num_layers: int = 1,
    dtype: torch.dtype = torch.bfloat16,
    kv_std: float = 1.0,
    device: str | torch.device = "cpu",
    seed: int = 0,
    device_rng: bool = False,
) -> DecodeBatch:
    """Build the inputs on the CPU generator (reproducible everywhere) and move
    them to ``device``; ``device_rng`` draws the pools with the device's own
    generator instead (fast for multi-GiB pools; values then differ from the
    CPU draw)."""
    gen = torch.Generator().manual_seed(seed)
    B = len(lens)
    tables = _tables(lens, num_blocks, BLOCK, gen)
    q = torch.randn(B, HQ, HEAD_DIM, generator=gen).to(dtype)
    new_k = (torch.randn(B, HKV, HEAD_DIM, generator=gen) * kv_std).to(dtype)
    new_v = (torch.randn(B, HKV, HEAD_DIM, generator=gen) * kv_std).to(dtype)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens_t, 0)
    slots = []
    for b, n in enumerate(lens):
        pos = n - 1
        slots.append(int(tables[b, pos // BLOCK]) * BLOCK + pos % BLOCK)
    dev = torch.device(device)
    k_pools, v_pools = [], []
    for layer in range(num_layers):
        shape = (num_blocks, BLOCK, HKV, HEAD_DIM)
        if device_rng and dev.type == "cuda":
            g = torch.Generator(device=dev).manual_seed(seed * 1000 + layer + 1)
            k = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).mul_(kv_std)
            v = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).mul_(kv_std)
            k_pools.append(k.to(dtype))
            v_pools.append(v.to(dtype))
            del k, v
        else:
            k_pools.append((torch.randn(shape, generator=gen) * kv_std).to(dtype).to(dev))
            v_pools.append((torch.randn(shape, generator=gen) * kv_std).to(dtype).to(dev))
    return DecodeBatch(
        q=q.to(dev),
        k_pools=k_pools,
        v_pools=v_pools,
        block_tables=tables.to(dev),
        context_lens=lens_t.to(dev),
        cu_seqlens_k=cu.to(dev),
        slot_mapping=torch.tensor(slots, dtype=torch.int32, device=dev),
        new_k=new_k.to(dev),
        new_v=new_v.to(dev),
        scale=1.0 / math.sqrt(HEAD_DIM),
        max_seq_len=max(lens),
        lens_list=list(lens),
    )


def cfg1_lens(seed: int = 0) -> list[int]:
    """Config 1: 4 sequences, context uniform in [17, 300]."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(17, 301, (4,), generator=gen).tolist()


def cfg2_lens(seed: int = 0, batch: int = 32) -> list[int]:
    """Config 2: batch 32, context uniform in [60, 600]."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(60, 601, (batch,), generator=gen).tolist()


def cfg5_lens(variant: str, seed: int = 0) -> list[int]:
    """Config 5: (i) one 16384-token context, (ii) 8 contexts uniform in [4096, 16384]."""
    if variant == "single":
        return [16384]
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(4096, 16385, (8,), generator=gen).tolist()


def decode_bytes(lens: list[int], hq: int = HQ, hkv: int = HKV, d: int = HEAD_DIM,
                 elem: int = 2, block: int = BLOCK) -> int:
    """Algorithmic HBM bytes of one decode call: K+V rows of every context
    token, q in, out, the used block-table entries and the lengths."""
    kv = sum(lens) * hkv * d * elem * 2
    qo = 2 * len(lens) * hq * d * elem
    tables = sum(math.ceil(n / block) for n in lens) * 4
    return kv + qo + tables + 4 * len(lens)


def store_bytes(num_tokens: int, hkv: int = HKV, d: int = HEAD_DIM, elem: int = 2) -> int:
    """Algorithmic bytes of store_kvcache: K and V rows read and written, slots read."""
    return 4 * num_tokens * hkv * d * elem + 4 * num_tokens


# ------------------------------------------------------------------ varlen
@dataclass
class VarlenBatch:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    cu_seqlens: torch.Tensor   # int32 [S + 1]
    max_seqlen: int
    lens: list[int]
    scale: float
    causal: bool


def make_varlen_batch(lens: list[int], heads: int, kv_heads: int, dim: int, *, causal: bool,
                      dtype=torch.bfloat16, device="cpu", seed: int = 0) -> VarlenBatch:
    gen = torch.Generator().manual_seed(seed)
    total = sum(lens)
    q = torch.randn(total, heads, dim, generator=gen).to(dtype)
    k = torch.randn(total, kv_heads, dim, generator=gen).to(dtype)
    v = torch.randn(total, kv_heads, dim, generator=gen).to(dtype)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    dev = torch.device(device)
    return VarlenBatch(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), max(lens), list(lens),
                       1.0 / math.sqrt(dim), causal)


def cfg3_lens(seed: int = 0) -> list[int]:
    """Config 3: 32 packed prompts, length uniform in [50, 450]."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(50, 451, (32,), generator=gen).tolist()


def cfg4_windows(seed: int = 0) -> list[int]:
    """Config 4: 32 clips of U[2, 30] s at 100 mel frames/s -> audio tokens ->
    104-token encoder windows (audio/tokens.py:30-37, audio/batcher.py:80-98)."""
    gen = torch.Generator().manual_seed(seed)
    secs = torch.rand(32, generator=gen) * 28.0 + 2.0
    frames = [int(s * 100) for s in secs.tolist()]
    tokens = [batcher.num_audio_tokens(f) for f in frames]
    bounds = batcher.build_window_boundaries(tokens, ENC_WINDOW)
    return [b - a for a, b in zip(bounds[:-1], bounds[1:])]


def causal_flops(lens: list[int], heads: int = HQ, dim: int = HEAD_DIM) -> int:
    """FLOPs of causal attention counting unmasked (query, key) pairs only."""
    return sum(4 * heads * dim * n * (n + 1) // 2 for n in lens)


def bidir_flops(lens: list[int], heads: int = ENC_HEADS, dim: int = ENC_DIM) -> int:
    return sum(4 * heads * dim * n * n for n in lens)


def varlen_bytes(lens: list[int], heads: int, kv_heads: int, dim: int, elem: int = 2) -> int:
    """q, k, v read once and out written once."""
    return sum(lens) * (2 * heads + 2 * kv_heads) * dim * elem
