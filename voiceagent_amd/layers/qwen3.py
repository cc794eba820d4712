"""Qwen3's attention core with the q/k prologue on the MI355X kernels.

``Qwen3AttentionCore`` is ``Qwen3Attention.forward`` between the fused qkv
projection and ``o_proj`` (qwen_asr_vllm/models/qwen3.py:42-50): per-head
RMSNorm of q and k, rotary embedding at the tokens' positions, then paged
attention with the KV store.  It subclasses :class:`PagedAttention`, so the
model runner binds its cache slices the same way
(engine/model_runner.py:129-131).

* Decode batches (one query per sequence, cache bound) run in ONE launch: the
  paged decode kernel normalises and rotates q and the new key in registers,
  writes the new K/V row and attends (reference: q_norm, k_norm, rotary,
  store_kvcache and attention as separate launches).
* Other batches run the standalone prologue kernel over q and k, then the
  varlen path of :class:`PagedAttention`.  With ``varlen_fuse_prologue``
  set (off by default: no faster over config 3), prefill batches with
  head_dim 128 and a 16-bit pool or none run the standalone kernel over the
  keys alone, and the varlen launch normalises and rotates the queries
  itself, in registers, at each item's first key tile.

The norm weights and the rotary table mirror the reference modules: weights
``q_norm.weight`` / ``k_norm.weight`` of shape [head_dim]
(layers/layernorm.py:16-17), and the fp32 cos|sin table built on the host by
the reference formula (layers/rotary_embedding.py:18-26).
"""

from __future__ import annotations

import torch
from torch import nn

from voiceagent_amd import ops
from voiceagent_amd.layers.attention import PagedAttention
from voiceagent_amd.layers.context import get_attention_context


def rotary_cos_sin_cache(head_dim: int, max_position: int, base: float) -> torch.Tensor:
    """[max_position, head_dim] fp32 = cos | sin of position x inv_freq
    (RotaryEmbedding.__init__, layers/rotary_embedding.py:18-26)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    positions = torch.arange(max_position, dtype=torch.float)
    freqs = torch.outer(positions, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


class Qwen3AttentionCore(PagedAttention):
    fuse_prologue = True

    def __init__(self, num_heads: int, head_dim: int, num_kv_heads: int, *, eps: float = 1e-6,
                 max_position: int = 32768, rope_theta: float = 1_000_000.0):
        super().__init__(num_heads, head_dim, head_dim ** -0.5, num_kv_heads)
        self.eps = eps
        self.q_norm_weight = nn.Parameter(torch.ones(head_dim))
        self.k_norm_weight = nn.Parameter(torch.ones(head_dim))
        self.register_buffer("cos_sin_cache",
                             rotary_cos_sin_cache(head_dim, max_position, rope_theta),
                             persistent=False)

    def prologue(self, positions: torch.Tensor) -> ops.QKPrologue:
        return ops.QKPrologue(self.q_norm_weight, self.k_norm_weight, self.eps,
                              self.cos_sin_cache, positions)

    def forward(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                v: torch.Tensor) -> torch.Tensor:
        """positions [T] (int64), q [T, Hq, D], k/v [T, Hkv, D]: raw projections."""
        context = get_attention_context()
        pro = self.prologue(positions)
        num_seqs = context.cu_seqlens_k.numel() - 1
        decode = context.max_seqlen_q == 1 and q.shape[0] == num_seqs
        if self.fuse_prologue and self.fuse_store and decode and self.k_cache.numel():
            return ops.paged_decode(
                q,
                self.k_cache,
                self.v_cache,
                context.block_tables,
                context.cu_seqlens_k,
                lens_cumulative=True,
                max_seq_len=context.max_seqlen_k,
                scale=self.scale,
                new_k=k,
                new_v=v,
                new_slots=context.slot_mapping,
                prologue=pro,
            )
        if self.fuse_prologue:
            # Prefill batches: the varlen launch applies the query prologue.
            return super().forward(q, k, v, prologue=pro)
        qn, kn = ops.qk_norm_rope(q, k, pro)
        return super().forward(qn, kn, v)
