"""Drop-in attention layers for the qwen_asr_vllm engine on MI355X.

Same classes, constructor arguments and forward signatures as
qwen_asr_vllm/layers/attention.py:52-139; the computation runs in the HIP
kernels of ``libvoiceagent_attn.so`` (there is no torch or CPU fallback).

``PagedAttention.forward(q, k, v)`` reads the batch metadata from
:func:`get_attention_context` exactly as the reference does
(layers/attention.py:87-107):

* with a bound cache and a decode-only batch (``max_seqlen_q == 1`` and one
  query per sequence) it launches the split-context paged decode kernel with
  the store of the new K/V rows fused in (one launch per layer);
* with a bound cache and any other batch it launches the causal varlen
  kernel over the paged prefix with the store fused;
* without a cache (``k_cache.numel() == 0``, the memory-profiling pass) it
  runs causal varlen attention over the packed k/v.

Fusing the store relies on the engine's invariant that ``slot_mapping[i]``
is the pool slot of query token i's position (model_runner.py:202-204,
graph_runner.py:165-168); ``fuse_store = False`` restores the reference's
store-then-attend order with two launches.

``forward(q, k, v, prologue=...)`` also takes Qwen3's q/k prologue
(:class:`voiceagent_amd.ops.QKPrologue`: the q_norm / k_norm weights and eps,
the rotary cos/sin cache and the tokens' positions): q and k are then the
raw projections, and the layer applies RMSNorm and RoPE to them as
Qwen3Attention.forward does before calling attention (models/qwen3.py:42-48).
A decode batch with the fused store applies it inside the decode launch.  A
prefill batch (head_dim 128, 16-bit pool or none) runs ``ops.qk_norm_rope``
over the keys alone and lets the varlen launch normalise and rotate the
queries itself; any other batch runs ``ops.qk_norm_rope`` over both first.
Qwen3Attention then passes the prologue instead of calling q_norm, k_norm and
rotary_emb itself.

``kv_layout`` names the pool layout: ``"nhd"`` ``[num_blocks, block_size,
Hkv, D]`` as model_runner.py:116-131 allocates it (the default), or
``"hnd"`` ``[num_blocks, Hkv, block_size, D]``, in which one (block, kv head)
is a contiguous 4 KiB run; decode reads it ~9% faster.  Every reader and
writer of the pool is a kernel of this package, so an engine may allocate
either layout and set ``PagedAttention.kv_layout`` to match.

The pool may also be FP8 (``torch.float8_e4m3fn``, half the bytes of bf16):
the layer's ``k_scale`` / ``v_scale`` (vLLM's per-tensor convention, 1.0 by
default) give each code's value, every store quantises and every read
dequantises.  The engine allocates the cache in that dtype
(model_runner.py:119) and sets the scales on the layers.
"""

from __future__ import annotations

import torch
from torch import nn

from voiceagent_amd import ops
from voiceagent_amd.layers.context import get_attention_context


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> None:
    """Scatter key/value rows [N, Hkv, D] into an NHD pool [nb, bs, Hkv, D].

    Mirrors qwen_asr_vllm/layers/attention.py:52-67, including its stride
    contract (assertions :61-64): rows may be strided (the engine's ``v`` is a
    view of the fused qkv output) but each row's heads are contiguous.  An FP8
    (float8_e4m3fn) pool receives the codes of key / k_scale and
    value / v_scale; the scales are ignored for a 16-bit or fp32 pool.
    """
    num_tokens, num_heads, head_dim = key.shape
    hidden = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == hidden and v_cache.stride(1) == hidden
    assert slot_mapping.numel() == num_tokens
    ops.store_kvcache(key, value, k_cache, v_cache, slot_mapping, layout=ops.LAYOUT_NHD,
                      k_scale=k_scale, v_scale=v_scale)


def _decode_split(context) -> int:
    """Decode split of this step: fixed partitions from an exact max_seqlen_k
    (an eager step's), the automatic split for a bound (a graph's
    max_model_len, or a context that does not say)."""
    return ops.SPLIT_EXACT if getattr(context, "max_seqlen_k_exact", False) else 0


class PagedAttention(nn.Module):
    fuse_store = True
    # True: prefill batches let the varlen launch apply the query prologue
    # (the keys alone go through the standalone kernel first).  Off by
    # default: over config 3 both ways take 66 us per layer, as each item
    # of the varlen launch fetches the cos / sin rows of its 64 positions
    # for one KV head (8 times the standalone kernel's rotary traffic per
    # position), which costs what the saved query round trip through HBM
    # saves.  False: the standalone kernel over q and k, then the launch.
    varlen_fuse_prologue = False
    kv_layout = ops.LAYOUT_NHD
    k_scale = 1.0  # FP8 pools: value of a key code = code * k_scale
    v_scale = 1.0

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        # Bound to slices of the engine-owned cache by the model runner.
        self.k_cache = torch.tensor([])
        self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                prologue: ops.QKPrologue | None = None) -> torch.Tensor:
        context = get_attention_context()
        num_seqs = context.cu_seqlens_k.numel() - 1
        decode = context.max_seqlen_q == 1 and q.shape[0] == num_seqs
        q_pro = None  # the prologue the varlen launch applies to q itself
        if prologue is not None:
            if self.k_cache.numel() and decode and self.fuse_store:
                return self._decode_fused(q, k, v, context, prologue)
            if not decode and self._varlen_takes_prologue(q):
                _, k = ops.qk_norm_rope(None, k, prologue)
                q_pro = prologue
            else:
                q, k = ops.qk_norm_rope(q, k, prologue)
        if not self.k_cache.numel():
            # Memory-profiling pass before the cache exists: packed causal varlen.
            return ops.varlen_attention(
                q,
                k,
                v,
                context.cu_seqlens_q,
                context.cu_seqlens_k,
                context.max_seqlen_q,
                context.max_seqlen_k,
                scale=self.scale,
                causal=True,
                prologue=q_pro,
            )
        if decode:
            if self.fuse_store:
                return self._decode_fused(q, k, v, context, None)
            self._store(k, v, context.slot_mapping)
            return ops.paged_decode(
                q,
                self.k_cache,
                self.v_cache,
                context.block_tables,
                context.cu_seqlens_k,
                lens_cumulative=True,
                max_seq_len=context.max_seqlen_k,
                scale=self.scale,
                layout=self.kv_layout,
                split_tokens=_decode_split(context),
                k_scale=self.k_scale,
                v_scale=self.v_scale,
            )
        if self.fuse_store:
            return ops.varlen_attention(
                q,
                k,
                v,
                context.cu_seqlens_q,
                context.cu_seqlens_k,
                context.max_seqlen_q,
                context.max_seqlen_k,
                scale=self.scale,
                causal=True,
                k_cache=self.k_cache,
                v_cache=self.v_cache,
                block_tables=context.block_tables,
                slot_mapping=context.slot_mapping,
                layout=self.kv_layout,
                k_scale=self.k_scale,
                v_scale=self.v_scale,
                prologue=q_pro,
            )
        self._store(k, v, context.slot_mapping)
        return ops.varlen_attention(
            q,
            None,
            None,
            context.cu_seqlens_q,
            context.cu_seqlens_k,
            context.max_seqlen_q,
            context.max_seqlen_k,
            scale=self.scale,
            causal=True,
            k_cache=self.k_cache,
            v_cache=self.v_cache,
            block_tables=context.block_tables,
            layout=self.kv_layout,
            k_scale=self.k_scale,
            v_scale=self.v_scale,
            prologue=q_pro,
        )

    def _varlen_takes_prologue(self, q: torch.Tensor) -> bool:
        """Whether the varlen launch can apply the query prologue itself:
        head_dim 128, 16-bit q, and a 16-bit pool or none."""
        return (self.varlen_fuse_prologue and q.shape[-1] == 128 and
                q.dtype in (torch.bfloat16, torch.float16) and
                (not self.k_cache.numel() or self.k_cache.dtype == q.dtype))

    def _decode_fused(self, q, k, v, context, prologue: ops.QKPrologue | None) -> torch.Tensor:
        """One launch: (prologue,) store of the new rows, paged decode."""
        return ops.paged_decode(
            q,
            self.k_cache,
            self.v_cache,
            context.block_tables,
            context.cu_seqlens_k,
            lens_cumulative=True,
            max_seq_len=context.max_seqlen_k,
            scale=self.scale,
            layout=self.kv_layout,
            new_k=k,
            new_v=v,
            new_slots=context.slot_mapping,
            prologue=prologue,
            split_tokens=_decode_split(context),
            k_scale=self.k_scale,
            v_scale=self.v_scale,
        )

    def _store(self, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Unfused store: the reference's store_kvcache (and its stride
        contract) for an NHD pool, the same scatter by layout otherwise."""
        if self.kv_layout == ops.LAYOUT_NHD and self.k_cache.dtype != ops.FP8_KV_DTYPE:
            store_kvcache(k, v, self.k_cache, self.v_cache, slot_mapping)
        else:
            ops.store_kvcache(k, v, self.k_cache, self.v_cache, slot_mapping,
                              layout=self.kv_layout, k_scale=self.k_scale, v_scale=self.v_scale)


class VarlenSelfAttention(nn.Module):
    """Non-causal block-diagonal varlen attention for the audio encoder (no KV cache)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale

    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        cu_seqlens: torch.Tensor,
        max_seqlen: int,
    ) -> torch.Tensor:
        return ops.varlen_attention(
            q,
            k,
            v,
            cu_seqlens,
            cu_seqlens,
            max_seqlen,
            max_seqlen,
            scale=self.scale,
            causal=False,
        )
