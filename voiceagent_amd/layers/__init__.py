from voiceagent_amd.layers.attention import PagedAttention, VarlenSelfAttention, store_kvcache
from voiceagent_amd.layers.context import (
    AttentionContext,
    attention_context,
    get_attention_context,
    set_attention_context,
)
from voiceagent_amd.layers.qwen3 import Qwen3AttentionCore, rotary_cos_sin_cache

__all__ = [
    "AttentionContext",
    "PagedAttention",
    "Qwen3AttentionCore",
    "VarlenSelfAttention",
    "attention_context",
    "get_attention_context",
    "rotary_cos_sin_cache",
    "set_attention_context",
    "store_kvcache",
]
