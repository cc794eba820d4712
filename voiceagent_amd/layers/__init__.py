from voiceagent_amd.layers.attention import PagedAttention, VarlenSelfAttention, store_kvcache
from voiceagent_amd.layers.context import (
    AttentionContext,
    attention_context,
    get_attention_context,
    set_attention_context,
)

__all__ = [
    "AttentionContext",
    "PagedAttention",
    "VarlenSelfAttention",
    "attention_context",
    "get_attention_context",
    "set_attention_context",
    "store_kvcache",
]
