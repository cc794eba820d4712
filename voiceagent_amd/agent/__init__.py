from voiceagent_amd.agent.paged_attention import PagedAttentionKernelError, paged_attention_decode

__all__ = ["PagedAttentionKernelError", "paged_attention_decode"]
