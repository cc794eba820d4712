"""MI355X-native attention core for qwen_asr_vllm.

Hand-written gfx950 HIP kernels behind a C ABI (include/voiceagent_attn.h),
with Python modules that keep the reference's call signatures:

* ``voiceagent_amd.layers.attention``: ``PagedAttention``, ``VarlenSelfAttention``,
  ``store_kvcache`` (qwen_asr_vllm/layers/attention.py)
* ``voiceagent_amd.layers.context``: ``AttentionContext`` (qwen_asr_vllm/layers/context.py)
* ``voiceagent_amd.agent.paged_attention``: ``paged_attention_decode``
  (qwen_asr_vllm/agent/qwen_tts_paged_attention.py)
* ``voiceagent_amd.audio.batcher``: encoder window ``cu_seqlens``
  (qwen_asr_vllm/audio/batcher.py)
"""

__version__ = "0.1.0"
