"""Encoder window metadata: the producer of the block-diagonal ``cu_seqlens``.

Restates the closed-form token accounting of qwen_asr_vllm/audio/tokens.py:16-37
and the window rule of qwen_asr_vllm/audio/batcher.py:75-98: each request's
audio tokens are cut into full windows of ``13 * (n_window_infer // 100)``
tokens plus a remainder, so a token never attends across a request boundary.
"""

from __future__ import annotations

import torch

CHUNK_FRAMES = 100
"""Mel frames per convolution chunk."""


def conv_output_len(length: int) -> int:
    """Output length of one Conv2d(kernel=3, stride=2, padding=1)."""
    return (length - 1) // 2 + 1


def after_cnn_len(frames: int) -> int:
    """Frames left after the three stride-2 convolutions."""
    return conv_output_len(conv_output_len(conv_output_len(frames)))


TOKENS_PER_FULL_CHUNK = after_cnn_len(CHUNK_FRAMES)  # 13


def num_audio_tokens(mel_frames: int, chunk_frames: int = CHUNK_FRAMES) -> int:
    """Audio tokens produced by ``mel_frames`` mel frames (tokens.py:30-37)."""
    full_chunks, tail = divmod(mel_frames, chunk_frames)
    return full_chunks * after_cnn_len(chunk_frames) + after_cnn_len(tail)


def attention_window_tokens(n_window_infer: int, chunk_frames: int = CHUNK_FRAMES) -> int:
    """Tokens per encoder attention window (batcher.py:75-77): 104 for 800 frames."""
    return TOKENS_PER_FULL_CHUNK * (n_window_infer // chunk_frames)


def build_window_boundaries(audio_token_lens: list[int], window_tokens: int) -> list[int]:
    """Cumulative window boundaries over the packed tokens (batcher.py:80-98)."""
    boundaries = [0]
    running = 0
    for token_len in audio_token_lens:
        full_windows, remainder = divmod(int(token_len), window_tokens)
        for _ in range(full_windows):
            running += window_tokens
            boundaries.append(running)
        if remainder:
            running += remainder
            boundaries.append(running)
    return boundaries


def window_cu_seqlens(
    audio_token_lens: list[int], window_tokens: int, device: torch.device | str = "cpu"
) -> tuple[torch.Tensor, int]:
    """int32 ``cu_seqlens`` of the encoder windows and the widest window."""
    bounds = build_window_boundaries(audio_token_lens, window_tokens)
    widest = max((b - a for a, b in zip(bounds[:-1], bounds[1:])), default=0)
    return torch.tensor(bounds, dtype=torch.int32, device=device), widest
