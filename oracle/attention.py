"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker / CPU baseline.  The
product path (``voiceagent_amd``) never calls it.

Each function restates the reference's per-sequence matmul/softmax fallback
in plain PyTorch on the CPU, evaluated in float32 (or float64 when asked):

* :func:`store_kvcache`   — qwen_asr_vllm/layers/attention.py:31-67
* :func:`write_current_kv` — qwen_asr_vllm/agent/qwen_tts_paged_attention.py:519-532
* :func:`paged_decode`     — _reference_paged_attention,
  qwen_asr_vllm/agent/qwen_tts_paged_attention.py:353-380 (kv head = h // G,
  :169-170 and :370-372), with the Triton kernel's masking (:229-234, :267)
* :func:`varlen_attention` — flash_attn_varlen_func semantics as the engine uses
  them: causal with bottom-right alignment (qwen_asr_vllm/layers/attention.py:1-11,
  92-107), non-causal block-diagonal windows (:121-139); equal to upstream
  eager_attention_forward + the causal or _prepare_attention_mask masks
  (reference/modeling_qwen3_asr.py:90-113, 649-667).
* :func:`quantize_fp8`, :func:`dequantize_fp8` — the FP8 KV pool format, OCP
  e4m3 (float8_e4m3fn) codes with one scale per pool: code =
  e4m3_rne(clamp(x * (1/scale), -448, 448)), value = code * scale.  The
  reference engine keeps K/V in the model dtype; this is the KV-quantisation
  lever its README names (README.md:427-435), with vLLM's per-tensor scale
  convention.  :func:`store_kvcache`, :func:`paged_decode` and
  :func:`varlen_attention` read and write FP8 pools through these two.
* :func:`rms_norm`, :func:`rope_cache`, :func:`apply_rope`, :func:`qk_norm_rope` —
  Qwen3's q/k prologue: RMSNorm._norm (qwen_asr_vllm/layers/layernorm.py:19-25),
  RotaryEmbedding's cache and apply_rotary_emb
  (qwen_asr_vllm/layers/rotary_embedding.py:9-32), in the order
  Qwen3Attention.forward applies them (qwen_asr_vllm/models/qwen3.py:42-48),
  evaluated by eager torch ops with the reference's dtype conversions.

Masking convention: masked scores are -inf; a query row with no attended key
returns 0 (the Triton kernel's result, qwen_tts_paged_attention.py:223-279).

Pinning (tests/test_oracle.py): golden vectors regenerated from the
reference tests' own seeded fixtures and checked against a float64 brute
force written with scalar loops; the reference's known-answer tests (exact
1.0/9.0 outputs, the SDPA comparison, window boundaries); torch's
scaled_dot_product_attention with independently built masks; closed forms
(single key, constant V, zero query, block-table permutation); and planted
mistakes (GQA mapping, causal alignment, block indexing) that must fail.
The prologue functions are pinned by closed forms (a constant row normalises
to +-1/sqrt(1 + eps/c^2); position 0 is the identity), by an independent
float64 complex-number rotation with the reference's frequency formula, and
by planted mistakes (swapped halves, flipped sign, a missing weight).
"""

from __future__ import annotations

import torch

NHD = "nhd"  # [num_blocks, block_size, Hkv, D]
HND = "hnd"  # [pages, Hkv, page_size, D]
FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def quantize_fp8(x: torch.Tensor, scale: float) -> torch.Tensor:
    """OCP e4m3 codes of x / scale: x * (1/scale) in fp32 (1/scale itself
    rounded to fp32), saturated to +-448, rounded to nearest even by torch's
    float8_e4m3fn conversion."""
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)
    y = x.float() * inv
    return y.clamp(-FP8_MAX, FP8_MAX).to(FP8)


def dequantize_fp8(codes: torch.Tensor, scale: float) -> torch.Tensor:
    """Values of e4m3 codes: code * scale, in fp32."""
    return codes.float() * torch.tensor(scale, dtype=torch.float32)


def _as_values(pool: torch.Tensor, scale: float | None) -> torch.Tensor:
    return dequantize_fp8(pool, scale) if pool.dtype == FP8 else pool


def _block_size(pool: torch.Tensor, layout: str) -> int:
    return int(pool.shape[1] if layout == NHD else pool.shape[2])


def gather_rows(pool: torch.Tensor, table_row: torch.Tensor, positions: torch.Tensor,
                layout: str = NHD) -> torch.Tensor:
    """Rows [len(positions), Hkv, D] of one sequence's paged K or V.

    Position p lives in block table_row[p // block_size], slot p % block_size
    (qwen_tts_paged_attention.py:366-369; model_runner.py:202-204).
    """
    bs = _block_size(pool, layout)
    pages = table_row.long().index_select(0, positions // bs)
    offsets = positions % bs
    if layout == NHD:
        return pool[pages, offsets]
    return pool[pages, :, offsets, :]


def store_kvcache(key, value, k_cache, v_cache, slot_mapping, layout: str = NHD,
                  k_scale: float = 1.0, v_scale: float = 1.0):
    """Return copies of the pools after the store (slot -1 skips; others must be valid).

    cache.view(-1, Hkv * D)[slot] = key[i]   (layers/attention.py:42-49); an
    FP8 pool receives quantize_fp8(key[i], k_scale) (and v_scale for values).
    """
    kc, vc = k_cache.clone(), v_cache.clone()
    if kc.dtype == FP8:
        key, value = quantize_fp8(key, k_scale), quantize_fp8(value, v_scale)
    bs = _block_size(kc, layout)
    for i, slot in enumerate(slot_mapping.tolist()):
        if slot == -1:
            continue
        blk, off = divmod(int(slot), bs)
        if layout == NHD:
            kc[blk, off] = key[i]
            vc[blk, off] = value[i]
        else:
            kc[blk, :, off] = key[i]
            vc[blk, :, off] = value[i]
    return kc, vc


def write_current_kv(key_pool, value_pool, page_table, seq_lens, new_key, new_value,
                     layout: str = HND, k_scale: float = 1.0, v_scale: float = 1.0):
    """Copies of the pools with row seq_len-1 of every sequence replaced
    (qwen_tts_paged_attention.py:519-532).  new_key: [B, Hkv, D]; an FP8
    pool receives the quantised rows."""
    kp, vp = key_pool.clone(), value_pool.clone()
    if kp.dtype == FP8:
        new_key, new_value = quantize_fp8(new_key, k_scale), quantize_fp8(new_value, v_scale)
    bs = _block_size(kp, layout)
    for row in range(new_key.shape[0]):
        position = int(seq_lens[row]) - 1
        page = int(page_table[row, position // bs])
        offset = position % bs
        if layout == NHD:
            kp[page, offset] = new_key[row]
            vp[page, offset] = new_value[row]
        else:
            kp[page, :, offset] = new_key[row]
            vp[page, :, offset] = new_value[row]
    return kp, vp


def _masked_softmax_av(scores: torch.Tensor, values: torch.Tensor, keep: torch.Tensor | None):
    """softmax over the last dim with -inf masking, rows with no key -> 0, then @ values."""
    if keep is not None:
        scores = scores.masked_fill(~keep, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    probs = torch.nan_to_num(probs, nan=0.0)  # fully masked rows
    return probs @ values


def paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale, *, layout: str = NHD,
                 valid_mask=None, key_limit=None, table_read_width=None,
                 compute_dtype=torch.float32, k_scale: float = 1.0, v_scale: float = 1.0):
    """One query token per sequence over a paged pool.  q: [B, Hq, D] -> [B, Hq, D].

    Per row (qwen_tts_paged_attention.py:363-379): gather the first L rows
    through the table, repeat_interleave the kv heads by G = Hq / Hkv, then
    softmax(q . K^T * scale) @ V.  ``valid_mask[b, t]`` masks token t when t is
    inside the mask's width (tokens past it count as valid); a masked token's
    value row counts as 0, as the Triton kernel loads it (:258-265), so that a
    non-finite value there does not reach the output.  ``key_limit`` and
    ``table_read_width`` are the Triton kernel's MAX_SEQ_LEN and
    num_page_slots (:223-241): tokens at or past key_limit are not attended,
    and table columns at or past table_read_width read as block 0.  FP8
    pools are read as dequantize_fp8(code, k_scale / v_scale).
    """
    k_cache, v_cache = _as_values(k_cache, k_scale), _as_values(v_cache, v_scale)
    B, hq, d = q.shape
    outs = []
    for b in range(B):
        length = int(context_lens[b])
        if key_limit is not None:
            length = min(length, int(key_limit))
        if length <= 0:
            outs.append(torch.zeros(1, hq, d, dtype=compute_dtype))
            continue
        pos = torch.arange(length)
        table_row = block_tables[b]
        if table_read_width is not None and table_row.shape[0] > table_read_width:
            table_row = table_row.clone()
            table_row[int(table_read_width):] = 0
        keys = gather_rows(k_cache, table_row, pos, layout).to(compute_dtype)
        values = gather_rows(v_cache, table_row, pos, layout).to(compute_dtype)
        group = hq // keys.shape[1]
        keys = keys.permute(1, 0, 2).repeat_interleave(group, dim=0)  # [Hq, L, D]
        values = values.permute(1, 0, 2).repeat_interleave(group, dim=0)
        qb = q[b].to(compute_dtype).unsqueeze(1)  # [Hq, 1, D]
        scores = (qb @ keys.transpose(-1, -2)) * scale  # [Hq, 1, L]
        keep = None
        if valid_mask is not None:
            width = valid_mask.shape[1]
            keep = torch.ones(length, dtype=torch.bool)
            n = min(width, length)
            keep[:n] = valid_mask[b, :n].bool()
            values = values.masked_fill(~keep.view(1, length, 1), 0.0)
            keep = keep.view(1, 1, length)
        outs.append(_masked_softmax_av(scores, values, keep).transpose(0, 1))
    return torch.cat(outs, dim=0)


def varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, causal, *, k_cache=None,
                     v_cache=None, block_tables=None, layout: str = NHD,
                     compute_dtype=torch.float32, k_scale: float = 1.0, v_scale: float = 1.0):
    """Packed variable-length attention.  q: [total_q, Hq, D] -> same shape.

    Sequence s owns queries [cu_q[s], cu_q[s+1]) and k_len = cu_k[s+1]-cu_k[s]
    keys.  Causal is bottom-right aligned: query i sees key j iff
    j <= k_len - q_len + i (layers/attention.py:8-10).  Keys come from packed
    k/v rows [cu_k[s], cu_k[s+1]) without a pool; with a pool, keys
    j < k_len - q_len are read through ``block_tables`` and the rest from k/v
    rows aligned with the queries (from the pool as well when k is None).
    FP8 pools are read as dequantize_fp8(code, k_scale / v_scale).
    """
    if k_cache is not None:
        k_cache, v_cache = _as_values(k_cache, k_scale), _as_values(v_cache, v_scale)
    total_q, hq, d = q.shape
    out = torch.zeros(total_q, hq, d, dtype=compute_dtype)
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    for s in range(len(cq) - 1):
        q0, q1 = cq[s], cq[s + 1]
        ql, kl = q1 - q0, ck[s + 1] - ck[s]
        if ql <= 0:
            continue
        if k_cache is None:
            keys = k[ck[s]:ck[s + 1]]
            values = v[ck[s]:ck[s + 1]]
        else:
            prefix = kl - ql if k is not None else kl
            pos = torch.arange(prefix)
            keys = gather_rows(k_cache, block_tables[s], pos, layout)
            values = gather_rows(v_cache, block_tables[s], pos, layout)
            if k is not None:
                keys = torch.cat([keys, k[q0:q1]], dim=0)
                values = torch.cat([values, v[q0:q1]], dim=0)
        keys = keys.to(compute_dtype)
        values = values.to(compute_dtype)
        group = hq // keys.shape[1]
        keys = keys.permute(1, 0, 2).repeat_interleave(group, dim=0)  # [Hq, kl, D]
        values = values.permute(1, 0, 2).repeat_interleave(group, dim=0)
        qs = q[q0:q1].to(compute_dtype).permute(1, 0, 2)  # [Hq, ql, D]
        scores = (qs @ keys.transpose(-1, -2)) * scale  # [Hq, ql, kl]
        keep = None
        if causal:
            i = torch.arange(ql).view(ql, 1)
            j = torch.arange(kl).view(1, kl)
            keep = (j <= kl - ql + i).view(1, ql, kl)
        out[q0:q1] = _masked_softmax_av(scores, values, keep).permute(1, 0, 2)
    return out


# ------------------------------------------------------------ q/k prologue
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm._norm (layers/layernorm.py:19-25): fp32 mean of squares and
    rsqrt, back to x's dtype, then an in-place product with the weight (the
    result keeps x's dtype)."""
    orig = x.dtype
    xf = x.float()
    variance = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    y = xf.to(orig)
    y.mul_(weight)
    return y


def rope_cache(head_dim: int, max_position: int, base: float) -> torch.Tensor:
    """The rotary table [max_position, head_dim] = cos | sin in fp32
    (RotaryEmbedding.__init__, layers/rotary_embedding.py:18-26, without the
    singleton head axis)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    positions = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j->ij", positions, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def apply_rope(x: torch.Tensor, cos_sin: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """apply_rotary_emb at per-token positions (layers/rotary_embedding.py:9-15,
    28-32): x [T, H, D], first half paired with the second, fp32 math, result
    in x's dtype."""
    cos, sin = cos_sin[positions.long()].unsqueeze(1).chunk(2, dim=-1)
    first, second = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((first * cos - second * sin, second * cos + first * sin), dim=-1).to(x.dtype)


def qk_norm_rope(q, k, positions, q_norm_weight, k_norm_weight, eps, cos_sin):
    """Qwen3Attention.forward's prologue (models/qwen3.py:44-48)."""
    return (apply_rope(rms_norm(q, q_norm_weight, eps), cos_sin, positions),
            apply_rope(rms_norm(k, k_norm_weight, eps), cos_sin, positions))
