/*
 * voiceagent_attn.h — C ABI of the MI355X (gfx950) attention core for qwen_asr_vllm.
 *
 * Every entry point takes one plain-old-data argument struct plus a HIP stream
 * handle (passed as void*, so this header needs no HIP include), launches on
 * that stream, never allocates, never synchronises the host, and returns
 * VA_OK (0) or a negative status.  The message for the last failure on the
 * calling thread is available from va_last_error().
 *
 * Tensors are described by device pointers and element (not byte) strides;
 * the innermost (head_dim) dimension is always contiguous.  Element type is
 * chosen by a va_dtype; index arrays (block tables, lengths, slot maps) by a
 * va_index_dtype.  The caller owns every buffer.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   va_store_kvcache      <- store_kvcache / _store_kvcache_kernel,
 *                            qwen_asr_vllm/layers/attention.py:31-67
 *   va_paged_decode       <- flash_attn_varlen_func(block_table=..., q_len 1),
 *                            qwen_asr_vllm/layers/attention.py:87-107, and
 *                            paged_attention_decode / _paged_decode_attention_kernel,
 *                            qwen_asr_vllm/agent/qwen_tts_paged_attention.py:130-287, 383-516
 *   va_varlen_attention   <- flash_attn_varlen_func(causal=True, block_table / no cache),
 *                            qwen_asr_vllm/layers/attention.py:92-107, and
 *                            flash_attn_varlen_func(causal=False),
 *                            qwen_asr_vllm/layers/attention.py:121-139
 *   va_qk_norm_rope       <- q_norm / k_norm + rotary_emb of Qwen3Attention.forward,
 *                            qwen_asr_vllm/models/qwen3.py:42-48 (RMSNorm._norm,
 *                            layers/layernorm.py:19-25; apply_rotary_emb and
 *                            RotaryEmbedding.forward, layers/rotary_embedding.py:9-32);
 *                            also fused into va_paged_decode (va_decode_args.prologue)
 */
#ifndef VOICEAGENT_ATTN_H
#define VOICEAGENT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VA_ATTN_ABI_VERSION 6

/* status codes */
#define VA_OK 0
#define VA_ERR_INVALID_ARG (-1)
#define VA_ERR_UNSUPPORTED (-2)
#define VA_ERR_WORKSPACE (-3)
#define VA_ERR_LAUNCH (-4)

/* element types */
#define VA_BF16 0
#define VA_F16 1
#define VA_F32 2

/* index types */
#define VA_I32 0
#define VA_I64 1

/* KV pool element formats (va_kv_pool.kv_format) */
#define VA_KV_NATIVE 0   /* the entry point's dtype (bf16 / f16 / f32)              */
#define VA_KV_FP8_E4M3 1 /* OCP float8 e4m3 (float8_e4m3fn); element = code * scale */

/* how va_decode_args.lens is read */
#define VA_LENS_PER_SEQ 0    /* lens[b] = context length of sequence b           */
#define VA_LENS_CUMULATIVE 1 /* lens[b+1] - lens[b] (cu_seqlens_k, num_seqs + 1) */

/*
 * KV pool addressing shared by all entry points.  Token slot s of a sequence
 * whose block table row is T lives at
 *     base + T[s / block_size] * stride_block + (s % block_size) * stride_slot
 *          + kv_head * stride_head + d
 * which covers the engine's NHD pool [num_blocks, block_size, Hkv, D]
 * (qwen_asr_vllm/engine/model_runner.py:116-131) and the TTS talker's HND
 * pool [pages, Hkv, page_size, D]
 * (qwen_asr_vllm/agent/qwen_tts_outer_paged_cache.py:116-119).
 */
typedef struct va_kv_pool {
  void* k;                /* key pool                                    */
  void* v;                /* value pool (same strides as k)              */
  int64_t stride_block;   /* elements between consecutive blocks/pages   */
  int64_t stride_slot;    /* elements between slots inside one block     */
  int64_t stride_head;    /* elements between kv heads                   */
  int32_t block_size;     /* tokens per block (any positive value)       */
  int32_t num_blocks;     /* blocks in the pool; out-of-range ids are    */
                          /* treated as masked and never dereferenced    */
  /* Element format (VA_KV_*).  An FP8 pool holds OCP e4m3 codes (strides
   * count bytes); a key element's value is code * k_scale, a value
   * element's code * v_scale (one scale per pool, > 0).  Every store into
   * it quantises: code = e4m3_rne(clamp(x * (1 / scale), -448, 448)), with
   * 1 / scale and the product rounded to fp32.  FP8 pools need 16-bit
   * q / k / v and, for decode, a block size that is a multiple of 16. */
  int32_t kv_format;
  float k_scale;
  float v_scale;
} va_kv_pool;

/* ---------------------------------------------------------------- store */
typedef struct va_store_args {
  uint32_t struct_size;   /* sizeof(va_store_args)                        */
  int32_t dtype;          /* VA_BF16 / VA_F16 / VA_F32                    */
  const void* key;        /* [num_tokens, Hkv, D]                         */
  const void* value;
  int64_t key_stride_tok, key_stride_head;
  int64_t value_stride_tok, value_stride_head;
  va_kv_pool pool;
  const void* slot_mapping; /* [num_tokens]; slot < 0 or >= capacity skips */
  int32_t slot_dtype;       /* VA_I32 / VA_I64                             */
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t head_dim;
} va_store_args;

/* Scatter key/value rows into the pool by slot_mapping (bit-exact copy).
 * Replaces store_kvcache, qwen_asr_vllm/layers/attention.py:52-67. */
int va_store_kvcache(const va_store_args* args, void* stream);

/* ------------------------------------------------------ q/k prologue */
/* Qwen3's per-head query/key prologue: RMSNorm over head_dim,
 *   n = to_dtype(x * 1/sqrt(mean(x^2) + eps)),  y = to_dtype(n * weight)
 * (layers/layernorm.py:19-25), then rotary embedding in the half-split
 * convention with the fp32 cache [max_position, head_dim] = [cos | sin],
 *   out[i]       = to_dtype(y[i] cos[i] - y[i + D/2] sin[i]),
 *   out[i + D/2] = to_dtype(y[i + D/2] cos[i] + y[i] sin[i]),    i < D/2
 * at the token's position (layers/rotary_embedding.py:9-32).  The rotation's
 * products are rounded before their sum (no fused multiply-add), as torch
 * evaluates them; the mean of squares is summed in another order than
 * torch's (with fused multiply-adds), so 1/sqrt(mean + eps) can differ from
 * torch's in its last bit. */
typedef struct va_qk_prologue {
  const void* q_norm_weight;  /* [head_dim] in weight_dtype                 */
  const void* k_norm_weight;  /* [head_dim] in weight_dtype                 */
  int32_t weight_dtype;       /* VA_BF16 / VA_F16 / VA_F32                  */
  float eps;
  const float* cos_sin_cache; /* [max_position, head_dim]: cos | sin halves */
  int64_t cos_sin_stride;     /* elements between consecutive positions     */
  int32_t max_position;       /* positions are clamped to [0, max_position) */
  int32_t positions_dtype;    /* VA_I32 / VA_I64                            */
  const void* positions;      /* decode: [num_seqs]; va_qk_norm_rope: [num_tokens] */
} va_qk_prologue;

typedef struct va_qk_norm_rope_args {
  uint32_t struct_size;   /* sizeof(va_qk_norm_rope_args)                 */
  int32_t dtype;          /* q, k and the outputs share it                */
  const void* q;          /* [num_tokens, Hq, D]                          */
  int64_t q_stride_tok, q_stride_head;
  const void* k;          /* [num_tokens, Hkv, D]                         */
  int64_t k_stride_tok, k_stride_head;
  void* q_out;            /* [num_tokens, Hq, D]; may equal q (in place)  */
  int64_t q_out_stride_tok, q_out_stride_head;
  void* k_out;            /* [num_tokens, Hkv, D]; may equal k            */
  int64_t k_out_stride_tok, k_out_stride_head;
  int32_t num_tokens, num_heads, num_kv_heads, head_dim;
  va_qk_prologue prologue; /* positions: one per token                    */
} va_qk_norm_rope_args;

/* Apply the prologue to every query and key row (prefill and any batch the
 * fused decode path does not take). */
int va_qk_norm_rope(const va_qk_norm_rope_args* args, void* stream);

/* --------------------------------------------------------------- decode */
typedef struct va_decode_args {
  uint32_t struct_size;   /* sizeof(va_decode_args)                       */
  int32_t dtype;          /* q, pool, out and new rows share it           */
  const void* q;          /* [num_seqs, Hq, D]: one query token per seq   */
  int64_t q_stride_seq, q_stride_head;
  void* out;              /* [num_seqs, Hq, D] in dtype                   */
  int64_t out_stride_seq, out_stride_head;
  va_kv_pool pool;
  const void* block_tables; /* [num_seqs, table_width]; entries at index  */
  int32_t table_dtype;      /* >= table_width read as block 0, as the TTS  */
  int64_t table_stride_seq; /* padding does (qwen_tts_paged_attention.py:458-465) */
  int32_t table_width;
  const void* lens;       /* see VA_LENS_*                                */
  int32_t lens_dtype;
  int32_t lens_kind;
  const uint8_t* valid_mask; /* optional [num_seqs, valid_len] bool; token */
  int64_t valid_stride_seq;  /* t < len is attended iff t >= valid_len or  */
  int32_t valid_len;         /* valid_mask[b, t] != 0                      */
  /* Optional current row, written to the pool at position len-1 and used
   * for that position in the same launch (the TTS fused write,
   * qwen_tts_paged_attention.py:181-221).  [num_seqs, Hkv, D]. */
  const void* new_k;
  int64_t new_k_stride_seq, new_k_stride_head;
  const void* new_v;
  int64_t new_v_stride_seq, new_v_stride_head;
  /* Optional destination slots for the current row ([num_seqs], slot < 0
   * skips the write and the substitution).  NULL: the slot of position len-1
   * through the block table. */
  const void* new_slots;
  int32_t new_slots_dtype;
  int32_t num_seqs, num_heads, num_kv_heads, head_dim;
  int32_t max_seq_len;    /* upper bound of every len; sizes the grid     */
  int32_t split_tokens;   /* tokens per context partition, 0 = automatic, */
                          /* VA_SPLIT_EXACT: automatic, exact bound       */
  float scale;            /* softmax scale                                */
  void* workspace;        /* partial results; see va_paged_decode_workspace_bytes */
  size_t workspace_bytes; /* (no initialisation needed; launches sharing one   */
                          /*  workspace must be ordered on one stream)         */
  /* Optional Qwen3 prologue (NULL: q and new_k are used as given).  When set,
   * q (and new_k, if given) are the raw projections: q is normalised and
   * rotated at positions[b] before attention, and new_k likewise before it
   * is written and attended (its position is also positions[b]). */
  const va_qk_prologue* prologue;
  /* Optional bounds of the attended keys, as the TTS kernel's MAX_SEQ_LEN
   * (kernel_seq_len) and num_page_slots (kernel_page_count) bound them
   * (qwen_tts_paged_attention.py:223-241): tokens at or past key_limit are
   * not attended (0: no bound), and block-table columns at or past
   * table_read_width read as block 0 when attending (0: table_width).  The
   * current row is still written at len - 1, through the table's own entry
   * (qwen_tts_paged_attention.py:182-221). */
  int32_t key_limit;
  int32_t table_read_width;
} va_decode_args;

/* Bytes of workspace va_paged_decode needs for these arguments (the
 * struct's workspace fields are ignored); 0 when no sequence can span more
 * than one context partition.  With split_tokens = 0 the partition size
 * depends on the current device's compute-unit count, so query the size with
 * the same device current as the launch. */
size_t va_paged_decode_workspace_bytes(const va_decode_args* args);

/* split_tokens = VA_SPLIT_EXACT: the automatic split, told that max_seq_len
 * is the exact longest context of the batch (an eager step's maximum, as
 * qwen_asr_vllm/engine/model_runner.py:213 computes it).  Its partitions are
 * then fixed from max_seq_len at any length, and each workgroup requests its
 * first tiles before the lengths arrive; with 0 that holds only up to 4096
 * tokens, above which each workgroup sizes its partition from its own
 * length (right for a bound that is only an upper limit, such as the
 * max_model_len a captured decode graph passes).  The workspace bound is
 * the automatic split's either way. */
#define VA_SPLIT_EXACT (-1)

/* One-token GQA attention over a paged pool: split-context partitions, then
 * (only when a context spans several) a merge pass.  Replaces the decode use of
 * flash_attn_varlen_func (qwen_asr_vllm/layers/attention.py:96-107) and
 * paged_attention_decode (qwen_tts_paged_attention.py:383-516).  head_dim
 * 64 / 128 / 256 with groups of 1 / 2 / 4 / 8 run the vector kernels (16-byte
 * aligned strides and pointers); any other head_dim up to 1024 and any group
 * run a scalar kernel that needs element alignment only and never splits
 * (no prologue, no FP8 pool there). */
int va_paged_decode(const va_decode_args* args, void* stream);

/* Size of the scratch buffer of va_paged_decode_noalloc, per GPU. */
#define VA_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

/* va_paged_decode without a caller workspace and without any allocation: the
 * split-context partials live in a scratch buffer of
 * VA_DECODE_NOALLOC_SCRATCH_BYTES that the library holds in device memory, one
 * per GPU, for the life of the process (its address is looked up on the first
 * call on each device).  The args' workspace fields are ignored.  A split
 * needing more than the buffer (only an explicit split_tokens can; every
 * automatic split fits) fails with VA_ERR_WORKSPACE.  Calls that overlap on
 * one GPU (on two streams, say) share the buffer and race: order them.  No
 * counterpart in the reference: it is for callers that cannot allocate, such
 * as code under HIP graph capture that must not touch an allocator, tight
 * serving loops and harnesses that forbid hipMalloc. */
int va_paged_decode_noalloc(const va_decode_args* args, void* stream);

/* --------------------------------------------------------------- varlen */
typedef struct va_varlen_args {
  uint32_t struct_size;   /* sizeof(va_varlen_args)                       */
  int32_t dtype;          /* VA_BF16 / VA_F16                             */
  const void* q;          /* [total_q, Hq, D]                             */
  int64_t q_stride_tok, q_stride_head;
  const void* k;          /* [total_k or total_q, Hkv, D]; NULL with a    */
  int64_t k_stride_tok, k_stride_head; /* pool = every key from the pool  */
  const void* v;
  int64_t v_stride_tok, v_stride_head;
  void* out;              /* [total_q, Hq, D]                             */
  int64_t out_stride_tok, out_stride_head;
  const int32_t* cu_seqlens_q; /* [num_seqs + 1]                          */
  const int32_t* cu_seqlens_k; /* [num_seqs + 1]                          */
  int32_t num_seqs, total_q;
  int32_t num_heads, num_kv_heads, head_dim;
  /* max_seqlen_q sizes the launch's query blocks and must be at least every
   * q_len (as flash_attn_varlen_func requires): query rows past it are not
   * computed.  max_seqlen_k is not read (key ranges come from cu_seqlens_k). */
  int32_t max_seqlen_q, max_seqlen_k;
  int32_t causal;         /* 1: bottom-right aligned causal mask          */
  float scale;
  /* Optional paged pool.  Keys j < k_len - q_len of a sequence come from the
   * pool; the rest from k/v rows aligned with the queries (or from the pool
   * too when k is NULL). */
  va_kv_pool pool;
  const void* block_tables;
  int32_t table_dtype;
  int64_t table_stride_seq;
  int32_t table_width;
  /* Optional fused store: q row i's k/v row is also written to slot
   * slot_mapping[i] (slot < 0 skips), as store_kvcache would. */
  const void* slot_mapping;
  int32_t slot_dtype;
  /* Unused (no varlen launch needs a workspace; va_varlen_workspace_bytes
   * returns 0).  An FP8 pool's prefix rows are converted to the 16-bit type
   * (code * scale, rounded once) inside the kernel, tile by tile, and its
   * new rows are stored quantised after the attention. */
  void* workspace;
  size_t workspace_bytes;
  /* Optional Qwen3 query prologue (NULL: q is used as given).  When set, q
   * holds the raw query projections: each query row is normalised with
   * q_norm_weight and rotated at positions[token] (one position per query
   * token, [total_q]) inside the launch, with the arithmetic of
   * va_qk_norm_rope; k and the pool must already hold normalised, rotated
   * keys (va_qk_norm_rope with num_heads = 0 does the keys alone).  Causal
   * launches with head_dim 128; k_norm_weight is not read. */
  const va_qk_prologue* prologue;
} va_varlen_args;

/* Variable-length attention over packed sequences: causal with bottom-right
 * alignment (prefill, optionally over a paged prefix, with the store and the
 * Qwen3 query prologue fused), or non-causal block-diagonal (audio encoder
 * windows). */
int va_varlen_attention(const va_varlen_args* args, void* stream);

/* Bytes of workspace va_varlen_attention needs: always 0 (kept for callers
 * written against the earlier contract). */
size_t va_varlen_workspace_bytes(const va_varlen_args* args);

/* ----------------------------------------------------------------- misc */
const char* va_last_error(void);
int va_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VOICEAGENT_ATTN_H */
