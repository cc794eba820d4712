// store_kvcache: scatter new K/V rows into the paged pool by slot_mapping.
//
// Semantics follow qwen_asr_vllm/layers/attention.py:31-67: for every token
// i with slot_mapping[i] != -1, cache row `slot` receives key[i] (and value[i])
// unchanged.  The copy moves raw 16-byte words, so it is bit-exact for every
// element type.  Slots outside [0, num_blocks * block_size) are skipped rather
// than written out of bounds.
//
// Launch shape: the K and V rows of all tokens are cut into 16-byte words and
// the flattened (token, K|V, word) space is spread over 256-lane workgroups,
// one word per lane (grid-stride beyond 65536 workgroups).  A 1024-element
// bf16 row (2 KiB) is moved by 128 lanes with one dwordx4 load and one
// dwordx4 store each; consecutive lanes touch consecutive 16-byte words, so
// both sides are fully coalesced.
//
// An FP8 pool (VA_KV_FP8_E4M3) receives each 16-byte word of 8 16-bit
// elements as 8 e4m3 codes, x * (1 / scale) saturated to +-448 and rounded
// to nearest even (one 8-byte store per lane).
#include "common.h"

namespace va {

struct StoreParams {
  const char* key;
  const char* value;
  int64_t key_stride_tok, key_stride_head;      // bytes
  int64_t value_stride_tok, value_stride_head;  // bytes
  char* k_pool;
  char* v_pool;
  int64_t stride_block, stride_slot, stride_head;  // bytes
  int64_t capacity;                                // num_blocks * block_size
  int32_t block_size;
  const void* slots;
  int32_t slot_i64;
  int32_t num_tokens;
  int32_t words_per_head;  // head_dim * elem_bytes / 16
  int32_t words_per_row;   // num_kv_heads * words_per_head
  float inv_k, inv_v;      // FP8 pools: 1 / k_scale, 1 / v_scale
};

constexpr int kStoreThreads = 256;

// kF8: the pool holds e4m3 codes of the 16-bit elements of ET.
template <bool kF8, typename ET>
__global__ __launch_bounds__(kStoreThreads) void store_kvcache_kernel(StoreParams p) {
  // Work items: (token, kv-tensor, word) flattened; each thread moves 16 B.
  const int64_t words_per_tok = 2 * (int64_t)p.words_per_row;
  const int64_t total = (int64_t)p.num_tokens * words_per_tok;
  for (int64_t w = (int64_t)blockIdx.x * kStoreThreads + threadIdx.x; w < total;
       w += (int64_t)gridDim.x * kStoreThreads) {
    const int tok = (int)(w / words_per_tok);
    int rem = (int)(w - (int64_t)tok * words_per_tok);
    const int is_v = rem >= p.words_per_row;
    if (is_v) rem -= p.words_per_row;
    const int head = rem / p.words_per_head;
    const int word = rem - head * p.words_per_head;
    const int64_t slot = load_index(p.slots, tok, p.slot_i64);
    if (slot < 0 || slot >= p.capacity) continue;
    const int64_t blk = slot / p.block_size;
    const int64_t off = slot - blk * p.block_size;
    const char* src = is_v ? p.value + tok * p.value_stride_tok + head * p.value_stride_head
                           : p.key + tok * p.key_stride_tok + head * p.key_stride_head;
    char* dst = (is_v ? p.v_pool : p.k_pool) + blk * p.stride_block + off * p.stride_slot +
                head * p.stride_head;
    if constexpr (kF8)
      *reinterpret_cast<uint2*>(dst + word * 8) =
          f8_quant8<ET>(ld16(src + word * 16), is_v ? p.inv_v : p.inv_k);
    else
      st16(dst + word * 16, ld16(src + word * 16));
  }
}

static int elem_bytes(int dtype) {
  switch (dtype) {
    case VA_BF16:
    case VA_F16:
      return 2;
    case VA_F32:
      return 4;
    default:
      return 0;
  }
}

}  // namespace va

extern "C" int va_store_kvcache(const va_store_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_store_kvcache: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_store_args),
               "va_store_kvcache: struct_size %u != %zu (header/library mismatch)",
               a->struct_size, sizeof(va_store_args));
  const int eb = elem_bytes(a->dtype);
  VA_CHECK_ARG(eb != 0, "va_store_kvcache: unknown dtype %d", a->dtype);
  const bool f8 = a->pool.kv_format == VA_KV_FP8_E4M3;
  VA_CHECK_ARG(a->pool.kv_format == VA_KV_NATIVE || f8, "va_store_kvcache: unknown kv_format %d",
               a->pool.kv_format);
  VA_CHECK_ARG(!f8 || a->dtype != VA_F32, "va_store_kvcache: an FP8 pool needs 16-bit key/value");
  VA_CHECK_ARG(!f8 || (a->pool.k_scale > 0.f && a->pool.v_scale > 0.f),
               "va_store_kvcache: FP8 pool scales must be positive");
  const int pb = f8 ? 1 : eb;  // bytes per pool element
  VA_CHECK_ARG(a->num_tokens >= 0, "va_store_kvcache: num_tokens < 0");
  if (a->num_tokens == 0) return VA_OK;
  VA_CHECK_ARG(a->key && a->value && a->pool.k && a->pool.v && a->slot_mapping,
               "va_store_kvcache: null pointer argument");
  VA_CHECK_ARG(a->num_kv_heads > 0 && a->head_dim > 0, "va_store_kvcache: bad head geometry");
  VA_CHECK_ARG((a->head_dim * eb) % 16 == 0,
               "va_store_kvcache: head_dim*elem_bytes must be a multiple of 16");
  VA_CHECK_ARG(a->pool.block_size > 0 && a->pool.num_blocks >= 0,
               "va_store_kvcache: bad pool geometry");
  VA_CHECK_ARG(a->slot_dtype == VA_I32 || a->slot_dtype == VA_I64,
               "va_store_kvcache: slot_dtype must be VA_I32 or VA_I64");
  // 16-byte alignment of every row start the kernel touches.
  const int64_t strides[] = {a->key_stride_tok, a->key_stride_head, a->value_stride_tok,
                             a->value_stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * eb) % 16 == 0, "va_store_kvcache: strides must be 16-byte multiples");
  const int64_t pstrides[] = {a->pool.stride_block, a->pool.stride_slot, a->pool.stride_head};
  for (int64_t s : pstrides)
    VA_CHECK_ARG((s * pb) % (f8 ? 8 : 16) == 0,
                 "va_store_kvcache: pool strides must be 16-byte (FP8: 8-byte) multiples");
  const uintptr_t ptrs[] = {(uintptr_t)a->key, (uintptr_t)a->value, (uintptr_t)a->pool.k,
                            (uintptr_t)a->pool.v};
  for (uintptr_t p : ptrs) VA_CHECK_ARG(p % 16 == 0, "va_store_kvcache: pointers must be 16-byte aligned");

  StoreParams p;
  p.key = (const char*)a->key;
  p.value = (const char*)a->value;
  p.key_stride_tok = a->key_stride_tok * eb;
  p.key_stride_head = a->key_stride_head * eb;
  p.value_stride_tok = a->value_stride_tok * eb;
  p.value_stride_head = a->value_stride_head * eb;
  p.k_pool = (char*)a->pool.k;
  p.v_pool = (char*)a->pool.v;
  p.stride_block = a->pool.stride_block * pb;
  p.stride_slot = a->pool.stride_slot * pb;
  p.stride_head = a->pool.stride_head * pb;
  p.inv_k = f8 ? 1.0f / a->pool.k_scale : 1.0f;
  p.inv_v = f8 ? 1.0f / a->pool.v_scale : 1.0f;
  p.capacity = (int64_t)a->pool.num_blocks * a->pool.block_size;
  p.block_size = a->pool.block_size;
  p.slots = a->slot_mapping;
  p.slot_i64 = a->slot_dtype == VA_I64;
  p.num_tokens = a->num_tokens;
  p.words_per_head = a->head_dim * eb / 16;
  p.words_per_row = a->num_kv_heads * p.words_per_head;

  const int64_t total = (int64_t)a->num_tokens * 2 * p.words_per_row;
  int64_t grid = (total + kStoreThreads - 1) / kStoreThreads;
  if (grid > 65536) grid = 65536;
  const hipStream_t s = (hipStream_t)stream;
  if (!f8)
    hipLaunchKernelGGL((store_kvcache_kernel<false, BF16>), dim3((unsigned)grid),
                       dim3(kStoreThreads), 0, s, p);
  else if (a->dtype == VA_BF16)
    hipLaunchKernelGGL((store_kvcache_kernel<true, BF16>), dim3((unsigned)grid),
                       dim3(kStoreThreads), 0, s, p);
  else
    hipLaunchKernelGGL((store_kvcache_kernel<true, F16>), dim3((unsigned)grid),
                       dim3(kStoreThreads), 0, s, p);
  return check_launch("va_store_kvcache");
}
