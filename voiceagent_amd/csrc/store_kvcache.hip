// store_kvcache: scatter new K/V rows into the paged pool by slot_mapping.
//
// Semantics follow qwen_asr_vllm/layers/attention.py:31-67: for every token
// i with slot_mapping[i] != -1, cache row `slot` receives key[i] (and value[i])
// unchanged.  The copy moves raw 16-byte words, so it is bit-exact for every
// element type.  Slots outside [0, num_blocks * block_size) are skipped rather
// than written out of bounds.
//
// Launch shape: the K and V rows of all tokens are cut into 16-byte words and
// the flattened (token, K|V, word) space is spread over 256-lane workgroups.
// A lane moves kStoreWords (4) words per pass, 256 words apart, so consecutive
// lanes touch consecutive 16-byte words (coalesced on both sides), and it
// issues every word's load (a DMA into LDS) and slot load before its first
// store: a wave keeps 4 KiB in flight and pays one round trip per pass.  (One
// word per lane, with the data load behind its slot check, kept 1 KiB per
// wave in flight behind two dependent round trips: config 3's 8561 rows ran
// at 4.05 TB/s.)  Rows are read and written non-temporally: each is touched
// once.  Indices are 32-bit (the host splits a launch whose words reach
// 2^31) and divide by multiply-and-shift.
//
// An FP8 pool (VA_KV_FP8_E4M3) receives each 16-byte word of 8 16-bit
// elements as 8 e4m3 codes, x * (1 / scale) saturated to +-448 and rounded
// to nearest even (one 8-byte store per lane).
#include "common.h"
#include "fastdiv.h"

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
  uint32_t total_words;    // num_tokens * 2 * words_per_row, below 2^31
  FastDiv tok_div;         // 2 * words_per_row: words per token
  FastDiv head_div;        // words_per_head
  FastDiv bs_div;          // block_size
  int32_t slot_small;      // capacity <= 2^31: slots divide by bs_div
};

constexpr int kStoreThreads = 256;

// kF8: the pool holds e4m3 codes of the 16-bit elements of ET.  kStoreWords:
// words a lane has in flight per pass (4; 1 for launches too small to give
// every CU a workgroup at 4, which one CU's rate would otherwise bound).
template <bool kF8, typename ET, int kStoreWords>
__global__ __launch_bounds__(kStoreThreads) void store_kvcache_kernel(StoreParams p) {
  // The words land in the wave's area of LDS by DMA: the compiler can neither
  // wait on an asm load early nor sink it into the store's branch (a register
  // load used only under the slot check was moved below it, so each word
  // waited for its slot first).  A lane reads back only what it loaded.
  __shared__ __align__(1024) char s_words[kStoreThreads / 64][kStoreWords][1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)&s_words[wave][0][0]);
  const uint32_t total = p.total_words;
  const uint32_t wpr = (uint32_t)p.words_per_row;
  const uint32_t* const sw = reinterpret_cast<const uint32_t*>(p.slots);
  for (uint32_t base = blockIdx.x * (kStoreThreads * kStoreWords) + threadIdx.x; base < total;
       base += gridDim.x * (kStoreThreads * kStoreWords)) {
    uint32_t part[kStoreWords], slo[kStoreWords], shi[kStoreWords];
    const char* src[kStoreWords];
    int64_t si[kStoreWords];
    // Every address first, then every load back to back: address arithmetic
    // between the loads made the compiler wait for the earlier ones when it
    // reused their registers.
#pragma unroll
    for (int u = 0; u < kStoreWords; ++u) {
      // Words past the end reload the last word and store nothing, so every
      // load is issued without a branch.
      uint32_t w = base + u * kStoreThreads;
      w = w < total ? w : total - 1;
      const uint32_t tok = fast_div(w, p.tok_div);
      part[u] = w - tok * p.tok_div.d;  // word within the token: K words, then V words
      const bool is_v = part[u] >= wpr;
      const uint32_t rem = is_v ? part[u] - wpr : part[u];
      const uint32_t head = fast_div(rem, p.head_div);
      const uint32_t word = rem - head * p.head_div.d;
      src[u] = (is_v ? p.value + (int64_t)tok * p.value_stride_tok +
                           (int64_t)head * p.value_stride_head
                     : p.key + (int64_t)tok * p.key_stride_tok +
                           (int64_t)head * p.key_stride_head) +
               word * 16;
      si[u] = (int64_t)tok << p.slot_i64;
    }
#pragma unroll
    for (int u = 0; u < kStoreWords; ++u) {
      dma16_nt(src[u], lds_wave + u * 1024);
      // The slot as raw words (both loads unconditional): the low word at
      // index tok << i64 and, for int64 slots, the high word after it.
      slo[u] = sw[si[u]];
      shi[u] = sw[si[u] + p.slot_i64];
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int u = 0; u < kStoreWords; ++u) {
      if (base + u * kStoreThreads >= total) break;
      const int64_t slot = p.slot_i64 ? (int64_t)(((uint64_t)shi[u] << 32) | slo[u])
                                      : (int64_t)(int32_t)slo[u];
      if (slot < 0 || slot >= p.capacity) continue;  // -1 (padding) and out-of-range slots
      const int64_t blk = p.slot_small ? (int64_t)fast_div((uint32_t)slot, p.bs_div)
                                       : slot / p.block_size;
      const int64_t off = slot - blk * p.block_size;
      const bool is_v = part[u] >= wpr;
      const uint32_t rem = is_v ? part[u] - wpr : part[u];
      const uint32_t head = fast_div(rem, p.head_div);
      const uint32_t word = rem - head * p.head_div.d;
      char* dst = (is_v ? p.v_pool : p.k_pool) + blk * p.stride_block + off * p.stride_slot +
                  (int64_t)head * p.stride_head;
      const uint4 data = *reinterpret_cast<const uint4*>(&s_words[wave][u][lane * 16]);
      if constexpr (kF8) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const uint2 codes = f8_quant8<ET>(data, is_v ? p.inv_v : p.inv_k);
        __builtin_nontemporal_store(u32x2{codes.x, codes.y},
                                    reinterpret_cast<u32x2*>(dst + word * 8));
      } else {
        st16_nt(dst + word * 16, data);
      }
    }
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
  const int64_t words_per_tok = 2 * (int64_t)p.words_per_row;
  VA_CHECK_ARG(words_per_tok < ((int64_t)1 << 31), "va_store_kvcache: rows too wide");
  p.tok_div = make_fastdiv((uint32_t)words_per_tok);
  p.head_div = make_fastdiv((uint32_t)p.words_per_head);
  p.bs_div = make_fastdiv((uint32_t)a->pool.block_size);
  p.slot_small = p.capacity <= ((int64_t)1 << 31);

  // One launch per chunk of tokens whose words stay below 2^31.
  const int64_t chunk = (((int64_t)1 << 31) - 1) / words_per_tok;
  const int slot_bytes = a->slot_dtype == VA_I64 ? 8 : 4;
  const hipStream_t s = (hipStream_t)stream;
  for (int64_t t0 = 0; t0 < a->num_tokens; t0 += chunk) {
    const int64_t n = a->num_tokens - t0 < chunk ? a->num_tokens - t0 : chunk;
    StoreParams q = p;
    q.key = p.key + t0 * p.key_stride_tok;
    q.value = p.value + t0 * p.value_stride_tok;
    q.slots = (const char*)p.slots + t0 * slot_bytes;
    q.num_tokens = (int32_t)n;
    q.total_words = (uint32_t)(n * words_per_tok);
    // Four words per lane once that still gives every CU a workgroup.
    const bool wide = q.total_words >= (uint32_t)current_device_cus() * kStoreThreads * 4u;
    const int64_t per_wg = (int64_t)kStoreThreads * (wide ? 4 : 1);
    int64_t grid = (q.total_words + per_wg - 1) / per_wg;
    if (grid > 65536) grid = 65536;
    const dim3 g((unsigned)grid), b(kStoreThreads);
    if (!f8) {
      if (wide) hipLaunchKernelGGL((store_kvcache_kernel<false, BF16, 4>), g, b, 0, s, q);
      else hipLaunchKernelGGL((store_kvcache_kernel<false, BF16, 1>), g, b, 0, s, q);
    } else if (a->dtype == VA_BF16) {
      if (wide) hipLaunchKernelGGL((store_kvcache_kernel<true, BF16, 4>), g, b, 0, s, q);
      else hipLaunchKernelGGL((store_kvcache_kernel<true, BF16, 1>), g, b, 0, s, q);
    } else {
      if (wide) hipLaunchKernelGGL((store_kvcache_kernel<true, F16, 4>), g, b, 0, s, q);
      else hipLaunchKernelGGL((store_kvcache_kernel<true, F16, 1>), g, b, 0, s, q);
    }
  }
  return check_launch("va_store_kvcache");
}
