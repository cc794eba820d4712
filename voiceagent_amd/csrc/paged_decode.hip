// Host side of the paged decode: argument checks, the context split and
// launch dispatch (kernels in paged_decode_kernel.h and paged_decode_mfma.h,
// instantiated per element type in paged_decode_{bf16,f16,f32}.hip).
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "paged_decode_mfma.h"

namespace va {

// ----------------------------------------------------------------- host side
// A context is split into at most kMaxParts partitions (the partition grows
// instead), which bounds the merge kernel's LDS and loops.

struct DecodePlan {
  int split_tokens;
  int max_parts;
  int dyn_split;
  size_t ml_bytes, o_bytes, total_bytes;
  int64_t wg_tokens;  // most tokens one workgroup attends (bound from max_seq_len)
};

// FP8 pools at head_dim 128 take twelve-wave workgroups when no workgroup
// attends more tokens than this (see MfmaWaves).
constexpr int64_t kWave12Tokens = 2048;

template <typename ET, int D, int G>
static int decode_unit() {
  // one round of CPW chunks on every wave of a workgroup
  return DecodeShape<ET, D, G>::NW * DecodeShape<ET, D, G>::CPW * kChunk;
}

static int decode_unit_for(int dtype, int D, int G);

// The matrix-core kernel serves 16-bit K/V with block sizes that are
// multiples of 16 (with or without a key_valid_mask and the prologue); every
// other call takes the general kernel.  VA_DECODE_KERNEL=general in the
// environment forces the general kernel (for comparisons).
static bool general_kernel_forced() {
  static const int forced = [] {
    const char* e = std::getenv("VA_DECODE_KERNEL");
    return (e != nullptr && std::strcmp(e, "general") == 0) ? 1 : 0;
  }();
  return forced != 0;
}

// Shapes neither the matrix-core nor the general kernel takes run on the
// small-head kernel (see launch_paged_decode_small).
static bool small_head_decode(const va_decode_args* a) {
  const bool d_ok = a->head_dim == 64 || a->head_dim == 128 || a->head_dim == 256;
  const int G = a->num_kv_heads > 0 ? a->num_heads / a->num_kv_heads : 0;
  return !d_ok || !(G == 1 || G == 2 || G == 4 || G == 8);
}

static bool use_mfma_decode(const va_decode_args* a) {
  if (a->dtype != VA_BF16 && a->dtype != VA_F16) return false;
  const int64_t kv_eb = a->pool.kv_format == VA_KV_FP8_E4M3 ? 1 : 2;
  if (a->pool.block_size <= 0 || a->pool.block_size % kChunk != 0) return false;
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return false;
  if (a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads != 0) return false;
  const int G = a->num_heads / a->num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return false;
  // Per-lane DMA offsets inside a 16-row tile are 32-bit.
  if (a->pool.stride_slot < 0 ||
      (kChunk - 1) * a->pool.stride_slot * kv_eb + (int64_t)a->head_dim * kv_eb >=
          ((int64_t)1 << 31))
    return false;
  // FP8 pools have no general-kernel path, so forcing it does not apply.
  return a->pool.kv_format == VA_KV_FP8_E4M3 || !general_kernel_forced();
}

static int mfma_unit_for(int D) {
  switch (D) {
    case 64: return mfma_decode_unit<64>();
    case 128: return mfma_decode_unit<128>();
    case 256: return mfma_decode_unit<256>();
    default: return 0;
  }
}

static int elem_bytes_of(int dtype);

// Contexts up to this many bytes of one kv head's K and V rows stay whole
// (see plan_decode).
constexpr int64_t kNoSplitBytes = 192 * 1024;

// Longest max_seq_len whose automatic split uses fixed partitions (see
// plan_decode).
constexpr int kStaticSplitMax = 4096;

// Context length whose K and V rows of one kv head fill kNoSplitBytes.
static int nosplit_tokens_for(const va_decode_args* a) {
  const int64_t per_token = (int64_t)a->head_dim * elem_bytes_of(a->dtype) * 2;
  return per_token > 0 ? (int)(kNoSplitBytes / per_token) : 0;
}

static DecodePlan plan_decode(const va_decode_args* a) {
  DecodePlan pl{};
  if (small_head_decode(a)) {  // one workgroup per (sequence, query head), no split
    pl.max_parts = 1;
    pl.split_tokens = a->max_seq_len > 0 ? a->max_seq_len : 1;
    pl.wg_tokens = pl.split_tokens;
    return pl;
  }
  const int G = a->num_kv_heads > 0 ? a->num_heads / a->num_kv_heads : 1;
  int unit = use_mfma_decode(a) ? mfma_unit_for(a->head_dim)
                                : decode_unit_for(a->dtype, a->head_dim, G);
  if (unit <= 0) unit = 128;
  int max_len = a->max_seq_len > 0 ? a->max_seq_len : 1;
  if (a->key_limit > 0 && a->key_limit < max_len) max_len = a->key_limit;
  const bool exact = a->split_tokens == VA_SPLIT_EXACT;
  int P = exact ? 0 : a->split_tokens;
  const int64_t pairs = (int64_t)a->num_seqs * a->num_kv_heads;
  if (P <= 0) {
    // Split contexts only as far as needed to give every CU one workgroup:
    // with at least as many (sequence, kv head) pairs as CUs, one partition
    // per pair.  Otherwise every context gets up to `want` partitions whose
    // size each workgroup derives from its own context length
    // (partition_tokens), so a max_seq_len that is only an upper bound (a
    // decode graph captured at max_model_len) still spreads short contexts.
    // When no pair can hold more than kNoSplitBytes * 8 / min(parts, 8) of
    // K/V (max_seq_len tokens), nothing is split: one CU streams that much
    // in less time than a split, its merge launch and the lost early
    // start-up cost, and with few partitions per pair (many pairs) the whole
    // launch is already near the HBM rate.  Fitted on 16 query / 8 kv heads,
    // head_dim 128, B = 1..16 x 128..1024 tokens (worst choice 0.24 us off
    // the better one): B <= 4 splits above 384 tokens, B = 8 (4 partitions)
    // above 768, B = 16 (2 partitions) above 1536.  A max_seq_len that is
    // only an upper bound (max_model_len) keeps the split.
    const int64_t cus = current_device_cus();
    const int64_t want = pairs >= cus ? 1 : cus / (pairs > 0 ? pairs : 1);
    int64_t parts = want;
    if (parts > 1 && (int64_t)max_len * (parts < 8 ? parts : 8) <= (int64_t)nosplit_tokens_for(a) * 8)
      parts = 1;
    const int64_t by_len = (max_len + kDynGrain - 1) / kDynGrain;
    if (parts > by_len) parts = by_len;
    if (parts > kMaxParts) parts = kMaxParts;
    if (parts > 1 && (exact || max_len <= kStaticSplitMax)) {
      // A short or exact (VA_SPLIT_EXACT) max_seq_len fixes the partitions:
      // each workgroup knows its tokens before the length arrives and
      // requests its first tiles at once, as an unsplit launch does.  (Short
      // bounds are the exact ones of eager steps and the TTS talker; a
      // decode graph captured at max_model_len has a long one and keeps
      // per-length partitions.)
      P = (int)((max_len + parts - 1) / parts);
      P = (P + kDynGrain - 1) / kDynGrain * kDynGrain;
      pl.split_tokens = P;
      pl.max_parts = (max_len + P - 1) / P;
      pl.wg_tokens = P;
      pl.ml_bytes = ((size_t)pairs * pl.max_parts * G * 2 * 4 + 255) / 256 * 256;
      pl.o_bytes = (size_t)pairs * pl.max_parts * G * a->head_dim * 4;
      pl.total_bytes = pl.ml_bytes + pl.o_bytes;
      return pl;
    }
    if (parts > 1) {
      pl.dyn_split = 1;
      pl.split_tokens = kDynGrain;
      pl.max_parts = (int)parts;
      pl.wg_tokens = (max_len + parts - 1) / parts;
      pl.ml_bytes = ((size_t)pairs * pl.max_parts * G * 2 * 4 + 255) / 256 * 256;
      pl.o_bytes = (size_t)pairs * pl.max_parts * G * a->head_dim * 4;
      pl.total_bytes = pl.ml_bytes + pl.o_bytes;
      return pl;
    }
    P = max_len;
  }
  // Any split (automatic or requested) keeps at most kMaxParts partitions.
  const int cap = (max_len + kMaxParts - 1) / kMaxParts;
  if (P < cap) P = cap;
  P = ((P + unit - 1) / unit) * unit;
  if (P < unit) P = unit;
  pl.split_tokens = P;
  pl.max_parts = (max_len + P - 1) / P;
  pl.wg_tokens = P < max_len ? P : max_len;
  if (pl.max_parts > 1) {
    pl.ml_bytes = ((size_t)pairs * pl.max_parts * G * 2 * 4 + 255) / 256 * 256;
    pl.o_bytes = (size_t)pairs * pl.max_parts * G * a->head_dim * 4;
  }
  pl.total_bytes = pl.ml_bytes + pl.o_bytes;
  return pl;
}

template <typename ET>
static int unit_for_d(int D, int G) {
#define VA_UNIT_G(DD)                                      \
  switch (G) {                                             \
    case 1: return decode_unit<ET, DD, 1>();               \
    case 2: return decode_unit<ET, DD, 2>();               \
    case 4: return decode_unit<ET, DD, 4>();               \
    case 8: return decode_unit<ET, DD, 8>();               \
    default: return 0;                                     \
  }
  switch (D) {
    case 64: VA_UNIT_G(64)
    case 128: VA_UNIT_G(128)
    case 256: VA_UNIT_G(256)
    default: return 0;
  }
#undef VA_UNIT_G
}

static int decode_unit_for(int dtype, int D, int G) {
  switch (dtype) {
    case VA_BF16: return unit_for_d<BF16>(D, G);
    case VA_F16: return unit_for_d<F16>(D, G);
    case VA_F32: return unit_for_d<F32>(D, G);
    default: return 0;
  }
}

static int elem_bytes_of(int dtype) {
  return dtype == VA_F32 ? 4 : (dtype == VA_BF16 || dtype == VA_F16) ? 2 : 0;
}

}  // namespace va

extern "C" size_t va_paged_decode_workspace_bytes(const va_decode_args* a) {
  if (a == nullptr || a->struct_size != sizeof(va_decode_args)) return 0;
  return va::plan_decode(a).total_bytes;
}

namespace va {

// The body of va_paged_decode; the workspace comes from the arguments.
static int paged_decode_impl(const va_decode_args* a, void* stream);

// ------------------------------------------------- allocation-free variant
// Scratch memory of va_paged_decode_noalloc: the split-context partials,
// `kDecodeScratchBytes` per GPU, in the library's own device memory (the
// loaded code object holds it for the life of the process).  Every
// automatic split needs at most (compute units) x group x (head_dim + 2) x 4
// bytes plus 256 of rounding: 2.1 MB at 256 compute units, group 8 and
// head_dim 256.  Host code never uses the array's name as an address: each
// device's copy is reached through the pointer hipGetSymbolAddress returns
// with that device current.
constexpr size_t kDecodeScratchBytes = VA_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

constexpr int kMaxScratchDevices = 64;
static void* g_scratch_ptr[kMaxScratchDevices];
static hipError_t g_scratch_status[kMaxScratchDevices];
static std::once_flag g_scratch_once[kMaxScratchDevices];

// The current device's copy of `scratch` (looked up once per device), or
// nullptr with the error set.
static void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    (void)hipGetLastError();
    set_error("va_paged_decode_noalloc: no usable current device (%d)", dev);
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_status[dev] = e;
    g_scratch_ptr[dev] = e == hipSuccess ? ptr : nullptr;
    if (e != hipSuccess) (void)hipGetLastError();
  });
  if (g_scratch_ptr[dev] == nullptr) {
    set_error("va_paged_decode_noalloc: hipGetSymbolAddress of the scratch buffer failed on "
              "device %d: %s",
              dev, hipGetErrorString(g_scratch_status[dev]));
    return nullptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace va

extern "C" int va_paged_decode_noalloc(const va_decode_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_paged_decode_noalloc: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_decode_args),
               "va_paged_decode_noalloc: struct_size %u != %zu (header/library mismatch)",
               a->struct_size, sizeof(va_decode_args));
  va_decode_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (b.num_seqs > 0) {
    const size_t need = plan_decode(&b).total_bytes;
    if (need > kDecodeScratchBytes) {
      set_error("va_paged_decode_noalloc: the split needs %zu bytes of workspace, above the "
                "%zu-byte scratch buffer (use va_paged_decode with a workspace, or a larger "
                "split_tokens)",
                need, kDecodeScratchBytes);
      return VA_ERR_WORKSPACE;
    }
    if (need > 0) {
      void* ptr = device_scratch();
      if (ptr == nullptr) return VA_ERR_WORKSPACE;
      b.workspace = ptr;
      b.workspace_bytes = kDecodeScratchBytes;
    }
  }
  return paged_decode_impl(&b, stream);
}

extern "C" int va_paged_decode(const va_decode_args* a, void* stream) {
  return va::paged_decode_impl(a, stream);
}

int va::paged_decode_impl(const va_decode_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_paged_decode: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_decode_args),
               "va_paged_decode: struct_size %u != %zu (header/library mismatch)", a->struct_size,
               sizeof(va_decode_args));
  const int eb = elem_bytes_of(a->dtype);
  VA_CHECK_ARG(eb != 0, "va_paged_decode: unknown dtype %d", a->dtype);
  const bool f8 = a->pool.kv_format == VA_KV_FP8_E4M3;
  VA_CHECK_ARG(a->pool.kv_format == VA_KV_NATIVE || f8, "va_paged_decode: unknown kv_format %d",
               a->pool.kv_format);
  VA_CHECK_ARG(!f8 || (a->pool.k_scale > 0.f && a->pool.v_scale > 0.f),
               "va_paged_decode: FP8 pool scales must be positive");
  const int kv_eb = f8 ? 1 : eb;  // bytes per pool element
  VA_CHECK_ARG(a->num_seqs >= 0, "va_paged_decode: num_seqs < 0");
  if (a->num_seqs == 0) return VA_OK;
  VA_CHECK_ARG(a->num_seqs <= 65535, "va_paged_decode: num_seqs > 65535");  // merge grid.y
  VA_CHECK_ARG(a->q && a->out && a->pool.k && a->pool.v && a->block_tables && a->lens,
               "va_paged_decode: null pointer argument");
  VA_CHECK_ARG(a->num_kv_heads > 0 && a->num_heads > 0 && a->num_heads % a->num_kv_heads == 0,
               "va_paged_decode: num_heads (%d) must be a positive multiple of num_kv_heads (%d)",
               a->num_heads, a->num_kv_heads);
  VA_CHECK_ARG(a->num_kv_heads <= 65535, "va_paged_decode: num_kv_heads > 65535");
  const int G = a->num_heads / a->num_kv_heads;
  VA_CHECK_ARG(a->pool.block_size > 0 && a->pool.num_blocks >= 0, "va_paged_decode: bad pool");
  VA_CHECK_ARG(a->table_dtype == VA_I32 || a->table_dtype == VA_I64, "va_paged_decode: table_dtype");
  VA_CHECK_ARG(a->lens_dtype == VA_I32 || a->lens_dtype == VA_I64, "va_paged_decode: lens_dtype");
  VA_CHECK_ARG(a->lens_kind == VA_LENS_PER_SEQ || a->lens_kind == VA_LENS_CUMULATIVE,
               "va_paged_decode: lens_kind");
  VA_CHECK_ARG((a->new_k == nullptr) == (a->new_v == nullptr),
               "va_paged_decode: new_k and new_v must be given together");
  VA_CHECK_ARG(a->new_slots == nullptr || a->new_k != nullptr,
               "va_paged_decode: new_slots requires new_k/new_v");
  VA_CHECK_ARG(a->new_slots == nullptr || a->new_slots_dtype == VA_I32 ||
                   a->new_slots_dtype == VA_I64,
               "va_paged_decode: new_slots_dtype");
  VA_CHECK_ARG(a->max_seq_len >= 0, "va_paged_decode: max_seq_len < 0");
  VA_CHECK_ARG(a->split_tokens >= VA_SPLIT_EXACT,
               "va_paged_decode: split_tokens %d (>= 0, or VA_SPLIT_EXACT)", a->split_tokens);
  VA_CHECK_ARG(a->table_width >= 0, "va_paged_decode: table_width < 0");
  VA_CHECK_ARG(a->key_limit >= 0 && a->table_read_width >= 0,
               "va_paged_decode: key_limit and table_read_width must be non-negative");
  VA_CHECK_ARG(a->valid_mask == nullptr || (a->valid_len >= 0 && a->valid_stride_seq >= 0),
               "va_paged_decode: valid_len and valid_stride_seq must be non-negative");
  // The vector kernels move 16-byte pieces; the small-head kernel moves
  // single elements.
  const bool small = small_head_decode(a);
  const int64_t align = small ? eb : 16, palign = small ? kv_eb : 16;
  VA_CHECK_ARG(!small || (a->head_dim >= 1 && a->head_dim <= kSmallMaxHeadDim),
               "va_paged_decode: head_dim %d outside [1, %d]", a->head_dim, kSmallMaxHeadDim);
  VA_CHECK_ARG(!small || (a->prologue == nullptr && !f8),
               "va_paged_decode: the q/k prologue and FP8 pools need head_dim 64|128|256 and "
               "group 1|2|4|8 (got head_dim %d, group %d)",
               a->head_dim, G);
  const int64_t strides[] = {a->q_stride_seq,      a->q_stride_head,     a->out_stride_seq,
                             a->out_stride_head,   a->new_k_stride_seq,  a->new_k_stride_head,
                             a->new_v_stride_seq,  a->new_v_stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * eb) % align == 0, "va_paged_decode: strides must be %lld-byte multiples",
                 (long long)align);
  const int64_t pstrides[] = {a->pool.stride_block, a->pool.stride_slot, a->pool.stride_head};
  for (int64_t s : pstrides)
    VA_CHECK_ARG((s * kv_eb) % palign == 0,
                 "va_paged_decode: pool strides must be %lld-byte multiples", (long long)palign);
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->out, (uintptr_t)a->new_k,
                            (uintptr_t)a->new_v};
  for (uintptr_t p : ptrs)
    VA_CHECK_ARG(p % align == 0, "va_paged_decode: pointers must be %lld-byte aligned",
                 (long long)align);
  const uintptr_t pptrs[] = {(uintptr_t)a->pool.k, (uintptr_t)a->pool.v};
  for (uintptr_t p : pptrs)
    VA_CHECK_ARG(p % palign == 0, "va_paged_decode: pool pointers must be %lld-byte aligned",
                 (long long)palign);

  const DecodePlan pl = plan_decode(a);
  if (pl.total_bytes > 0) {
    if (a->workspace == nullptr || a->workspace_bytes < pl.total_bytes) {
      set_error("va_paged_decode: workspace of %zu bytes needed, %zu given", pl.total_bytes,
                a->workspace_bytes);
      return VA_ERR_WORKSPACE;
    }
    VA_CHECK_ARG((uintptr_t)a->workspace % 16 == 0, "va_paged_decode: workspace alignment");
  }
  VA_CHECK_ARG(pl.max_parts <= kMaxParts, "va_paged_decode: too many context partitions");

  DecodeParams p;
  p.q = (const char*)a->q;
  p.q_sb = a->q_stride_seq * eb;
  p.q_sh = a->q_stride_head * eb;
  p.out = (char*)a->out;
  p.o_sb = a->out_stride_seq * eb;
  p.o_sh = a->out_stride_head * eb;
  p.kp = (char*)a->pool.k;
  p.vp = (char*)a->pool.v;
  p.s_blk = a->pool.stride_block * kv_eb;
  p.s_slot = a->pool.stride_slot * kv_eb;
  p.s_head = a->pool.stride_head * kv_eb;
  p.block_size = a->pool.block_size;
  p.num_blocks = a->pool.num_blocks;
  p.block_is_chunk_aligned = a->pool.block_size % kChunk == 0;
  p.bs_div = make_fastdiv((uint32_t)a->pool.block_size);
  p.slot_small = (int64_t)a->pool.num_blocks * a->pool.block_size <= ((int64_t)1 << 31);
  {
    // Largest byte offset inside one pool: the last slot of the last head of
    // the last block, plus a row.
    const int64_t last = (int64_t)(a->pool.num_blocks > 0 ? a->pool.num_blocks - 1 : 0) *
                             a->pool.stride_block +
                         (int64_t)(a->pool.block_size - 1) * a->pool.stride_slot +
                         (int64_t)(a->num_kv_heads - 1) * a->pool.stride_head + a->head_dim;
    p.pool_off32 = last * kv_eb < ((int64_t)1 << 32) && a->pool.stride_block >= 0 &&
                   a->pool.stride_slot >= 0 && a->pool.stride_head >= 0;
  }
  p.table = a->block_tables;
  p.t_sb = a->table_stride_seq;
  p.table_i64 = a->table_dtype == VA_I64;
  p.table_width_full = a->table_width;
  p.table_width = (a->table_read_width > 0 && a->table_read_width < a->table_width)
                      ? a->table_read_width
                      : a->table_width;
  p.key_limit = a->key_limit;
  p.lens = a->lens;
  p.lens_i64 = a->lens_dtype == VA_I64;
  p.lens_cum = a->lens_kind == VA_LENS_CUMULATIVE;
  p.valid = a->valid_mask;
  p.valid_sb = a->valid_stride_seq;
  p.valid_len = a->valid_mask ? a->valid_len : 0;
  p.new_k = (const char*)a->new_k;
  p.new_v = (const char*)a->new_v;
  p.nk_sb = a->new_k_stride_seq * eb;
  p.nk_sh = a->new_k_stride_head * eb;
  p.nv_sb = a->new_v_stride_seq * eb;
  p.nv_sh = a->new_v_stride_head * eb;
  p.new_slots = a->new_slots;
  p.new_slots_i64 = a->new_slots_dtype == VA_I64;
  p.num_kv_heads = a->num_kv_heads;
  p.split_tokens = pl.split_tokens;
  p.max_parts = pl.max_parts;
  p.dyn_split = pl.dyn_split;
  // An FP8 pool's key scale multiplies every logit; its value scale the
  // output (applied after the weighted sum).
  p.scale_log2 = a->scale * (f8 ? a->pool.k_scale : 1.0f) * 1.4426950408889634f;
  p.kv_fp8 = f8;
  // Matrix-core workgroup shape (MfmaWaves): four waves when the launch has
  // more workgroups than CUs, so that several share a CU; otherwise twelve
  // over FP8 pools whose workgroups attend few tokens.
  const int64_t wgs = (int64_t)a->num_seqs * a->num_kv_heads * pl.max_parts;
  p.waves = a->head_dim != 128                ? 0
            : wgs > current_device_cus()      ? 4
            : f8 && pl.wg_tokens <= kWave12Tokens ? 12
                                              : 0;
  p.v_scale = f8 ? a->pool.v_scale : 1.0f;
  p.inv_k = f8 ? 1.0f / a->pool.k_scale : 1.0f;
  p.inv_v = f8 ? 1.0f / a->pool.v_scale : 1.0f;
  p.has_pro = a->prologue != nullptr;
  p.pro = PrologueParams{};
  if (a->prologue != nullptr) {
    const va_qk_prologue& pr = *a->prologue;
    VA_CHECK_ARG(pr.cos_sin_cache && pr.positions && pr.max_position > 0 &&
                     pr.cos_sin_stride >= a->head_dim,
                 "va_paged_decode: prologue rotary cache / positions");
    VA_CHECK_ARG(pr.q_norm_weight && (a->new_k == nullptr || pr.k_norm_weight),
                 "va_paged_decode: prologue norm weights missing");
    VA_CHECK_ARG(pr.weight_dtype == VA_BF16 || pr.weight_dtype == VA_F16 ||
                     pr.weight_dtype == VA_F32,
                 "va_paged_decode: prologue weight_dtype");
    VA_CHECK_ARG(pr.positions_dtype == VA_I32 || pr.positions_dtype == VA_I64,
                 "va_paged_decode: prologue positions_dtype");
    VA_CHECK_ARG((uintptr_t)pr.q_norm_weight % 16 == 0 && (uintptr_t)pr.k_norm_weight % 16 == 0,
                 "va_paged_decode: prologue norm weights must be 16-byte aligned");
    p.pro.q_w = pr.q_norm_weight;
    p.pro.k_w = pr.k_norm_weight;
    p.pro.w_dtype = pr.weight_dtype;
    p.pro.eps = pr.eps;
    p.pro.cs = pr.cos_sin_cache;
    p.pro.cs_stride = pr.cos_sin_stride;
    p.pro.max_pos = pr.max_position;
    p.pro.pos_i64 = pr.positions_dtype == VA_I64;
    p.pro.pos = pr.positions;
  }
  char* ws = (char*)a->workspace;
  p.part_ml = pl.total_bytes ? (float*)ws : nullptr;
  p.part_o = pl.total_bytes ? (float*)(ws + pl.ml_bytes) : nullptr;

  const dim3 grid(a->num_seqs, a->num_kv_heads, pl.max_parts);
  const hipStream_t s = (hipStream_t)stream;
  bool ok = false;
  if (small) {
    ok = launch_paged_decode_small(a->dtype, a->head_dim, G, p, dim3(a->num_seqs, a->num_heads),
                                   s);
    if (!ok) {
      set_error("va_paged_decode: unsupported dtype %d / head_dim %d", a->dtype, a->head_dim);
      return VA_ERR_UNSUPPORTED;
    }
    return check_launch("va_paged_decode");
  }
  if (f8 && !use_mfma_decode(a)) {
    set_error("va_paged_decode: an FP8 pool needs bf16/f16 q, a block size that is a multiple "
              "of 16, head_dim 64|128|256 and group 1|2|4|8 (got dtype %d, block %d, head_dim %d, "
              "group %d)",
              a->dtype, a->pool.block_size, a->head_dim, G);
    return VA_ERR_UNSUPPORTED;
  }
  if (f8) {
    ok = a->dtype == VA_BF16 ? launch_paged_decode_mfma_f8<BF16>(a->head_dim, G, p, grid, s)
                             : launch_paged_decode_mfma_f8<F16>(a->head_dim, G, p, grid, s);
  } else if (use_mfma_decode(a)) {
    ok = a->dtype == VA_BF16 ? launch_paged_decode_mfma<BF16>(a->head_dim, G, p, grid, s)
                             : launch_paged_decode_mfma<F16>(a->head_dim, G, p, grid, s);
  } else {
    switch (a->dtype) {
      case VA_BF16: ok = launch_paged_decode<BF16>(a->head_dim, G, p, grid, s); break;
      case VA_F16: ok = launch_paged_decode<F16>(a->head_dim, G, p, grid, s); break;
      case VA_F32: ok = launch_paged_decode<F32>(a->head_dim, G, p, grid, s); break;
    }
  }
  if (!ok) {
    set_error("va_paged_decode: unsupported head_dim %d / group size %d (head_dim 64|128|256, "
              "group 1|2|4|8)",
              a->head_dim, G);
    return VA_ERR_UNSUPPORTED;
  }
  return check_launch("va_paged_decode");
}
