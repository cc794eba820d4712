// Variable-length attention over packed sequences on CDNA4 bf16/f16 MFMA:
// causal prefill (bottom-right aligned, optionally over a paged prefix with
// the KV store fused) and non-causal block-diagonal encoder windows.
//
// Semantics (flash_attn_varlen_func as qwen_asr_vllm/layers/attention.py
// calls it, :1-11, 92-107, 121-139): sequence s owns queries
// [cu_q[s], cu_q[s+1]) and k_len = cu_k[s+1] - cu_k[s] keys.  Query i of head
// hq sees key j of kv head hq / G iff j < k_len and, when causal,
// j <= k_len - q_len + i; out = softmax(scale * q.K^T) V over visible keys
// (0 when none is visible).  The non-causal case with cu_q = cu_k is the
// block-diagonal mask of reference/modeling_qwen3_asr.py:649-667.
//
// Tiling (one workgroup = 4 wave64 = 256 lanes): a workgroup owns one
// (sequence, kv head, query block) and serves all G query heads of the kv
// group, so its 128 MFMA rows are BQ = 128 / G query positions x G heads.
// Each wave owns two 16-row tiles.  Keys stream through LDS in 64-key tiles
// (K and V row-major, rows padded to avoid bank conflicts).  Per tile:
//   S^T = K Q^T  with v_mfma_f32_16x16x32 (A = K rows from LDS via
//                ds_read_b128, B = Q^T held in registers for the whole loop);
//   online softmax in the exp2 domain on the S^T accumulators: each lane
//                holds 4 consecutive keys of one query row, so the row max /
//                sum need only two cross-lane steps;
//   O^T += V^T P^T with the same MFMA: P^T is the S^T accumulator converted
//                to 16-bit in place (the MFMA's k index is permuted to match),
//                and V^T comes from row-major V through ds_read_b64_tr_b16.
// With a paged pool, keys j < k_len - q_len are gathered through the block
// table while the tile is loaded; the new keys come from k/v.  The fused
// store copies this workgroup's new K/V rows to slot_mapping before the loop.
#include "common.h"

namespace va {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

struct VarlenParams {
  const char* q;
  int64_t q_st, q_sh;  // bytes
  const char* k;
  int64_t k_st, k_sh;
  const char* v;
  int64_t v_st, v_sh;
  char* out;
  int64_t o_st, o_sh;
  const int32_t* cu_q;
  const int32_t* cu_k;
  float scale_log2;
  int32_t has_pool;
  char* kp;
  char* vp;
  int64_t s_blk, s_slot, s_head;  // bytes
  int32_t block_size, num_blocks;
  const void* table;
  int64_t t_sb;
  int32_t table_i64, table_width;
  const void* slots;
  int32_t slot_i64;
  int32_t num_qblocks;
};

template <bool kBF16>
struct Mma {
  __device__ static inline f32x4_t mfma(uint4 a, uint4 b, f32x4_t c) {
    if constexpr (kBF16)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                     __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                    __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    if constexpr (kBF16)
      return (uint32_t)BF16::from_float(lo) | ((uint32_t)BF16::from_float(hi) << 16);
    else
      return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
  }
};

constexpr int kVarlenThreads = 256;
constexpr int kRowsPerWG = 128;
constexpr int kKeyTile = 64;

__device__ inline uint4 lds_read16(const char* base, int off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

__device__ inline s16x4_t lds_read_tr(const char* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(base + off));
}

template <bool kBF16, int D, int G, bool kCausal>
__global__ __launch_bounds__(kVarlenThreads, 2) void varlen_attention_kernel(VarlenParams p) {
  constexpr int BQ = kRowsPerWG / G;       // query positions per workgroup
  constexpr int DS = D / 32;               // k-steps of the S^T MFMA
  constexpr int DT = D / 16;               // 16-wide d tiles of O^T
  constexpr int CPR = D * 2 / 16;          // 16-byte chunks per K/V row
  constexpr int LDS_ROW = D * 2 + 32;      // padded row pitch in bytes
  constexpr int KT = kKeyTile / 16;        // 16-key tiles per key tile
  constexpr int KS = kKeyTile / 32;        // 32-key MFMA steps per key tile
  constexpr int LOADS = kKeyTile * CPR / kVarlenThreads;
  static_assert(BQ % 16 == 0, "query block must hold whole 16-row tiles");
  static_assert(LOADS * kVarlenThreads == kKeyTile * CPR, "tile load split");
  using M = Mma<kBF16>;

  __shared__ __align__(16) char s_kv[2 * kKeyTile * LDS_ROW];
  char* s_k = s_kv;
  char* s_v = s_kv + kKeyTile * LDS_ROW;

  const int qb = p.num_qblocks - 1 - (int)blockIdx.x;  // heavy (late) blocks first
  const int h = blockIdx.y;
  const int s = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;

  const int q0 = p.cu_q[s];
  const int ql = p.cu_q[s + 1] - q0;
  const int k0 = p.cu_k[s];
  const int kl = p.cu_k[s + 1] - k0;
  const int pos0 = qb * BQ;
  if (pos0 >= ql) return;
  const int pos_end = min(ql, pos0 + BQ);
  const int diag = kl - ql;  // bottom-right alignment offset
  const int pool_prefix = p.has_pool ? (p.k != nullptr ? kl - ql : kl) : 0;

  // ---- fused store of this block's new K/V rows (kv head h) ----
  if (p.slots != nullptr) {
    const int nrows = pos_end - pos0;
    const int64_t cap = (int64_t)p.num_blocks * p.block_size;
    for (int c = tid; c < nrows * CPR * 2; c += kVarlenThreads) {
      const int is_v = c >= nrows * CPR;
      const int cc = is_v ? c - nrows * CPR : c;
      const int row = cc / CPR, chunk = cc % CPR;
      const int tok = q0 + pos0 + row;
      const int64_t slot = load_index(p.slots, tok, p.slot_i64);
      if (slot < 0 || slot >= cap) continue;
      const int64_t blk = slot / p.block_size;
      const char* src = (is_v ? p.v + tok * p.v_st + h * p.v_sh : p.k + tok * p.k_st + h * p.k_sh) +
                        chunk * 16;
      char* dst = (is_v ? p.vp : p.kp) + blk * p.s_blk + (slot - blk * p.block_size) * p.s_slot +
                  h * p.s_head + chunk * 16;
      st16(dst, ld16(src));
    }
  }

  // ---- per-lane row bookkeeping: two 16-row tiles per wave ----
  int qpos[2], qhead[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int row = 16 * (2 * wave + tt) + r16;
    qhead[tt] = h * G + row / BQ;
    qpos[tt] = pos0 + row % BQ;
  }

  uint4 qreg[2][DS];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      if (qpos[tt] < ql)
        qreg[tt][ds] = ld16(p.q + (int64_t)(q0 + qpos[tt]) * p.q_st +
                            (int64_t)qhead[tt] * p.q_sh + (32 * ds + 8 * g4) * 2);
      else
        qreg[tt][ds] = make_uint4(0, 0, 0, 0);
    }

  float m[2] = {-1.0e30f, -1.0e30f};
  float l[2] = {0.f, 0.f};
  f32x4_t o[2][DT];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[tt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int kend = kCausal ? max(0, min(kl, diag + pos_end)) : kl;
  const int64_t table_row = (int64_t)s * p.t_sb;

  for (int kb = 0; kb < kend; kb += kKeyTile) {
    // ---- stage K/V tile [kb, kb + 64) into LDS ----
    uint4 kbuf[LOADS], vbuf[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * kVarlenThreads;
      const int key = c / CPR, chunk = c % CPR;
      const int j = kb + key;
      kbuf[i] = make_uint4(0, 0, 0, 0);
      vbuf[i] = make_uint4(0, 0, 0, 0);
      if (j < kend) {
        const char* ka = nullptr;
        const char* va_ = nullptr;
        if (j < pool_prefix) {
          const int col = j / p.block_size;
          const int64_t blk =
              col < p.table_width ? load_index(p.table, table_row + col, p.table_i64) : 0;
          if (blk >= 0 && blk < p.num_blocks) {
            const int64_t off = blk * p.s_blk + (int64_t)(j % p.block_size) * p.s_slot +
                                h * p.s_head + chunk * 16;
            ka = p.kp + off;
            va_ = p.vp + off;
          }
        } else {
          const int64_t row = p.has_pool ? (int64_t)q0 + (j - pool_prefix) : (int64_t)k0 + j;
          ka = p.k + row * p.k_st + h * p.k_sh + chunk * 16;
          va_ = p.v + row * p.v_st + h * p.v_sh + chunk * 16;
        }
        if (ka != nullptr) {
          kbuf[i] = ld16(ka);
          vbuf[i] = ld16(va_);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * kVarlenThreads;
      const int key = c / CPR, chunk = c % CPR;
      *reinterpret_cast<uint4*>(s_k + key * LDS_ROW + chunk * 16) = kbuf[i];
      *reinterpret_cast<uint4*>(s_v + key * LDS_ROW + chunk * 16) = vbuf[i];
    }
    __syncthreads();

    // ---- S^T = K Q^T for both row tiles ----
    f32x4_t sacc[2][KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      sacc[0][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      sacc[1][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const uint4 a = lds_read16(s_k, (16 * kt + r16) * LDS_ROW + (32 * ds + 8 * g4) * 2);
        sacc[0][kt] = M::mfma(a, qreg[0][ds], sacc[0][kt]);
        sacc[1][kt] = M::mfma(a, qreg[1][ds], sacc[1][kt]);
      }
    }

    // ---- online softmax (exp2 domain) and P^T packing ----
    uint4 pb[2][KS];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      float sv[KT][4];
      float mx = -INFINITY;
      const int lim = kCausal ? min(kend, diag + qpos[tt] + 1) : kend;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = kb + 16 * kt + 4 * g4 + i;
          const float x = sacc[tt][kt][i] * p.scale_log2;
          sv[kt][i] = (j < lim && qpos[tt] < ql) ? x : -INFINITY;
          mx = fmaxf(mx, sv[kt][i]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m[tt], mx);
      const float alpha = fast_exp2(m[tt] - mnew);
      m[tt] = mnew;
      l[tt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[tt][dt] *= alpha;
      float pr[KT][4];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[kt][i] = fast_exp2(sv[kt][i] - mnew);
          l[tt] += pr[kt][i];
        }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        pb[tt][ks].x = M::pack2(pr[2 * ks][0], pr[2 * ks][1]);
        pb[tt][ks].y = M::pack2(pr[2 * ks][2], pr[2 * ks][3]);
        pb[tt][ks].z = M::pack2(pr[2 * ks + 1][0], pr[2 * ks + 1][1]);
        pb[tt][ks].w = M::pack2(pr[2 * ks + 1][2], pr[2 * ks + 1][3]);
      }
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int off = (32 * ks + 4 * g4 + (r16 >> 2)) * LDS_ROW + (16 * dt + 4 * (r16 & 3)) * 2;
        const s16x4_t lo = lds_read_tr(s_v, off);
        const s16x4_t hi = lds_read_tr(s_v, off + 16 * LDS_ROW);
        uint4 a;
        a.x = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
        a.y = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
        a.z = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
        a.w = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
        o[0][dt] = M::mfma(a, pb[0][ks], o[0][dt]);
        o[1][dt] = M::mfma(a, pb[1][ks], o[1][dt]);
      }
    __syncthreads();
  }

  // ---- normalise and write: lane holds O[row r16][16 dt + 4 g4 + i] ----
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    float lt = l[tt];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    if (qpos[tt] >= ql) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    char* dst = p.out + (int64_t)(q0 + qpos[tt]) * p.o_st + (int64_t)qhead[tt] * p.o_sh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint2 w;
      w.x = M::pack2(o[tt][dt][0] * inv, o[tt][dt][1] * inv);
      w.y = M::pack2(o[tt][dt][2] * inv, o[tt][dt][3] * inv);
      *reinterpret_cast<uint2*>(dst + (16 * dt + 4 * g4) * 2) = w;
    }
  }
}

template <bool kBF16, int D, int G>
static void launch_varlen(const VarlenParams& p, bool causal, dim3 grid, hipStream_t st) {
  if (causal)
    hipLaunchKernelGGL((varlen_attention_kernel<kBF16, D, G, true>), grid, dim3(kVarlenThreads), 0,
                       st, p);
  else
    hipLaunchKernelGGL((varlen_attention_kernel<kBF16, D, G, false>), grid, dim3(kVarlenThreads),
                       0, st, p);
}

template <bool kBF16, int D>
static bool dispatch_varlen_g(int G, const VarlenParams& p, bool causal, dim3 grid,
                              hipStream_t st) {
  switch (G) {
    case 1: launch_varlen<kBF16, D, 1>(p, causal, grid, st); return true;
    case 2: launch_varlen<kBF16, D, 2>(p, causal, grid, st); return true;
    case 4: launch_varlen<kBF16, D, 4>(p, causal, grid, st); return true;
    case 8: launch_varlen<kBF16, D, 8>(p, causal, grid, st); return true;
    default: return false;
  }
}

template <bool kBF16>
static bool dispatch_varlen(int D, int G, const VarlenParams& p, bool causal, dim3 grid,
                            hipStream_t st) {
  switch (D) {
    case 64: return dispatch_varlen_g<kBF16, 64>(G, p, causal, grid, st);
    case 128: return dispatch_varlen_g<kBF16, 128>(G, p, causal, grid, st);
    default: return false;
  }
}

}  // namespace va

extern "C" int va_varlen_attention(const va_varlen_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_varlen_attention: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_varlen_args),
               "va_varlen_attention: struct_size %u != %zu (header/library mismatch)",
               a->struct_size, sizeof(va_varlen_args));
  VA_CHECK_ARG(a->num_seqs >= 0, "va_varlen_attention: num_seqs < 0");
  if (a->num_seqs == 0 || a->total_q == 0) return VA_OK;
  VA_CHECK_ARG(a->dtype == VA_BF16 || a->dtype == VA_F16,
               "va_varlen_attention: dtype must be VA_BF16 or VA_F16 (MFMA path)");
  VA_CHECK_ARG(a->q && a->out && a->cu_seqlens_q && a->cu_seqlens_k,
               "va_varlen_attention: null pointer argument");
  VA_CHECK_ARG(a->num_seqs <= 65535, "va_varlen_attention: num_seqs > 65535");
  VA_CHECK_ARG(a->num_kv_heads > 0 && a->num_kv_heads <= 65535 && a->num_heads > 0 &&
                   a->num_heads % a->num_kv_heads == 0,
               "va_varlen_attention: num_heads (%d) must be a positive multiple of "
               "num_kv_heads (%d)",
               a->num_heads, a->num_kv_heads);
  const bool has_pool = a->pool.k != nullptr;
  VA_CHECK_ARG(has_pool || (a->k && a->v), "va_varlen_attention: k/v required without a pool");
  VA_CHECK_ARG(!has_pool || (a->pool.v && a->block_tables && a->pool.block_size > 0 &&
                             a->pool.num_blocks >= 0 && a->table_width >= 0),
               "va_varlen_attention: incomplete pool description");
  VA_CHECK_ARG((a->k == nullptr) == (a->v == nullptr),
               "va_varlen_attention: k and v must be given together");
  VA_CHECK_ARG(a->slot_mapping == nullptr || (has_pool && a->k),
               "va_varlen_attention: slot_mapping needs a pool and k/v");
  VA_CHECK_ARG(a->max_seqlen_q >= 0 && a->max_seqlen_k >= 0, "va_varlen_attention: max_seqlen");
  VA_CHECK_ARG(!has_pool || a->table_dtype == VA_I32 || a->table_dtype == VA_I64,
               "va_varlen_attention: table_dtype");
  VA_CHECK_ARG(a->slot_mapping == nullptr || a->slot_dtype == VA_I32 || a->slot_dtype == VA_I64,
               "va_varlen_attention: slot_dtype");
  const int64_t strides[] = {a->q_stride_tok,  a->q_stride_head,      a->k_stride_tok,
                             a->k_stride_head, a->v_stride_tok,       a->v_stride_head,
                             a->out_stride_tok, a->out_stride_head,   a->pool.stride_block,
                             a->pool.stride_slot, a->pool.stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * 2) % 16 == 0, "va_varlen_attention: strides must be 16-byte multiples");
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->v, (uintptr_t)a->out,
                            (uintptr_t)a->pool.k, (uintptr_t)a->pool.v};
  for (uintptr_t p : ptrs)
    VA_CHECK_ARG(p % 16 == 0, "va_varlen_attention: pointers must be 16-byte aligned");
  const int G = a->num_heads / a->num_kv_heads;
  if (!((a->head_dim == 64 || a->head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8))) {
    set_error("va_varlen_attention: unsupported head_dim %d / group size %d (head_dim 64|128, "
              "group 1|2|4|8)",
              a->head_dim, G);
    return VA_ERR_UNSUPPORTED;
  }
  const int BQ = kRowsPerWG / G;
  const int nqb = (a->max_seqlen_q + BQ - 1) / BQ;
  if (nqb == 0) return VA_OK;
  VA_CHECK_ARG(nqb <= 65535 * 16, "va_varlen_attention: max_seqlen_q too large");

  VarlenParams p;
  p.q = (const char*)a->q;
  p.q_st = a->q_stride_tok * 2;
  p.q_sh = a->q_stride_head * 2;
  p.k = (const char*)a->k;
  p.k_st = a->k_stride_tok * 2;
  p.k_sh = a->k_stride_head * 2;
  p.v = (const char*)a->v;
  p.v_st = a->v_stride_tok * 2;
  p.v_sh = a->v_stride_head * 2;
  p.out = (char*)a->out;
  p.o_st = a->out_stride_tok * 2;
  p.o_sh = a->out_stride_head * 2;
  p.cu_q = a->cu_seqlens_q;
  p.cu_k = a->cu_seqlens_k;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.has_pool = has_pool;
  p.kp = (char*)a->pool.k;
  p.vp = (char*)a->pool.v;
  p.s_blk = a->pool.stride_block * 2;
  p.s_slot = a->pool.stride_slot * 2;
  p.s_head = a->pool.stride_head * 2;
  p.block_size = has_pool ? a->pool.block_size : 1;
  p.num_blocks = a->pool.num_blocks;
  p.table = a->block_tables;
  p.t_sb = a->table_stride_seq;
  p.table_i64 = a->table_dtype == VA_I64;
  p.table_width = a->table_width;
  p.slots = a->slot_mapping;
  p.slot_i64 = a->slot_dtype == VA_I64;
  p.num_qblocks = nqb;

  const dim3 grid(nqb, a->num_kv_heads, a->num_seqs);
  const hipStream_t st = (hipStream_t)stream;
  const bool ok = a->dtype == VA_BF16
                      ? dispatch_varlen<true>(a->head_dim, G, p, a->causal != 0, grid, st)
                      : dispatch_varlen<false>(a->head_dim, G, p, a->causal != 0, grid, st);
  if (!ok) {
    set_error("va_varlen_attention: unsupported configuration");
    return VA_ERR_UNSUPPORTED;
  }
  return check_launch("va_varlen_attention");
}
