// Paged decode for the shapes the matrix-core and general kernels do not
// take: a head_dim other than 64 / 128 / 256, or a query group other than
// 1 / 2 / 4 / 8.  The reference's Triton kernel pads any head_dim to a power
// of two (qwen_tts_paged_attention.py:470-480), and its own tests run at
// head_dim 4 with pages of 2 tokens (tests/test_qwen_tts_paged_attention_kernel.py:16-57);
// this kernel runs those shapes on the GPU.  It is correct for any size and
// built for small ones: scalar loads, no matrix cores, no context split.
//
// Semantics are the other decode kernels': attended length min(L, key_limit);
// table columns at or past table_width read block 0; a block id outside
// [0, num_blocks) or a false key_valid_mask byte (tokens past valid_len are
// valid) masks the token; the current row (new_k / new_v) goes to new_slots[b]
// or to the table slot of position L - 1 and is attended there in place of the
// pool's row, or, when it lies past the attended range (current_row_detached),
// is written and not attended; a row with no visible key gives 0.
//
// One workgroup per (sequence, query head).  Keys go in chunks of kChunkKeys:
// thread t scores keys t, t + 256, ... with a dot product over head_dim and
// keeps the key's V row offset in LDS; block reductions give the chunk's
// maximum and sum (online softmax in the exp2 domain); thread d then adds
// p_t v_t[d] over the chunk for its output elements d, d + 256, ...  The
// workgroup of the group's first query head writes the current row.
#include "paged_decode_kernel.h"

namespace va {
namespace {

constexpr int kSmallThreads = 256;
constexpr int kChunkKeys = 1024;
constexpr int kMaxPerThread = kSmallMaxHeadDim / kSmallThreads;  // output elements per thread
static_assert(kMaxPerThread * kSmallThreads == kSmallMaxHeadDim, "head_dim bound");

template <typename ET>
__device__ inline float ld_elem(const char* p) {
  if constexpr (ET::kBytes == 4)
    return *reinterpret_cast<const float*>(p);
  else if constexpr (ET::kIsBF16)
    return (float)*reinterpret_cast<const __bf16*>(p);
  else
    return (float)*reinterpret_cast<const _Float16*>(p);
}

template <typename ET>
__device__ inline void st_elem(char* p, float x) {
  if constexpr (ET::kBytes == 4)
    *reinterpret_cast<float*>(p) = x;
  else if constexpr (ET::kIsBF16)
    *reinterpret_cast<__bf16*>(p) = (__bf16)x;
  else
    *reinterpret_cast<_Float16*>(p) = (_Float16)x;
}

// Raw element copy (the current-row write is bit-exact).
template <typename ET>
__device__ inline void copy_elem(char* dst, const char* src) {
  if constexpr (ET::kBytes == 4)
    *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
  else
    *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
}

// Block-wide maximum / sum of one float per thread (every thread gets it).
__device__ inline float block_reduce(float x, bool is_max, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float y = __shfl_xor(x, o, 64);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kSmallThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  __syncthreads();  // red is reused by the next reduction
  return r;
}

template <typename ET>
__global__ __launch_bounds__(kSmallThreads) void paged_decode_small_kernel(DecodeParams p, int D,
                                                                          int G) {
  constexpr int EB = ET::kBytes;
  constexpr int64_t kNewRow = -2;  // V offset marker: the current row, read from new_v
  const int b = blockIdx.x;
  const int hq = blockIdx.y;
  const int h = hq / G;
  const int tid = threadIdx.x;
  __shared__ float s_q[kSmallMaxHeadDim];
  __shared__ float s_p[kChunkKeys];
  __shared__ int64_t s_voff[kChunkKeys];  // byte offset of the key's V row, -1 masked
  __shared__ float s_red[kSmallThreads / 64];

  const int L = p.lens_cum ? (int)(load_index(p.lens, b + 1, p.lens_i64) -
                                   load_index(p.lens, b, p.lens_i64))
                           : (int)load_index(p.lens, b, p.lens_i64);
  const int La = attend_len(p, L);
  const int64_t table_row = (int64_t)b * p.t_sb;
  const int col_new = L >= 1 ? (L - 1) / p.block_size : 0;
  const bool detached = current_row_detached(p, L, La, col_new);
  const int64_t cap = (int64_t)p.num_blocks * p.block_size;

  // Slot of the current row: new_slots[b]; otherwise the table slot of
  // position L - 1, through the table's own entry when detached and through
  // the entry the attention reads (block 0 past table_width) when in place.
  int64_t cur_slot = -1;
  if (p.new_k != nullptr && L >= 1) {
    if (p.new_slots != nullptr) {
      cur_slot = load_index(p.new_slots, b, p.new_slots_i64);
    } else {
      const int64_t blk =
          detached ? (col_new < p.table_width_full ? load_index(p.table, table_row + col_new,
                                                                p.table_i64)
                                                   : 0)
                   : table_entry(p, table_row, col_new);
      cur_slot = (blk >= 0 && blk < p.num_blocks) ? blk * p.block_size + (L - 1) % p.block_size
                                                  : -1;
    }
    if (cur_slot >= cap) cur_slot = -1;
  }
  const char* new_k = p.new_k ? p.new_k + b * p.nk_sb + h * p.nk_sh : nullptr;
  const char* new_v = p.new_v ? p.new_v + b * p.nv_sb + h * p.nv_sh : nullptr;
  if (cur_slot >= 0 && hq % G == 0) {
    const int64_t sb = cur_slot / p.block_size;
    const int64_t dst = sb * p.s_blk + (cur_slot - sb * p.block_size) * p.s_slot + h * p.s_head;
    for (int d = tid; d < D; d += kSmallThreads) {
      copy_elem<ET>(p.kp + dst + d * EB, new_k + d * EB);
      copy_elem<ET>(p.vp + dst + d * EB, new_v + d * EB);
    }
  }
  // Attended in place of the pool's row: position L - 1, when its slot is valid.
  const int cur_tok = (!detached && cur_slot >= 0 && L - 1 < La) ? L - 1 : -1;

  for (int d = tid; d < D; d += kSmallThreads)
    s_q[d] = ld_elem<ET>(p.q + b * p.q_sb + hq * p.q_sh + d * EB);
  __syncthreads();

  float m = -INFINITY, l = 0.f;
  float acc[kMaxPerThread];
#pragma unroll
  for (int i = 0; i < kMaxPerThread; ++i) acc[i] = 0.f;

  for (int c0 = 0; c0 < La; c0 += kChunkKeys) {
    const int n = min(kChunkKeys, La - c0);
    float cmax = -INFINITY;
    for (int t = tid; t < n; t += kSmallThreads) {
      const int tok = c0 + t;
      float s = -INFINITY;
      int64_t voff = -1;
      const bool on = tok >= p.valid_len || p.valid[(int64_t)b * p.valid_sb + tok] != 0;
      if (on) {
        const char* krow = nullptr;
        if (tok == cur_tok) {
          krow = new_k;
          voff = kNewRow;
        } else {
          const int64_t blk = table_entry(p, table_row, tok / p.block_size);
          if (blk >= 0 && blk < p.num_blocks) {
            voff = blk * p.s_blk + (int64_t)(tok % p.block_size) * p.s_slot + h * p.s_head;
            krow = p.kp + voff;
          }
        }
        if (krow != nullptr) {
          float dot = 0.f;
          for (int d = 0; d < D; ++d) dot = fmaf(s_q[d], ld_elem<ET>(krow + d * EB), dot);
          s = dot * p.scale_log2;
        }
      }
      s_p[t] = s;
      s_voff[t] = voff;
      cmax = fmaxf(cmax, s);
    }
    cmax = block_reduce(cmax, true, s_red);
    const float mn = fmaxf(m, cmax);
    float csum = 0.f;
    if (mn != -INFINITY) {
      for (int t = tid; t < n; t += kSmallThreads) {
        const float e = s_p[t] == -INFINITY ? 0.f : exp2f(s_p[t] - mn);
        s_p[t] = e;
        csum += e;
      }
    }
    csum = block_reduce(csum, false, s_red);  // its barrier publishes s_p
    if (mn != -INFINITY) {
      const float alpha = exp2f(m - mn);  // 0 while nothing was visible (m = -inf)
      l = l * alpha + csum;
#pragma unroll
      for (int i = 0; i < kMaxPerThread; ++i) {
        const int d = tid + i * kSmallThreads;
        if (d >= D) break;
        float a = acc[i] * alpha;
        for (int t = 0; t < n; ++t) {
          const float pt = s_p[t];
          if (pt == 0.f) continue;
          const int64_t vo = s_voff[t];
          const char* vrow = vo == kNewRow ? new_v : p.vp + vo;
          a = fmaf(pt, ld_elem<ET>(vrow + d * EB), a);
        }
        acc[i] = a;
      }
      m = mn;
    }
    __syncthreads();  // every thread is done with s_p / s_voff of this chunk
  }

  const float inv = l > 0.f ? p.v_scale / l : 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPerThread; ++i) {
    const int d = tid + i * kSmallThreads;
    if (d >= D) break;
    st_elem<ET>(p.out + b * p.o_sb + hq * p.o_sh + d * EB, acc[i] * inv);
  }
}

}  // namespace

bool launch_paged_decode_small(int dtype, int D, int G, const DecodeParams& p, dim3 grid,
                               hipStream_t s) {
  if (D < 1 || D > kSmallMaxHeadDim || G < 1) return false;
  switch (dtype) {
    case VA_BF16:
      hipLaunchKernelGGL(paged_decode_small_kernel<BF16>, grid, dim3(kSmallThreads), 0, s, p, D, G);
      return true;
    case VA_F16:
      hipLaunchKernelGGL(paged_decode_small_kernel<F16>, grid, dim3(kSmallThreads), 0, s, p, D, G);
      return true;
    case VA_F32:
      hipLaunchKernelGGL(paged_decode_small_kernel<F32>, grid, dim3(kSmallThreads), 0, s, p, D, G);
      return true;
    default:
      return false;
  }
}

}  // namespace va
