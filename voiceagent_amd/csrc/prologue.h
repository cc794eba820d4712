// Qwen3's per-head query/key prologue on the lanes that hold one head row:
// RMSNorm over head_dim (qwen_asr_vllm/layers/layernorm.py:19-25) and the
// half-split rotary embedding (qwen_asr_vllm/layers/rotary_embedding.py:9-32).
//
// A row of D elements is spread over LPR consecutive lanes, E = 16 / sizeof(T)
// contiguous elements per lane (lane c of the row holds elements
// [c E, c E + E)).  The row's sum of squares is a DPP reduction over those
// lanes; the rotary partner of element i (i +- D/2) sits in lane c ^ (LPR/2)
// at the same slot.  Every rounding the reference performs in the element
// type is reproduced (to_dtype after the normalisation, after the weight,
// after the rotation), and products and sums are rounded separately.
#pragma once

#include "common.h"

namespace va {

struct PrologueParams {
  const void* q_w;
  const void* k_w;
  int32_t w_dtype;
  float eps;
  const float* cs;
  int64_t cs_stride;
  int32_t max_pos;
  int32_t pos_i64;
  const void* pos;
};

template <typename ET>
__device__ inline float round_to(float x) {
  if constexpr (ET::kBytes == 4) {
    return x;
  } else if constexpr (ET::kIsBF16) {
    return __uint_as_float((uint32_t)BF16::from_float(x) << 16);
  } else {
    return (float)(_Float16)x;
  }
}

// E weights starting at element `start`, as floats.
template <int E>
__device__ inline void load_weights(const void* w, int dtype, int start, float (&out)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (dtype == VA_F32) {
      out[e] = reinterpret_cast<const float*>(w)[start + e];
    } else if (dtype == VA_BF16) {
      out[e] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(w)[start + e] << 16);
    } else {
      out[e] = (float)reinterpret_cast<const _Float16*>(w)[start + e];
    }
  }
}

// The cos / sin factors of this lane's slice at `pos` (col = lane's index in
// its row of LPR lanes).
template <int E, int LPR>
__device__ inline void load_rotary(const PrologueParams& pp, int64_t pos, int col, int D,
                                   float (&c)[E], float (&s)[E]) {
  const float* row = pp.cs + pos * pp.cs_stride;
  const int i0 = (col % (LPR / 2)) * E;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    c[e] = row[i0 + e];
    s[e] = row[D / 2 + i0 + e];
  }
}

// In place on the lane's E floats of one row: normalise, weight, rotate.
template <typename ET, int LPR, int E>
__device__ inline void qk_prologue(float (&x)[E], const float (&w)[E], float eps, int D,
                                   const float (&c)[E], const float (&s)[E], bool first_half) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss = __fadd_rn(ss, __fmul_rn(x[e], x[e]));
  ss = group_sum<LPR>(ss);
  const float r = 1.0f / sqrtf(__fadd_rn(ss / (float)D, eps));
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = round_to<ET>(__fmul_rn(round_to<ET>(__fmul_rn(x[e], r)), w[e]));
  float pt[E];
#pragma unroll
  for (int e = 0; e < E; ++e) pt[e] = __shfl_xor(x[e], LPR / 2, 64);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float a = __fmul_rn(x[e], c[e]), b = __fmul_rn(pt[e], s[e]);
    x[e] = round_to<ET>(first_half ? __fsub_rn(a, b) : __fadd_rn(a, b));
  }
}

}  // namespace va
