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
// and, by the caller's pack, after the rotation), and the rotation's products
// are rounded before their sum.
#pragma once

#include <type_traits>

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

// An fp32 value the compiler may not fold into the operation that consumes
// it.  On gfx950 a conversion to half can absorb the multiply or add that
// produced its operand (v_fma_mixlo_f16), rounding once where the reference
// rounds to fp32 first; whether it does depends on the surrounding code, so
// two kernels running the same arithmetic could differ in the last bit.  No
// instruction is emitted.
__device__ inline void pin(float& x) { asm("" : "+v"(x)); }

// Every element of x rounded to the element type (nearest even) and widened
// back to float, two at a time (one packed conversion per pair; bf16 through
// gfx950's v_cvt_pk_bf16_f32).  Each operand is first rounded to fp32, as the
// reference's fp32 result is (pin).
template <typename ET, int E>
__device__ inline void round_to(float (&x)[E]) {
  static_assert(E % 2 == 0, "pairs");
  if constexpr (ET::kBytes == 2) {
#pragma unroll
    for (int i = 0; i < E; ++i) pin(x[i]);
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
      if constexpr (ET::kIsBF16) {
        bf16x2_t v;
        v.x = (__bf16)x[2 * i];
        v.y = (__bf16)x[2 * i + 1];
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        x[2 * i] = __uint_as_float(u << 16);
        x[2 * i + 1] = __uint_as_float(u & 0xffff0000u);
      } else {
        f16x2_t v;
        v.x = (_Float16)x[2 * i];
        v.y = (_Float16)x[2 * i + 1];
        x[2 * i] = (float)v.x;
        x[2 * i + 1] = (float)v.y;
      }
    }
  }
}

// The value held by lane (lane ^ (LPR / 2)) of the same LPR-lane row: the
// rotary partner.  A 16-lane row (D = 128 in 16-bit types) is one DPP row,
// rotated by 8; other widths use a cross-lane permute.
template <int LPR>
__device__ inline float rotary_partner(float x) {
  if constexpr (LPR == 16) {
    // Every lane of the row has a source, so no fallback value is needed
    // (update_dpp would first move one into the destination).
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128 /* row_ror:8 */, 0xF,
                                                   0xF, false));
  } else {
    return __shfl_xor(x, LPR / 2, 64);
  }
}

// The E norm weights from element `start`, as raw bytes: two loads of E * 2
// bytes each, issued without a branch (a loaded value that meets a branch
// join makes the compiler wait for every outstanding load).  16-bit weights
// sit in `a` (`b` repeats it); fp32 weights are `a` then `b`.  The weight
// array must be aligned to 2 E bytes.
template <int E>
struct WeightRaw {
  using V = typename std::conditional<E == 8, uint4, uint2>::type;
  V a, b;
};

template <int E>
__device__ inline WeightRaw<E> load_weights_raw(const void* w, int dtype, int start) {
  using V = typename WeightRaw<E>::V;
  const int wb = dtype == VA_F32 ? 4 : 2;
  const char* ptr = reinterpret_cast<const char*>(w) + (int64_t)start * wb;
  WeightRaw<E> r;
  r.a = *reinterpret_cast<const V*>(ptr);
  r.b = *reinterpret_cast<const V*>(ptr + (wb == 4 ? E * 2 : 0));
  return r;
}

template <int E>
__device__ inline void convert_weights(const WeightRaw<E>& r, int dtype, float (&out)[E]) {
  uint32_t wa[E / 2], wbv[E / 2];
  __builtin_memcpy(wa, &r.a, sizeof(wa));
  __builtin_memcpy(wbv, &r.b, sizeof(wbv));
  if (dtype == VA_F32) {
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      out[e] = __uint_as_float(wa[e]);
      out[E / 2 + e] = __uint_as_float(wbv[e]);
    }
  } else if (dtype == VA_BF16) {
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      out[2 * e] = __uint_as_float(wa[e] << 16);
      out[2 * e + 1] = __uint_as_float(wa[e] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      const f16x2_t hv = __builtin_bit_cast(f16x2_t, wa[e]);
      out[2 * e] = (float)hv.x;
      out[2 * e + 1] = (float)hv.y;
    }
  }
}

// The E norm weights of one row from raw words: 16-bit weights (kW16) from
// r.a, as bfloat16 when `bf` is set and as half otherwise; fp32 weights from
// r.a then r.b.  The values convert_weights gives.  A kernel that unpacks
// 16-bit weights row by row keeps E/2 words per weight array in registers
// instead of E floats (the qk prologue kernel's occupancy depends on it).
template <int E, bool kW16>
__device__ inline void row_weights(const WeightRaw<E>& r, bool bf, float (&out)[E]) {
  uint32_t wa[E / 2];
  __builtin_memcpy(wa, &r.a, sizeof(wa));
  if constexpr (kW16) {
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      const f16x2_t hv = __builtin_bit_cast(f16x2_t, wa[e]);
      out[2 * e] = bf ? __uint_as_float(wa[e] << 16) : (float)hv.x;
      out[2 * e + 1] = bf ? __uint_as_float(wa[e] & 0xffff0000u) : (float)hv.y;
    }
  } else {
    uint32_t wb[E / 2];
    __builtin_memcpy(wb, &r.b, sizeof(wb));
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      out[e] = __uint_as_float(wa[e]);
      out[E / 2 + e] = __uint_as_float(wb[e]);
    }
  }
}

// Norm weight i of a weight array of `dtype`, widened to float.
__device__ inline float load_weight(const void* w, int dtype, int i) {
  if (dtype == VA_F32) return reinterpret_cast<const float*>(w)[i];
  const uint32_t u = reinterpret_cast<const uint16_t*>(w)[i];
  if (dtype == VA_BF16) return __uint_as_float(u << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
}

// The cos / sin factors of this lane's slice at `pos` (col = lane's index in
// its row of LPR lanes).  The sin factors of the row's first half come
// negated: element i < D/2 rotates to x_i cos - x_(i+D/2) sin, and
// x cos + p (-sin) rounds exactly as x cos - p sin does.
template <int E, int LPR>
__device__ inline void load_rotary(const PrologueParams& pp, int64_t pos, int col, int D,
                                   float (&c)[E], float (&s)[E]) {
  const float* row = pp.cs + pos * pp.cs_stride;
  // Both halves through a pointer each, so that each loads as whole vectors
  // (indexing the sin half from `row` left eight scalar loads, each with its
  // own address held in registers).
  const float* srow = row + D / 2;
  const int i0 = (col % (LPR / 2)) * E;
  const bool first_half = col < LPR / 2;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    c[e] = row[i0 + e];
    const float sv = srow[i0 + e];
    s[e] = first_half ? -sv : sv;
  }
}

// In place on the lane's E floats of one row: normalise, weight, rotate, with
// s from load_rotary.  The result is left unrounded: every caller packs it
// to the element type, which is the reference's last rounding.
template <typename ET, int LPR, int E>
__device__ inline void qk_prologue(float (&x)[E], const float (&w)[E], float eps, int D,
                                   const float (&c)[E], const float (&s)[E]) {
  // The sum of squares is reduced in another order than the reference's
  // mean, so it is not bit-exact either way; it takes fused multiply-adds.
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss = fmaf(x[e], x[e], ss);
  ss = group_sum<LPR>(ss);
  const float r = 1.0f / sqrtf(__fadd_rn(ss / (float)D, eps));
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = __fmul_rn(x[e], r);
  round_to<ET>(x);
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = __fmul_rn(x[e], w[e]);
  round_to<ET>(x);
  float pt[E];
#pragma unroll
  for (int e = 0; e < E; ++e) pt[e] = rotary_partner<LPR>(x[e]);
  {
    // x cos and p sin rounded apart before their sum, as the reference's
    // elementwise ops round them: no fused multiply-add here.
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = x[e] * c[e] + pt[e] * s[e];
  }
  // The caller's pack rounds the fp32 sums, not a fused form of them.
#pragma unroll
  for (int e = 0; e < E; ++e) pin(x[e]);
}

}  // namespace va
