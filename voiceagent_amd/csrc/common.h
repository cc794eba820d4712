// Shared device helpers for the gfx950 attention kernels: element types,
// 16-byte vector loads, wave64 lane reductions (DPP within a 16-lane row,
// cross-row permutes above that) and the error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/voiceagent_attn.h"

namespace va {

// ------------------------------------------------------------------ errors
void set_error(const char* fmt, ...);

#define VA_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::va::set_error(__VA_ARGS__);      \
      return VA_ERR_INVALID_ARG;         \
    }                                    \
  } while (0)

int check_launch(const char* what);

// Compute units of the current device (cached per device; 256, the MI355X
// count, when no device is visible).
int current_device_cus();

// ------------------------------------------------------------ element types
// Each type describes how 16 bytes (one dwordx4 lane load) unpack to floats
// and how floats pack back.  bf16 -> f32 is exact (bit shift); f32 -> bf16
// rounds to nearest even, as torch does (hardware conversion on gfx950).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// dot(q, k, acc): acc + sum over the 16-byte vectors' elements, fp32
// accumulation.  16-bit types use v_dot2_f32_{bf16,f16} on raw (unscaled)
// q; F32 uses FMAs.
struct BF16 {
  static constexpr int kBytes = 2;
  static constexpr int kPerVec = 8;
  static constexpr bool kIsBF16 = true;
  __device__ static inline float dot(const uint4 q, const uint4 k, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.x),
                                          __builtin_bit_cast(bf16x2_t, k.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.y),
                                          __builtin_bit_cast(bf16x2_t, k.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.z),
                                          __builtin_bit_cast(bf16x2_t, k.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q.w),
                                          __builtin_bit_cast(bf16x2_t, k.w), acc, false);
    return acc;
  }
  __device__ static inline void unpack(const uint4 u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  // Round to nearest even (NaN stays NaN) with gfx950's v_cvt_pk_bf16_f32.
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  __device__ static inline uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x2_t v;
      v.x = (__bf16)f[2 * i];
      v.y = (__bf16)f[2 * i + 1];
      w[i] = __builtin_bit_cast(uint32_t, v);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};

struct F16 {
  static constexpr int kBytes = 2;
  static constexpr int kPerVec = 8;
  static constexpr bool kIsBF16 = false;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  __device__ static inline float dot(const uint4 q, const uint4 k, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.x), __builtin_bit_cast(f16x2_t, k.x),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.y), __builtin_bit_cast(f16x2_t, k.y),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.z), __builtin_bit_cast(f16x2_t, k.z),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q.w), __builtin_bit_cast(f16x2_t, k.w),
                                 acc, false);
    return acc;
  }
  __device__ static inline void unpack(const uint4 u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h2 h = __builtin_bit_cast(h2, w[i]);
      f[2 * i] = (float)h.x;
      f[2 * i + 1] = (float)h.y;
    }
  }
  __device__ static inline uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h2 h;
      h.x = (_Float16)f[2 * i];
      h.y = (_Float16)f[2 * i + 1];
      w[i] = __builtin_bit_cast(uint32_t, h);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};

struct F32 {
  static constexpr int kBytes = 4;
  static constexpr int kPerVec = 4;
  static constexpr bool kIsBF16 = false;
  __device__ static inline float dot(const uint4 q, const uint4 k, float acc) {
    acc = fmaf(__uint_as_float(q.x), __uint_as_float(k.x), acc);
    acc = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), acc);
    acc = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), acc);
    acc = fmaf(__uint_as_float(q.w), __uint_as_float(k.w), acc);
    return acc;
  }
  __device__ static inline void unpack(const uint4 u, float* f) {
    f[0] = __uint_as_float(u.x);
    f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z);
    f[3] = __uint_as_float(u.w);
  }
  __device__ static inline uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                      __float_as_uint(f[3]));
  }
};

// ------------------------------------------------------------- FP8 pools
// OCP e4m3 (float8_e4m3fn) codes of FP8 KV pools.  Quantisation saturates to
// +-448, the largest finite e4m3 value, before gfx950's round-to-nearest-even
// conversion (v_cvt_pk_fp8_f32); a NaN stays NaN.  Every e4m3 value is
// exactly representable in bf16 and f16, so dequantisation to either
// (v_cvt_scalef32_pk_{bf16,f16}_fp8 with a unit scale) is exact.
constexpr float kF8Max = 448.0f;
__device__ inline float f8_sat(float x) {
  return x > kF8Max ? kF8Max : (x < -kF8Max ? -kF8Max : x);
}
// Four floats (already multiplied by 1 / scale) to four e4m3 bytes, the
// first in the low byte.
__device__ inline uint32_t f8_pack4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(f8_sat(a), f8_sat(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(f8_sat(c), f8_sat(d), w, true);
  return (uint32_t)w;
}

// ------------------------------------------------------------ memory access
__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Non-temporal 16-byte load (the nt cache policy): for data read exactly once,
// such as the K/V rows of a decode step.  One CU streams ~80 GB/s with it and
// ~60 GB/s without it on MI355X.
typedef unsigned va_u32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld16_nt(const void* p) {
  const va_u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const va_u32x4*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ inline void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// Non-temporal 16-byte store: for results nothing in the launch reads back,
// such as attention output rows (measured: the encoder's launch 17.2 -> 16.0 us
// with its output stored this way).
__device__ inline void st16_nt(void* p, uint4 v) {
  __builtin_nontemporal_store(va_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<va_u32x4*>(p));
}

__device__ inline int64_t load_index(const void* p, int64_t i, int is_i64) {
  return is_i64 ? reinterpret_cast<const int64_t*>(p)[i]
                : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// The 16-bit word u of 8 elements of ET (BF16 or F16), each multiplied by
// inv in fp32, as 8 e4m3 codes (element i in byte i).
template <typename ET>
__device__ inline uint2 f8_quant8(uint4 u, float inv) {
  float f[8];
  ET::unpack(u, f);
  return make_uint2(f8_pack4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                    f8_pack4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv));
}
// 8 e4m3 codes (byte i = element i) as 8 elements of ET (BF16 or F16),
// exactly.
template <typename ET>
__device__ inline uint4 f8_dequant8(uint2 c) {
  uint32_t w[4];
  if constexpr (ET::kIsBF16) {
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, false));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, true));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, false));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, true));
  } else {
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.x, 1.0f, false));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.x, 1.0f, true));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.y, 1.0f, false));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.y, 1.0f, true));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------- lane reductions
// DPP control words (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ inline float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum / max over aligned groups of W lanes (W in 1..64, power of two).  Every
// lane of a group ends with the group's result.  Groups of <= 16 stay inside
// a DPP row; wider groups add cross-row permutes.
template <int W>
__device__ inline float group_sum(float x) {
  if constexpr (W >= 2) x += dpp<kDppQuadXor1>(x);
  if constexpr (W >= 4) x += dpp<kDppQuadXor2>(x);
  if constexpr (W >= 8) x += dpp<kDppRowHalfMirror>(x);
  if constexpr (W >= 16) x += dpp<kDppRowMirror>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (W >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

template <int W>
__device__ inline float group_max(float x) {
  if constexpr (W >= 2) x = fmaxf(x, dpp<kDppQuadXor1>(x));
  if constexpr (W >= 4) x = fmaxf(x, dpp<kDppQuadXor2>(x));
  if constexpr (W >= 8) x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
  if constexpr (W >= 16) x = fmaxf(x, dpp<kDppRowMirror>(x));
  if constexpr (W >= 32) x = fmaxf(x, __shfl_xor(x, 16, 64));
  if constexpr (W >= 64) x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

// Reduce across the lanes that share (lane % STRIDE), i.e. over lanes
// l, l+STRIDE, l+2*STRIDE, ... (STRIDE a power of two dividing 64).
template <int STRIDE>
__device__ inline float strided_sum(float x) {
#pragma unroll
  for (int s = STRIDE; s < 64; s <<= 1) x += __shfl_xor(x, s, 64);
  return x;
}
template <int STRIDE>
__device__ inline float strided_max(float x) {
#pragma unroll
  for (int s = STRIDE; s < 64; s <<= 1) x = fmaxf(x, __shfl_xor(x, s, 64));
  return x;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum / sum of x over lanes l and l ^ 32 (or l ^ 16) through gfx950's
// v_permlane32_swap / v_permlane16_swap (VALU, no LDS round trip).
// permlane32_swap(a, a) swaps lanes 32..63 of its first operand with lanes
// 0..31 of its second, so in every lane its two results hold x[l] and
// x[l ^ 32], in one order or the other: the reduction of the two needs no
// lane test.  permlane16_swap does the same for the odd / even 16-lane rows
// of each half.  The maximum is a plain v_max_f32: fmaxf would canonicalise
// both swapped values first (two more instructions per step).
__device__ inline float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(r[0]), "v"(r[1]));
  return m;
}
__device__ inline float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(r[0]), "v"(r[1]));
  return m;
}
__device__ inline float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------- global -> LDS DMA
// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane l's
// bytes land at lds + 16 l.  Inline asm, so the compiler neither waits on it
// nor moves memory accesses across it; callers wait with wait_vmcnt.
// The compiler's hazard recognizer does not look inside inline asm, so each
// asm pads the wait states the ISA requires before the load itself: five
// after a VALU write of an SGPR the load reads (uniform bases come from
// v_readfirstlane) and one after the SALU write of M0.
__device__ inline void dma16(uint32_t off, const void* base, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}
// The same with the non-temporal cache policy (data read exactly once).
__device__ inline void dma16_nt(uint32_t off, const void* base, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}
// The same from a per-lane 64-bit address.
__device__ inline void dma16(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}
__device__ inline void dma16_nt(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(lds)
               : "memory");
}

// s_waitcnt vmcnt(N) / lgkmcnt(0) as inline asm with a memory clobber: no
// memory access moves across the wait (the waitcnt builtin is not a memory
// barrier for the compiler).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A wave-uniform pointer in SGPRs (readfirstlane of both halves).
__device__ inline const char* uniform_ptr(const char* ptr) {
  const uint64_t u = (uint64_t)(uintptr_t)ptr;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (const char*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

}  // namespace va
