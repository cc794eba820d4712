// Standalone Qwen3 q/k prologue: RMSNorm + half-split rotary embedding of
// every query and key head row of a batch of tokens (the prefill side of
// Qwen3Attention.forward, qwen_asr_vllm/models/qwen3.py:42-48; the decode side
// is fused into the paged decode kernel).  One group of LPR lanes per head
// row, a token's rows over one or more waves (or, with few rows per token,
// several tokens per wave); the per-row math lives in prologue.h.
#include <algorithm>

#include "prologue.h"

namespace va {

struct QkParams {
  const char* q;
  int64_t q_st, q_sh;  // bytes
  const char* k;
  int64_t k_st, k_sh;
  char* qo;
  int64_t qo_st, qo_sh;
  char* ko;
  int64_t ko_st, ko_sh;
  int32_t num_tokens, hq, hkv;
  int32_t waves_per_token, groups_per_wave;  // row groups split over waves
  PrologueParams pp;
};

constexpr int kQkThreads = 256;
// Row groups whose loads a lane of qk_norm_rope_kernel keeps in flight at
// once: six hold a token of 16 + 8 heads in one round trip and keep the
// kernel at 90 VGPRs, five waves per SIMD (eight groups: 108 VGPRs, four).
constexpr int kQkChunk = 6;
// Head rows per token up to which prompt-sized batches take
// qk_norm_rope_tokens_kernel (keys alone: 8 heads).
constexpr int kQkTokenRows = 8;
constexpr int64_t kQkTargetWaves = 4096;  // ~16 per CU: below it a token spreads over waves

// A token's Hq + Hkv head rows go RPW at a time (one row per LPR-lane group)
// over waves_per_token waves, groups_per_wave row groups each, all of a
// wave's row loads in flight at once (up to kQkChunk groups at a time).
// Large batches take one wave per token; small ones spread a token over
// several waves, so that no wave computes a long chain alone.  What the rows
// of a token share is loaded once per wave: the position, the two norm weight
// slices and this lane's cos / sin slice (the same for every row, as a lane
// keeps its column).  Row loads are issued together with the position,
// before the rotary loads that depend on it, so a wave costs two round trips
// whatever its row count; rows past the wave's last read its last row and are
// not stored, so no load sits behind a branch (row groups wholly past it are
// not computed either).  The norm weights stay as loaded and are unpacked
// row by row (kW16: 16-bit weights, E/2 words per array instead of E
// floats): at one wave per token, prompt batches run in rounds of the
// resident waves, so the registers set the number of rounds (config 3's 8561
// tokens: 25.5 us at 164 VGPRs, three waves per SIMD; 24.4 at 98, four; 23.8
// at 90, five).
template <typename ET, int D, bool kW16>
__global__ __launch_bounds__(kQkThreads) void qk_norm_rope_kernel(QkParams p) {
  constexpr int E = ET::kPerVec;
  constexpr int LPR = D / E;     // lanes per head row
  constexpr int RPW = 64 / LPR;  // rows per wave instruction
  static_assert(LPR >= 2 && LPR <= 64 && 64 % LPR == 0, "unsupported head_dim");
  const int lane = threadIdx.x & 63;
  const int col = lane % LPR;
  const int sub = lane / LPR;
  const int64_t w = (int64_t)blockIdx.x * (kQkThreads / 64) + threadIdx.x / 64;
  const int64_t tok = w / p.waves_per_token;
  if (tok >= p.num_tokens) return;  // whole waves
  const int heads = p.hq + p.hkv;
  const int r0 = (int)(w % p.waves_per_token) * p.groups_per_wave * RPW;  // first row
  const int r1 = r0 + p.groups_per_wave * RPW < heads ? r0 + p.groups_per_wave * RPW : heads;
  if (r0 >= heads) return;  // whole waves
  int64_t pos = load_index(p.pp.pos, tok, p.pp.pos_i64);
  // With no query (key) heads the other side's weights stand in; unused.
  const WeightRaw<E> wqr = load_weights_raw<E>(p.hq > 0 ? p.pp.q_w : p.pp.k_w, p.pp.w_dtype, col * E);
  const WeightRaw<E> wkr = load_weights_raw<E>(p.hkv > 0 ? p.pp.k_w : p.pp.q_w, p.pp.w_dtype, col * E);
  const char* const qrow = p.q + tok * p.q_st + col * 16;
  const char* const krow = p.k + tok * p.k_st + col * 16;
  char* const qdst = p.qo + tok * p.qo_st + col * 16;
  char* const kdst = p.ko + tok * p.ko_st + col * 16;
  // Rows are read and written non-temporally: each is touched once here.
  // Over 8561 prompt tokens (16 + 8 heads of 128) the launch takes 25.4 us
  // against 27.7 with the default policy; non-temporal loads alone lose
  // (28.3), stores alone win less (26.1), and a decode that reads the rows
  // next runs as before.
  const bool wbf = p.pp.w_dtype == VA_BF16;
  float c[E], s[E];
  for (int h0 = r0; h0 < r1; h0 += kQkChunk * RPW) {
    uint4 raw[kQkChunk];
#pragma unroll
    for (int j = 0; j < kQkChunk; ++j) {
      int hh = h0 + j * RPW + sub;
      hh = hh < r1 ? hh : r1 - 1;
      raw[j] = ld16_nt(hh < p.hq ? qrow + hh * p.q_sh : krow + (int64_t)(hh - p.hq) * p.k_sh);
    }
    if (h0 == r0) {
      pos = pos < 0 ? 0 : (pos >= p.pp.max_pos ? p.pp.max_pos - 1 : pos);
      load_rotary<E, LPR>(p.pp, pos, col, D, c, s);
    }
#pragma unroll
    for (int j = 0; j < kQkChunk; ++j) {
      if (h0 + j * RPW >= r1) break;  // whole row groups past the wave's last row
      const int hh = h0 + j * RPW + sub;
      const bool isq = hh < p.hq;
      float x[E], wv[E];
      ET::unpack(raw[j], x);
      WeightRaw<E> wr;
      wr.a = isq ? wqr.a : wkr.a;
      if constexpr (!kW16) wr.b = isq ? wqr.b : wkr.b;
      row_weights<E, kW16>(wr, wbf, wv);
      qk_prologue<ET, LPR, E>(x, wv, p.pp.eps, D, c, s);
      if (hh < r1)
        st16_nt(isq ? qdst + hh * p.qo_sh : kdst + (int64_t)(hh - p.hq) * p.ko_sh, ET::pack(x));
    }
  }
}

// Few head rows per token (at most kQkTokenRows, as for keys alone): a wave takes
// RPW tokens, one per LPR-lane group, and every head row of them, all of its
// row loads in flight at once.  A token per wave would leave each wave a
// kilobyte or two behind two dependent round trips (position, then rotary);
// over config 3's 8561 prompt tokens, 8 key heads of 128, that layout took
// 15.0 us.  Each lane loads the position and rotary slice of its own token;
// lanes past the last token read it and store nothing.
template <typename ET, int D>
__global__ __launch_bounds__(kQkThreads) void qk_norm_rope_tokens_kernel(QkParams p) {
  constexpr int E = ET::kPerVec;
  constexpr int LPR = D / E;
  constexpr int RPW = 64 / LPR;  // tokens per wave
  static_assert(LPR >= 2 && LPR <= 64 && 64 % LPR == 0, "unsupported head_dim");
  const int lane = threadIdx.x & 63;
  const int col = lane % LPR;
  const int64_t w = (int64_t)blockIdx.x * (kQkThreads / 64) + threadIdx.x / 64;
  if (w * RPW >= p.num_tokens) return;  // whole waves
  const int64_t tok_raw = w * RPW + lane / LPR;
  const bool live = tok_raw < p.num_tokens;
  const int64_t tok = live ? tok_raw : p.num_tokens - 1;
  const int heads = p.hq + p.hkv;  // <= kQkTokenRows (host)
  int64_t pos = load_index(p.pp.pos, tok, p.pp.pos_i64);
  const WeightRaw<E> wqr = load_weights_raw<E>(p.hq > 0 ? p.pp.q_w : p.pp.k_w, p.pp.w_dtype, col * E);
  const WeightRaw<E> wkr = load_weights_raw<E>(p.hkv > 0 ? p.pp.k_w : p.pp.q_w, p.pp.w_dtype, col * E);
  const char* const qrow = p.q + tok * p.q_st + col * 16;
  const char* const krow = p.k + tok * p.k_st + col * 16;
  char* const qdst = p.qo + tok * p.qo_st + col * 16;
  char* const kdst = p.ko + tok * p.ko_st + col * 16;
  uint4 raw[kQkTokenRows];
#pragma unroll
  for (int j = 0; j < kQkTokenRows; ++j) {
    const int hh = j < heads ? j : heads - 1;
    raw[j] = ld16_nt(hh < p.hq ? qrow + hh * p.q_sh : krow + (int64_t)(hh - p.hq) * p.k_sh);
  }
  pos = pos < 0 ? 0 : (pos >= p.pp.max_pos ? p.pp.max_pos - 1 : pos);
  float c[E], s[E], wq[E], wk[E];
  load_rotary<E, LPR>(p.pp, pos, col, D, c, s);
  convert_weights<E>(wqr, p.pp.w_dtype, wq);
  convert_weights<E>(wkr, p.pp.w_dtype, wk);
#pragma unroll
  for (int j = 0; j < kQkTokenRows; ++j) {
    if (j >= heads) break;
    const bool isq = j < p.hq;
    float x[E], wv[E];
    ET::unpack(raw[j], x);
#pragma unroll
    for (int e = 0; e < E; ++e) wv[e] = isq ? wq[e] : wk[e];
    qk_prologue<ET, LPR, E>(x, wv, p.pp.eps, D, c, s);
    if (live) st16_nt(isq ? qdst + j * p.qo_sh : kdst + (int64_t)(j - p.hq) * p.ko_sh, ET::pack(x));
  }
}

template <typename ET, bool kW16>
static bool launch_qk_w(int D, const QkParams& p, dim3 grid, hipStream_t st) {
  switch (D) {
    case 64: hipLaunchKernelGGL((qk_norm_rope_kernel<ET, 64, kW16>), grid, dim3(kQkThreads), 0, st, p); return true;
    case 128: hipLaunchKernelGGL((qk_norm_rope_kernel<ET, 128, kW16>), grid, dim3(kQkThreads), 0, st, p); return true;
    case 256: hipLaunchKernelGGL((qk_norm_rope_kernel<ET, 256, kW16>), grid, dim3(kQkThreads), 0, st, p); return true;
    default: return false;
  }
}

template <typename ET>
static bool launch_qk(int D, const QkParams& p, dim3 grid, hipStream_t st) {
  return p.pp.w_dtype == VA_F32 ? launch_qk_w<ET, false>(D, p, grid, st)
                                : launch_qk_w<ET, true>(D, p, grid, st);
}

template <typename ET>
static bool launch_qk_tokens(int D, const QkParams& p, dim3 grid, hipStream_t st) {
  switch (D) {
    case 64: hipLaunchKernelGGL((qk_norm_rope_tokens_kernel<ET, 64>), grid, dim3(kQkThreads), 0, st, p); return true;
    case 128: hipLaunchKernelGGL((qk_norm_rope_tokens_kernel<ET, 128>), grid, dim3(kQkThreads), 0, st, p); return true;
    case 256: hipLaunchKernelGGL((qk_norm_rope_tokens_kernel<ET, 256>), grid, dim3(kQkThreads), 0, st, p); return true;
    default: return false;
  }
}

}  // namespace va

extern "C" int va_qk_norm_rope(const va_qk_norm_rope_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_qk_norm_rope: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_qk_norm_rope_args),
               "va_qk_norm_rope: struct_size %u != %zu (header/library mismatch)", a->struct_size,
               sizeof(va_qk_norm_rope_args));
  VA_CHECK_ARG(a->num_tokens >= 0, "va_qk_norm_rope: num_tokens < 0");
  if (a->num_tokens == 0) return VA_OK;
  const int eb = a->dtype == VA_F32 ? 4 : (a->dtype == VA_BF16 || a->dtype == VA_F16) ? 2 : 0;
  VA_CHECK_ARG(eb != 0, "va_qk_norm_rope: unknown dtype %d", a->dtype);
  VA_CHECK_ARG(a->head_dim == 64 || a->head_dim == 128 || a->head_dim == 256,
               "va_qk_norm_rope: head_dim %d (64, 128 or 256)", a->head_dim);
  VA_CHECK_ARG(a->num_heads >= 0 && a->num_kv_heads >= 0 && a->num_heads + a->num_kv_heads > 0,
               "va_qk_norm_rope: head counts");
  VA_CHECK_ARG(a->num_heads == 0 || (a->q && a->q_out), "va_qk_norm_rope: q / q_out missing");
  VA_CHECK_ARG(a->num_kv_heads == 0 || (a->k && a->k_out), "va_qk_norm_rope: k / k_out missing");
  const va_qk_prologue& pr = a->prologue;
  VA_CHECK_ARG(pr.cos_sin_cache && pr.positions && pr.max_position > 0 && pr.cos_sin_stride >= a->head_dim,
               "va_qk_norm_rope: rotary cache / positions");
  VA_CHECK_ARG((a->num_heads == 0 || pr.q_norm_weight) && (a->num_kv_heads == 0 || pr.k_norm_weight),
               "va_qk_norm_rope: norm weights missing");
  VA_CHECK_ARG(pr.weight_dtype == VA_BF16 || pr.weight_dtype == VA_F16 || pr.weight_dtype == VA_F32,
               "va_qk_norm_rope: weight_dtype");
  VA_CHECK_ARG(pr.positions_dtype == VA_I32 || pr.positions_dtype == VA_I64,
               "va_qk_norm_rope: positions_dtype");
  const int64_t strides[] = {a->q_stride_tok,     a->q_stride_head,     a->k_stride_tok,
                             a->k_stride_head,    a->q_out_stride_tok,  a->q_out_stride_head,
                             a->k_out_stride_tok, a->k_out_stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * eb) % 16 == 0, "va_qk_norm_rope: strides must be 16-byte multiples");
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->q_out,
                            (uintptr_t)a->k_out};
  for (uintptr_t p : ptrs)
    VA_CHECK_ARG(p % 16 == 0, "va_qk_norm_rope: pointers must be 16-byte aligned");
  VA_CHECK_ARG((uintptr_t)pr.q_norm_weight % 16 == 0 && (uintptr_t)pr.k_norm_weight % 16 == 0,
               "va_qk_norm_rope: norm weights must be 16-byte aligned");

  QkParams p;
  p.q = (const char*)a->q;
  p.q_st = a->q_stride_tok * eb;
  p.q_sh = a->q_stride_head * eb;
  p.k = (const char*)a->k;
  p.k_st = a->k_stride_tok * eb;
  p.k_sh = a->k_stride_head * eb;
  p.qo = (char*)a->q_out;
  p.qo_st = a->q_out_stride_tok * eb;
  p.qo_sh = a->q_out_stride_head * eb;
  p.ko = (char*)a->k_out;
  p.ko_st = a->k_out_stride_tok * eb;
  p.ko_sh = a->k_out_stride_head * eb;
  p.num_tokens = a->num_tokens;
  p.hq = a->num_heads;
  p.hkv = a->num_kv_heads;
  p.pp.q_w = pr.q_norm_weight;
  p.pp.k_w = pr.k_norm_weight;
  p.pp.w_dtype = pr.weight_dtype;
  p.pp.eps = pr.eps;
  p.pp.cs = pr.cos_sin_cache;
  p.pp.cs_stride = pr.cos_sin_stride;
  p.pp.max_pos = pr.max_position;
  p.pp.pos_i64 = pr.positions_dtype == VA_I64;
  p.pp.pos = pr.positions;

  const int E = 16 / eb;
  const int rpw = 64 / (a->head_dim / E);
  const int heads = a->num_heads + a->num_kv_heads;
  const hipStream_t st = (hipStream_t)stream;
  if (heads <= kQkTokenRows && a->num_tokens >= kQkTargetWaves) {
    // Prompt-sized batches with few rows per token: RPW tokens per wave.
    const int64_t waves = ((int64_t)a->num_tokens + rpw - 1) / rpw;
    const dim3 grid((unsigned)((waves + kQkThreads / 64 - 1) / (kQkThreads / 64)));
    bool ok = false;
    switch (a->dtype) {
      case VA_BF16: ok = launch_qk_tokens<BF16>(a->head_dim, p, grid, st); break;
      case VA_F16: ok = launch_qk_tokens<F16>(a->head_dim, p, grid, st); break;
      case VA_F32: ok = launch_qk_tokens<F32>(a->head_dim, p, grid, st); break;
    }
    if (!ok) {
      set_error("va_qk_norm_rope: unsupported configuration");
      return VA_ERR_UNSUPPORTED;
    }
    return check_launch("va_qk_norm_rope");
  }
  // Waves per token: enough for ~16 waves per CU when the batch is small
  // (decode-sized), one per token when it is large.
  const int groups = (heads + rpw - 1) / rpw;
  int wpt = (int)std::min<int64_t>(groups, std::max<int64_t>(1, (kQkTargetWaves + a->num_tokens - 1) / a->num_tokens));
  const int gpw = (groups + wpt - 1) / wpt;
  wpt = (groups + gpw - 1) / gpw;
  const int64_t waves = (int64_t)a->num_tokens * wpt;
  const int64_t blocks = (waves + kQkThreads / 64 - 1) / (kQkThreads / 64);
  VA_CHECK_ARG(blocks <= INT32_MAX, "va_qk_norm_rope: too many tokens");
  p.waves_per_token = wpt;
  p.groups_per_wave = gpw;
  const dim3 grid((unsigned)blocks);
  bool ok = false;
  switch (a->dtype) {
    case VA_BF16: ok = launch_qk<BF16>(a->head_dim, p, grid, st); break;
    case VA_F16: ok = launch_qk<F16>(a->head_dim, p, grid, st); break;
    case VA_F32: ok = launch_qk<F32>(a->head_dim, p, grid, st); break;
  }
  if (!ok) {
    set_error("va_qk_norm_rope: unsupported configuration");
    return VA_ERR_UNSUPPORTED;
  }
  return check_launch("va_qk_norm_rope");
}
