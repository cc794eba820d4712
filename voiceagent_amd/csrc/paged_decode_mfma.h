// Paged-KV decode attention on CDNA4 matrix cores, for 16-bit K/V whose
// block size is a multiple of 16: the engine's decode and the TTS decode
// with its key_valid_mask.  The general kernel in paged_decode_kernel.h
// covers the rest.
//
// Same semantics and partial/merge protocol as paged_decode_kernel; the grid
// is (kv head, sequence, partition) here (see `h` below).  A workgroup owns P
// consecutive tokens of one (sequence, kv head) pair and all G query heads
// of its group.
//
// Work decomposition.  A workgroup is W wave64s (8, two per SIMD, for head
// dims up to 128; 4 for 256; at head_dim 128, 12 over FP8 pools when a
// workgroup attends few tokens and 4 when a launch has
// more workgroups than CUs (16-bit or FP8 pools), see MfmaWaves).  The partition's 16-token
// tiles go round robin to the waves (tile c to wave c % W), and each wave
// runs its own pipeline with no workgroup barrier:
//   * the K and V rows of a tile (16 rows of one block) are copied from HBM
//     straight into the wave's LDS ring of S stages with
//     global_load_lds_dwordx4 (1 KiB per instruction, 16-byte chunks stored
//     XOR-swizzled by row so the matrix-core reads below are conflict-free);
//     S - 1 tiles are in flight while one is reduced;
//   * S^T = K Q^T  (16 tokens x 16 columns, G of them real query heads) with
//     v_mfma_f32_16x16x32: A = K rows from LDS (ds_read_b128), B = Q^T held
//     in registers for the whole loop;
//   * online softmax in the exp2 domain on the four scores each lane holds
//     (tokens 4 (lane / 16) + i of column lane % 16); the reference maximum is
//     raised only when a column's new maximum exceeds it by more than kLazy;
//   * O^T += V^T P^T with v_mfma_f32_16x16x16: P^T is the S^T accumulator
//     packed to 16 bits in place (its layout is already the B operand's),
//     V^T comes from the row-major V tile through ds_read_b64_tr_b16.
// Nearly all arithmetic runs on the matrix cores, so two waves per SIMD keep
// HBM busy and a workgroup can pull several times its fair share of
// bandwidth once shorter contexts have finished.  With one partition per
// pair the first tiles are requested before the context length has
// arrived (see `early` below).  The waves merge through
// LDS at the end; partitioned contexts write (m, l, o) partials that
// paged_decode_merge_kernel combines.
#pragma once

#include "paged_decode_kernel.h"

namespace va {

typedef __bf16 mf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_f16x4 __attribute__((ext_vector_type(4)));
typedef short mf_s16x4 __attribute__((ext_vector_type(4)));
typedef float mf_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) mf_s16x4 mf_lds_s16x4;
typedef int mf_s32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) mf_s32x2 mf_lds_s32x2;

template <typename ET>
struct DecodeMma;

template <>
struct DecodeMma<BF16> {
  __device__ static inline mf_f32x4 qk(uint4 a, uint4 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mf_bf16x8, a),
                                                   __builtin_bit_cast(mf_bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline mf_f32x4 pv(mf_s16x4 a, uint2 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, __builtin_bit_cast(mf_s16x4, b), c, 0, 0,
                                                     0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <>
struct DecodeMma<F16> {
  __device__ static inline mf_f32x4 qk(uint4 a, uint4 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf_f16x8, a),
                                                  __builtin_bit_cast(mf_f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline mf_f32x4 pv(mf_s16x4 a, uint2 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mf_f16x4, a),
                                                 __builtin_bit_cast(mf_f16x4, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    f16x2_t v;
    v.x = (_Float16)lo;
    v.y = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Geometry of the matrix-core decode for head_dim D (16-bit elements).
template <int D>
struct MfmaDecodeShape {
  static constexpr int ROWB = D * 2;           // bytes per K/V row
  static constexpr int CPR = ROWB / 16;        // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;         // rows per DMA instruction (1 KiB)
  static constexpr int NI = kChunk / RPI;      // DMA instructions per tile, K or V
  static constexpr int TILE_B = kChunk * ROWB; // bytes of one K (or V) tile
  // Two waves per SIMD with two stages each (128 KiB of LDS) where the tiles
  // allow; head_dim 256 keeps one wave per SIMD.
  static constexpr int W = 8 * 2 * 2 * TILE_B <= 131072 ? 8 : 4;  // waves per workgroup
  static constexpr int S = 131072 / (W * 2 * TILE_B) < 2 ? 2 : 131072 / (W * 2 * TILE_B);
  static constexpr int WAVE_B = S * 2 * TILE_B;  // LDS bytes per wave
  static constexpr int DS = D / 32;            // k-steps of S^T = K Q^T
  static constexpr int DT = D / 16;            // 16-row d tiles of O^T
  static constexpr int LPR = D / 8;            // lanes per row in the row layout
  static constexpr int RPL = 64 / LPR;         // rows per wave in the row layout
};

// Waves per workgroup and the most LDS bytes a wave's ring may take, for
// the host's choice kWaves (DecodeParams::waves): 0 takes the default for D.
//   12: twelve waves (three per SIMD) with two stages of codes each, for FP8
//   pools at head_dim 128 when a workgroup streams few tokens.  Over FP8 a
//   long context's tail is bound by its tiles' arithmetic (code reads and
//   conversions wait on LDS), and a third wave per SIMD hides more of it
//   (config 2 over FP8 pools 11.5 -> 10.7 us/layer, one 16K context 14.3 ->
//   13.8, measured when V still went through a 16-bit conversion area).
//   With ~4K tokens per workgroup (config 5's eight long contexts) two stages
//   are too few (44.6 -> 45.6 us/layer), so those keep eight waves with three
//   stages.  (Measured and dropped: sixteen waves with two stages, config 2
//   10.5 and one 16K context 14.0 against 10.3 and 13.5.)
//   4: four waves with two stages each, at head_dim 128 when the launch has
//   more workgroups than CUs: several workgroups share a CU (two over 16-bit
//   pools, 64 KiB of ring each; four over FP8 pools, 32 KiB), so one's
//   start-up round trips overlap the others' streams instead of following
//   them.  Batch 64 x U[60,600] 22.2 -> 20.7 us/layer, 256: 72.3 -> 65.9;
//   over FP8 pools (against twelve waves) 18.4 -> 15.2 and 61.7 -> 40.7.
//   With one workgroup per CU (config 2's 256) eight waves stay faster over
//   16-bit pools (13.1 against 13.9).
template <int D, int kWaves>
struct MfmaWaves {
  static_assert(kWaves == 0 || D == 128, "twelve or four waves at head_dim 128 only");
  static_assert(kWaves == 0 || kWaves == 12 || kWaves == 4, "0, 12 or 4 waves");
  static constexpr int W = kWaves == 0 ? MfmaDecodeShape<D>::W : kWaves;
  static constexpr int WAVE_B = kWaves == 12 ? 8 * 1024 : MfmaDecodeShape<D>::WAVE_B;
};

// Tokens per partition unit of the matrix-core kernel: one round of S tiles
// on every wave.
template <int D>
constexpr int mfma_decode_unit() {
  return MfmaDecodeShape<D>::W * MfmaDecodeShape<D>::S * kChunk;
}

// LDS position of 16-byte chunk c of row r in a staged tile: c ^ swz(r).
// The XOR spreads the 16 rows of a K read (one chunk per row) and the four
// rows x four half-chunks of a transposed V read over distinct banks.
template <int D>
__device__ inline int dec_swz(int row) {
  if constexpr (D == 64)
    return (((row >> 1) & 3) << 1) | ((row >> 3) & 1);
  else
    return ((row & 7) << 1) | ((row >> 3) & 1);
}

__device__ __align__(16) const uint4 kDecZeroRow = {0u, 0u, 0u, 0u};

// Lazy-rescale slack of the online softmax in log2 units (p <= 2^kDecLazy).
constexpr float kDecLazy = 8.0f;


// kMask: the launch has a key_valid_mask (a separate instantiation, so the
// kernel without one carries none of its loads or branches).  kF8: the pool
// holds OCP e4m3 codes.  S^T reads a staged K tile's codes, eight per lane,
// and converts them, exactly, in registers; V^T is read from the staged V
// codes with ds_read_b64_tr_b8, one read giving the lane its four tokens of
// two 16-dim blocks, converted in registers as well.  k_scale is folded
// into the softmax scale and v_scale into the output.
template <typename ET, int D, int G, bool kProlog, bool kMask, bool kF8, int kWaves = 0>
__global__ __launch_bounds__((MfmaWaves<D, kWaves>::W * 64), 1) void paged_decode_mfma_kernel(
    DecodeParams p) {
  static_assert(kWaves != 12 || kF8, "twelve waves over FP8 pools only");
  using Sh = MfmaDecodeShape<D>;
  using M = DecodeMma<ET>;
  constexpr int W = MfmaWaves<D, kWaves>::W, ROWB = Sh::ROWB;
  constexpr int RING_B = MfmaWaves<D, kWaves>::WAVE_B;  // LDS bytes per wave
  constexpr int TILE_B = Sh::TILE_B, DS = Sh::DS, DT = Sh::DT;
  constexpr int LPR = Sh::LPR, RPL = Sh::RPL, E = 8;
  // A tile as the DMA stages it: 16-bit rows, or rows of D e4m3 codes.
  constexpr int PROWB = kF8 ? D : ROWB;     // staged bytes per row
  constexpr int CPR = PROWB / 16;           // 16-byte chunks per staged row
  constexpr int RPI = 64 / CPR;             // rows per DMA instruction (1 KiB)
  constexpr int NI = kChunk / RPI;          // DMA instructions per tile, K or V
  constexpr int PTILE = kChunk * PROWB;     // staged bytes of one K (or V) tile
  constexpr int STAGE_B = 2 * PTILE;
  // FP8: K and V are read as codes straight from their stage, half the bytes
  // of 16-bit rows, and the wave keeps at most three stages of them: a
  // fourth (a third with twelve waves) only enlarges the launch's first
  // burst of requests, whose last tiles then land later (config 2 over FP8
  // pools 10.3 -> 11.0 us/layer, one 16K context 13.5 -> 14.2).
  // Four-wave workgroups keep two, so that four share a CU (with three
  // stages, ~53 KB of LDS each: batch 256 over FP8 pools 42.8 against 40.7
  // us/layer).
  constexpr int S_F8 = kWaves == 4 ? 2 : (RING_B / STAGE_B < 3 ? RING_B / STAGE_B : 3);
  constexpr int S = kF8 ? S_F8 : Sh::S;  // stages of the wave's ring
  static_assert(S >= 2, "two stages at least");
  constexpr int WAVE_B = S * STAGE_B;  // LDS bytes per wave
  static_assert(WAVE_B <= RING_B, "the stages fit the wave's LDS");
  constexpr int NT = W * 64;
  static_assert(W % 4 == 0, "the wave merge reads (m, l) of four waves at a time");
  constexpr int QROWS = (G + RPL - 1) / RPL;  // query rows per lane in the row layout
  static_assert(G <= 16, "at most 16 query heads per kv head");
  // The waves' partial results for the merge: o [W][G][D], then m and l
  // [G][W].  They get their own LDS beside the tile ring when it fits, so a
  // wave can write its partial as soon as its loop ends; otherwise they
  // reuse the ring once every wave is done with it.
  constexpr int MERGE_B = W * G * D * 4 + 2 * G * W * 4;
  constexpr int Q_B = kProlog ? W * G * ROWB : 16;
  constexpr bool kOwnMerge = W * WAVE_B + MERGE_B + Q_B <= 160 * 1024;
  static_assert(MERGE_B <= W * WAVE_B, "merge scratch");

  __shared__ __align__(1024) char s_buf[W * WAVE_B];
  // Apart from the tile ring, so that early tile DMAs cannot land on them:
  // the query rows of the prologue (per wave).
  __shared__ __align__(16) char s_q[Q_B];
  __shared__ __align__(16) char s_mrg[kOwnMerge ? MERGE_B : 16];

  // Grid (kv head, sequence, partition), kv head fastest: workgroup i runs
  // on XCD i % 8, so each XCD takes the same kv heads of every sequence and
  // reads an equal share of the step's bytes however the lengths vary
  // (sequence-major, an XCD held all heads of a few sequences: config 2
  // 13.33-13.42 us against 12.95-12.99).
  const int b = blockIdx.y;
  const int h = blockIdx.x;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;   // MFMA row / column index of this lane
  const int c4 = lane >> 4;    // MFMA k-group of this lane
  const int rg = lane / LPR;   // row-layout row of this lane
  const int col = lane % LPR;  // row-layout 16-byte column of this lane
  int P = p.split_tokens;  // placeholder in dyn_split mode, fixed below from L
  int start = part * P;
  const int64_t table_row = (int64_t)b * p.t_sb;

  // ---- independent loads, all issued before the first wait: this wave's
  // block ids, the query, the current K/V row, the length and the slot.
  // Index arrays are read as raw 32-bit words (the low word of an int64
  // entry) and combined only after the last load is issued, so that no load
  // waits behind another one's arithmetic. ----
  // Block of the wave's tile `lane` (tile 64 i + lane after refills): `tab`
  // serves the DMA issue, which runs S tiles ahead; `tab_proc` is the copy
  // the tile being reduced reads (refreshed when it reaches the refill).
  const uint32_t* const tabw = reinterpret_cast<const uint32_t*>(p.table);
  auto block_of = [&](int tok) -> int {  // table entry of token tok's block, 0 past the width
    const int idx = (int)fast_div((uint32_t)tok, p.bs_div);
    return idx < p.table_width ? (int)tabw[(table_row + idx) << p.table_i64] : 0;
  };
  int tab = 0;
  {
    const int c = wave + W * lane;
    if (c * kChunk < P || part == p.max_parts - 1) tab = block_of(start + c * kChunk);
  }
  // The query: in the B-operand layout of S^T = K Q^T (lane holds
  // q[head r16][32 j + 8 c4, +8)), or, for the prologue, as rows in the row
  // layout, which go through LDS into the B layout after normalisation.
  uint4 qb[DS];
  uint4 qrow[QROWS];
  if constexpr (!kProlog) {
#pragma unroll
    for (int j = 0; j < DS; ++j)
      qb[j] = r16 < G ? ld16(p.q + b * p.q_sb + (int64_t)(h * G + r16) * p.q_sh +
                             (32 * j + 8 * c4) * 2)
                      : make_uint4(0, 0, 0, 0);
  } else {
#pragma unroll
    for (int k = 0; k < QROWS; ++k) {
      const int g = rg + RPL * k;
      qrow[k] = g < G ? ld16(p.q + b * p.q_sb + (int64_t)(h * G + g) * p.q_sh + col * 16)
                      : make_uint4(0, 0, 0, 0);
    }
  }
  // key_valid_mask: lane l holds the validity of the 16 tokens of this
  // wave's tile l (of the current 64-tile group, like `tab`) as 16 bits,
  // token i of the tile at bit i; tokens at or past the mask's width count
  // as valid.  The tile's 16 bytes are read as the aligned 4-byte words that
  // cover them (five when the row does not start on a word boundary); a
  // word holding a byte of the row lies in the page holding that byte, so
  // reading it whole stays within mapped memory.
  constexpr bool has_mask = kMask;  // the host launches it only with a mask
  const int mlen = has_mask ? p.valid_len : 0;
  const uint8_t* const mrow = p.valid + (has_mask ? (int64_t)b * p.valid_sb : 0);
  const int moff = (int)((uintptr_t)mrow & 3);
  const uint32_t* const mwords = reinterpret_cast<const uint32_t*>(mrow - moff);
  uint32_t mraw[5] = {~0u, ~0u, ~0u, ~0u, ~0u};
  int mtb = 0;  // first token of the tile whose words mraw holds
  auto mask_load = [&](int tb) {
    mtb = tb;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      const int rb = tb + 4 * j - moff;  // row byte at the word's start
      mraw[j] = rb < mlen && (j < 4 || moff != 0) ? mwords[(tb >> 2) + j] : 0xffffffffu;
    }
  };
  auto mask_bits = [&]() -> uint32_t {
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t x = __builtin_amdgcn_alignbyte(mraw[j + 1], mraw[j], (uint32_t)moff);
      x |= x >> 4;  // bit 0 of each byte becomes the OR of the byte's bits
      x |= x >> 2;
      x |= x >> 1;
      x &= 0x01010101u;
      bits |= ((x * 0x01020408u) >> 24) << (4 * j);  // byte i's bit to bit 24 + i
    }
    const int rem = mlen - mtb;  // tokens of the tile inside the mask's width
    if (rem < 16) bits |= rem <= 0 ? 0xffffu : (0xffffu << rem) & 0xffffu;
    return bits;
  };
  uint32_t mbits = 0xffffu;
  // With fixed partitions the partition's start is known, so the words go
  // out with the other start-up loads (see `early` below).
  if (has_mask && !p.dyn_split) mask_load(start + (wave + W * lane) * kChunk);
  uint4 kcur = make_uint4(0, 0, 0, 0), vcur = make_uint4(0, 0, 0, 0);
  if (p.new_k != nullptr) {
    kcur = ld16(p.new_k + b * p.nk_sb + h * p.nk_sh + col * 16);
    vcur = ld16(p.new_v + b * p.nv_sb + h * p.nv_sh + col * 16);
  }
  // Length: lens[b] or cu[b + 1] - cu[b]; only the low words matter for a
  // 32-bit length.
  const uint32_t* const lensw = reinterpret_cast<const uint32_t*>(p.lens);
  const uint32_t len_hi = lensw[(int64_t)(b + p.lens_cum) << p.lens_i64];
  const uint32_t len_lo = lensw[(int64_t)b << p.lens_i64];
  uint32_t slot_lo = ~0u, slot_hi = ~0u;  // new_slots[b] (-1 without one)
  if (p.new_slots != nullptr) {
    const uint32_t* const sw = reinterpret_cast<const uint32_t*>(p.new_slots);
    slot_lo = sw[(int64_t)b << p.new_slots_i64];
    slot_hi = sw[((int64_t)b << p.new_slots_i64) + p.new_slots_i64];
  }
  float pro_c[E], pro_s[E];
  WeightRaw<E> pro_wq{}, pro_wk{};
  int64_t pos = 0;
  if constexpr (kProlog) {
    pos = load_index(p.pro.pos, b, p.pro.pos_i64);
    pos = pos < 0 ? 0 : (pos >= p.pro.max_pos ? p.pro.max_pos - 1 : pos);
    pro_wq = load_weights_raw<E>(p.pro.q_w, p.pro.w_dtype, col * E);
    pro_wk = load_weights_raw<E>(p.pro.k_w != nullptr ? p.pro.k_w : p.pro.q_w, p.pro.w_dtype,
                                 col * E);
  }

  char* const s_wave = s_buf + wave * WAVE_B;
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)s_wave);

  // ---- tile DMA: instruction i of a tile moves rows RPI i .. RPI i + RPI - 1;
  // lane l writes row RPI i + l / CPR at chunk position l % CPR, i.e. reads
  // logical chunk (l % CPR) ^ swz(row) of that row ----
  // FP8: code chunks of K and V go to chunk (c ^ row % CPR) of their row, so
  // that the 8-code reads of S^T and the transposed V reads spread over the
  // banks.
  uint32_t loff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = RPI * i + lane / CPR;
    const int pos = kF8 ? (lane % CPR) ^ (row % CPR) : (lane % CPR) ^ dec_swz<D>(row);
    loff[i] = (uint32_t)(row * p.s_slot) + (uint32_t)(pos << 4);
  }
  const char* zero_row = reinterpret_cast<const char*>(&kDecZeroRow);
  const int64_t head_off = (int64_t)h * p.s_head;
  int span = 0;  // tokens of this partition (set once the length is known)
  // Issue tile k of this wave into stage k % S.  Tiles whose block id is
  // outside [0, num_blocks) read zeros (their scores are masked).
  auto issue = [&](int k) {
    if (k > 0 && (k & 63) == 0) {
      // Next 64 tiles of this wave: refill the block-id prefetch.
      const int c = wave + W * (k + lane);
      tab = c * kChunk < span ? block_of(start + c * kChunk) : 0;
      if (has_mask) {
        mask_load(start + c * kChunk);
        mbits = mask_bits();
      }
    }
    const int tb = start + (wave + W * k) * kChunk;
    const int32_t blk = __builtin_amdgcn_readlane(tab, k & 63);
    const uint32_t dst = lds_wave + (uint32_t)((k % S) * STAGE_B);
    if (blk >= 0 && blk < p.num_blocks) {
      const int64_t off = (int64_t)blk * p.s_blk + (int64_t)fast_mod((uint32_t)tb, p.bs_div) * p.s_slot +
                          head_off;
      const char* kb = uniform_ptr(p.kp + off);
      const char* vb = uniform_ptr(p.vp + off);
#pragma unroll
      for (int i = 0; i < NI; ++i) dma16_nt(loff[i], kb, dst + i * 1024);
#pragma unroll
      for (int i = 0; i < NI; ++i) dma16_nt(loff[i], vb, dst + PTILE + i * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < 2 * NI; ++i) dma16(zero_row, dst + i * 1024);
    }
  };

  // With fixed partitions (one per pair, the common decode batch, or a split
  // planned from a short or exact max_seq_len) the first S tiles of the partition are
  // issued now, before the length is known: a block id outside
  // [0, num_blocks) reads zeros, tokens past the context are masked, and a
  // partition wholly past it only waits for its tiles and exits, so the
  // early tiles are safe to fetch, and the length's round trip leaves the
  // critical path.  The vector loads above are waited for first, so the
  // compiler's own waits for them do not fall after the DMA (where they
  // would also wait for it).  With the prologue only the block ids are: its
  // rotary rows depend on the position and are requested after the DMA, so
  // the prologue arithmetic waits for the early tiles anyway, which it
  // precedes only by a few hundred cycles.
  const bool early = !p.dyn_split;
  if (early) {
    if constexpr (!kProlog) {
#pragma unroll
      for (int j = 0; j < DS; ++j)
        asm volatile("" ::"v"(qb[j].x), "v"(qb[j].y), "v"(qb[j].z), "v"(qb[j].w));
      asm volatile("" ::"v"(kcur.x), "v"(kcur.y), "v"(kcur.z), "v"(kcur.w), "v"(vcur.x),
                   "v"(vcur.y), "v"(vcur.z), "v"(vcur.w));
    }
    asm volatile("" ::"v"(tab));
    if constexpr (kMask)
      asm volatile("" ::"v"(mraw[0]), "v"(mraw[1]), "v"(mraw[2]), "v"(mraw[3]), "v"(mraw[4]));
    // Only tiles inside the partition: a short one leaves most waves' slots
    // past it.  The last partition also takes any tokens past its P, so it
    // requests all of its first tiles.
    for (int k = 0; k < S; ++k)
      if (part == p.max_parts - 1 || (wave + W * k) * kChunk < P) issue(k);
  }
  if constexpr (kProlog) load_rotary<E, LPR>(p.pro, pos, col, D, pro_c, pro_s);

  int L = (int)(p.lens_cum ? len_hi - len_lo : len_lo);
  L = __builtin_amdgcn_readfirstlane(L);
  // L becomes the attended length; the current row sits at Lr - 1.
  const int Lr = L;
  L = attend_len(p, L);
  const int col_new = Lr >= 1 ? (int)fast_div((uint32_t)(Lr - 1), p.bs_div) : 0;
  const bool detached = current_row_detached(p, Lr, L, col_new);
  const int64_t new_slot = p.new_slots_i64 ? (int64_t)(((uint64_t)slot_hi << 32) | slot_lo)
                                           : (int64_t)(int32_t)slot_lo;

  if (L <= 0) {
    wait_vmcnt<0>();  // early tiles land before the workgroup's LDS is released
    // Nothing to attend: the output is defined as 0.
    if (part == 0) {
      for (int idx = tid; idx < G * D / E; idx += NT) {
        const int g = idx / (D / E), d = (idx % (D / E)) * E;
        st16(p.out + b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d * 2, make_uint4(0, 0, 0, 0));
      }
    }
    return;
  }
  if (p.dyn_split) {
    // The partition follows from L: re-read this wave's block ids for it.
    P = partition_tokens(p, L);
    start = part * P;
    if (start < L) {
      const int c = wave + W * lane;
      tab = c * kChunk < P ? block_of(start + c * kChunk) : 0;
    }
  }
  if (start >= L) {
    wait_vmcnt<0>();
    return;
  }
  int nparts = (L + P - 1) / P;
  const bool last_grid_part = part == p.max_parts - 1;
  if (nparts > p.max_parts) nparts = p.max_parts;  // the last partition absorbs the rest
  const int end = last_grid_part ? L : min(start + P, L);
  span = end - start;
  const int nch = (end - start + kChunk - 1) / kChunk;
  const int ntw = nch > wave ? (nch - wave + W - 1) / W : 0;  // tiles of this wave

  // The current row is position L - 1 when this partition holds it: it is
  // stored to its slot and replaces the pool row in the staged tile.
  const int new_tok =
      (!detached && p.new_k != nullptr && L - 1 >= start && L - 1 < end) ? L - 1 : -1;
  const int new_tile = new_tok >= 0 ? (new_tok - start) / kChunk : -1;  // partition chunk
  const int64_t cap = (int64_t)p.num_blocks * p.block_size;

  // ---- prologue (Qwen3 q/k RMSNorm + RoPE) in the row layout, then the
  // query rows go through LDS into the B-operand layout ----
  if constexpr (kProlog) {
    float w[E];
    convert_weights<E>(pro_wq, p.pro.w_dtype, w);
#pragma unroll
    for (int k = 0; k < QROWS; ++k) {
      float x[E];
      ET::unpack(qrow[k], x);
      qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, pro_c, pro_s);
      qrow[k] = ET::pack(x);
    }
    if (new_tok >= 0 || (detached && part == 0 && wave == 0)) {
      convert_weights<E>(pro_wk, p.pro.w_dtype, w);
      float x[E];
      ET::unpack(kcur, x);
      qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, pro_c, pro_s);
      kcur = ET::pack(x);
    }
#pragma unroll
    for (int k = 0; k < QROWS; ++k) {
      const int g = rg + RPL * k;
      if (g < G) st16(s_q + (wave * G + g) * ROWB + col * 16, qrow[k]);
    }
#pragma unroll
    for (int j = 0; j < DS; ++j)
      qb[j] = r16 < G ? *reinterpret_cast<const uint4*>(s_q + (wave * G + r16) * ROWB +
                                                         (4 * j + c4) * 16)
                      : make_uint4(0, 0, 0, 0);
  }

  // FP8 pool: the current row is stored as codes and attended as their
  // values, as a later step reads it back.
  uint2 kq = make_uint2(0u, 0u), vq = make_uint2(0u, 0u);
  if constexpr (kF8) {
    if (p.new_k != nullptr) {
      kq = f8_quant8<ET>(kcur, p.inv_k);
      vq = f8_quant8<ET>(vcur, p.inv_v);
      kcur = f8_dequant8<ET>(kq);
      vcur = f8_dequant8<ET>(vq);
    }
  }
  // The current row is not attended in place: wave 0 of the first partition
  // writes it.
  if (detached && part == 0 && wave == 0 && rg == 0) {
    if constexpr (kF8)
      store_detached_row_f8(p, h, table_row, Lr, col_new, new_slot, col * 8, kq, vq);
    else
      store_detached_row(p, h, table_row, Lr, col_new, new_slot, col * 16, kcur, vcur);
  }

  if (!early) {
    for (int k = 0; k < S; ++k)
      if (k < ntw) issue(k);
    // The partition's start follows from the length here, so the mask words
    // are requested behind the first tiles.
    if (has_mask) mask_load(start + (wave + W * lane) * kChunk);
  }
  if (has_mask) mbits = mask_bits();
  int tab_proc = tab;
  uint32_t mbits_proc = mbits;

  float m = kNegBig, l = 0.f;  // running max (scaled, log2) and sum of this lane's column
  mf_f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  // Pool offset of this lane's 16 bytes of the current row (-1: none).  The
  // row is written after the last workgroup barrier: a barrier waits for
  // every store the wave has in flight, so a write issued in the loop would
  // hold up the merge below by a whole HBM write round trip.
  int64_t cur_dst = -1;
  const int kswz = dec_swz<D>(r16);
  const int vrow = 4 * c4 + (r16 >> 2);
  const int vswz = dec_swz<D>(vrow);

  for (int k = 0; k < ntw; ++k) {
    if (k + S - 1 < ntw)
      wait_vmcnt<2 * NI * (S - 1)>();  // tiles k + 1 .. k + S - 1 may stay in flight
    else
      wait_vmcnt<0>();
    char* sK = s_wave + (k % S) * STAGE_B;
    char* sV = sK + PTILE;
    const int c = wave + W * k;  // partition chunk of this tile
    const int tb = start + c * kChunk;
    if (k > 0 && (k & 63) == 0) {
      tab_proc = tab;
      mbits_proc = mbits;
    }
    const int32_t blk = __builtin_amdgcn_readlane(tab_proc, k & 63);
    const bool blk_ok = blk >= 0 && blk < p.num_blocks;

    if (c == new_tile) {
      // The current row: put it in place of the staged pool row, and note
      // its slot (new_slots[b], or the table slot of L - 1) for the pool
      // write at the end.
      int64_t slot = new_slot;
      if (p.new_slots == nullptr)
        slot = blk_ok ? (int64_t)blk * p.block_size + fast_mod((uint32_t)new_tok, p.bs_div) : -1;
      if (slot >= 0 && slot < cap && rg == 0) {
        const int r = new_tok - tb;
        const int pos16 = (col ^ dec_swz<D>(r)) << 4;
        if constexpr (kF8) {  // the lane's eight codes, in the stages' layout
          const int off8 = r * PROWB + (((col >> 1) ^ (r % CPR)) << 4) + (col & 1) * 8;
          *reinterpret_cast<uint2*>(sK + off8) = kq;
          *reinterpret_cast<uint2*>(sV + off8) = vq;
        } else {
          *reinterpret_cast<uint4*>(sK + r * ROWB + pos16) = kcur;
          *reinterpret_cast<uint4*>(sV + r * ROWB + pos16) = vcur;
        }
        const int64_t sb = p.slot_small ? (int64_t)fast_div((uint32_t)slot, p.bs_div)
                                        : slot / p.block_size;
        cur_dst = sb * p.s_blk + (slot - sb * p.block_size) * p.s_slot + head_off +
                  col * (kF8 ? 8 : 16);
      }
    }

    // S^T = K Q^T: lane holds scores of tokens tb + 4 c4 + i for head r16.
    mf_f32x4 sacc = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < DS; ++j) {
      uint4 a;
      if constexpr (kF8) {
        // Codes 8 u .. 8 u + 7 of row r16 (u = 4 j + c4): half u & 1 of
        // staged chunk (u / 2) ^ (r16 % CPR).
        const int u = 4 * j + c4;
        a = f8_dequant8<ET>(*reinterpret_cast<const uint2*>(
            sK + r16 * PROWB + (((u >> 1) ^ (r16 % CPR)) << 4) + (u & 1) * 8));
      } else {
        a = *reinterpret_cast<const uint4*>(sK + r16 * ROWB + (((4 * j + c4) ^ kswz) << 4));
      }
      sacc = M::qk(a, qb[j], sacc);
    }
    // FP8: V^T's codes, read now so that the stage can take the wave's tile
    // k + S before the softmax.  Read q gives lane (r16, c4) the codes of
    // tokens 4 c4 .. 4 c4 + 3 at dim 16 (2 q) + r16 (bytes 0-3) and at dim
    // 16 (2 q + 1) + r16 (bytes 4-7): the A operands of two 16x16x16
    // products.  Byte j of lane 16 c4 + i is byte i % 8 of the word lane
    // 16 c4 + 2 j + i / 8 points at, so lane (t, c4) points at token
    // 4 c4 + (t / 2) % 4, dims 16 (2 q + t / 8) + 8 (t % 2) .. + 7.
    uint2 vraw[kF8 ? DT / 2 : 1];
    if constexpr (kF8) {
      const int trow = 4 * c4 + ((r16 >> 1) & 3);
#pragma unroll
      for (int q = 0; q < DT / 2; ++q) {
        const int dt = 2 * q + (r16 >> 3);
        const int off = trow * PROWB + ((dt ^ (trow % CPR)) << 4) + (r16 & 1) * 8;
        vraw[q] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((mf_lds_s32x2*)(sV + off)));
      }
      // Both halves of the stage have been read: it takes tile k + S.
      wait_lgkmcnt0();
      if (k + S < ntw) issue(k + S);
    }
    float sv[4];
    const int rel = blk_ok ? end - tb - 4 * c4 : 0;  // token 4 c4 + i is live iff i < rel
    uint32_t live = 0;  // bit i: token 4 c4 + i is attended
#pragma unroll
    for (int i = 0; i < 4; ++i) live |= (i < rel ? 1u : 0u) << i;
    if (has_mask) {
      // Validity bits of tokens 4 c4 .. 4 c4 + 3 of this tile.
      const uint32_t mb = (uint32_t)__builtin_amdgcn_readlane((int)mbits_proc, k & 63) >> (4 * c4);
      live &= mb;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = ((live >> i) & 1u) ? sacc[i] : -INFINITY;
    // Dead tokens (past the context, masked) keep their staged V rows, which
    // may hold anything, non-finite values included: their P is 0, and the
    // V^T operand elements of this lane (tokens 4 c4 .. 4 c4 + 3, the same
    // tokens as its scores) are zeroed for them so that 0 * inf never enters
    // the sum.
    const uint32_t keep0 = ((live & 1u) ? 0xffffu : 0u) | ((live & 2u) ? 0xffff0000u : 0u);
    const uint32_t keep1 = ((live & 4u) ? 0xffffu : 0u) | ((live & 8u) ? 0xffff0000u : 0u);
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    const float mxs = mx * p.scale_log2;
    if (__builtin_amdgcn_ballot_w64(mxs > m + kDecLazy) != 0) {
      const float mnew = fmaxf(m, mxs);
      const float alpha = fast_exp2(m - mnew);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = fast_exp2(fmaf(sv[i], p.scale_log2, -m));
      l += pr[i];
    }
    uint2 pb;
    pb.x = M::pack2(pr[0], pr[1]);
    pb.y = M::pack2(pr[2], pr[3]);

    // O^T += V^T P^T over this tile's 16 tokens.
    if constexpr (kF8) {
#pragma unroll
      for (int q = 0; q < DT / 2; ++q) {
        const uint4 u = f8_dequant8<ET>(vraw[q]);
        o[2 * q] = M::pv(__builtin_bit_cast(mf_s16x4, make_uint2(u.x & keep0, u.y & keep1)), pb,
                         o[2 * q]);
        o[2 * q + 1] = M::pv(__builtin_bit_cast(mf_s16x4, make_uint2(u.z & keep0, u.w & keep1)),
                             pb, o[2 * q + 1]);
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int off =
            vrow * ROWB + (((2 * dt + ((r16 >> 1) & 1)) ^ vswz) << 4) + ((r16 & 1) << 3);
        uint2 au = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((mf_lds_s16x4*)(sV + off)));
        au.x &= keep0;
        au.y &= keep1;
        o[dt] = M::pv(__builtin_bit_cast(mf_s16x4, au), pb, o[dt]);
      }
    }
    // The stage is free once its LDS reads have returned (an FP8 stage was
    // reissued after its V reads above).
    if constexpr (!kF8) {
      wait_lgkmcnt0();
      if (k + S < ntw) issue(k + S);
    }
  }

  // ---- merge the waves through LDS ----
  // A wave with fewer tiles than the early issue fetched still has them in
  // flight: they land before the merge reuses the LDS.
  wait_vmcnt<0>();
  l = sum_xor16(l);
  l = sum_xor32(l);
  if constexpr (!kOwnMerge) __syncthreads();  // every wave is done with its stages
  float* s_o = reinterpret_cast<float*>(kOwnMerge ? s_mrg : s_buf);  // [W][G][D]
  float* s_m = s_o + W * G * D;                                       // [G][W]
  float* s_l = s_m + G * W;                                           // [G][W]
  if (r16 < G) {
    // Lane (r16, c4) holds o of head r16 at d = 16 dt + 4 c4 + i.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<mf_f32x4*>(s_o + (wave * G + r16) * D + 16 * dt + 4 * c4) = o[dt];
    if (c4 == 0) {
      s_m[r16 * W + wave] = ntw > 0 ? m : kNegBig;
      s_l[r16 * W + wave] = ntw > 0 ? l : 0.f;
    }
  }
  __syncthreads();

  // Each lane combines four consecutive outputs of one query head.
  const int64_t pair = (int64_t)b * p.num_kv_heads + h;
  for (int qd = tid; qd < G * D / 4; qd += NT) {
    const int g = qd / (D / 4), d = (qd % (D / 4)) * 4;
    float mw[W], lw[W];
#pragma unroll
    for (int w = 0; w < W; w += 4) {
      const mf_f32x4 mv = *reinterpret_cast<const mf_f32x4*>(s_m + g * W + w);
      const mf_f32x4 lv = *reinterpret_cast<const mf_f32x4*>(s_l + g * W + w);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mw[w + i] = mv[i];
        lw[w + i] = lv[i];
      }
    }
    float Mx = kNegBig;
#pragma unroll
    for (int w = 0; w < W; ++w) Mx = fmaxf(Mx, mw[w]);
    float Lt = 0.f;
    mf_f32x4 acc = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = fast_exp2(mw[w] - Mx);
      Lt += lw[w] * f;
      acc += f * *reinterpret_cast<const mf_f32x4*>(s_o + (w * G + g) * D + d);
    }
    if (nparts == 1) {
      const float inv = Lt > 0.f ? p.v_scale / Lt : 0.f;
      uint2 u;
      u.x = M::pack2(acc[0] * inv, acc[1] * inv);
      u.y = M::pack2(acc[2] * inv, acc[3] * inv);
      *reinterpret_cast<uint2*>(p.out + b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d * 2) = u;
    } else {
      const int64_t slot = (pair * p.max_parts + part) * G + g;
      *reinterpret_cast<mf_f32x4*>(p.part_o + slot * D + d) = acc * p.v_scale;
      if (d == 0) {
        p.part_ml[slot * 2] = Mx;
        p.part_ml[slot * 2 + 1] = Lt;
      }
    }
  }
  if (cur_dst >= 0) {
    if constexpr (kF8) {
      *reinterpret_cast<uint2*>(p.kp + cur_dst) = kq;
      *reinterpret_cast<uint2*>(p.vp + cur_dst) = vq;
    } else {
      st16(p.kp + cur_dst, kcur);
      st16(p.vp + cur_dst, vcur);
    }
  }
}

// ------------------------------------------------------------- launching
template <typename ET, int D, int G, bool kF8, int kWaves>
static void launch_decode_mfma_w(const DecodeParams& p, dim3 grid, hipStream_t s) {
  constexpr int NT = MfmaWaves<D, kWaves>::W * 64;
  const dim3 hgrid(grid.y, grid.x, grid.z);  // (kv head, sequence, partition)
  const bool mask = p.valid != nullptr && p.valid_len > 0;
  if (p.has_pro && mask)
    hipLaunchKernelGGL((paged_decode_mfma_kernel<ET, D, G, true, true, kF8, kWaves>), hgrid,
                       dim3(NT), 0, s, p);
  else if (p.has_pro)
    hipLaunchKernelGGL((paged_decode_mfma_kernel<ET, D, G, true, false, kF8, kWaves>), hgrid,
                       dim3(NT), 0, s, p);
  else if (mask)
    hipLaunchKernelGGL((paged_decode_mfma_kernel<ET, D, G, false, true, kF8, kWaves>), hgrid,
                       dim3(NT), 0, s, p);
  else
    hipLaunchKernelGGL((paged_decode_mfma_kernel<ET, D, G, false, false, kF8, kWaves>), hgrid,
                       dim3(NT), 0, s, p);
}

template <typename ET, int D, int G, bool kF8>
static void launch_decode_mfma(const DecodeParams& p, dim3 grid, hipStream_t s) {
  // Twelve waves: FP8 pools at head_dim 128 and groups up to 4 (a G = 8
  // prologue's query rows would not fit beside twelve waves' LDS).  Four
  // waves: head_dim 128.
  bool done = false;
  if constexpr (D == 128 && kF8 && G <= 4) {
    if (p.waves == 12) {
      launch_decode_mfma_w<ET, D, G, kF8, 12>(p, grid, s);
      done = true;
    }
  }
  if constexpr (D == 128) {
    if (p.waves == 4) {
      launch_decode_mfma_w<ET, D, G, kF8, 4>(p, grid, s);
      done = true;
    }
  }
  if (!done) launch_decode_mfma_w<ET, D, G, kF8, 0>(p, grid, s);
  if (p.max_parts > 1)
    hipLaunchKernelGGL((paged_decode_merge_kernel<ET, D, G, kF8 ? 1 : 0>), dim3(grid.y, grid.x),
                       dim3(256), 0, s, p);
}

template <typename ET, int D, bool kF8>
static bool dispatch_mfma_g(int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_decode_mfma<ET, D, 1, kF8>(p, grid, s); return true;
    case 2: launch_decode_mfma<ET, D, 2, kF8>(p, grid, s); return true;
    case 4: launch_decode_mfma<ET, D, 4, kF8>(p, grid, s); return true;
    case 8: launch_decode_mfma<ET, D, 8, kF8>(p, grid, s); return true;
    default: return false;
  }
}

template <typename ET, bool kF8>
static bool dispatch_mfma_d(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_mfma_g<ET, 64, kF8>(G, p, grid, s);
    case 128: return dispatch_mfma_g<ET, 128, kF8>(G, p, grid, s);
    case 256: return dispatch_mfma_g<ET, 256, kF8>(G, p, grid, s);
    default: return false;
  }
}

// Launch the matrix-core decode (and, when partitioned, the merge) for one
// 16-bit element type over a 16-bit pool (launch_paged_decode_mfma) or an
// FP8 pool (launch_paged_decode_mfma_f8, in its own translation units);
// false for an unsupported (head_dim, group) pair.
template <typename ET>
bool launch_paged_decode_mfma(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s);
template <typename ET>
bool launch_paged_decode_mfma_f8(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s);

}  // namespace va
