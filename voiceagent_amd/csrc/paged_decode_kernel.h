// Paged-KV decode attention (one query token per sequence) for GQA, with
// optional split-context partitions merged by a second, small kernel.
//
// Semantics: for sequence b with context length L and query head hq,
//     out[b, hq] = softmax_j( scale * q[b, hq] . K[j, hq / G] ) @ V[j, hq / G]
// over the tokens j < L that are not masked, where G = Hq / Hkv, K/V row j
// lives at block_table[b][j / block_size], slot j % block_size.  This is the
// per-sequence matmul/softmax of _reference_paged_attention
// (qwen_asr_vllm/agent/qwen_tts_paged_attention.py:353-380) and the q_len = 1
// case of flash_attn_varlen_func with bottom-right causal alignment
// (qwen_asr_vllm/layers/attention.py:1-11, 96-107).  Masking follows the
// Triton kernel (qwen_tts_paged_attention.py:229-234, 267): a token is
// attended iff j < L and key_valid_mask[b, j] (tokens past the mask width
// count as valid, qwen_tts_paged_attention.py:466-474); a row with no
// attended token yields 0.
//
// Work decomposition (MI355X): the grid is (partition, kv head, sequence).
// One workgroup of NW wavefronts owns P = split_tokens consecutive tokens of
// one (sequence, kv head) pair and serves all G query heads of the group, so
// every K/V byte is read from HBM once.  Tokens are processed in 16-token
// chunks; the 64 lanes of a wave split a chunk as (row group, 16-byte column):
// a D = 128 bf16 row is 16 lanes x 16 B, four rows per dwordx4 load, so each
// load instruction moves 1 KiB of fully used 128-byte lines.  Chunk c of the
// partition goes to wave c % NW; a wave issues the K/V loads of CPW chunks
// before reducing the first of them.  Scores (v_dot2 on 16-bit inputs) are
// reduced over the row's lanes with DPP, the running max over row groups
// with cross-row permutes; softmax runs in the exp2 domain (scores scaled by
// scale * log2 e).  Waves merge through LDS.  A sequence split into several
// partitions writes unnormalised partials (m, l, o) to the workspace, and a
// small second kernel (one workgroup per sequence x kv head) merges them with
// the log-sum-exp rule.  The kernel boundary publishes the partials, so no
// workgroup ever waits on another.  Partitions are used only when there are
// too few (sequence, kv head) pairs to give every CU a workgroup: one
// 8-wave workgroup fills a CU, and a second round of workgroups costs more
// than the imbalance between long and short contexts.
#pragma once

#include "fastdiv.h"
#include "prologue.h"

namespace va {

struct DecodeParams {
  const char* q;
  int64_t q_sb, q_sh;  // bytes
  char* out;
  int64_t o_sb, o_sh;  // bytes
  char* kp;
  char* vp;
  int64_t s_blk, s_slot, s_head;  // bytes
  int32_t block_size, num_blocks;
  int32_t block_is_chunk_aligned;  // block_size % 16 == 0
  FastDiv bs_div;                  // block_size
  int32_t slot_small;              // num_blocks * block_size <= 2^31
  int32_t pool_off32;              // every pool byte offset fits 32 bits
  const void* table;
  int64_t t_sb;  // elements
  int32_t table_i64;
  int32_t table_width;       // columns attention reads (past it: block 0)
  int32_t table_width_full;  // columns the current-row write may read
  int32_t key_limit;         // > 0: tokens at or past it are not attended
  const void* lens;
  int32_t lens_i64, lens_cum;
  const uint8_t* valid;
  int64_t valid_sb;
  int32_t valid_len;
  const char* new_k;
  const char* new_v;
  int64_t nk_sb, nk_sh, nv_sb, nv_sh;  // bytes
  const void* new_slots;
  int32_t new_slots_i64;
  int32_t num_kv_heads;
  int32_t split_tokens;
  int32_t max_parts;
  int32_t dyn_split;  // partition size from each context's length (see partition_tokens)
  float scale_log2;
  float* part_ml;
  float* part_o;
  int32_t has_pro;  // apply the Qwen3 q/k prologue to q and the current row
  PrologueParams pro;
  int32_t kv_fp8;        // the pool holds e4m3 codes (matrix-core kernel only)
  int32_t waves;         // matrix-core kernel: 0 (the default for head_dim), 12 or 4
  float v_scale;         // output factor: v_scale of an FP8 pool, else 1
  float inv_k, inv_v;    // FP8 pool: 1 / k_scale, 1 / v_scale (current-row quantisation)
};

constexpr int kChunk = 16;

// Block id at table column `idx` of row `row`; columns past the table width
// read as block 0.
__device__ inline int64_t table_entry(const DecodeParams& p, int64_t row, int idx) {
  return idx < p.table_width ? load_index(p.table, row + idx, p.table_i64) : 0;
}
constexpr float kNegBig = -1.0e30f;

// Tokens per context partition.  Fixed (split_tokens), or with dyn_split
// derived on the device from the context length L, so that the max_parts
// partitions of a pair share its context evenly in multiples of kDynGrain
// tokens.  The dynamic form serves launches whose max_seq_len is only an
// upper bound, such as a decode graph captured at max_model_len.  One
// 16-token tile: a short context spreads over as many workgroups as the
// split allows (the TTS talker's B = 1 x 600 step: 8.01 us/layer with
// 64-token partitions, 7.66 with 16).
constexpr int kDynGrain = 16;

// Attended length of a context of L tokens: L, or key_limit when that is
// smaller (the TTS kernel's MAX_SEQ_LEN = kernel_seq_len bound,
// qwen_tts_paged_attention.py:223-230).
__device__ inline int attend_len(const DecodeParams& p, int L) {
  return (p.key_limit > 0 && L > p.key_limit) ? p.key_limit : L;
}

// Where the current row (position L - 1) goes when it is not attended in
// place: past key_limit, or (written through the table) in a column at or
// past the attention's read width but inside the table, where attention
// reads block 0 while the write takes the table's entry
// (qwen_tts_paged_attention.py:182-187 reads the table unbounded, :236-241
// bounds the attention's reads by num_page_slots).
__device__ inline bool current_row_detached(const DecodeParams& p, int L, int La, int col_new) {
  if (p.new_k == nullptr || L < 1) return false;
  if (L - 1 >= La) return true;
  return p.new_slots == nullptr && col_new >= p.table_width && col_new < p.table_width_full;
}

// The detached current-row write: this lane's 16 bytes (at byte column
// `col16`) of kv head h's row go to new_slots[b], or to the slot of
// position L - 1 through the table's own entry (block 0 past the table);
// a slot outside the pool skips the write.
__device__ inline void store_detached_row(const DecodeParams& p, int h, int64_t table_row, int L,
                                          int col_new, int64_t new_slot, int col16, uint4 kr,
                                          uint4 vr) {
  int64_t slot = new_slot;
  if (p.new_slots == nullptr) {
    const int64_t blk =
        col_new < p.table_width_full ? load_index(p.table, table_row + col_new, p.table_i64) : 0;
    slot = (blk >= 0 && blk < p.num_blocks) ? blk * p.block_size + (L - 1) % p.block_size : -1;
  }
  if (slot < 0 || slot >= (int64_t)p.num_blocks * p.block_size) return;
  const int64_t sb = slot / p.block_size;
  const int64_t dst =
      sb * p.s_blk + (slot - sb * p.block_size) * p.s_slot + (int64_t)h * p.s_head + col16;
  st16(p.kp + dst, kr);
  st16(p.vp + dst, vr);
}

// The same for an FP8 pool: this lane's 8 codes (at byte column col8).
__device__ inline void store_detached_row_f8(const DecodeParams& p, int h, int64_t table_row,
                                             int L, int col_new, int64_t new_slot, int col8,
                                             uint2 kr, uint2 vr) {
  int64_t slot = new_slot;
  if (p.new_slots == nullptr) {
    const int64_t blk =
        col_new < p.table_width_full ? load_index(p.table, table_row + col_new, p.table_i64) : 0;
    slot = (blk >= 0 && blk < p.num_blocks) ? blk * p.block_size + (L - 1) % p.block_size : -1;
  }
  if (slot < 0 || slot >= (int64_t)p.num_blocks * p.block_size) return;
  const int64_t sb = slot / p.block_size;
  const int64_t dst =
      sb * p.s_blk + (slot - sb * p.block_size) * p.s_slot + (int64_t)h * p.s_head + col8;
  *reinterpret_cast<uint2*>(p.kp + dst) = kr;
  *reinterpret_cast<uint2*>(p.vp + dst) = vr;
}

__device__ inline int partition_tokens(const DecodeParams& p, int L) {
  if (!p.dyn_split) return p.split_tokens;
  int P = (L + p.max_parts - 1) / p.max_parts;
  P = (P + kDynGrain - 1) / kDynGrain * kDynGrain;
  return P > kDynGrain ? P : kDynGrain;
}

__device__ inline float uniform(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// Per-configuration launch shape: NW = 8 wavefronts per workgroup (two per
// SIMD, so a wave may hold up to 256 VGPRs and the state never spills), CPW
// chunks whose K/V loads are in flight together per wave (8 * NR data VGPRs
// each).  Measured on MI355X at B = 32: 8 waves x 2 chunks beat 16 waves
// (128-VGPR cap, spills) and deeper per-wave prefetch (3-4 chunks).
template <typename ET, int D, int G>
struct DecodeShape {
  static constexpr int E = ET::kPerVec;       // elements per 16-byte lane load
  static constexpr int LPR = D / E;           // lanes per K/V row
  static constexpr int RPL = 64 / LPR;        // rows per load instruction
  static constexpr int NR = kChunk / RPL;     // rows per lane per chunk
  static constexpr int CPW = (8 * NR >= 64) ? 1 : 64 / (8 * NR);
  static constexpr int NW = 8;
  static constexpr int kWavesPerSimd = 2;     // occupancy the register budget is sized for
};

// kAligned: block_size % 16 == 0 (one block per chunk).  kProlog: apply the
// Qwen3 q/k prologue (a separate instantiation, so the kernels without it
// carry none of its loads or branches).
template <typename ET, int D, int G, bool kAligned, bool kProlog>
__global__ __launch_bounds__((DecodeShape<ET, D, G>::NW * 64),
                             (DecodeShape<ET, D, G>::kWavesPerSimd)) void paged_decode_kernel(
    DecodeParams p) {
  using S = DecodeShape<ET, D, G>;
  constexpr int E = S::E, LPR = S::LPR, RPL = S::RPL, NR = S::NR, CPW = S::CPW, NW = S::NW;
  static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "unsupported head_dim");
  static_assert(RPL <= kChunk, "unsupported head_dim");
  constexpr int NT = NW * 64;

  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ float s_o[NW][G][D];

  // Partition-major grid: every sequence's first partition is dispatched
  // before any second one, so workgroups past the end of short contexts
  // (which exit after reading the length) queue behind the live ones.
  // Grid (kv head, sequence, partition), as the matrix-core kernel's: each
  // XCD takes the same kv heads of every sequence.
  const int b = blockIdx.y;
  const int h = blockIdx.x;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int rg = lane / LPR;
  const int col = lane % LPR;
  int P = p.split_tokens;  // placeholder in dyn_split mode, fixed below from L
  int start = part * P;
  const int64_t table_row = (int64_t)b * p.t_sb;

  // Independent loads first, none depending on another: the context length,
  // this wave's block-table entries (lane k holds the block of the wave's
  // k-th chunk), the query, the current K/V row, its slot and the prologue's
  // position.  The first K/V loads then wait for one round trip only.
  int L;
  if (p.lens_cum)
    L = (int)(load_index(p.lens, b + 1, p.lens_i64) - load_index(p.lens, b, p.lens_i64));
  else
    L = (int)load_index(p.lens, b, p.lens_i64);
  int tab = 0;  // block of the wave's chunk `lane` (chunks 64 i + lane after refills)
  if constexpr (kAligned) {
    // The last grid partition runs to the context's end, which may lie past
    // P when max_seq_len underestimates; table_entry bounds the read.
    const int c = wave + NW * lane;
    const int tok = start + c * kChunk;
    if (c * kChunk < P || part == p.max_parts - 1)
      tab = (int)table_entry(p, table_row, tok / p.block_size);
  }
  // The query slice of this lane, as loaded (16-bit types feed v_dot2 and
  // are scaled after the row reduction; fp32 is pre-scaled before use).
  uint4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = ld16(p.q + b * p.q_sb + (int64_t)(h * G + g) * p.q_sh + col * 16);
  uint4 kcur = make_uint4(0, 0, 0, 0), vcur = make_uint4(0, 0, 0, 0);
  if (p.new_k != nullptr) {
    kcur = ld16(p.new_k + b * p.nk_sb + h * p.nk_sh + col * 16);
    vcur = ld16(p.new_v + b * p.nv_sb + h * p.nv_sh + col * 16);
  }
  int64_t new_slot = -1;
  if (p.new_slots != nullptr) new_slot = load_index(p.new_slots, b, p.new_slots_i64);
  int64_t pos = 0;
  if (kProlog) pos = load_index(p.pro.pos, b, p.pro.pos_i64);
  L = __builtin_amdgcn_readfirstlane(L);
  // L becomes the attended length; the current row sits at Lr - 1.
  const int Lr = L;
  L = attend_len(p, L);
  const int col_new = Lr >= 1 ? (Lr - 1) / p.block_size : 0;
  const bool detached = current_row_detached(p, Lr, L, col_new);

  if (L <= 0) {
    // Nothing to attend: the output is defined as 0.
    if (part == 0) {
      for (int idx = tid; idx < G * D; idx += NT) {
        const int g = idx / D, d = idx % D;
        float z[E] = {};
        if (d % E == 0)
          st16(p.out + b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d * ET::kBytes,
               ET::pack(z));
      }
    }
    return;
  }
  if (p.dyn_split) {
    // The partition follows from L: re-read this wave's block ids for it.
    P = partition_tokens(p, L);
    start = part * P;
    if (kAligned && start < L) {
      const int c = wave + NW * lane;
      tab = c * kChunk < P ? (int)table_entry(p, table_row, (start + c * kChunk) / p.block_size)
                           : 0;
    }
  }
  if (start >= L) return;
  int nparts = (L + P - 1) / P;
  const bool last_grid_part = part == p.max_parts - 1;
  if (nparts > p.max_parts) nparts = p.max_parts;  // the last partition absorbs the rest
  const int end = last_grid_part ? L : min(start + P, L);

  // The current row (TTS fused write, engine fused store) is position L - 1
  // of the partition that holds it.  It is written to its slot and attended
  // in place of the pool's row when the slot is valid: new_slots[b], or the
  // block-table slot of L - 1 (resolved at the row's chunk from the same
  // block id its loads use).  A slot < 0 skips the write and the
  // substitution.
  const int new_tok =
      (!detached && p.new_k != nullptr && L - 1 >= start && L - 1 < end) ? L - 1 : -1;
  const int64_t cap = (int64_t)p.num_blocks * p.block_size;

  // Prologue factors of this lane's slice (the math runs once the first
  // chunk group's K/V loads are in flight).
  float pro_c[E], pro_s[E];
  WeightRaw<E> pro_wq{}, pro_wk{};
  if constexpr (kProlog) {
    pro_wq = load_weights_raw<E>(p.pro.q_w, p.pro.w_dtype, col * E);
    pro_wk = load_weights_raw<E>(p.pro.k_w != nullptr ? p.pro.k_w : p.pro.q_w, p.pro.w_dtype,
                                 col * E);
    pos = pos < 0 ? 0 : (pos >= p.pro.max_pos ? p.pro.max_pos - 1 : pos);
    load_rotary<E, LPR>(p.pro, pos, col, D, pro_c, pro_s);
  }
  if (detached && part == 0 && wave == 0) {
    // The current row is not attended in place: wave 0 of the first
    // partition writes it (after the prologue, when there is one).
    uint4 kw = kcur;
    if constexpr (kProlog) {
      float w[E], x[E];
      convert_weights<E>(pro_wk, p.pro.w_dtype, w);
      ET::unpack(kw, x);
      qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, pro_c, pro_s);
      kw = ET::pack(x);
    }
    if (rg == 0) store_detached_row(p, h, table_row, Lr, col_new, new_slot, col * 16, kw, vcur);
  }

  constexpr bool kScaleAfter = ET::kBytes == 2;
  float m[G], l[G], o[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) o[g][e] = 0.f;
  }

  const int64_t head_off = (int64_t)h * p.s_head + col * 16;
  const int nch = (end - start + kChunk - 1) / kChunk;
  const int my_chunks = nch > wave ? (nch - wave + NW - 1) / NW : 0;

  // Issue the K/V loads of the wave's k-th chunk.  `cb` is the chunk's block
  // (16-aligned blocks) and `rbk` the per-row blocks (other block sizes),
  // both read before the chunk group's first K/V load.  No loaded value is
  // consumed here: a value needed at a branch join makes the compiler wait
  // for every outstanding load (s_waitcnt vmcnt(0)), which would serialise
  // the K/V traffic.  `valid` gets bit r for every row inside the context
  // with a mapped block (the key_valid_mask is applied after the loads).
  auto load_chunk = [&](int k, int32_t cb, const int32_t* rbk, uint4 (&kr)[NR], uint4 (&vr)[NR],
                        uint32_t& valid) {
    const int tb = start + (wave + NW * k) * kChunk;
    valid = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int tok = tb + rg + r * RPL;
      const int32_t blk = kAligned ? cb : rbk[r];
      const bool ok = tok < end && blk >= 0 && blk < p.num_blocks;
      valid |= (ok ? 1u : 0u) << r;
      kr[r] = make_uint4(0, 0, 0, 0);
      vr[r] = make_uint4(0, 0, 0, 0);
      if (p.pool_off32) {
        // 32-bit offsets from the pool bases: one VGPR per address.
        if (ok) {
          const uint32_t off = (uint32_t)blk * (uint32_t)p.s_blk +
                               (uint32_t)(tok % p.block_size) * (uint32_t)p.s_slot +
                               (uint32_t)head_off;
          kr[r] = ld16_nt(p.kp + off);
          vr[r] = ld16_nt(p.vp + off);
        }
      } else if (ok) {
        const int64_t off =
            (int64_t)blk * p.s_blk + (int64_t)(tok % p.block_size) * p.s_slot + head_off;
        kr[r] = ld16_nt(p.kp + off);
        vr[r] = ld16_nt(p.vp + off);
      }
    }
  };

  // The chunk holding the current row: substitute the register copy for the
  // row and note its slot's pool offset (exactly one lane group in the grid
  // does).  The pool write itself comes after the last workgroup barrier: a
  // barrier waits for every store the wave has in flight, so a write issued
  // here would hold up the merge by a whole HBM write round trip.
  int64_t cur_dst = -1;
  auto current_row = [&](int k, int32_t cb, const int32_t* rbk, uint4 (&kr)[NR],
                         uint4 (&vr)[NR]) {
    const int tb = start + (wave + NW * k) * kChunk;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (tb + rg + r * RPL != new_tok) continue;
      int64_t slot = new_slot;
      if (p.new_slots == nullptr) {
        const int32_t blk = kAligned ? cb : rbk[r];
        slot = (blk >= 0 && blk < p.num_blocks) ? (int64_t)blk * p.block_size +
                                                      new_tok % p.block_size
                                                : -1;
      }
      if (slot >= 0 && slot < cap) {
        kr[r] = kcur;
        vr[r] = vcur;
        const int64_t blk = slot / p.block_size;
        cur_dst = blk * p.s_blk + (slot - blk * p.block_size) * p.s_slot + head_off;
      }
    }
  };

  auto process_chunk = [&](const uint4 (&kr)[NR], const uint4 (&vr)[NR], uint32_t valid) {
    float s[NR][G];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int g = 0; g < G; ++g) s[r][g] = ET::dot(qv[g], kr[r], 0.f);
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float t = group_sum<LPR>(s[r][g]);
        if constexpr (kScaleAfter) t *= p.scale_log2;
        s[r][g] = ((valid >> r) & 1u) ? t : -INFINITY;
      }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[0][g];
#pragma unroll
      for (int r = 1; r < NR; ++r) mx = fmaxf(mx, s[r][g]);
      mx = uniform(strided_max<LPR>(mx));
      if (mx > m[g]) {
        const float alpha = fast_exp2(m[g] - mx);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < E; ++e) o[g][e] *= alpha;
        m[g] = mx;
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float vf[E];
      ET::unpack(vr[r], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = fast_exp2(s[r][g] - m[g]);
        l[g] += pr;
#pragma unroll
        for (int e = 0; e < E; ++e) o[g][e] = fmaf(pr, vf[e], o[g][e]);
      }
    }
  };

  // The query (and current key) transform and the fp32 pre-scale: run once,
  // after the first chunk group's loads are issued, so their inputs' round
  // trip overlaps that of the K/V rows.
  auto prepare_query = [&]() {
    if constexpr (kProlog) {
      float w[E];
      convert_weights<E>(pro_wq, p.pro.w_dtype, w);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float x[E];
        ET::unpack(qv[g], x);
        qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, pro_c, pro_s);
        qv[g] = ET::pack(x);
      }
      if (new_tok >= 0) {
        convert_weights<E>(pro_wk, p.pro.w_dtype, w);
        float x[E];
        ET::unpack(kcur, x);
        qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, pro_c, pro_s);
        kcur = ET::pack(x);
      }
    }
    if constexpr (!kScaleAfter) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        qv[g].x = __float_as_uint(__uint_as_float(qv[g].x) * p.scale_log2);
        qv[g].y = __float_as_uint(__uint_as_float(qv[g].y) * p.scale_log2);
        qv[g].z = __float_as_uint(__uint_as_float(qv[g].z) * p.scale_log2);
        qv[g].w = __float_as_uint(__uint_as_float(qv[g].w) * p.scale_log2);
      }
    }
  };

  // One group of CPW chunks: read their block ids (and mask bits) first, then
  // issue all their K/V loads, then reduce them in order.
  constexpr int kRbk = kAligned ? 1 : CPW * NR;
  auto run_group = [&](int k0, bool first) {
    if (kAligned && k0 > 0 && (k0 & 63) == 0) {
      // Next 64 chunks of this wave: refill the block-id prefetch (every
      // earlier load of this wave has been consumed by now).
      const int c = wave + NW * (k0 + lane);
      tab = c * kChunk < end - start
                ? (int)table_entry(p, table_row, (start + c * kChunk) / p.block_size)
                : 0;
    }
    int32_t cb[CPW];
    int32_t rbk[kRbk];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int k = k0 + j;
      const int tb = start + (wave + NW * k) * kChunk;
      cb[j] = 0;
      if (k >= my_chunks) continue;
      if constexpr (kAligned) {
        cb[j] = __builtin_amdgcn_readlane(tab, k & 63);
      } else {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int tok = tb + rg + r * RPL;
          rbk[j * NR + r] = tok < end ? (int32_t)table_entry(p, table_row, tok / p.block_size) : 0;
        }
      }
    }
    uint4 kr[CPW][NR], vr[CPW][NR];
    uint32_t valid[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (k0 + j < my_chunks) {
        load_chunk(k0 + j, cb[j], kAligned ? rbk : rbk + (kAligned ? 0 : j * NR), kr[j], vr[j],
                   valid[j]);
      } else {
        valid[j] = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) kr[j][r] = vr[j][r] = make_uint4(0, 0, 0, 0);
      }
    }
    if (p.valid != nullptr && p.valid_len > 0) {
      // key_valid_mask bits of the rows, read after the K/V loads are issued
      // (the rows are loaded either way; a cleared bit only drops the score).
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int tb = start + (wave + NW * (k0 + j)) * kChunk;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int tok = tb + rg + r * RPL;
          const int idx = tok < p.valid_len ? tok : p.valid_len - 1;
          const uint8_t byte = p.valid[b * p.valid_sb + (idx < 0 ? 0 : idx)];
          if (tok < p.valid_len && byte == 0) valid[j] &= ~(1u << r);
        }
      }
      // Masked rows were loaded: zero their values, so that a non-finite
      // value in a masked slot cannot reach the output through 0 * inf.
#pragma unroll
      for (int j = 0; j < CPW; ++j)
#pragma unroll
        for (int r = 0; r < NR; ++r)
          if (!((valid[j] >> r) & 1u)) vr[j][r] = make_uint4(0, 0, 0, 0);
    }
    if (first) prepare_query();
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (k0 + j < my_chunks) {
        const int tb = start + (wave + NW * (k0 + j)) * kChunk;
        if (new_tok >= tb && new_tok < tb + kChunk)  // uniform
          current_row(k0 + j, cb[j], kAligned ? rbk : rbk + (kAligned ? 0 : j * NR), kr[j],
                      vr[j]);
        process_chunk(kr[j], vr[j], valid[j]);
      }
    }
  };
  if (my_chunks > 0) run_group(0, true);
  for (int k0 = CPW; k0 < my_chunks; k0 += CPW) run_group(k0, false);

  // Wave result: sum l and o over row groups (lanes sharing `col`).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = strided_sum<LPR>(l[g]);
#pragma unroll
    for (int e = 0; e < E; ++e) o[g][e] = strided_sum<LPR>(o[g][e]);
  }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < E; ++e) s_o[wave][g][col * E + e] = o[g][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = l[g];
    }
  }
  __syncthreads();

  const int64_t pair = (int64_t)b * p.num_kv_heads + h;
  for (int idx = tid; idx < G * D; idx += NT) {
    const int g = idx / D, d = idx % D;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
    float Lt = 0.f, Ot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = fast_exp2(s_m[w][g] - M);
      Lt += s_l[w][g] * f;
      Ot += s_o[w][g][d] * f;
    }
    if (nparts == 1) {
      const float val = Lt > 0.f ? Ot / Lt : 0.f;
      char* dst = p.out + b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d * ET::kBytes;
      if constexpr (ET::kBytes == 4) {
        *reinterpret_cast<float*>(dst) = val;
      } else {
        float tmp[E] = {};
        tmp[0] = val;
        const uint4 u = ET::pack(tmp);
        *reinterpret_cast<uint16_t*>(dst) = (uint16_t)(u.x & 0xffffu);
      }
    } else {
      const int64_t slot = (pair * p.max_parts + part) * G + g;
      p.part_o[slot * D + d] = Ot;
      if (d == 0) {
        p.part_ml[slot * 2] = M;
        p.part_ml[slot * 2 + 1] = Lt;
      }
    }
  }
  if (cur_dst >= 0) {
    st16(p.kp + cur_dst, kcur);
    st16(p.vp + cur_dst, vcur);
  }
}

// Most partitions one context is split into (the host grows the partition
// beyond this), which bounds the merge kernel's LDS.
constexpr int kMaxParts = 256;

// Merge of the partitions of one (sequence, kv head) pair: for each query head
//   out = sum_q 2^(m_q - M) o_q / sum_q 2^(m_q - M) l_q,  M = max_q m_q.
// Pairs that fit one partition were written by the attention kernel and are
// skipped.  Every wave serves one query head g over 64 of its D outputs
// (idx = (g, d) in 64-wide slices).  Lane q of the wave holds (m, l) of
// partitions q, q + 64, ..., and the o values of the first kBatch
// partitions are loaded by every lane for its d in the same breath, together
// with the length, so the merge costs one round trip.  The weights
// 2^(m_q - M) reach the o sums through readlane (q is wave-uniform).  Loads
// use clamped indices and are masked afterwards, so no load sits behind a
// branch.
// kTag only separates the instantiations of the translation units that
// launch the kernel (native and FP8 pools), which then never share a name.
template <typename ET, int D, int G, int kTag = 0>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p) {
  constexpr int E = ET::kPerVec;
  constexpr int kPerLane = kMaxParts / 64;
  constexpr int kBatch = 32;
  static_assert(D % 64 == 0, "a wave covers 64 outputs of one query head");
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Every load is issued before the first wait: the length (raw low words,
  // as in the attention kernels) and the partials of all max_parts slots of
  // the pair, whether or not this context filled them.  Slots past the
  // context's partition count hold stale data; they are read (the workspace
  // has them) but never enter the arithmetic.
  const uint32_t* const lensw = reinterpret_cast<const uint32_t*>(p.lens);
  const uint32_t len_hi = lensw[(int64_t)(b + p.lens_cum) << p.lens_i64];
  const uint32_t len_lo = lensw[(int64_t)b << p.lens_i64];
  const int64_t pair_slot0 = ((int64_t)b * p.num_kv_heads + h) * p.max_parts;

  for (int idx0 = tid & ~63; idx0 < G * D; idx0 += 256) {
    const int g = idx0 / D;                // uniform per wave
    const int d = idx0 % D + lane;
    float mq[kPerLane], lq[kPerLane], oq[kBatch];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int q = lane + 64 * i;
      const int64_t slot = (pair_slot0 + (q < p.max_parts ? q : p.max_parts - 1)) * G + g;
      mq[i] = p.part_ml[slot * 2];
      lq[i] = p.part_ml[slot * 2 + 1];
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int q = j < p.max_parts ? j : p.max_parts - 1;
      oq[j] = p.part_o[((pair_slot0 + q) * G + g) * D + d];
    }
    int L = (int)(p.lens_cum ? len_hi - len_lo : len_lo);
    L = attend_len(p, __builtin_amdgcn_readfirstlane(L));
    if (L <= 0) return;
    const int P = partition_tokens(p, L);
    int nparts = (L + P - 1) / P;
    if (nparts > p.max_parts) nparts = p.max_parts;
    if (nparts <= 1) return;  // the attention kernel wrote the output itself
    float M = kNegBig;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)
      if (lane + 64 * i < nparts) M = fmaxf(M, mq[i]);
    M = group_max<64>(M);
    float w[kPerLane], Lt = 0.f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const bool live = lane + 64 * i < nparts;
      w[i] = live ? fast_exp2(mq[i] - M) : 0.f;
      if (live) Lt = fmaf(w[i], lq[i], Lt);
    }
    Lt = group_sum<64>(Lt);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (j < nparts)
        acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[0]), j)), oq[j], acc);
    for (int q0 = kBatch; q0 < nparts; q0 += kBatch) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int q = q0 + j < nparts ? q0 + j : nparts - 1;
        oq[j] = p.part_o[((pair_slot0 + q) * G + g) * D + d];
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int q = q0 + j;
        if (q < nparts) {
          float wq = 0.f;
#pragma unroll
          for (int i = 0; i < kPerLane; ++i)
            if ((q >> 6) == i) wq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[i]), q & 63));
          acc = fmaf(wq, oq[j], acc);
        }
      }
    }
    const float val = Lt > 0.f ? acc / Lt : 0.f;
    char* dst = p.out + b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d * ET::kBytes;
    if constexpr (ET::kBytes == 4) {
      *reinterpret_cast<float*>(dst) = val;
    } else {
      float tmp[E] = {};
      tmp[0] = val;
      const uint4 u = ET::pack(tmp);
      *reinterpret_cast<uint16_t*>(dst) = (uint16_t)(u.x & 0xffffu);
    }
  }
}

// ------------------------------------------------------------- launching
template <typename ET, int D, int G, bool kProlog>
static void launch_decode_kernel(const DecodeParams& p, dim3 grid, hipStream_t s) {
  const dim3 hgrid(grid.y, grid.x, grid.z);  // (kv head, sequence, partition)
  if (p.block_is_chunk_aligned)
    hipLaunchKernelGGL((paged_decode_kernel<ET, D, G, true, kProlog>), hgrid,
                       dim3(DecodeShape<ET, D, G>::NW * 64), 0, s, p);
  else
    hipLaunchKernelGGL((paged_decode_kernel<ET, D, G, false, kProlog>), hgrid,
                       dim3(DecodeShape<ET, D, G>::NW * 64), 0, s, p);
}

template <typename ET, int D, int G>
static void launch_decode(const DecodeParams& p, dim3 grid, hipStream_t s) {
  if (p.has_pro)
    launch_decode_kernel<ET, D, G, true>(p, grid, s);
  else
    launch_decode_kernel<ET, D, G, false>(p, grid, s);
  if (p.max_parts > 1)
    hipLaunchKernelGGL((paged_decode_merge_kernel<ET, D, G>), dim3(grid.y, grid.x), dim3(256), 0,
                       s, p);
}

template <typename ET, int D>
static bool dispatch_g(int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_decode<ET, D, 1>(p, grid, s); return true;
    case 2: launch_decode<ET, D, 2>(p, grid, s); return true;
    case 4: launch_decode<ET, D, 4>(p, grid, s); return true;
    case 8: launch_decode<ET, D, 8>(p, grid, s); return true;
    default: return false;
  }
}

template <typename ET>
static bool dispatch_d(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<ET, 64>(G, p, grid, s);
    case 128: return dispatch_g<ET, 128>(G, p, grid, s);
    case 256: return dispatch_g<ET, 256>(G, p, grid, s);
    default: return false;
  }
}

// Launch the decode (and, when partitioned, the merge) kernels for one
// element type; defined in paged_decode_<type>.hip so the instantiations
// compile in parallel.  False for an unsupported (head_dim, group) pair.
template <typename ET>
bool launch_paged_decode(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s);

// Shapes the two kernels above do not take (head_dim other than 64 / 128 /
// 256, or a group other than 1 / 2 / 4 / 8) go to the small-head kernel
// (paged_decode_small.hip): grid (num_seqs, num_heads), no context split.
// False for a head_dim outside [1, kSmallMaxHeadDim] or an unknown dtype.
constexpr int kSmallMaxHeadDim = 1024;
bool launch_paged_decode_small(int dtype, int D, int G, const DecodeParams& p, dim3 grid,
                               hipStream_t s);

}  // namespace va

