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
#include <atomic>

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
  int32_t pool_off32;              // every pool byte offset fits 32 bits
  const void* table;
  int64_t t_sb;  // elements
  int32_t table_i64;
  int32_t table_width;
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
  float scale_log2;
  float* part_ml;
  float* part_o;
  int32_t has_pro;  // apply the Qwen3 q/k prologue to q and the current row
  PrologueParams pro;
};

constexpr int kChunk = 16;

// Block id at table column `idx` of row `row`; columns past the table width
// read as block 0.
__device__ inline int64_t table_entry(const DecodeParams& p, int64_t row, int idx) {
  return idx < p.table_width ? load_index(p.table, row + idx, p.table_i64) : 0;
}
constexpr float kNegBig = -1.0e30f;

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

template <typename ET, int D, int G, bool kAligned>
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
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int rg = lane / LPR;
  const int col = lane % LPR;
  const int P = p.split_tokens;
  const int start = part * P;
  const int64_t table_row = (int64_t)b * p.t_sb;

  // Independent loads first: the context length, this wave's block-table
  // entries (lane k holds the block of the wave's k-th chunk) and the query.
  int L;
  if (p.lens_cum)
    L = (int)(load_index(p.lens, b + 1, p.lens_i64) - load_index(p.lens, b, p.lens_i64));
  else
    L = (int)load_index(p.lens, b, p.lens_i64);
  int tab = 0;
  if constexpr (kAligned) {
    const int c = wave + NW * lane;
    const int tok = start + c * kChunk;
    if (c * kChunk < P) tab = (int)table_entry(p, table_row, tok / p.block_size);
  }
  // The query slice of this lane, as loaded (16-bit types feed v_dot2 and
  // are scaled after the row reduction; fp32 is pre-scaled below).
  uint4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = ld16(p.q + b * p.q_sb + (int64_t)(h * G + g) * p.q_sh + col * 16);
  L = __builtin_amdgcn_readfirstlane(L);

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
  if (start >= L) return;
  int nparts = (L + P - 1) / P;
  const bool last_grid_part = part == p.max_parts - 1;
  if (nparts > p.max_parts) nparts = p.max_parts;  // the last partition absorbs the rest
  const int end = last_grid_part ? L : min(start + P, L);

  // Current-row substitution / write (TTS fused write, engine fused store).
  int64_t new_dst = -1;  // byte offset of the destination slot (block/slot part)
  int new_tok = -1;
  if (p.new_k != nullptr && L - 1 >= start && L - 1 < end) {
    int64_t slot;
    if (p.new_slots != nullptr) {
      slot = load_index(p.new_slots, b, p.new_slots_i64);
    } else {
      const int64_t blk = table_entry(p, table_row, (L - 1) / p.block_size);
      slot = (blk < 0 || blk >= p.num_blocks) ? -1
                                              : blk * p.block_size + (L - 1) % p.block_size;
    }
    if (slot >= 0 && slot < (int64_t)p.num_blocks * p.block_size) {
      const int64_t blk = slot / p.block_size;
      new_dst = blk * p.s_blk + (slot - blk * p.block_size) * p.s_slot;
      new_tok = L - 1;
    }
  }
  // This lane's slice of the current row (attended at new_tok and written to
  // new_dst); loaded up front, so no K/V load waits on it.
  uint4 kcur = make_uint4(0, 0, 0, 0), vcur = make_uint4(0, 0, 0, 0);
  if (new_tok >= 0) {
    kcur = ld16(p.new_k + b * p.nk_sb + h * p.nk_sh + col * 16);
    vcur = ld16(p.new_v + b * p.nv_sb + h * p.nv_sh + col * 16);
  }

  // Qwen3 prologue: q and the current key are raw projections; normalise and
  // rotate them at the sequence's position (one head row per LPR lanes).
  if (p.has_pro) {
    int64_t pos = load_index(p.pro.pos, b, p.pro.pos_i64);
    pos = pos < 0 ? 0 : (pos >= p.pro.max_pos ? p.pro.max_pos - 1 : pos);
    float c[E], sn[E], w[E];
    load_rotary<E, LPR>(p.pro, pos, col, D, c, sn);
    load_weights<E>(p.pro.q_w, p.pro.w_dtype, col * E, w);
    const bool first_half = col < LPR / 2;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x[E];
      ET::unpack(qv[g], x);
      qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, c, sn, first_half);
      qv[g] = ET::pack(x);
    }
    if (new_tok >= 0) {
      load_weights<E>(p.pro.k_w, p.pro.w_dtype, col * E, w);
      float x[E];
      ET::unpack(kcur, x);
      qk_prologue<ET, LPR, E>(x, w, p.pro.eps, D, c, sn, first_half);
      kcur = ET::pack(x);
    }
  }

  constexpr bool kScaleAfter = ET::kBytes == 2;
  if constexpr (!kScaleAfter) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      qv[g].x = __float_as_uint(__uint_as_float(qv[g].x) * p.scale_log2);
      qv[g].y = __float_as_uint(__uint_as_float(qv[g].y) * p.scale_log2);
      qv[g].z = __float_as_uint(__uint_as_float(qv[g].z) * p.scale_log2);
      qv[g].w = __float_as_uint(__uint_as_float(qv[g].w) * p.scale_log2);
    }
  }


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
  // `mbits` the key_valid_mask bits of its rows; all were read before the
  // chunk group's first K/V load.  No loaded value is consumed here: a value
  // needed at a branch join makes the compiler wait for every outstanding
  // load (s_waitcnt vmcnt(0)), which would serialise the K/V traffic.
  // `valid` gets bit r for every attended row.
  auto load_chunk = [&](int k, int32_t cb, const int32_t* rbk, uint32_t mbits, uint4 (&kr)[NR],
                        uint4 (&vr)[NR], uint32_t& valid) {
    const int tb = start + (wave + NW * k) * kChunk;
    valid = 0;
    // Uniform: does this chunk hold the current row (read from new_k/new_v)?
    const bool has_cur = new_tok >= tb && new_tok < tb + kChunk;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int tok = tb + rg + r * RPL;
      const int32_t blk = kAligned ? cb : rbk[r];
      const bool ok = tok < end && blk >= 0 && blk < p.num_blocks && ((mbits >> r) & 1u);
      valid |= (ok ? 1u : 0u) << r;
      kr[r] = make_uint4(0, 0, 0, 0);
      vr[r] = make_uint4(0, 0, 0, 0);
      if (p.pool_off32 && !has_cur) {
        // 32-bit offsets from the pool bases: one VGPR per address.
        if (ok) {
          const uint32_t off = (uint32_t)blk * (uint32_t)p.s_blk +
                               (uint32_t)(tok % p.block_size) * (uint32_t)p.s_slot +
                               (uint32_t)head_off;
          kr[r] = ld16(p.kp + off);
          vr[r] = ld16(p.vp + off);
        }
      } else if (tok == new_tok) {
        // The current row comes from registers (also when it is masked, so
        // the store below always has it).
        kr[r] = kcur;
        vr[r] = vcur;
      } else if (ok) {
        const int64_t off =
            (int64_t)blk * p.s_blk + (int64_t)(tok % p.block_size) * p.s_slot + head_off;
        kr[r] = ld16(p.kp + off);
        vr[r] = ld16(p.vp + off);
      }
    }
  };

  // Fused write of the current row from its register copy (exactly one lane
  // group in the grid holds it).
  auto store_current_row = [&](int k, const uint4 (&kr)[NR], const uint4 (&vr)[NR]) {
    const int tb = start + (wave + NW * k) * kChunk;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (tb + rg + r * RPL == new_tok) {
        st16(p.kp + new_dst + head_off, kr[r]);
        st16(p.vp + new_dst + head_off, vr[r]);
      }
    }
  };

  auto process_chunk = [&](int k, const uint4 (&kr)[NR], const uint4 (&vr)[NR], uint32_t valid) {
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

  // CPW chunks per group: read their block ids (and mask bits) first, then
  // issue all their K/V loads, then reduce them in order.
  constexpr int kRbk = kAligned ? 1 : CPW * NR;
  for (int k0 = 0; k0 < my_chunks; k0 += CPW) {
    int32_t cb[CPW];
    int32_t rbk[kRbk];
    uint32_t mbits[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int k = k0 + j;
      const int c = wave + NW * k;
      const int tb = start + c * kChunk;
      cb[j] = 0;
      mbits[j] = (1u << NR) - 1;
      if (k >= my_chunks) continue;
      if constexpr (kAligned) {
        cb[j] = (k < 64 && c * kChunk < P) ? __builtin_amdgcn_readlane(tab, k)
                                          : (int32_t)table_entry(p, table_row, tb / p.block_size);
      } else {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int tok = tb + rg + r * RPL;
          rbk[j * NR + r] = tok < end ? (int32_t)table_entry(p, table_row, tok / p.block_size) : 0;
        }
      }
      if (p.valid != nullptr) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int tok = tb + rg + r * RPL;
          if (tok < end && tok < p.valid_len && p.valid[b * p.valid_sb + tok] == 0)
            mbits[j] &= ~(1u << r);
        }
      }
    }
    uint4 kr[CPW][NR], vr[CPW][NR];
    uint32_t valid[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (k0 + j < my_chunks) {
        load_chunk(k0 + j, cb[j], kAligned ? rbk : rbk + (kAligned ? 0 : j * NR), mbits[j], kr[j],
                   vr[j], valid[j]);
      } else {
        valid[j] = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) kr[j][r] = vr[j][r] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (k0 + j < my_chunks) {
        process_chunk(k0 + j, kr[j], vr[j], valid[j]);
        // After the chunk's reduction, so the store adds no wait in front of it.
        if (new_tok >= 0) store_current_row(k0 + j, kr[j], vr[j]);
      }
    }
  }

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
}

// Merge of the partitions of one (sequence, kv head) pair: out = sum_q
// 2^(m_q - M) o_q / sum_q 2^(m_q - M) l_q with M = max_q m_q.  Pairs that
// fit one partition were written by the first kernel and are skipped.
template <typename ET, int D, int G>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p) {
  constexpr int E = ET::kPerVec;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int L;
  if (p.lens_cum)
    L = (int)(load_index(p.lens, b + 1, p.lens_i64) - load_index(p.lens, b, p.lens_i64));
  else
    L = (int)load_index(p.lens, b, p.lens_i64);
  L = __builtin_amdgcn_readfirstlane(L);
  if (L <= 0) return;
  int nparts = (L + p.split_tokens - 1) / p.split_tokens;
  if (nparts > p.max_parts) nparts = p.max_parts;
  if (nparts <= 1) return;
  const int64_t pair = (int64_t)b * p.num_kv_heads + h;
  constexpr int kBatch = 8;  // partials whose loads are in flight together
  for (int idx = threadIdx.x; idx < G * D; idx += 256) {
    const int g = idx / D, d = idx % D;
    float M = kNegBig, Lt = 0.f, Ot = 0.f;
    for (int q0 = 0; q0 < nparts; q0 += kBatch) {
      float mq[kBatch], lq[kBatch], oq[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        mq[j] = kNegBig;
        lq[j] = 0.f;
        oq[j] = 0.f;
        if (q0 + j < nparts) {
          const int64_t slot = (pair * p.max_parts + q0 + j) * G + g;
          mq[j] = p.part_ml[slot * 2];
          lq[j] = p.part_ml[slot * 2 + 1];
          oq[j] = p.part_o[slot * D + d];
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const float Mn = fmaxf(M, mq[j]);
        const float a = fast_exp2(M - Mn), bq = fast_exp2(mq[j] - Mn);
        Lt = Lt * a + lq[j] * bq;
        Ot = Ot * a + oq[j] * bq;
        M = Mn;
      }
    }
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
  }
}

// ----------------------------------------------------------------- host side
// Longest context a sequence may be split into without growing the
// partition: beyond kMaxParts partitions the partition grows instead, which
// bounds the merge kernel's loop.
constexpr int kMaxParts = 256;

struct DecodePlan {
  int split_tokens;
  int max_parts;
  size_t ml_bytes, o_bytes, total_bytes;
};

template <typename ET, int D, int G>
static int decode_unit() {
  // one round of CPW chunks on every wave of a workgroup
  return DecodeShape<ET, D, G>::NW * DecodeShape<ET, D, G>::CPW * kChunk;
}

static int decode_unit_for(int dtype, int D, int G);

// Compute units of the current device (cached per device; 256, the MI355X
// count, when no device is visible, e.g. when only the workspace size is
// queried on a host without a GPU).
static int current_device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < 64) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

static DecodePlan plan_decode(const va_decode_args* a) {
  DecodePlan pl{};
  const int G = a->num_kv_heads > 0 ? a->num_heads / a->num_kv_heads : 1;
  int unit = decode_unit_for(a->dtype, a->head_dim, G);
  if (unit <= 0) unit = 128;
  const int max_len = a->max_seq_len > 0 ? a->max_seq_len : 1;
  int P = a->split_tokens;
  const int64_t pairs = (int64_t)a->num_seqs * a->num_kv_heads;
  if (P <= 0) {
    // Split contexts only as far as needed to give every CU one workgroup:
    // with at least as many (sequence, kv head) pairs as CUs, one partition
    // per pair.  Partitions are at least one round of in-flight chunks and
    // at most kMaxParts per context.
    const int64_t cus = current_device_cus();
    const int64_t want = pairs >= cus ? 1 : cus / (pairs > 0 ? pairs : 1);
    P = (int)((max_len + want - 1) / want);
    if (P < unit) P = unit;
    const int cap = (max_len + kMaxParts - 1) / kMaxParts;
    if (P < cap) P = cap;
  }
  P = ((P + unit - 1) / unit) * unit;
  if (P < unit) P = unit;
  pl.split_tokens = P;
  pl.max_parts = (max_len + P - 1) / P;
  if (pl.max_parts > 1) {
    pl.ml_bytes = ((size_t)pairs * pl.max_parts * G * 2 * 4 + 255) / 256 * 256;
    pl.o_bytes = (size_t)pairs * pl.max_parts * G * a->head_dim * 4;
  }
  pl.total_bytes = pl.ml_bytes + pl.o_bytes;
  return pl;
}

template <typename ET, int D, int G>
static void launch_decode(const DecodeParams& p, dim3 grid, hipStream_t s) {
  if (p.block_is_chunk_aligned)
    hipLaunchKernelGGL((paged_decode_kernel<ET, D, G, true>), grid,
                       dim3(DecodeShape<ET, D, G>::NW * 64), 0, s, p);
  else
    hipLaunchKernelGGL((paged_decode_kernel<ET, D, G, false>), grid,
                       dim3(DecodeShape<ET, D, G>::NW * 64), 0, s, p);
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

extern "C" int va_paged_decode(const va_decode_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_paged_decode: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_decode_args),
               "va_paged_decode: struct_size %u != %zu (header/library mismatch)", a->struct_size,
               sizeof(va_decode_args));
  const int eb = elem_bytes_of(a->dtype);
  VA_CHECK_ARG(eb != 0, "va_paged_decode: unknown dtype %d", a->dtype);
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
  VA_CHECK_ARG(a->table_width >= 0, "va_paged_decode: table_width < 0");
  const int64_t strides[] = {a->q_stride_seq,        a->q_stride_head,        a->out_stride_seq,
                             a->out_stride_head,     a->pool.stride_block,    a->pool.stride_slot,
                             a->pool.stride_head,    a->new_k_stride_seq,     a->new_k_stride_head,
                             a->new_v_stride_seq,    a->new_v_stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * eb) % 16 == 0, "va_paged_decode: strides must be 16-byte multiples");
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->out, (uintptr_t)a->pool.k,
                            (uintptr_t)a->pool.v, (uintptr_t)a->new_k, (uintptr_t)a->new_v};
  for (uintptr_t p : ptrs)
    VA_CHECK_ARG(p % 16 == 0, "va_paged_decode: pointers must be 16-byte aligned");

  const DecodePlan pl = plan_decode(a);
  if (pl.total_bytes > 0) {
    if (a->workspace == nullptr || a->workspace_bytes < pl.total_bytes) {
      set_error("va_paged_decode: workspace of %zu bytes needed, %zu given", pl.total_bytes,
                a->workspace_bytes);
      return VA_ERR_WORKSPACE;
    }
    VA_CHECK_ARG((uintptr_t)a->workspace % 16 == 0, "va_paged_decode: workspace alignment");
  }
  VA_CHECK_ARG(pl.max_parts <= 65535, "va_paged_decode: too many context partitions");

  DecodeParams p;
  p.q = (const char*)a->q;
  p.q_sb = a->q_stride_seq * eb;
  p.q_sh = a->q_stride_head * eb;
  p.out = (char*)a->out;
  p.o_sb = a->out_stride_seq * eb;
  p.o_sh = a->out_stride_head * eb;
  p.kp = (char*)a->pool.k;
  p.vp = (char*)a->pool.v;
  p.s_blk = a->pool.stride_block * eb;
  p.s_slot = a->pool.stride_slot * eb;
  p.s_head = a->pool.stride_head * eb;
  p.block_size = a->pool.block_size;
  p.num_blocks = a->pool.num_blocks;
  p.block_is_chunk_aligned = a->pool.block_size % kChunk == 0;
  {
    // Largest byte offset inside one pool: the last slot of the last head of
    // the last block, plus a row.
    const int64_t last = (int64_t)(a->pool.num_blocks > 0 ? a->pool.num_blocks - 1 : 0) *
                             a->pool.stride_block +
                         (int64_t)(a->pool.block_size - 1) * a->pool.stride_slot +
                         (int64_t)(a->num_kv_heads - 1) * a->pool.stride_head + a->head_dim;
    p.pool_off32 = last * eb < ((int64_t)1 << 32) && a->pool.stride_block >= 0 &&
                   a->pool.stride_slot >= 0 && a->pool.stride_head >= 0;
  }
  p.table = a->block_tables;
  p.t_sb = a->table_stride_seq;
  p.table_i64 = a->table_dtype == VA_I64;
  p.table_width = a->table_width;
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
  p.scale_log2 = a->scale * 1.4426950408889634f;
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
  switch (a->dtype) {
    case VA_BF16: ok = dispatch_d<BF16>(a->head_dim, G, p, grid, s); break;
    case VA_F16: ok = dispatch_d<F16>(a->head_dim, G, p, grid, s); break;
    case VA_F32: ok = dispatch_d<F32>(a->head_dim, G, p, grid, s); break;
  }
  if (!ok) {
    set_error("va_paged_decode: unsupported head_dim %d / group size %d (head_dim 64|128|256, "
              "group 1|2|4|8)",
              a->head_dim, G);
    return VA_ERR_UNSUPPORTED;
  }
  return check_launch("va_paged_decode");
}
