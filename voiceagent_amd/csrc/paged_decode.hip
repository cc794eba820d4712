// Paged-KV decode attention (one query token per sequence) for GQA, with
// split-context partitions merged inside the same launch.
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
// partition goes to wave c % NW and the next chunk's K/V loads are issued
// before the current chunk is reduced.  Scores are reduced over the row's
// lanes with DPP, the running max over row groups with cross-row permutes;
// softmax runs in the exp2 domain (q pre-scaled by scale * log2 e).  Waves
// merge through LDS; a sequence split into several partitions writes
// unnormalised partials (m, l, o) to the workspace, and the last workgroup
// to arrive (device-scope counter, reset by that workgroup) merges them and
// writes the output — no second launch.
#include "common.h"

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
  int64_t n_sb, n_sh;  // bytes
  const void* new_slots;
  int32_t new_slots_i64;
  int32_t num_kv_heads;
  int32_t split_tokens;
  int32_t max_parts;
  float scale_log2;
  int32_t* counters;
  float* part_ml;
  float* part_o;
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

// Per-configuration launch shape.  NW wavefronts per workgroup and CPW chunks
// whose K/V loads are in flight together per wave, sized so that the data
// registers (8 * NR per chunk) plus the query/accumulator state fit 128 VGPRs
// at NW = 16 (four waves per SIMD).
template <typename ET, int D, int G>
struct DecodeShape {
  static constexpr int E = ET::kPerVec;       // elements per 16-byte lane load
  static constexpr int LPR = D / E;           // lanes per K/V row
  static constexpr int RPL = 64 / LPR;        // rows per load instruction
  static constexpr int NR = kChunk / RPL;     // rows per lane per chunk
  static constexpr int CPW = (8 * NR >= 64) ? 1 : 64 / (8 * NR);
  static constexpr int NW = (2 * G * E + CPW * 8 * NR <= 96) ? 16 : 8;
};

template <typename ET, int D, int G>
__global__ __launch_bounds__((DecodeShape<ET, D, G>::NW * 64)) void paged_decode_kernel(
    DecodeParams p) {
  using S = DecodeShape<ET, D, G>;
  constexpr int E = S::E, LPR = S::LPR, RPL = S::RPL, NR = S::NR, CPW = S::CPW, NW = S::NW;
  static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "unsupported head_dim");
  static_assert(RPL <= kChunk, "unsupported head_dim");
  constexpr int NT = NW * 64;

  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ float s_o[NW][G][D];
  __shared__ int s_last;

  const int part = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
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
  if (p.block_is_chunk_aligned) {
    const int c = wave + NW * lane;
    const int tok = start + c * kChunk;
    if (c * kChunk < P) tab = (int)table_entry(p, table_row, tok / p.block_size);
  }
  float qv[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 u = ld16(p.q + b * p.q_sb + (int64_t)(h * G + g) * p.q_sh + col * 16);
    ET::unpack(u, qv[g]);
  }
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

#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < E; ++e) qv[g][e] *= p.scale_log2;

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

  // Issue the K/V loads of the wave's k-th chunk; `valid` gets bit r for every
  // attended row.
  auto load_chunk = [&](int k, uint4 (&kr)[NR], uint4 (&vr)[NR], uint32_t& valid) {
    const int c = wave + NW * k;
    const int tb = start + c * kChunk;
    int64_t chunk_blk = 0;
    if (p.block_is_chunk_aligned)
      chunk_blk = (k < 64 && c * kChunk < P) ? (int64_t)__builtin_amdgcn_readlane(tab, k)
                                             : table_entry(p, table_row, tb / p.block_size);
    valid = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int tok = tb + rg + r * RPL;
      bool ok = tok < end;
      int64_t blk = chunk_blk;
      if (!p.block_is_chunk_aligned && ok) blk = table_entry(p, table_row, tok / p.block_size);
      ok = ok && blk >= 0 && blk < p.num_blocks;
      if (ok && p.valid != nullptr && tok < p.valid_len)
        ok = p.valid[b * p.valid_sb + tok] != 0;
      // The current row is loaded (and later written) even when it is masked.
      if (ok || tok == new_tok) {
        const char* kaddr;
        const char* vaddr;
        if (tok == new_tok) {
          kaddr = p.new_k + b * p.n_sb + h * p.n_sh + col * 16;
          vaddr = p.new_v + b * p.n_sb + h * p.n_sh + col * 16;
        } else {
          const int64_t off = blk * p.s_blk + (int64_t)(tok % p.block_size) * p.s_slot + head_off;
          kaddr = p.kp + off;
          vaddr = p.vp + off;
        }
        kr[r] = ld16(kaddr);
        vr[r] = ld16(vaddr);
        valid |= (ok ? 1u : 0u) << r;
      } else {
        kr[r] = make_uint4(0, 0, 0, 0);
        vr[r] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  auto process_chunk = [&](int k, const uint4 (&kr)[NR], const uint4 (&vr)[NR], uint32_t valid) {
    // Fused write of the current row (exactly one lane group in the grid).
    if (new_tok >= 0) {
      const int tb = start + (wave + NW * k) * kChunk;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (tb + rg + r * RPL == new_tok) {
          st16(p.kp + new_dst + head_off, kr[r]);
          st16(p.vp + new_dst + head_off, vr[r]);
        }
      }
    }
    float s[NR][G];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float kf[E];
      ET::unpack(kr[r], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc = fmaf(qv[g][e], kf[e], acc);
        s[r][g] = acc;
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float t = group_sum<LPR>(s[r][g]);
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

  // CPW chunks per group: all their loads are issued before the first is reduced.
  for (int k0 = 0; k0 < my_chunks; k0 += CPW) {
    uint4 kr[CPW][NR], vr[CPW][NR];
    uint32_t valid[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (k0 + j < my_chunks) {
        load_chunk(k0 + j, kr[j], vr[j], valid[j]);
      } else {
        valid[j] = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) kr[j][r] = vr[j][r] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < CPW; ++j)
      if (k0 + j < my_chunks) process_chunk(k0 + j, kr[j], vr[j], valid[j]);
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
      __hip_atomic_store(p.part_o + slot * D + d, Ot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(p.part_ml + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.part_ml + slot * 2 + 1, Lt, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (nparts == 1) return;

  // Cross-workgroup merge: the last partition to finish combines all of them.
  // The partials above were written with device-scope stores, which write
  // through the per-XCD L2 to the device coherence point, and the merge below
  // reads them with device-scope loads, which do not hit stale L2 lines.  So
  // publishing only needs this workgroup's stores to have completed before
  // its counter increment (s_waitcnt 0 + barrier); a __threadfence() here
  // would instead write back the whole L2 of the XCD in every merging
  // workgroup, which measured ~6x slower on MI355X.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(p.counters + pair, 1);
    s_last = prev == nparts - 1;
  }
  __syncthreads();
  if (!s_last) return;

  constexpr int kBatch = 8;  // partials whose loads are in flight together
  for (int idx = tid; idx < G * D; idx += NT) {
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
          mq[j] = __hip_atomic_load(p.part_ml + slot * 2, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
          lq[j] = __hip_atomic_load(p.part_ml + slot * 2 + 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
          oq[j] = __hip_atomic_load(p.part_o + slot * D + d, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
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
  if (tid == 0) __hip_atomic_store(p.counters + pair, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------- host side
// Workgroups resident at once on the 256 CUs of an MI355X (one 16-wave
// workgroup per CU); the split aims to give every CU one workgroup.
constexpr int kDecodeTargetWorkgroups = 256;

struct DecodePlan {
  int split_tokens;
  int max_parts;
  size_t ml_bytes, o_bytes, total_bytes;
};

template <typename ET, int D, int G>
static int decode_unit() {
  return DecodeShape<ET, D, G>::NW * kChunk;  // one chunk per wave
}

static int decode_unit_for(int dtype, int D, int G);

static DecodePlan plan_decode(const va_decode_args* a) {
  DecodePlan pl{};
  const int G = a->num_kv_heads > 0 ? a->num_heads / a->num_kv_heads : 1;
  int unit = decode_unit_for(a->dtype, a->head_dim, G);
  if (unit <= 0) unit = 256;
  const int max_len = a->max_seq_len > 0 ? a->max_seq_len : 1;
  int P = a->split_tokens;
  if (P <= 0) {
    const int64_t pairs = (int64_t)a->num_seqs * a->num_kv_heads;
    int64_t want = (kDecodeTargetWorkgroups + pairs - 1) / (pairs > 0 ? pairs : 1);
    if (want < 1) want = 1;
    P = (int)((max_len + want - 1) / want);
  }
  P = ((P + unit - 1) / unit) * unit;
  if (P < unit) P = unit;
  pl.split_tokens = P;
  pl.max_parts = (max_len + P - 1) / P;
  const int64_t pairs = (int64_t)a->num_seqs * a->num_kv_heads;
  if (pl.max_parts > 1) {
    pl.ml_bytes = ((size_t)pairs * pl.max_parts * G * 2 * 4 + 255) / 256 * 256;
    pl.o_bytes = (size_t)pairs * pl.max_parts * G * a->head_dim * 4;
  }
  pl.total_bytes = pl.ml_bytes + pl.o_bytes;
  return pl;
}

template <typename ET, int D, int G>
static void launch_decode(const DecodeParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((paged_decode_kernel<ET, D, G>), grid,
                     dim3(DecodeShape<ET, D, G>::NW * 64), 0, s, p);
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
  VA_CHECK_ARG(a->num_seqs <= 65535, "va_paged_decode: num_seqs > 65535");
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
                             a->pool.stride_head,    a->new_stride_seq,       a->new_stride_head};
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
    const int64_t pairs = (int64_t)a->num_seqs * a->num_kv_heads;
    if (a->counters == nullptr || a->counters_len < pairs) {
      set_error("va_paged_decode: %lld zero-initialised counters needed, %lld given",
                (long long)pairs, (long long)a->counters_len);
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
  p.n_sb = a->new_stride_seq * eb;
  p.n_sh = a->new_stride_head * eb;
  p.new_slots = a->new_slots;
  p.new_slots_i64 = a->new_slots_dtype == VA_I64;
  p.num_kv_heads = a->num_kv_heads;
  p.split_tokens = pl.split_tokens;
  p.max_parts = pl.max_parts;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  char* ws = (char*)a->workspace;
  p.counters = pl.total_bytes ? a->counters : nullptr;
  p.part_ml = pl.total_bytes ? (float*)ws : nullptr;
  p.part_o = pl.total_bytes ? (float*)(ws + pl.ml_bytes) : nullptr;

  const dim3 grid(pl.max_parts, a->num_kv_heads, a->num_seqs);
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
