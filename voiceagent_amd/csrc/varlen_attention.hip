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
// Tiling (one workgroup = 4 wave64 = 256 lanes): an item is one
// (sequence, kv head, query block) with all G query heads of the kv group,
// so its 128 MFMA rows are BQ = 128 / G query positions x G heads.  Each wave
// owns two 16-row tiles.  Workgroups are persistent: the grid fills the
// GPU's workgroup slots once and each workgroup works through a list of
// items.  Keys stream through LDS in 64-key tiles (K and V row-major,
// 16-byte chunks XOR-swizzled by row against bank conflicts) over a ring of
// two stages filled by global_load_lds DMA, so one tile is in flight while
// one is reduced; the ring runs on from one item into the next.  Per tile:
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
// store copies an item's new K/V rows from the staged tiles to slot_mapping.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "fastdiv.h"
#include "prologue.h"

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
  int32_t num_seqs, num_kv_heads;
  FastDiv bs_div, hkv_div;  // block_size, num_kv_heads
  int32_t slot_small;       // num_blocks * block_size <= 2^31: slots divide in 32 bits
  float k_scale, v_scale;   // FP8 pool: element = code * scale
  int32_t kv_f8;            // the pool holds e4m3 codes (strides in bytes of codes)
  int32_t has_pro;          // the Qwen3 query prologue runs on every query row
  PrologueParams pro;
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
  // Two floats to a packed 16-bit pair, round to nearest even (bf16 through
  // gfx950's v_cvt_pk_bf16_f32).
  __device__ static inline uint32_t pack2(float lo, float hi) {
    if constexpr (kBF16) {
      bf16x2_t v;
      v.x = (__bf16)lo;
      v.y = (__bf16)hi;
      return __builtin_bit_cast(uint32_t, v);
    } else
      return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
  }
};

constexpr int kVarlenThreads = 256;
constexpr int kRowsPerWG = 128;
constexpr int kKeyTile = 64;
// Stages of the K/V ring: one tile streams in while one is reduced.
constexpr int kStages = 2;
// MI355X hands workgroup i of a launch to XCD i % 8; each XCD has its own L2.
constexpr int kXcds = 8;
// Lazy-rescale slack of the online softmax, in log2 units (p <= 2^kLazy).
constexpr float kLazy = 8.0f;

// 16 zero bytes: the DMA source of every lane whose key row is past the end
// of the visible keys or unmapped, so every tile takes the same number of
// DMA instructions (the pipeline's vmcnt waits count them).
__device__ __align__(16) const uint4 kZeroRow = {0u, 0u, 0u, 0u};

// LDS layout of a staged K or V tile: kKeyTile rows of 2 D bytes, unpadded;
// the 16-byte chunk c of row r sits at chunk position c ^ swz(r).  The XOR
// spreads the 16 rows of one K read (ds_read_b128, one chunk per row) and
// the 8 rows x 2 chunks of half a V read (ds_read_b64_tr_b16) over distinct
// banks.  swz depends on r % 16 only.
template <int D>
__device__ inline int swz(int row) {
  if constexpr (D == 128)
    return ((row & 7) << 1) | ((row >> 3) & 1);
  else
    return (((row >> 1) & 3) << 1) | ((row >> 3) & 1);
}

__device__ inline uint4 lds_read16(const char* base, int off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

__device__ inline s16x4_t lds_read_tr(const char* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(base + off));
}

// kPaged: keys j < k_len - q_len come from the pool through the block table
// (launches with a pool); otherwise every key comes from k/v.  kF8 (with
// kPaged): the pool holds OCP e4m3 codes.  A tile's pool rows are copied as
// codes into a code area of LDS and converted, at the top of the tile's
// step, into the 16-bit stage as code * scale rounded to the 16-bit type
// (every e4m3 value converts exactly; the product is rounded once), before
// the next tile's copy may reuse the code area.  Rows from k/v are staged
// as 16-bit rows, as without a pool.
//
// kPro: q holds raw projections; each item's query rows are normalised and
// rotated (Qwen3's q_norm + rotary_emb, prologue.h's arithmetic) in registers
// at the item's first tile, with positions loaded beside the rows.
template <bool kBF16, int D, int G, bool kCausal, bool kPaged, bool kOnce, bool kF8 = false,
          bool kPro = false>
__global__ __launch_bounds__(kVarlenThreads, 2) void varlen_attention_kernel(VarlenParams p) {
  constexpr int BQ = kRowsPerWG / G;       // query positions per workgroup
  constexpr int DS = D / 32;               // k-steps of the S^T MFMA
  constexpr int DT = D / 16;               // 16-wide d tiles of O^T
  constexpr int ROWB = D * 2;              // bytes per K/V row
  constexpr int CPR = ROWB / 16;           // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;            // rows per DMA instruction (1 KiB)
  constexpr int TILE_B = kKeyTile * ROWB;  // bytes of one K (or V) tile
  constexpr int NI = TILE_B / 1024 / 4;    // DMA instructions per wave per tile, K or V
  constexpr int KT = kKeyTile / 16;        // 16-key tiles per key tile
  constexpr int KS = kKeyTile / 32;        // 32-key MFMA steps per key tile
  static_assert(BQ % 16 == 0, "query block must hold whole 16-row tiles");
  static_assert(NI * 4 * 1024 == TILE_B, "tile DMA split");
  using M = Mma<kBF16>;

  // Two stages of (K tile, V tile): one streams in while the other is
  // reduced.
  static_assert(kStages == 2, "the tile loop alternates two stages");
  __shared__ __align__(1024) char s_kv[kStages * 2 * TILE_B];
  // FP8 pool: the codes of one tile's pool rows (K, then V), row-major and
  // unswizzled: row r's 16-code chunk c at r D + 16 c.
  static_assert(!kF8 || kPaged, "FP8 codes come from a pool");
  constexpr int CODE_B = kKeyTile * D;     // bytes of one tile of codes, K or V
  constexpr int CCPR = D / 16;             // 16-code chunks per code row
  constexpr int CRPI = 64 / CCPR;          // code rows per DMA instruction
  constexpr int NIC = CODE_B / 1024 / 4;   // code DMA instructions per wave per tile, K or V
  static_assert(!kF8 || NIC * 4 * 1024 == CODE_B, "code DMA split");
  __shared__ __align__(1024) char s_code[kF8 ? 2 * CODE_B : 16];
  // kPro: the query norm weights as fp32, written once per workgroup here and
  // read by every item's prologue (the first tile's barrier orders them).
  __shared__ __align__(16) float s_qw[kPro ? D : 4];
  using ET = std::conditional_t<kBF16, BF16, F16>;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  if constexpr (kPro) {
    for (int i = tid; i < D; i += kVarlenThreads) s_qw[i] = load_weight(p.pro.q_w, p.pro.w_dtype, i);
  }

  // ---- persistent schedule ----
  // Workgroup 8 j + x runs on XCD x (MI355X hands workgroup i of a launch to
  // XCD i % 8, and each XCD has its own L2) and takes items from XCD x's
  // list: the query blocks of pairs x, x + 8, ... (pair = sequence *
  // num_kv_heads + kv head), so the blocks that share a pair's K/V rows
  // share one L2.  The list is level-major: every pair's last block, then
  // every pair's second to last, ... (late blocks are the heavy ones under
  // causal masking).  It is dealt to the XCD's nslots workgroups in snake
  // order: in round r workgroup j takes item r nslots + j when r is even and
  // r nslots + nslots - 1 - j when r is odd, which evens out the sums of a
  // list sorted heavy first.  A workgroup keeps its K/V ring running from
  // one item into the next: the next item's first tile, query rows and store
  // slots are loading while the current item's last tile is reduced.
  const int nqb = p.num_qblocks;
  // kOnce: one query block per sequence (the host launches it for the
  // encoder's windows), so every K/V row is read by one item only and the
  // tiles stream in non-temporally (config 4: 16.2 -> 15.5 us).  Otherwise a
  // pair's later blocks re-read them from L2, which the default policy keeps
  // them in (non-temporal there: config 3's prefill 40.6 -> 45.3 us).
  constexpr bool kv_once = kOnce;
  const int npairs = p.num_seqs * p.num_kv_heads;
  const int xcd = (int)blockIdx.x % kXcds;
  const int wslot = (int)blockIdx.x / kXcds;
  const int nslots = (int)gridDim.x / kXcds;
  const int ppx = (npairs - xcd + kXcds - 1) / kXcds;  // pairs on this XCD
  // With at most 64 pairs per XCD (lane_pairs), lane k holds pair k's
  // query and key ranges and the list is walked with wave ballots, no memory
  // access per item.  Otherwise the list holds every (pair, block), blocks
  // past a sequence's end are skipped, and lane k holds the ranges of this
  // workgroup's item 64 i + k (refilled every 64 items).
  const bool lane_pairs = ppx <= 64;
  int lq0 = 0, lql = 0, lk0 = 0, lkl = 0, lnq = 0, lpair = 0;
  auto load_ranges = [&](int pair) {
    const int ls = (int)fast_div((uint32_t)pair, p.hkv_div);
    lq0 = p.cu_q[ls];
    lql = p.cu_q[ls + 1] - lq0;
    lk0 = p.cu_k[ls];
    lkl = p.cu_k[ls + 1] - lk0;
  };
  const int64_t total = (int64_t)ppx * nqb;  // list length without lane_pairs
  auto item_index = [&](int r) -> int64_t {  // list index of this workgroup's round r
    return (int64_t)r * nslots + ((r & 1) ? nslots - 1 - wslot : wslot);
  };
  auto refill = [&](int r0) {
    const int64_t li = item_index(r0 + lane);
    lnq = -1;
    if (li < total) {
      const int li32 = (int)li;  // list indices stay below 2^31 (host check)
      lpair = xcd + kXcds * (li32 % ppx);
      lnq = nqb - 1 - li32 / ppx;  // the item's query block
      load_ranges(lpair);
    }
  };
  if (lane_pairs) {
    if (lane < ppx) {
      load_ranges(xcd + kXcds * lane);
      lnq = (lql + BQ - 1) / BQ;
    }
  } else {
    refill(0);
  }

  struct Item {
    int h, qb, q0, ql, k0, kl;
    int pos0, pos_end, diag, pool_prefix, kend, ntiles;
    int64_t new_base, table_row;
  };
  int round = 0;                         // this workgroup's next round
  int lev = nqb - 1, cum = 0;            // lane_pairs walk: level and items above it
  auto next_item = [&](Item& it) -> bool {
    int ksel, qb;
    if (lane_pairs) {
      const int64_t li = item_index(round);
      // Levels are walked downwards once over the workgroup's life: the
      // list indices of its rounds increase.
      int cnt = 0;
      while (lev >= 0) {
        cnt = __popcll(__builtin_amdgcn_ballot_w64(lnq > lev));
        if (li < cum + cnt) break;
        cum += cnt;
        --lev;
      }
      if (lev < 0) return false;
      ++round;
      const int rem = (int)(li - cum);
      const uint64_t live = __builtin_amdgcn_ballot_w64(lnq > lev);
      const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(live >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)live, 0));
      ksel = __builtin_ctzll(__builtin_amdgcn_ballot_w64(lnq > lev && below == rem));
      qb = lev;
      const int pair = xcd + kXcds * ksel;
      it.h = (int)fast_mod((uint32_t)pair, p.hkv_div);
    } else {
      for (;;) {
        if (item_index(round) >= total) return false;
        if (round > 0 && (round & 63) == 0) refill(round);
        ksel = round & 63;
        ++round;
        qb = __builtin_amdgcn_readlane(lnq, ksel);
        if (qb * BQ < __builtin_amdgcn_readlane(lql, ksel)) break;  // else past the end
      }
      it.h = (int)fast_mod((uint32_t)__builtin_amdgcn_readlane(lpair, ksel), p.hkv_div);
    }
    const int pair = lane_pairs ? xcd + kXcds * ksel : __builtin_amdgcn_readlane(lpair, ksel);
    const int s = (int)fast_div((uint32_t)pair, p.hkv_div);
    it.qb = qb;
    it.q0 = __builtin_amdgcn_readlane(lq0, ksel);
    it.ql = __builtin_amdgcn_readlane(lql, ksel);
    it.k0 = __builtin_amdgcn_readlane(lk0, ksel);
    it.kl = __builtin_amdgcn_readlane(lkl, ksel);
    it.pos0 = qb * BQ;
    it.pos_end = min(it.ql, it.pos0 + BQ);
    it.diag = it.kl - it.ql;  // bottom-right alignment offset
    it.pool_prefix = kPaged ? (p.k != nullptr ? it.kl - it.ql : it.kl) : 0;
    it.kend = kCausal ? max(0, min(it.kl, it.diag + it.pos_end)) : it.kl;
    it.ntiles = (it.kend + kKeyTile - 1) / kKeyTile;
    // Keys from k/v: key j is row new_base + j of k and v.
    it.new_base = kPaged ? (int64_t)it.q0 - it.pool_prefix : (int64_t)it.k0;
    it.table_row = (int64_t)s * p.t_sb;
    return true;
  };

  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)s_kv);
  const uint32_t code_base = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)s_code);

  // ---- DMA of key tile [kb, kb + 64) into stage st ----
  // (h, pool_prefix, kend, new_base, table_row) are the item's; all uniform.
  // Wave w fills 1 KiB blocks w NI .. w NI + NI - 1 of the K and V tiles;
  // lane l of a block writes row RPI * block + l / CPR, chunk position l % CPR,
  // so it reads logical chunk (l % CPR) ^ swz(row) of that key.  Every lane
  // issues exactly 2 NI DMAs per tile.
  uint32_t koff[NI], voff[NI];  // per-lane byte offsets inside a tile of k/v rows
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (wave * NI + i) * RPI + lane / CPR;
    const int chunk = (lane % CPR) ^ swz<D>(row);
    koff[i] = (uint32_t)(row * p.k_st + chunk * 16);
    voff[i] = (uint32_t)(row * p.v_st + chunk * 16);
  }
  const char* zero_row = reinterpret_cast<const char*>(&kZeroRow);
  auto issue_tile = [&](int h, int pool_prefix, int kend, int64_t new_base, int64_t table_row,
                        int kb, int st) {
    const uint32_t dst0 = lds_base + (uint32_t)(st * 2 * TILE_B + wave * NI * 1024);
    if (kb >= pool_prefix && kb + kKeyTile <= kend) {
      // Whole tile from k/v: uniform bases, constant lane offsets.
      const char* kbase = uniform_ptr(p.k + (new_base + kb) * p.k_st + h * p.k_sh);
      const char* vbase = uniform_ptr(p.v + (new_base + kb) * p.v_st + h * p.v_sh);
      if constexpr (kv_once) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          dma16_nt(koff[i], kbase, dst0 + i * 1024);
          dma16_nt(voff[i], vbase, dst0 + TILE_B + i * 1024);
        }
      } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          dma16(koff[i], kbase, dst0 + i * 1024);
          dma16(voff[i], vbase, dst0 + TILE_B + i * 1024);
        }
      }
      return;
    }
    // Tile with pool keys or past kend: per-lane addresses; rows past kend
    // or with an unmapped block read kZeroRow.  The lane's first row is
    // made opaque so that the per-lane address arithmetic stays here
    // instead of being hoisted out of the tile loop into live registers.
    // Block ids are loaded as raw words and widened after the last load, and
    // every address is formed before the first DMA: a register still
    // awaiting its load when a DMA has been issued would make the compiler's
    // wait for it also wait for that DMA.
    int row0 = wave * NI * RPI + lane / CPR;
    asm volatile("" : "+v"(row0));
    uint2 braw[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) braw[i] = make_uint2(0u, 0u);
    if (kPaged && !kF8 && kb < pool_prefix) {
      int64_t e[NI];
      bool ok[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int j = kb + row0 + i * RPI;
        const int col = (int)fast_div((uint32_t)j, p.bs_div);
        ok[i] = j < pool_prefix && j < kend && col < p.table_width;
        e[i] = table_row + col;
      }
      if (p.table_i64) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (ok[i]) braw[i] = reinterpret_cast<const uint2*>(p.table)[e[i]];
      } else {
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (ok[i]) braw[i].x = reinterpret_cast<const uint32_t*>(p.table)[e[i]];
      }
    }
    // FP8 pool: the tile's pool rows as codes.  Lane l of code instruction i
    // copies chunk l % CCPR of code row (wave NIC + i) CRPI + l / CCPR.
    const char* kc[kF8 ? NIC : 1];
    const char* vc[kF8 ? NIC : 1];
    if constexpr (kF8) {
#pragma unroll
      for (int i = 0; i < NIC; ++i) {
        kc[i] = zero_row;
        vc[i] = zero_row;
      }
      if (kb < pool_prefix) {
        int crow0 = wave * NIC * CRPI + lane / CCPR;
        asm volatile("" : "+v"(crow0));
        uint2 craw[NIC];
        bool cok[NIC];
        int64_t ce[NIC];
#pragma unroll
        for (int i = 0; i < NIC; ++i) {
          const int j = kb + crow0 + i * CRPI;
          const int col = (int)fast_div((uint32_t)j, p.bs_div);
          cok[i] = j < pool_prefix && j < kend && col < p.table_width;
          ce[i] = table_row + col;
          craw[i] = make_uint2(0u, 0u);
        }
        if (p.table_i64) {
#pragma unroll
          for (int i = 0; i < NIC; ++i)
            if (cok[i]) craw[i] = reinterpret_cast<const uint2*>(p.table)[ce[i]];
        } else {
#pragma unroll
          for (int i = 0; i < NIC; ++i)
            if (cok[i]) craw[i].x = reinterpret_cast<const uint32_t*>(p.table)[ce[i]];
        }
        // As for 16-bit rows: a column at or past the table width keeps
        // block id 0 (read as block 0, the TTS padding semantics).
#pragma unroll
        for (int i = 0; i < NIC; ++i) {
          const int j = kb + crow0 + i * CRPI;
          const int64_t bid = p.table_i64 ? (int64_t)(((uint64_t)craw[i].y << 32) | craw[i].x)
                                          : (int64_t)(int32_t)craw[i].x;
          if (j < pool_prefix && j < kend && bid >= 0 && bid < p.num_blocks) {
            const int64_t off = bid * p.s_blk +
                                (int64_t)fast_mod((uint32_t)j, p.bs_div) * p.s_slot +
                                h * p.s_head + (lane % CCPR) * 16;
            kc[i] = p.kp + off;
            vc[i] = p.vp + off;
          }
        }
      }
    }
    const char* ka[NI];
    const char* va_[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = row0 + i * RPI;
      const int chunk = (lane % CPR) ^ swz<D>(row);
      const int j = kb + row;
      ka[i] = zero_row;
      va_[i] = zero_row;
      if (j < kend) {
        if (kPaged && j < pool_prefix) {
          // An FP8 pool row is staged by the code copy and its conversion.
          if constexpr (kF8) continue;
          const int64_t bid = p.table_i64 ? (int64_t)(((uint64_t)braw[i].y << 32) | braw[i].x)
                                          : (int64_t)(int32_t)braw[i].x;
          if (bid >= 0 && bid < p.num_blocks) {
            const int64_t off = bid * p.s_blk + (int64_t)fast_mod((uint32_t)j, p.bs_div) * p.s_slot +
                                h * p.s_head + chunk * 16;
            ka[i] = p.kp + off;
            va_[i] = p.vp + off;
          }
        } else {
          ka[i] = p.k + (new_base + j) * p.k_st + h * p.k_sh + chunk * 16;
          va_[i] = p.v + (new_base + j) * p.v_st + h * p.v_sh + chunk * 16;
        }
      }
    }
    if constexpr (kv_once) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        dma16_nt(ka[i], dst0 + i * 1024);
        dma16_nt(va_[i], dst0 + TILE_B + i * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        dma16(ka[i], dst0 + i * 1024);
        dma16(va_[i], dst0 + TILE_B + i * 1024);
      }
    }
    if constexpr (kF8) {
      if (kb < pool_prefix) {
        const uint32_t cdst = code_base + (uint32_t)(wave * NIC * 1024);
#pragma unroll
        for (int i = 0; i < NIC; ++i) {
          dma16(kc[i], cdst + i * 1024);
          dma16(vc[i], cdst + CODE_B + i * 1024);
        }
      }
    }
  };

  // ---- query rows and store slots of an item ----
  // Two 16-row tiles per wave: row 16 (2 wave + tt) + r16 of the block is
  // query position pos0 + row % BQ of head h G + row / BQ.
  uint4 qreg[2][DS];
  // kPro: the rotary position of each of the lane's two query rows (the row
  // of the item's last query for rows past the end, whose output is unused).
  int64_t qrot[2] = {0, 0};
  auto load_q = [&](const Item& it) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int row = 16 * (2 * wave + tt) + r16;
      const int qpos = it.pos0 + row % BQ;
      const int qhead = it.h * G + row / BQ;
      if constexpr (kPro)
        qrot[tt] = load_index(p.pro.pos, (int64_t)it.q0 + (qpos < it.ql ? qpos : it.ql - 1),
                              p.pro.pos_i64);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        if (qpos < it.ql)
          qreg[tt][ds] = ld16(p.q + (int64_t)(it.q0 + qpos) * p.q_st +
                              (int64_t)qhead * p.q_sh + (32 * ds + 8 * g4) * 2);
        else
          qreg[tt][ds] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  // Fused store: the item's new rows are keys [pool_prefix + pos0,
  // pool_prefix + pos_end), which the tile loop stages in LDS anyway: each is
  // copied from there to its slot, so k/v are read once.  The block's rows
  // are BQ x CPR 16-byte chunks, e = row CPR + chunk; store step k of wave w
  // takes e = 256 k + 64 w + lane, so each step writes RPS = 64 / CPR whole
  // rows of K and the same rows of V.  Lane j < NSTEP RPS of a wave loads
  // the slot of the wave's row j (step j / RPS, row j % RPS of the step), and
  // a store step reads the slots it needs from those lanes.  The slot is
  // loaded with the item's query rows, as the raw 32-bit word(s) of the
  // mapping (all ones for no row), and widened only where it is used, once
  // the tile holding the row has landed: widening at the load would wait for
  // it there, behind the tile DMA just issued.
  constexpr int RPS = 64 / CPR;  // rows per store step
  constexpr int NSTEP = (BQ * CPR + kVarlenThreads - 1) / kVarlenThreads;
  static_assert(NSTEP * RPS <= 64, "one slot lane per row");
  const bool fused_store = kPaged && p.slots != nullptr;
  auto st_base = [&](int k) {  // first block row of store step k (BQ: none)
    const int e0 = k * kVarlenThreads + 64 * wave;
    return e0 < BQ * CPR ? e0 / CPR : BQ;
  };
  const int st_row = lane < NSTEP * RPS ? min(st_base(lane / RPS) + lane % RPS, BQ) : BQ;
  auto load_slot = [&](const Item& it) -> uint2 {
    uint2 raw = make_uint2(~0u, ~0u);
    if (fused_store && it.pos0 + st_row < it.pos_end) {
      const int64_t i = (int64_t)it.q0 + it.pos0 + st_row;
      if (p.slot_i64)
        raw = reinterpret_cast<const uint2*>(p.slots)[i];
      else
        raw.x = reinterpret_cast<const uint32_t*>(p.slots)[i];
    }
    return raw;
  };

  // Swizzled chunk positions of this lane's reads (row % 16 is fixed per lane).
  const int kswz = swz<D>(r16);
  const int vswz = swz<D>(4 * g4 + (r16 >> 2));

  Item cur, nxt;
  if (!next_item(cur)) return;
  if (cur.ntiles > 0)
    issue_tile(cur.h, cur.pool_prefix, cur.kend, cur.new_base, cur.table_row, 0, 0);
  load_q(cur);
  uint2 st_slot = load_slot(cur);
  int stage = 0;  // stage holding the current item's next tile to reduce

  for (;;) {
    const bool has_next = next_item(nxt);

    int qpos[2], qhead[2], lim[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int row = 16 * (2 * wave + tt) + r16;
      qhead[tt] = cur.h * G + row / BQ;
      qpos[tt] = cur.pos0 + row % BQ;
      // Visible keys per row: j < lim[tt].  Rows past the end of the
      // sequence have zero queries; their outputs are never written.
      lim[tt] = kCausal ? min(cur.kend, cur.diag + qpos[tt] + 1) : cur.kend;
    }
    // Tiles ending at or below lim_lo (the smallest limit in the block) need
    // no mask.
    const int lim_lo = kCausal ? min(cur.kend, cur.diag + cur.pos0 + 1) : cur.kend;
    const int st_key0 = cur.pool_prefix + cur.pos0;  // key of the block's first row

    float m[2] = {-1.0e30f, -1.0e30f};
    float l[2] = {0.f, 0.f};
    f32x4_t o[2][DT];
    // With the query prologue the accumulators are zeroed after it, at the
    // item's first tile, so they hold no registers while it runs.
    if constexpr (!kPro) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[tt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    for (int t = 0; t < cur.ntiles; ++t) {
      const int kb = t * kKeyTile;
      // Tile t (and, in order, everything issued before it) has landed once
      // nothing is pending; the barrier makes every wave's part of it
      // visible and tells that every wave is done with the other stage,
      // which then takes the next tile: this item's tile t + 1, or the next
      // item's first tile.
      wait_vmcnt<0>();
      __syncthreads();
      // The query rows and slot were loaded before the wait: make the
      // compiler's own wait for them fall here, before the next DMA, where
      // it is free (a later wait would also stall on that DMA).
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
          asm volatile("" ::"v"(qreg[tt][ds].x), "v"(qreg[tt][ds].y), "v"(qreg[tt][ds].z),
                       "v"(qreg[tt][ds].w));
      asm volatile("" ::"v"(st_slot.x), "v"(st_slot.y));
      // Qwen3 query prologue on the item's rows, in the B-operand layout:
      // lane (r16, g4) holds elements 32 ds + 8 g4 + e of its row (ds < DS,
      // e < 8), so element i < D/2 and its rotary partner i + D/2 sit in the
      // same lane (ds and ds + DS/2), and a row's sum of squares is the sum
      // over the four lanes r16 + 16 g4.  It runs before the next tile is
      // requested: the compiler's wait for the cos / sin loads would
      // otherwise also wait for that request.  Both rows' cos / sin are
      // requested together (one round trip per item), into the registers
      // the output accumulators take after this block; the weights come
      // from LDS.
      if constexpr (kPro) {
        if (t == 0) {
          static_assert(DS % 2 == 0, "rotary halves");
          constexpr int HD = DS / 2;
          f32x4_t cv[2][HD][2], sv[2][HD][2];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            int64_t P = qrot[tt];
            P = P < 0 ? 0 : (P >= p.pro.max_pos ? p.pro.max_pos - 1 : P);
            const float* crow = p.pro.cs + P * p.pro.cs_stride;
#pragma unroll
            for (int hh = 0; hh < HD; ++hh)
#pragma unroll
              for (int e4 = 0; e4 < 2; ++e4) {
                cv[tt][hh][e4] = *reinterpret_cast<const f32x4_t*>(crow + 32 * hh + 8 * g4 + 4 * e4);
                sv[tt][hh][e4] =
                    *reinterpret_cast<const f32x4_t*>(crow + D / 2 + 32 * hh + 8 * g4 + 4 * e4);
              }
          }
          // One row at a time, each called with a constant row index so that
          // qreg and the factors stay in registers.
          auto pro_row = [&](auto TT) {
            constexpr int tt = decltype(TT)::value;
            float x[DS][8];
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) ET::unpack(qreg[tt][ds], x[ds]);
            // The sum of squares in va_qk_norm_rope's order, so that the
            // queries come out bit for bit as that kernel's do: there a lane
            // holds one 8-element chunk c of the row (a fused multiply-add
            // chain) and the 16 chunk sums meet in the tree
            // ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)) + ...  Here
            // chunk c = 4 ds + g4 sits in lane g4 at ds: pairs (g4, g4 ^ 1)
            // are lanes l, l ^ 16, quads lanes l ^ 32, and the rest is in
            // the lane.
            static_assert(DS == 4, "the standalone kernel's tree for head_dim 128");
            float cs4[DS];
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
              cs4[ds] = 0.f;
#pragma unroll
              for (int e = 0; e < 8; ++e) cs4[ds] = fmaf(x[ds][e], x[ds][e], cs4[ds]);
              cs4[ds] = sum_xor16(cs4[ds]);
              cs4[ds] = sum_xor32(cs4[ds]);
            }
            const float ss = (cs4[0] + cs4[1]) + (cs4[2] + cs4[3]);
            const float r = 1.0f / sqrtf(__fadd_rn(ss / (float)D, p.pro.eps));
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
#pragma unroll
              for (int e = 0; e < 8; ++e) x[ds][e] = __fmul_rn(x[ds][e], r);
              round_to<ET>(x[ds]);
              const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(s_qw + 32 * ds + 8 * g4);
              const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(s_qw + 32 * ds + 8 * g4 + 4);
#pragma unroll
              for (int e = 0; e < 8; ++e) x[ds][e] = __fmul_rn(x[ds][e], e < 4 ? w0[e] : w1[e - 4]);
              round_to<ET>(x[ds]);
            }
            {
              // Products rounded apart before their sum (no fused multiply-add).
#pragma clang fp contract(off)
#pragma unroll
              for (int hh = 0; hh < HD; ++hh)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  const float c = e < 4 ? cv[tt][hh][0][e] : cv[tt][hh][1][e - 4];
                  const float sn = e < 4 ? sv[tt][hh][0][e] : sv[tt][hh][1][e - 4];
                  const float a = x[hh][e], b2 = x[hh + HD][e];
                  x[hh][e] = a * c - b2 * sn;
                  x[hh + HD][e] = b2 * c + a * sn;
                }
            }
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
#pragma unroll
              for (int e = 0; e < 8; ++e) pin(x[ds][e]);  // pack the fp32 sums
              qreg[tt][ds] = ET::pack(x[ds]);
            }
          };
          pro_row(std::integral_constant<int, 0>{});
          pro_row(std::integral_constant<int, 1>{});
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[tt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
      // FP8 pool: convert this tile's pool rows from the code area into the
      // stage (16-byte chunks at their swizzled positions), then free the
      // code area for the next tile's copy below.
      if constexpr (kF8) {
        if (kb < cur.pool_prefix) {
          char* const s_kt = s_kv + stage * 2 * TILE_B;
          for (int e = tid; e < 2 * kKeyTile * CCPR; e += kVarlenThreads) {
            const int is_v = e >= kKeyTile * CCPR ? 1 : 0;
            const int rc = e - is_v * kKeyTile * CCPR;
            const int r = rc / CCPR, c = rc % CCPR;
            if (kb + r < cur.pool_prefix) {
              const uint4 codes = lds_read16(s_code + is_v * CODE_B, r * D + c * 16);
              const float sc = is_v ? p.v_scale : p.k_scale;
              char* const dst = s_kt + is_v * TILE_B + r * ROWB;
              float f[8];
              ET::unpack(f8_dequant8<ET>(make_uint2(codes.x, codes.y)), f);
#pragma unroll
              for (int i = 0; i < 8; ++i) f[i] *= sc;
              *reinterpret_cast<uint4*>(dst + (((2 * c) ^ swz<D>(r)) << 4)) = ET::pack(f);
              ET::unpack(f8_dequant8<ET>(make_uint2(codes.z, codes.w)), f);
#pragma unroll
              for (int i = 0; i < 8; ++i) f[i] *= sc;
              *reinterpret_cast<uint4*>(dst + (((2 * c + 1) ^ swz<D>(r)) << 4)) = ET::pack(f);
            }
          }
          wait_lgkmcnt0();
          __syncthreads();
        }
      }
      // The next tile (this item's tile t + 1, or the next item's first)
      // goes to the other stage.  A whole tile from k/v is issued in NI
      // pairs spread over the S^T loop below: issued back to back, its DMAs
      // stall the wave on the vector memory queue for as long as the
      // MFMAs of half a tile take.  Other tiles are issued here.
      const bool same = t + 1 < cur.ntiles;
      const bool next_tile = same || (has_next && nxt.ntiles > 0);
      const int n_h = same ? cur.h : nxt.h;
      const int n_prefix = same ? cur.pool_prefix : nxt.pool_prefix;
      const int n_kend = same ? cur.kend : nxt.kend;
      const int64_t n_base = same ? cur.new_base : nxt.new_base;
      const int n_kb = same ? kb + kKeyTile : 0;
      const bool spread = next_tile && n_kb >= n_prefix && n_kb + kKeyTile <= n_kend;
      const char* n_kbase = nullptr;
      const char* n_vbase = nullptr;
      if (spread) {
        n_kbase = uniform_ptr(p.k + (n_base + n_kb) * p.k_st + n_h * p.k_sh);
        n_vbase = uniform_ptr(p.v + (n_base + n_kb) * p.v_st + n_h * p.v_sh);
      } else if (next_tile) {
        issue_tile(n_h, n_prefix, n_kend, n_base, same ? cur.table_row : nxt.table_row, n_kb,
                   stage ^ 1);
      }
      const uint32_t n_dst = lds_base + (uint32_t)((stage ^ 1) * 2 * TILE_B + wave * NI * 1024);
      const char* s_k = s_kv + stage * 2 * TILE_B;
      const char* s_v = s_k + TILE_B;

      // Store steps run only on tiles that hold some of the block's new rows.
      // The rows go out non-temporally: nothing in the launch reads them back
      // (config 3: 40.4 -> 39.6 us per launch).
      if (fused_store && st_key0 < kb + kKeyTile &&
          st_key0 + (cur.pos_end - cur.pos0) > kb) {
        const int64_t cap = (int64_t)p.num_blocks * p.block_size;
        const int c = lane % CPR;
#pragma unroll 4
        for (int k = 0; k < NSTEP; ++k) {
          const int holder = k * RPS + lane / CPR;
          const uint32_t sx = (uint32_t)__shfl((int)st_slot.x, holder, 64);
          const uint32_t sy = (uint32_t)__shfl((int)st_slot.y, holder, 64);
          const int64_t slot = p.slot_i64 ? (int64_t)(((uint64_t)sy << 32) | sx)
                                          : (int64_t)(int32_t)sx;
          const int row = st_base(k) + lane / CPR;
          const int key = st_key0 + row;
          if (row < BQ && slot >= 0 && slot < cap && key >= kb && key < kb + kKeyTile) {
            const int64_t blk = p.slot_small ? (int64_t)fast_div((uint32_t)slot, p.bs_div)
                                             : slot / p.block_size;
            const int64_t dst = blk * p.s_blk + (slot - blk * p.block_size) * p.s_slot +
                                cur.h * p.s_head + c * 16;
            const int r = key - kb;
            const int off = r * ROWB + ((c ^ swz<D>(r)) << 4);
            st16_nt(p.kp + dst, lds_read16(s_k, off));
            st16_nt(p.vp + dst, lds_read16(s_v, off));
          }
        }
      }

      // ---- S^T = K Q^T for both row tiles ----
      // K rows of 16-key group kt + 1 are read before group kt's DMA pair:
      // no LDS read moves across a DMA.
      static_assert(KT % NI == 0 || NI % KT == 0, "DMA pairs spread evenly over the key groups");
      constexpr int PAIRS = NI >= KT ? NI / KT : 1;  // DMA pairs after each chosen group
      constexpr int EVERY = NI >= KT ? 1 : KT / NI;  // every EVERY-th group gets them
      f32x4_t sacc[2][KT];
      uint4 ka[2][DS];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        ka[0][ds] = lds_read16(s_k, r16 * ROWB + (((4 * ds + g4) ^ kswz) << 4));
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT) {
#pragma unroll
          for (int ds = 0; ds < DS; ++ds)
            ka[(kt + 1) & 1][ds] =
                lds_read16(s_k, (16 * (kt + 1) + r16) * ROWB + (((4 * ds + g4) ^ kswz) << 4));
        }
        sacc[0][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        sacc[1][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          sacc[0][kt] = M::mfma(ka[kt & 1][ds], qreg[0][ds], sacc[0][kt]);
          sacc[1][kt] = M::mfma(ka[kt & 1][ds], qreg[1][ds], sacc[1][kt]);
        }
        if (spread && kt % EVERY == 0) {
#pragma unroll
          for (int j = 0; j < PAIRS; ++j) {
            const int i = (kt / EVERY) * PAIRS + j;
            if constexpr (kv_once) {
              dma16_nt(koff[i], n_kbase, n_dst + i * 1024);
              dma16_nt(voff[i], n_vbase, n_dst + TILE_B + i * 1024);
            } else {
              dma16(koff[i], n_kbase, n_dst + i * 1024);
              dma16(voff[i], n_vbase, n_dst + TILE_B + i * 1024);
            }
          }
        }
      }
      // The query rows are dead now: on the item's last tile, start the next
      // item's loads.  Its store slot goes straight into st_slot (this item's
      // store steps ran at the top of this tile): a copy at the item's end
      // would have to wait for the load, and with it for every store issued
      // after it.
      if (t + 1 == cur.ntiles && has_next) {
        load_q(nxt);
        st_slot = load_slot(nxt);
      }

      // ---- online softmax (exp2 domain) and P^T packing ----
      // Scores stay unscaled until the exponent: p = 2^(s c - m) with
      // c = scale log2 e > 0 and m the row's running max of s c.  The max used
      // as reference is raised only when a row's new max exceeds it by more
      // than kLazy (or on the first scores); in between, p <= 2^kLazy, which
      // the fp32 sums and 16-bit P hold exactly as well.  Key masking is
      // applied only on tiles that cross a row's limit.
      const bool need_mask = kb + kKeyTile > lim_lo;
      uint4 pb[2][KS];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float sv[KT][4];
        if (need_mask) {
          const int rel = lim[tt] - kb - 4 * g4;  // key 16 kt + i of this lane is visible iff < rel
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[kt][i] = 16 * kt + i < rel ? sacc[tt][kt][i] : -INFINITY;
        } else {
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[kt][i] = sacc[tt][kt][i];
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[kt][i]);
        mx = max_xor16(mx);
        mx = max_xor32(mx);
        const float mxs = mx * p.scale_log2;
        if (__builtin_amdgcn_ballot_w64(mxs > m[tt] + kLazy) != 0) {
          const float mnew = fmaxf(m[tt], mxs);
          const float alpha = fast_exp2(m[tt] - mnew);
          m[tt] = mnew;
          l[tt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[tt][dt] *= alpha;
        }
        float pr[KT][4];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pr[kt][i] = fast_exp2(fmaf(sv[kt][i], p.scale_log2, -m[tt]));
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
          const int off = (32 * ks + 4 * g4 + (r16 >> 2)) * ROWB +
                          (((2 * dt + ((r16 >> 1) & 1)) ^ vswz) << 4) + ((r16 & 1) << 3);
          const s16x4_t lo = lds_read_tr(s_v, off);
          const s16x4_t hi = lds_read_tr(s_v, off + 16 * ROWB);
          uint4 a;
          a.x = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
          a.y = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
          a.z = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
          a.w = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
          o[0][dt] = M::mfma(a, pb[0][ks], o[0][dt]);
          o[1][dt] = M::mfma(a, pb[1][ks], o[1][dt]);
        }
      stage ^= 1;
    }
    if (cur.ntiles == 0 && has_next) {
      // No visible keys in this item: its output is 0 and the next item's
      // loads start here.  `stage` is free: no wave has read it since the
      // last barrier.
      if (nxt.ntiles > 0)
        issue_tile(nxt.h, nxt.pool_prefix, nxt.kend, nxt.new_base, nxt.table_row, 0, stage);
      load_q(nxt);
      st_slot = load_slot(nxt);
    }

    // ---- normalise and write: lane holds O[row r16][16 dt + 4 g4 + i] ----
    // The rows go out through LDS so that each store instruction writes whole
    // rows (16 bytes per lane, CPR lanes per row) instead of 8-byte pieces of
    // 16 rows: the narrow pattern cost more per byte.  The staging area is
    // the stage of the item's last tile (the next item's first tile is
    // landing in the other one); wave w uses its own 32 rows of it, so the
    // only barrier needed is the one that tells every wave is done reading
    // that stage's K and V.  Chunks are XOR-swizzled by row against bank
    // conflicts.
    if (cur.ntiles > 0) {
      __syncthreads();
      char* s_o = s_kv + (stage ^ 1) * 2 * TILE_B + wave * 32 * ROWB;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float lt = l[tt];
        lt = sum_xor16(lt);
        lt = sum_xor32(lt);
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          uint2 w;
          w.x = M::pack2(o[tt][dt][0] * inv, o[tt][dt][1] * inv);
          w.y = M::pack2(o[tt][dt][2] * inv, o[tt][dt][3] * inv);
          const int chunk = (2 * dt + (g4 >> 1)) ^ (r16 % CPR);
          *reinterpret_cast<uint2*>(s_o + (16 * tt + r16) * ROWB + chunk * 16 + (g4 & 1) * 8) = w;
        }
      }
      __builtin_amdgcn_wave_barrier();
      constexpr int RPS = 64 / CPR;  // rows per store instruction
#pragma unroll 2
      for (int j = 0; j < 32 / RPS; ++j) {
        const int rw = RPS * j + lane / CPR;  // row within the wave's 32
        const int c = lane % CPR;
        const uint4 v = lds_read16(s_o, rw * ROWB + ((c ^ ((rw % 16) % CPR)) << 4));
        const int row = 32 * wave + rw;  // MFMA row of the block
        const int qp = cur.pos0 + row % BQ;
        if (qp < cur.ql)
          st16_nt(p.out + (int64_t)(cur.q0 + qp) * p.o_st + (int64_t)(cur.h * G + row / BQ) * p.o_sh +
                   c * 16,
               v);
      }
    } else {
      // No visible keys: the rows are 0 (the other stage may be receiving the
      // next item's first tile, so nothing is staged).
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int row = 16 * (2 * wave + tt) + r16;
        const int qp = cur.pos0 + row % BQ;
        if (qp >= cur.ql) continue;
        char* dst = p.out + (int64_t)(cur.q0 + qp) * p.o_st + (int64_t)(cur.h * G + row / BQ) * p.o_sh;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          *reinterpret_cast<uint2*>(dst + (16 * dt + 4 * g4) * 2) = make_uint2(0u, 0u);
      }
    }
    if (!has_next) break;
    cur = nxt;
  }
}

// Launch the persistent grid: per XCD, as many workgroups as the kernel
// keeps resident on one XCD's CUs, or fewer when the XCD's item list (at
// most items_per_xcd long) is shorter.
template <bool kBF16, int D, int G, bool kCausal, bool kPaged, bool kOnce = false,
          bool kF8 = false, bool kPro = false>
static void launch_persistent(const VarlenParams& p, int64_t items_per_xcd, hipStream_t st) {
  const auto kern = varlen_attention_kernel<kBF16, D, G, kCausal, kPaged, kOnce, kF8, kPro>;
  // Resident workgroups per CU, queried once (a failed query is not cached:
  // the launch then assumes 1, which is correct but leaves slots idle).
  static std::atomic<int> cached{0};
  int per_cu = cached.load(std::memory_order_relaxed);
  if (per_cu <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kVarlenThreads, 0) ==
            hipSuccess &&
        per_cu > 0) {
      cached.store(per_cu, std::memory_order_relaxed);
    } else {
      (void)hipGetLastError();
      per_cu = 1;
    }
  }
  int64_t cus_per_xcd = current_device_cus() / kXcds;
  if (cus_per_xcd < 1) cus_per_xcd = 1;
  int64_t per_xcd = (int64_t)per_cu * cus_per_xcd;
  if (per_xcd > items_per_xcd) per_xcd = items_per_xcd;
  if (per_xcd < 1) per_xcd = 1;
  hipLaunchKernelGGL(kern, dim3((unsigned)(per_xcd * kXcds)), dim3(kVarlenThreads), 0, st, p);
}

template <bool kBF16, int D, int G, bool kCausal>
static void launch_varlen_c(const VarlenParams& p, int64_t items_per_xcd, hipStream_t st) {
  // The fused query prologue: causal launches at head_dim 128 over a 16-bit
  // pool or none (the host checks this before launching).
  if constexpr (kCausal && D == 128) {
    if (p.has_pro) {
      if (p.has_pool)
        launch_persistent<kBF16, D, G, true, true, false, false, true>(p, items_per_xcd, st);
      else
        launch_persistent<kBF16, D, G, true, false, false, false, true>(p, items_per_xcd, st);
      return;
    }
  }
  if (p.has_pool && p.kv_f8)
    launch_persistent<kBF16, D, G, kCausal, true, false, true>(p, items_per_xcd, st);
  else if (p.has_pool)
    launch_persistent<kBF16, D, G, kCausal, true>(p, items_per_xcd, st);
  else if (!kCausal && p.num_qblocks == 1)
    launch_persistent<kBF16, D, G, kCausal, false, true>(p, items_per_xcd, st);
  else
    launch_persistent<kBF16, D, G, kCausal, false>(p, items_per_xcd, st);
}

template <bool kBF16, int D, int G>
static void launch_varlen(const VarlenParams& p, bool causal, int64_t items_per_xcd,
                          hipStream_t st) {
  if (causal)
    launch_varlen_c<kBF16, D, G, true>(p, items_per_xcd, st);
  else
    launch_varlen_c<kBF16, D, G, false>(p, items_per_xcd, st);
}

template <bool kBF16, int D>
static bool dispatch_varlen_g(int G, const VarlenParams& p, bool causal, int64_t items_per_xcd,
                              hipStream_t st) {
  switch (G) {
    case 1: launch_varlen<kBF16, D, 1>(p, causal, items_per_xcd, st); return true;
    case 2: launch_varlen<kBF16, D, 2>(p, causal, items_per_xcd, st); return true;
    case 4: launch_varlen<kBF16, D, 4>(p, causal, items_per_xcd, st); return true;
    case 8: launch_varlen<kBF16, D, 8>(p, causal, items_per_xcd, st); return true;
    default: return false;
  }
}

template <bool kBF16>
static bool dispatch_varlen(int D, int G, const VarlenParams& p, bool causal,
                            int64_t items_per_xcd, hipStream_t st) {
  switch (D) {
    case 64: return dispatch_varlen_g<kBF16, 64>(G, p, causal, items_per_xcd, st);
    case 128: return dispatch_varlen_g<kBF16, 128>(G, p, causal, items_per_xcd, st);
    default: return false;
  }
}

static int varlen_native(const va_varlen_args* a, void* stream);

}  // namespace va

// No launch needs a workspace: an FP8 pool's prefix rows are converted
// inside the attention kernel, tile by tile.
extern "C" size_t va_varlen_workspace_bytes(const va_varlen_args* a) {
  (void)a;
  return 0;
}

extern "C" int va_varlen_attention(const va_varlen_args* a, void* stream) {
  using namespace va;
  VA_CHECK_ARG(a != nullptr, "va_varlen_attention: null args");
  VA_CHECK_ARG(a->struct_size == sizeof(va_varlen_args),
               "va_varlen_attention: struct_size %u != %zu (header/library mismatch)",
               a->struct_size, sizeof(va_varlen_args));
  VA_CHECK_ARG(a->num_seqs >= 0, "va_varlen_attention: num_seqs < 0");
  if (a->num_seqs == 0 || a->total_q == 0) return VA_OK;
  const bool has_pool = a->pool.k != nullptr;
  VA_CHECK_ARG(!has_pool || a->pool.kv_format == VA_KV_NATIVE ||
                   a->pool.kv_format == VA_KV_FP8_E4M3,
               "va_varlen_attention: unknown kv_format %d", a->pool.kv_format);
  if (!has_pool || a->pool.kv_format == VA_KV_NATIVE) return varlen_native(a, stream);

  // ---- FP8 pool: attention with the prefix converted in the kernel, then
  // the quantising store of the new rows ----
  VA_CHECK_ARG(a->pool.k_scale > 0.f && a->pool.v_scale > 0.f,
               "va_varlen_attention: FP8 pool scales must be positive");
  va_varlen_args b = *a;
  b.slot_mapping = nullptr;
  int rc = varlen_native(&b, stream);
  if (rc != VA_OK || a->slot_mapping == nullptr) return rc;

  va_store_args sa{};
  sa.struct_size = sizeof(va_store_args);
  sa.dtype = a->dtype;
  sa.key = a->k;
  sa.value = a->v;
  sa.key_stride_tok = a->k_stride_tok;
  sa.key_stride_head = a->k_stride_head;
  sa.value_stride_tok = a->v_stride_tok;
  sa.value_stride_head = a->v_stride_head;
  sa.pool = a->pool;
  sa.slot_mapping = a->slot_mapping;
  sa.slot_dtype = a->slot_dtype;
  sa.num_tokens = a->total_q;
  sa.num_kv_heads = a->num_kv_heads;
  sa.head_dim = a->head_dim;
  return va_store_kvcache(&sa, stream);
}

int va::varlen_native(const va_varlen_args* a, void* stream) {
  using namespace va;
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
  // An FP8 pool holds one byte per element (its strides count bytes).
  const bool f8 = has_pool && a->pool.kv_format == VA_KV_FP8_E4M3;
  VA_CHECK_ARG(!f8 || a->head_dim % 16 == 0,
               "va_varlen_attention: FP8 pool head_dim must be a multiple of 16");
  const int64_t kv_eb = f8 ? 1 : 2;
  const int64_t strides[] = {a->q_stride_tok,  a->q_stride_head,      a->k_stride_tok,
                             a->k_stride_head, a->v_stride_tok,       a->v_stride_head,
                             a->out_stride_tok, a->out_stride_head};
  for (int64_t s : strides)
    VA_CHECK_ARG((s * 2) % 16 == 0, "va_varlen_attention: strides must be 16-byte multiples");
  const int64_t pstrides[] = {a->pool.stride_block, a->pool.stride_slot, a->pool.stride_head};
  for (int64_t s : pstrides)
    VA_CHECK_ARG((s * kv_eb) % 16 == 0,
                 "va_varlen_attention: pool strides must be 16-byte multiples");
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->v, (uintptr_t)a->out,
                            (uintptr_t)a->pool.k, (uintptr_t)a->pool.v};
  for (uintptr_t p : ptrs)
    VA_CHECK_ARG(p % 16 == 0, "va_varlen_attention: pointers must be 16-byte aligned");
  VA_CHECK_ARG(a->scale > 0.f && a->scale < INFINITY, "va_varlen_attention: scale must be > 0");
  if (a->k != nullptr) {
    // Per-lane DMA offsets inside a 64-key tile are 32-bit.
    const int64_t span = (int64_t)(kKeyTile - 1) * (a->k_stride_tok > a->v_stride_tok
                                                        ? a->k_stride_tok
                                                        : a->v_stride_tok) * 2 +
                         (int64_t)a->head_dim * 2;
    VA_CHECK_ARG(a->k_stride_tok >= 0 && a->v_stride_tok >= 0 && span < ((int64_t)1 << 32),
                 "va_varlen_attention: k/v token strides must be non-negative and below 64 MiB");
  }
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
  p.s_blk = a->pool.stride_block * kv_eb;
  p.s_slot = a->pool.stride_slot * kv_eb;
  p.s_head = a->pool.stride_head * kv_eb;
  p.kv_f8 = f8;
  p.k_scale = f8 ? a->pool.k_scale : 1.0f;
  p.v_scale = f8 ? a->pool.v_scale : 1.0f;
  p.has_pro = a->prologue != nullptr;
  p.pro = PrologueParams{};
  if (a->prologue != nullptr) {
    const va_qk_prologue& pr = *a->prologue;
    VA_CHECK_ARG(a->causal != 0 && a->head_dim == 128 && !f8,
                 "va_varlen_attention: the fused query prologue needs a causal launch, "
                 "head_dim 128 and a 16-bit pool or none");
    VA_CHECK_ARG(pr.q_norm_weight && pr.cos_sin_cache && pr.positions && pr.max_position > 0 &&
                     pr.cos_sin_stride >= a->head_dim,
                 "va_varlen_attention: prologue weight / rotary cache / positions");
    VA_CHECK_ARG(pr.weight_dtype == VA_BF16 || pr.weight_dtype == VA_F16 ||
                     pr.weight_dtype == VA_F32,
                 "va_varlen_attention: prologue weight_dtype");
    VA_CHECK_ARG(pr.positions_dtype == VA_I32 || pr.positions_dtype == VA_I64,
                 "va_varlen_attention: prologue positions_dtype");
    VA_CHECK_ARG((uintptr_t)pr.q_norm_weight % 16 == 0 && (uintptr_t)pr.cos_sin_cache % 16 == 0 &&
                     (pr.cos_sin_stride * 4) % 16 == 0,
                 "va_varlen_attention: prologue weight and rotary cache must be 16-byte aligned "
                 "(rows too)");
    p.pro.q_w = pr.q_norm_weight;
    p.pro.k_w = pr.q_norm_weight;
    p.pro.w_dtype = pr.weight_dtype;
    p.pro.eps = pr.eps;
    p.pro.cs = pr.cos_sin_cache;
    p.pro.cs_stride = pr.cos_sin_stride;
    p.pro.max_pos = pr.max_position;
    p.pro.pos_i64 = pr.positions_dtype == VA_I64;
    p.pro.pos = pr.positions;
  }
  p.block_size = has_pool ? a->pool.block_size : 1;
  p.num_blocks = a->pool.num_blocks;
  p.table = a->block_tables;
  p.t_sb = a->table_stride_seq;
  p.table_i64 = a->table_dtype == VA_I64;
  p.table_width = a->table_width;
  p.slots = a->slot_mapping;
  p.slot_i64 = a->slot_dtype == VA_I64;
  p.num_qblocks = nqb;
  p.num_seqs = a->num_seqs;
  p.num_kv_heads = a->num_kv_heads;
  p.bs_div = make_fastdiv((uint32_t)p.block_size);
  p.hkv_div = make_fastdiv((uint32_t)a->num_kv_heads);
  p.slot_small = (int64_t)p.num_blocks * p.block_size <= ((int64_t)1 << 31);

  // Persistent 1-D grid over kXcds interleaved item lists; see the kernel.
  const int64_t npairs = (int64_t)a->num_seqs * a->num_kv_heads;
  const int64_t items_per_xcd = (npairs + kXcds - 1) / kXcds * nqb;
  VA_CHECK_ARG(npairs <= INT32_MAX / 2 && items_per_xcd * kXcds <= INT32_MAX,
               "va_varlen_attention: too many (sequence, kv head, query block) items");
  const hipStream_t st = (hipStream_t)stream;
  const bool ok =
      a->dtype == VA_BF16
          ? dispatch_varlen<true>(a->head_dim, G, p, a->causal != 0, items_per_xcd, st)
          : dispatch_varlen<false>(a->head_dim, G, p, a->causal != 0, items_per_xcd, st);
  if (!ok) {
    set_error("va_varlen_attention: unsupported configuration");
    return VA_ERR_UNSUPPORTED;
  }
  return check_launch("va_varlen_attention");
}
