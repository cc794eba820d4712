// HBM read floor: a streaming read of `bytes` contiguous bytes in one launch,
// through one of three load paths.  It gives the decode kernel's bandwidth a
// machine-measured reference: what one launch reading the same number of
// bytes, with nothing else to do, reaches on this GPU.  Bench-only (built
// into libvoiceagent_bench.so, declared in include/voiceagent_bench.h); it
// has no counterpart in the reference.
//
// Workgroup w (8 wave64s) reads the contiguous slice [w per_wg, (w + 1)
// per_wg) of 16-byte words:
//   VA_PROBE_PLAIN    each lane keeps four plain 16-byte loads in flight;
//   VA_PROBE_NT       each lane keeps eight non-temporal 16-byte loads in
//                     flight;
//   VA_PROBE_LDS_DMA  1 KiB units of the slice go round robin to the waves,
//                     each copied by one non-temporal global_load_lds_dwordx4
//                     into a 16-unit LDS ring per wave, 16 KiB in flight per
//                     wave (the decode kernel's load path and depth).
// Register loads are XOR-folded and the fold is written to sink[w] only when
// it equals a fixed value, so the loads cannot be removed and, in practice,
// nothing is written; the DMA path writes only LDS.
//
// va_bench_hbm_copy is the mixed floor for the varlen launches: it reads and
// writes given byte counts in one launch (for prefill, its q, k, v reads and
// its output and stored-row writes).  va_bench_empty launches a kernel that
// does nothing: the fixed cost of a launch of a given grid.
#include <stdarg.h>
#include <stdio.h>

#include "../common.h"
#include "../../../include/voiceagent_bench.h"

namespace va {
namespace {

thread_local char g_bench_error[256] = "";

int bench_fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_bench_error, sizeof(g_bench_error), fmt, ap);
  va_end(ap);
  return -1;
}

constexpr int kProbeThreads = 512;
constexpr uint32_t kProbeMagic = 0x9e3779b9u;

template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(
    const uint4* __restrict__ src, int64_t nvec, int64_t per_wg, uint32_t* sink) {
  const int64_t beg = (int64_t)blockIdx.x * per_wg;
  const int64_t end = beg + per_wg < nvec ? beg + per_wg : nvec;
  uint32_t acc = 0;
  for (int64_t i = beg + threadIdx.x; i < end; i += kUnroll * kProbeThreads) {
    uint4 w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kProbeThreads;
      if (j < end)
        w[u] = kNt ? ld16_nt(src + j) : src[j];
      else
        w[u] = make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= w[u].x ^ w[u].y ^ w[u].z ^ w[u].w;
  }
  if (acc == kProbeMagic) sink[blockIdx.x] = acc;
}

constexpr int kDmaRing = 16;  // 1 KiB units in flight per wave

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_dma_kernel(const char* src,
                                                                           int64_t nvec,
                                                                           int64_t per_wg) {
  __shared__ __align__(1024) char ring[kProbeThreads / 64 * kDmaRing * 1024];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t beg = (int64_t)blockIdx.x * per_wg;
  const int64_t end = beg + per_wg < nvec ? beg + per_wg : nvec;
  const int64_t units = end > beg ? (end - beg + 63) / 64 : 0;  // 64 words per unit
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(ring +
                                                                     wave * kDmaRing * 1024));
  int issued = 0;
  for (int64_t u = wave; u < units; u += kProbeThreads / 64) {
    // Lane l copies word beg + 64 u + l; past the slice it re-reads the
    // slice's last word, so every address stays inside the buffer.
    int64_t word = beg + 64 * u + lane;
    if (word >= end) word = end - 1;
    const char* base = uniform_ptr(src + (beg + 64 * u) * 16);
    const uint32_t off = (uint32_t)((word - (beg + 64 * u)) * 16);
    dma16_nt(off, base, lds + (uint32_t)((issued % kDmaRing) * 1024));
    ++issued;
    if (issued >= kDmaRing) wait_vmcnt<kDmaRing - 1>();
  }
  wait_vmcnt<0>();
}

// Mixed read/write stream: workgroup w covers the slice [w per_wg, (w + 1)
// per_wg) of max(nr, nw) 16-byte words; word j is read from src when j < nr
// and written to dst when j < nw (the word read, so that no load can be
// dropped).  Eight non-temporal loads per lane are in flight before their
// non-temporal stores, as an attention epilogue stores rows it has no further
// use for.
template <int kUnroll>
__global__ __launch_bounds__(kProbeThreads) void hbm_copy_probe_kernel(
    const uint4* __restrict__ src, int64_t nr, uint4* __restrict__ dst, int64_t nw,
    int64_t per_wg) {
  const int64_t n = nr > nw ? nr : nw;
  const int64_t beg = (int64_t)blockIdx.x * per_wg;
  const int64_t end = beg + per_wg < n ? beg + per_wg : n;
  for (int64_t i = beg + threadIdx.x; i < end; i += kUnroll * kProbeThreads) {
    uint4 w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kProbeThreads;
      w[u] = (j < end && j < nr) ? ld16_nt(src + j) : make_uint4((uint32_t)j, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kProbeThreads;
      if (j < end && j < nw) st16_nt(dst + j, w[u]);
    }
  }
}

// Does nothing: the fixed cost of a launch of its grid.
__global__ __launch_bounds__(kProbeThreads) void empty_probe_kernel() {}

// Per-workgroup read rate against the bytes in flight.  Workgroup w (8
// wave64s) reads `rounds` rounds of its slice src + w slice_stride; in each
// round a wave takes NL + NV consecutive 1 KiB units of its own (unit j of
// wave v at byte (8 j + v) KiB): the first NL through non-temporal LDS DMA
// into the wave's NL KiB of a 128 KiB ring (so one workgroup fills a CU's
// LDS and workgroups land on distinct CUs), the next NV through
// non-temporal 16-byte register loads (XOR-folded, written to sink only on a
// fixed value, so never in practice).  Before each request the wave waits
// until at most NL + NV - 1 of its requests are in flight: 8 (NL + NV) KiB
// per CU stay in flight.  The DMA uses the builtin form; with both kinds in
// a round the compiler still waits for all in-flight requests once per round
// before folding the registers (it does not count the DMAs issued after a
// register load), so mixed depths hold only between those drains.  Thread 0
// writes s_memrealtime (100 MHz) at the start and the end to times[2 w],
// times[2 w + 1].
constexpr int kDepthMaxDma = 16;  // KiB of LDS DMA per wave
constexpr int kDepthWaves = kProbeThreads / 64;

template <int NL, int NV>
__global__ __launch_bounds__(kProbeThreads, 1) void hbm_depth_probe_kernel(
    const char* src, int64_t slice_stride, int64_t rounds, uint64_t* times, uint32_t* sink) {
  static_assert(NL >= 0 && NL <= kDepthMaxDma && NV >= 0 && NL + NV >= 1 && NL + NV < 64,
                "depth");
  __shared__ __align__(1024) char ring[kDepthWaves * kDepthMaxDma * 1024];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const char* const base = src + (int64_t)blockIdx.x * slice_stride + lane * 16;
  char* const myring = ring + wave * kDepthMaxDma * 1024 + lane * 16;
  // Every round is the same code (the registers start at zero and are
  // folded before each reload): a first round without the fold made the
  // compiler's own wait for the loop-carried registers a full drain.
  uint4 r[NV > 0 ? NV : 1];
#pragma unroll
  for (int s = 0; s < (NV > 0 ? NV : 1); ++s) r[s] = make_uint4(0u, 0u, 0u, 0u);
  uint32_t acc = 0;
  uint64_t t0 = 0;
  __syncthreads();
  if (threadIdx.x == 0) t0 = __builtin_amdgcn_s_memrealtime();
  for (int64_t rd = 0; rd < rounds; ++rd) {
    const int64_t j0 = rd * (NL + NV);
#pragma unroll
    for (int s = 0; s < NL; ++s) {
      wait_vmcnt<NL + NV - 1>();
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void*>(base + (((j0 + s) * kDepthWaves + wave) << 10)),
          reinterpret_cast<__attribute__((address_space(3))) void*>(
              (__attribute__((address_space(3))) char*)(myring + s * 1024)),
          16, 0, /*aux: nt*/ 2);
    }
#pragma unroll
    for (int s = 0; s < NV; ++s) {
      wait_vmcnt<NL + NV - 1>();
      uint32_t f = r[s].x ^ r[s].y ^ r[s].z ^ r[s].w;
      asm volatile("" : "+v"(f));
      acc ^= f;
      r[s] = ld16_nt(reinterpret_cast<const uint4*>(
          base + (((j0 + NL + s) * kDepthWaves + wave) << 10)));
    }
  }
#pragma unroll
  for (int s = 0; s < NV; ++s) acc ^= r[s].x ^ r[s].y ^ r[s].z ^ r[s].w;
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    times[2 * blockIdx.x] = t0;
    times[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
  }
  if (acc == kProbeMagic) sink[blockIdx.x] = acc;
}

template <int NL>
static bool launch_depth_nv(int nv, dim3 grid, hipStream_t s, const char* src, int64_t stride,
                            int64_t rounds, uint64_t* times, uint32_t* sink) {
  switch (nv) {
    case 0:
      if constexpr (NL > 0) {
        hipLaunchKernelGGL((hbm_depth_probe_kernel<NL, 0>), grid, dim3(kProbeThreads), 0, s, src, stride, rounds, times, sink);
        return true;
      }
      return false;
    case 4: hipLaunchKernelGGL((hbm_depth_probe_kernel<NL, 4>), grid, dim3(kProbeThreads), 0, s, src, stride, rounds, times, sink); return true;
    case 8: hipLaunchKernelGGL((hbm_depth_probe_kernel<NL, 8>), grid, dim3(kProbeThreads), 0, s, src, stride, rounds, times, sink); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace va

extern "C" int va_bench_hbm_copy(const void* src, size_t read_bytes, void* dst,
                                 size_t write_bytes, int workgroups, void* stream) {
  using namespace va;
  if ((read_bytes > 0 && src == nullptr) || (write_bytes > 0 && dst == nullptr))
    return bench_fail("va_bench_hbm_copy: null pointer");
  if ((uintptr_t)src % 16 != 0 || (uintptr_t)dst % 16 != 0 || read_bytes % 16 != 0 ||
      write_bytes % 16 != 0)
    return bench_fail("va_bench_hbm_copy: pointers and sizes must be 16-byte aligned");
  if (workgroups < 1 || workgroups > 65536)
    return bench_fail("va_bench_hbm_copy: workgroups must be in [1, 65536]");
  const int64_t nr = (int64_t)(read_bytes / 16), nw = (int64_t)(write_bytes / 16);
  const int64_t n = nr > nw ? nr : nw;
  if (n == 0) return 0;
  const int64_t per_wg = (n + workgroups - 1) / workgroups;
  hipLaunchKernelGGL((hbm_copy_probe_kernel<8>), dim3((unsigned)workgroups), dim3(kProbeThreads),
                     0, (hipStream_t)stream, reinterpret_cast<const uint4*>(src), nr,
                     reinterpret_cast<uint4*>(dst), nw, per_wg);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bench_fail("va_bench_hbm_copy: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int va_bench_hbm_read(const void* src, size_t bytes, int workgroups, int mode,
                                 void* sink, void* stream) {
  using namespace va;
  if (src == nullptr || sink == nullptr) return bench_fail("va_bench_hbm_read: null pointer");
  if ((uintptr_t)src % 16 != 0 || bytes % 16 != 0)
    return bench_fail("va_bench_hbm_read: src and bytes must be 16-byte aligned");
  if (workgroups < 1 || workgroups > 65536)
    return bench_fail("va_bench_hbm_read: workgroups must be in [1, 65536]");
  if (mode != VA_PROBE_PLAIN && mode != VA_PROBE_NT && mode != VA_PROBE_LDS_DMA)
    return bench_fail("va_bench_hbm_read: unknown mode %d", mode);
  if (bytes == 0) return 0;
  const int64_t nvec = (int64_t)(bytes / 16);
  const int64_t per_wg = (nvec + workgroups - 1) / workgroups;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)workgroups), block(kProbeThreads);
  const uint4* v = reinterpret_cast<const uint4*>(src);
  uint32_t* out = reinterpret_cast<uint32_t*>(sink);
  if (mode == VA_PROBE_PLAIN)
    hipLaunchKernelGGL((hbm_read_probe_kernel<4, false>), grid, block, 0, s, v, nvec, per_wg, out);
  else if (mode == VA_PROBE_NT)
    hipLaunchKernelGGL((hbm_read_probe_kernel<8, true>), grid, block, 0, s, v, nvec, per_wg, out);
  else
    hipLaunchKernelGGL(hbm_read_probe_dma_kernel, grid, block, 0, s,
                       reinterpret_cast<const char*>(src), nvec, per_wg);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bench_fail("va_bench_hbm_read: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int va_bench_empty(int workgroups, void* stream) {
  using namespace va;
  if (workgroups < 1 || workgroups > 65536)
    return bench_fail("va_bench_empty: workgroups must be in [1, 65536]");
  hipLaunchKernelGGL(empty_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeThreads), 0,
                     (hipStream_t)stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bench_fail("va_bench_empty: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int va_bench_hbm_depth(const void* src, size_t src_bytes, size_t bytes_per_wg,
                                  int workgroups, int dma_kib_per_wave, int vgpr_kib_per_wave,
                                  void* times, void* sink, void* stream) {
  using namespace va;
  if (src == nullptr || times == nullptr || sink == nullptr)
    return bench_fail("va_bench_hbm_depth: null pointer");
  if ((uintptr_t)src % 1024 != 0 || bytes_per_wg % 1024 != 0)
    return bench_fail("va_bench_hbm_depth: src and bytes_per_wg must be 1 KiB aligned");
  if (workgroups < 1 || workgroups > 4096)
    return bench_fail("va_bench_hbm_depth: workgroups must be in [1, 4096]");
  if ((dma_kib_per_wave != 0 && dma_kib_per_wave != 4 && dma_kib_per_wave != 8 &&
       dma_kib_per_wave != 16) ||
      (vgpr_kib_per_wave != 0 && vgpr_kib_per_wave != 4 && vgpr_kib_per_wave != 8) ||
      dma_kib_per_wave + vgpr_kib_per_wave == 0)
    return bench_fail("va_bench_hbm_depth: depths must be 0|4|8|16 KiB (DMA) and 0|4|8 KiB "
                      "(registers) per wave, not both 0");
  const int64_t per_round = (int64_t)kDepthWaves * (dma_kib_per_wave + vgpr_kib_per_wave) * 1024;
  const int64_t rounds = (int64_t)bytes_per_wg / per_round;
  if (rounds < 2) return bench_fail("va_bench_hbm_depth: bytes_per_wg below two rounds");
  if ((uint64_t)bytes_per_wg * (uint64_t)workgroups > src_bytes)
    return bench_fail("va_bench_hbm_depth: %d slices of %zu bytes exceed the %zu-byte buffer",
                      workgroups, bytes_per_wg, src_bytes);
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)workgroups);
  const char* c = reinterpret_cast<const char*>(src);
  uint64_t* t = reinterpret_cast<uint64_t*>(times);
  uint32_t* k = reinterpret_cast<uint32_t*>(sink);
  const int64_t stride = (int64_t)bytes_per_wg;
  bool ok = false;
  switch (dma_kib_per_wave) {
    case 0: ok = vgpr_kib_per_wave > 0 && launch_depth_nv<0>(vgpr_kib_per_wave, grid, s, c, stride, rounds, t, k); break;
    case 4: ok = launch_depth_nv<4>(vgpr_kib_per_wave, grid, s, c, stride, rounds, t, k); break;
    case 8: ok = launch_depth_nv<8>(vgpr_kib_per_wave, grid, s, c, stride, rounds, t, k); break;
    case 16: ok = launch_depth_nv<16>(vgpr_kib_per_wave, grid, s, c, stride, rounds, t, k); break;
  }
  if (!ok) return bench_fail("va_bench_hbm_depth: unsupported depth");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bench_fail("va_bench_hbm_depth: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" const char* va_bench_last_error(void) { return va::g_bench_error; }
