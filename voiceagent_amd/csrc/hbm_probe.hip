// HBM read floor: a plain streaming read of `bytes` contiguous bytes in one
// launch.  It gives the decode kernel's bandwidth a machine-measured
// reference: what one launch reading the same number of bytes, with nothing
// else to do, reaches on this GPU.  Diagnostic only; it has no counterpart in
// the reference.
//
// Workgroup w reads the contiguous slice [w per_wg, (w + 1) per_wg) of 16-byte
// words; each of its 512 lanes keeps four 16-byte loads in flight per step.
// The words are XOR-folded and the fold is written to sink[w] only when it
// equals a fixed value, so the loads cannot be removed and, in practice,
// nothing is written.
#include "common.h"

namespace va {

constexpr int kProbeThreads = 512;
constexpr int kProbeUnroll = 4;
constexpr uint32_t kProbeMagic = 0x9e3779b9u;

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(const uint4* __restrict__ src,
                                                                       int64_t nvec,
                                                                       int64_t per_wg,
                                                                       uint32_t* sink) {
  const int64_t beg = (int64_t)blockIdx.x * per_wg;
  const int64_t end = beg + per_wg < nvec ? beg + per_wg : nvec;
  uint32_t acc = 0;
  for (int64_t i = beg + threadIdx.x; i < end; i += kProbeUnroll * kProbeThreads) {
    uint4 w[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t j = i + (int64_t)u * kProbeThreads;
      w[u] = j < end ? src[j] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= w[u].x ^ w[u].y ^ w[u].z ^ w[u].w;
  }
  if (acc == kProbeMagic) sink[blockIdx.x] = acc;
}

}  // namespace va

extern "C" int va_hbm_read_probe(const void* src, size_t bytes, int workgroups, void* sink,
                                 void* stream) {
  using namespace va;
  VA_CHECK_ARG(src != nullptr && sink != nullptr, "va_hbm_read_probe: null pointer argument");
  VA_CHECK_ARG((uintptr_t)src % 16 == 0 && bytes % 16 == 0,
               "va_hbm_read_probe: src and bytes must be 16-byte aligned");
  VA_CHECK_ARG(workgroups >= 1 && workgroups <= 65536,
               "va_hbm_read_probe: workgroups must be in [1, 65536]");
  if (bytes == 0) return VA_OK;
  const int64_t nvec = (int64_t)(bytes / 16);
  const int64_t per_wg = (nvec + workgroups - 1) / workgroups;
  hipLaunchKernelGGL(hbm_read_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeThreads), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint4*>(src), nvec, per_wg,
                     reinterpret_cast<uint32_t*>(sink));
  return check_launch("va_hbm_read_probe");
}
