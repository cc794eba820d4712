// F16 instantiations of the paged decode kernels (general kernel in
// paged_decode_kernel.h, matrix-core kernel in paged_decode_mfma.h).
#include "paged_decode_mfma.h"

namespace va {

template <>
bool launch_paged_decode<F16>(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  return dispatch_d<F16>(D, G, p, grid, s);
}

template <>
bool launch_paged_decode_mfma<F16>(int D, int G, const DecodeParams& p, dim3 grid,
                                    hipStream_t s) {
  return dispatch_mfma_d<F16, false>(D, G, p, grid, s);
}

}  // namespace va
