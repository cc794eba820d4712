// F16 instantiations of the paged decode kernels (see paged_decode_kernel.h).
#include "paged_decode_kernel.h"

namespace va {

template <>
bool launch_paged_decode<F16>(int D, int G, const DecodeParams& p, dim3 grid, hipStream_t s) {
  return dispatch_d<F16>(D, G, p, grid, s);
}

}  // namespace va
