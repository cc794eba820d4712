// BF16 instantiations of the matrix-core paged decode over FP8 (e4m3) pools
// (paged_decode_mfma.h), apart from the 16-bit-pool ones so that both compile
// in parallel.
#include "paged_decode_mfma.h"

namespace va {

template <>
bool launch_paged_decode_mfma_f8<BF16>(int D, int G, const DecodeParams& p, dim3 grid,
                                      hipStream_t s) {
  return dispatch_mfma_d<BF16, true>(D, G, p, grid, s);
}

}  // namespace va
