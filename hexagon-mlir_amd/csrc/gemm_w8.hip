// Instantiations of the MFMA GEMM with int8 [N,K] weights and per-column
// scales (weight-only int8, fp16 activations).
#include "gemm_impl.h"

namespace hxmi {
namespace gemm {

hipError_t launch_fast_w8(int tile, int epi, bool out_f32, const KArgs& k, hipStream_t s) {
  if (out_f32) {
    if (epi != EPI_NONE) return hipErrorNotSupported;
    return launch_tile<false, _Float16, EPI_NONE, true, true>(tile, k, s);
  }
  switch (epi) {
    case EPI_NONE: return launch_tile<false, _Float16, EPI_NONE, false, true>(tile, k, s);
    case EPI_BIAS: return launch_tile<false, _Float16, EPI_BIAS, false, true>(tile, k, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace gemm
}  // namespace hxmi
