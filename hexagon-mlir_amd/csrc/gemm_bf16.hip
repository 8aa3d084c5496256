// Instantiations of the MFMA GEMM for bf16 operands.
#include "gemm_impl.h"

namespace hxmi {
namespace gemm {

hipError_t launch_fast_bf16(int tile, bool nn, int epi, bool out_f32, bool rms, const KArgs& k, hipStream_t s) {
  using T = __bf16;
  if (rms) {  // RMSNorm folded into the GEMM: NT, bf16 out, the LLaMA / Qwen2 projection epilogues
    if (nn || out_f32) return hipErrorNotSupported;
    switch (epi) {
      case EPI_NONE: return launch_tile<false, T, EPI_NONE, false, false, true>(tile, k, s);
      case EPI_BIAS: return launch_tile<false, T, EPI_BIAS, false, false, true>(tile, k, s);
      case EPI_SILU_MUL: return launch_tile<false, T, EPI_SILU_MUL, false, false, true>(tile, k, s);
      default: return hipErrorNotSupported;
    }
  }
  if (out_f32) {
    if (epi != EPI_NONE) return hipErrorNotSupported;
    return nn ? launch_tile<true, T, EPI_NONE, true>(tile, k, s) : launch_tile<false, T, EPI_NONE, true>(tile, k, s);
  }
  if (nn) {
    switch (epi) {
      case EPI_NONE: return launch_tile<true, T, EPI_NONE, false>(tile, k, s);
      case EPI_BIAS: return launch_tile<true, T, EPI_BIAS, false>(tile, k, s);
      default: return hipErrorNotSupported;
    }
  }
  switch (epi) {
    case EPI_NONE: return launch_tile<false, T, EPI_NONE, false>(tile, k, s);
    case EPI_BIAS: return launch_tile<false, T, EPI_BIAS, false>(tile, k, s);
    case EPI_SILU_MUL: return launch_tile<false, T, EPI_SILU_MUL, false>(tile, k, s);
    case EPI_GELU_TANH: return launch_tile<false, T, EPI_GELU_TANH, false>(tile, k, s);
    case EPI_BIAS_GELU_TANH: return launch_tile<false, T, EPI_BIAS_GELU_TANH, false>(tile, k, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace gemm
}  // namespace hxmi
