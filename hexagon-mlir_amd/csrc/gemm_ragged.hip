// Instantiations of the MFMA GEMM for K not a multiple of 8 (fp16 / bf16):
// the fragments of the last K-step keep only their elements below K.
// Two tiles: 128x128 (4 waves) for problems with enough of them to cover the
// CUs, 64x64 otherwise.
#include "gemm_impl.h"

namespace hxmi {
namespace gemm {
namespace {

template <bool NN, typename T, int EPI, bool OUTF32>
hipError_t ragged_tile(int tile, const KArgs& k, hipStream_t s) {
  if (tile == TILE_128x128) return launch_one<TILE_128x128, NN, T, EPI, OUTF32, false, false, true>(k, s);
  return launch_one<TILE_64x64, NN, T, EPI, OUTF32, false, false, true>(k, s);
}

template <typename T>
hipError_t ragged_t(int tile, bool nn, int epi, bool out_f32, const KArgs& k, hipStream_t s) {
  if (out_f32) {
    if (epi != EPI_NONE) return hipErrorNotSupported;
    return nn ? ragged_tile<true, T, EPI_NONE, true>(tile, k, s) : ragged_tile<false, T, EPI_NONE, true>(tile, k, s);
  }
  if (nn) {
    switch (epi) {
      case EPI_NONE: return ragged_tile<true, T, EPI_NONE, false>(tile, k, s);
      case EPI_BIAS: return ragged_tile<true, T, EPI_BIAS, false>(tile, k, s);
      default: return hipErrorNotSupported;
    }
  }
  switch (epi) {
    case EPI_NONE: return ragged_tile<false, T, EPI_NONE, false>(tile, k, s);
    case EPI_BIAS: return ragged_tile<false, T, EPI_BIAS, false>(tile, k, s);
    case EPI_SILU_MUL: return ragged_tile<false, T, EPI_SILU_MUL, false>(tile, k, s);
    case EPI_GELU_TANH: return ragged_tile<false, T, EPI_GELU_TANH, false>(tile, k, s);
    case EPI_BIAS_GELU_TANH: return ragged_tile<false, T, EPI_BIAS_GELU_TANH, false>(tile, k, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace

hipError_t launch_fast_ragged(int tile, bool bf16, bool nn, int epi, bool out_f32, const KArgs& k, hipStream_t s) {
  return bf16 ? ragged_t<__bf16>(tile, nn, epi, out_f32, k, s) : ragged_t<_Float16>(tile, nn, epi, out_f32, k, s);
}

}  // namespace gemm
}  // namespace hxmi
