// Per-output-channel symmetric int8 quantisation of fp16 weights [N, K] into
// the codes + scales layout the weight-only int8 GEMV / GEMM reads.
//
// One wave per row, two passes over the row: the first takes max |w|, the
// second writes the codes (the row comes back from L2).  Lanes move 16 bytes
// of weights and 8 bytes of codes per step, consecutive lanes consecutive
// chunks.  A load-time transform, HBM-bound; not on the per-token path.
#include <hip/hip_runtime.h>

#include "hxmi_internal.h"

namespace hxmi {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Smallest fp16 s with s >= fp16(amax / 127) and 127 * s >= amax: round to
// nearest, then one fp16 step up when that fell below, so that |w| / s <= 127
// and no code clips.  127 * s is exact in fp32 (7 x 11 significant bits).  A
// zero row gets s = 1; a row too small for any normal scale gets the fp16
// subnormal that covers it.
__device__ inline _Float16 row_scale(float amax) {
  if (amax == 0.f) return (_Float16)1.f;
  _Float16 s = (_Float16)__fdiv_rn(amax, 127.f);
  if ((float)s * 127.f < amax) {
    const unsigned short bits = __builtin_bit_cast(unsigned short, s);
    s = __builtin_bit_cast(_Float16, (unsigned short)(bits + 1));  // s >= 0: next representable up
  }
  return s;
}

__global__ __launch_bounds__(256) void quantize_int8_rows(const _Float16* __restrict__ W, int8_t* __restrict__ q,
                                                          _Float16* __restrict__ s, int64_t N, int64_t K, int64_t ldw,
                                                          int64_t ldq) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // whole wave leaves together: n is wave-uniform
  const _Float16* w = W + n * ldw;
  float amax = 0.f;
  for (int64_t k = 8 * (int64_t)lane; k < K; k += 512) {
    const half8 v = *reinterpret_cast<const half8*>(w + k);
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf((float)v[j]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const _Float16 sh = row_scale(amax);
  const float sf = (float)sh;
  if (lane == 0) s[n] = sh;
  int8_t* qr = q + n * ldq;
  for (int64_t k = 8 * (int64_t)lane; k < K; k += 512) {
    const half8 v = *reinterpret_cast<const half8*>(w + k);
    unsigned int lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float c = rintf(__fdiv_rn((float)v[j], sf));  // round half to even
      c = fminf(fmaxf(c, -127.f), 127.f);
      const unsigned int b = (unsigned int)(int)c & 0xffu;
      if (j < 4) lo |= b << (8 * j);
      else hi |= b << (8 * (j - 4));
    }
    *reinterpret_cast<uint2*>(qr + k) = make_uint2(lo, hi);
  }
}

}  // namespace

hipError_t launch_quantize_int8_rows(const void* W, int8_t* q, void* s, int64_t N, int64_t K, int64_t ldw,
                                     int64_t ldq, hipStream_t stream) {
  const int64_t blocks = (N + 3) / 4;
  if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_int8_rows, dim3((unsigned)blocks), dim3(256), 0, stream, (const _Float16*)W, q,
                     (_Float16*)s, N, K, ldw, ldq);
  return hipGetLastError();
}

}  // namespace hxmi
