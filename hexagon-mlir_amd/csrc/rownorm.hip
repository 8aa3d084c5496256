// Row reductions: RMSNorm and (scaled) softmax, one wave64 per row.
//
// The reference turns these into HVX split reductions (a 32-wide partial
// accumulator generic plus linalg.reduce, SplitReductionUtils.cpp,
// TilingPass.cpp:261-289) over VTCM tiles.  On CDNA the row lives in the
// registers of one wave: 16-byte loads (or 2-byte loads for unaligned rows)
// spread the row across the 64 lanes, the reduction is a butterfly over
// lanes, and every element is read from HBM once and written once.  All
// arithmetic is fp32.
#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {

struct RArgs {
  const char* x;
  const char* g;
  char* y;
  int64_t rows;
  int cols;
  int64_t ldx, ldy;
  float eps, scale;
};

template <typename T>
__device__ __forceinline__ void unpack8(int4v raw, float* f) {
  T t[8];
  __builtin_memcpy(t, &raw, 16);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)t[i];
}

template <typename T>
__device__ __forceinline__ int4v pack8(const float* f) {
  T t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = (T)f[i];
  int4v raw;
  __builtin_memcpy(&raw, t, 16);
  return raw;
}

// ---- RMSNorm: y = g * T(x * rsqrt(mean(x^2) + eps)) -------------------------
// (the normalised value is rounded to the I/O type before the weight multiply,
// as in the HF LlamaRMSNorm forward the TinyLlama benchmark runs)

// Row held in registers: CPL 16-byte chunks per lane (cols <= 512 * CPL).
template <typename T, int CPL>
__global__ __launch_bounds__(256) void rmsnorm_vec(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int nch = a.cols >> 3;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + row * a.ldx * 2, 0x7fffffff);
  int4v v[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = load16(rx, c < nch ? (uint32_t)c * 16 : kOOB);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float f[8];
    unpack8<T>(v[i], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
  }
  ss = wave_sum_dpp(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)a.cols + a.eps);
  char* yrow = a.y + row * a.ldy * 2;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float f[8], gf[8];
      unpack8<T>(v[i], f);
      unpack8<T>(*(const int4v*)(a.g + (int64_t)c * 16), gf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = gf[e] * (float)(T)(f[e] * r);
      *(int4v*)(yrow + (int64_t)c * 16) = pack8<T>(f);
    }
  }
}

// Any width / alignment: two passes over the row, element at a time.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_any(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* x = (const T*)a.x + row * a.ldx;
  T* y = (T*)a.y + row * a.ldy;
  const T* g = (const T*)a.g;
  float ss = 0.f;
  for (int c = lane; c < a.cols; c += 64) {
    const float f = (float)x[c];
    ss += f * f;
  }
  ss = wave_sum_dpp(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)a.cols + a.eps);
  for (int c = lane; c < a.cols; c += 64) y[c] = (T)((float)g[c] * (float)(T)((float)x[c] * r));
}

// ---- softmax: y = exp(s*x - max) / sum ---------------------------------------

// EPL elements per lane, strided by 64 (coalesced 2-byte loads; any
// alignment).  The max and the sum go through DPP and lane-swap reductions
// (no LDS round trip): softmax [18912, 197] 7.07 -> 6.27 us on one MI355X.
// Several rows per wave, all loads issued first, measured slower (2 rows
// 6.57 us, 4 rows 7.75 us), as did staging blocks of rows through LDS with
// 16-byte global accesses (11-15 us).
template <typename T, int EPL>
__global__ __launch_bounds__(256) void softmax_reg(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* x = (const T*)a.x + row * a.ldx;
  T* y = (T*)a.y + row * a.ldy;
  float v[EPL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < a.cols ? (float)x[c] * a.scale : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max_dpp(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < a.cols ? fast_exp(v[i] - mx) : 0.f;
    sum += v[i];
  }
  sum = wave_sum_dpp(sum);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int c = lane + 64 * i;
    if (c < a.cols) y[c] = (T)(v[i] * inv);
  }
}

// Wide rows: three passes (max, sum, write), re-reading x from cache.
template <typename T>
__global__ __launch_bounds__(256) void softmax_any(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* x = (const T*)a.x + row * a.ldx;
  T* y = (T*)a.y + row * a.ldy;
  float mx = -INFINITY;
  for (int c = lane; c < a.cols; c += 64) mx = fmaxf(mx, (float)x[c] * a.scale);
  mx = wave_max_dpp(mx);
  float sum = 0.f;
  for (int c = lane; c < a.cols; c += 64) sum += fast_exp((float)x[c] * a.scale - mx);
  sum = wave_sum_dpp(sum);
  const float inv = 1.0f / sum;
  for (int c = lane; c < a.cols; c += 64) y[c] = (T)(fast_exp((float)x[c] * a.scale - mx) * inv);
}

RArgs make_args(const RowProblem& p) {
  RArgs a;
  a.x = (const char*)p.x;
  a.g = (const char*)p.g;
  a.y = (char*)p.y;
  a.rows = p.rows;
  a.cols = (int)p.cols;
  a.ldx = p.ldx;
  a.ldy = p.ldy;
  a.eps = p.eps;
  a.scale = p.scale;
  return a;
}

template <typename T>
hipError_t rms_launch(const RowProblem& p, hipStream_t stream) {
  const RArgs a = make_args(p);
  const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
  const bool vec = (p.cols % 8 == 0) && (p.ldx % 8 == 0) && (p.ldy % 8 == 0) && ((uintptr_t)p.x % 16 == 0) &&
                   ((uintptr_t)p.y % 16 == 0) && ((uintptr_t)p.g % 16 == 0) && p.ldx * 2 * 4 < (1ll << 31);
  const int64_t nch = p.cols / 8;
  if (vec && nch <= 64) hipLaunchKernelGGL((rmsnorm_vec<T, 1>), grid, block, 0, stream, a);
  else if (vec && nch <= 128) hipLaunchKernelGGL((rmsnorm_vec<T, 2>), grid, block, 0, stream, a);
  else if (vec && nch <= 256) hipLaunchKernelGGL((rmsnorm_vec<T, 4>), grid, block, 0, stream, a);
  else if (vec && nch <= 512) hipLaunchKernelGGL((rmsnorm_vec<T, 8>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((rmsnorm_any<T>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t softmax_launch(const RowProblem& p, hipStream_t stream) {
  const RArgs a = make_args(p);
  const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
  const int64_t epl = (p.cols + 63) / 64;
  if (epl <= 1) hipLaunchKernelGGL((softmax_reg<T, 1>), grid, block, 0, stream, a);
  else if (epl <= 2) hipLaunchKernelGGL((softmax_reg<T, 2>), grid, block, 0, stream, a);
  else if (epl <= 4) hipLaunchKernelGGL((softmax_reg<T, 4>), grid, block, 0, stream, a);
  else if (epl <= 8) hipLaunchKernelGGL((softmax_reg<T, 8>), grid, block, 0, stream, a);
  else if (epl <= 16) hipLaunchKernelGGL((softmax_reg<T, 16>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((softmax_any<T>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rmsnorm(const RowProblem& p, hipStream_t stream) {
  if (p.rows == 0 || p.cols == 0) return hipSuccess;
  return p.dtype == DT_BF16 ? rms_launch<__bf16>(p, stream) : rms_launch<_Float16>(p, stream);
}

hipError_t launch_softmax(const RowProblem& p, hipStream_t stream) {
  if (p.rows == 0 || p.cols == 0) return hipSuccess;
  return p.dtype == DT_BF16 ? softmax_launch<__bf16>(p, stream) : softmax_launch<_Float16>(p, stream);
}

namespace {

template <typename T>
__global__ __launch_bounds__(256) void fold_rms_weight(const T* W, const T* g, T* Wg, int64_t N, int64_t K,
                                                       int64_t ldw, int64_t ldwg) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N * K) return;
  const int64_t n = i / K, k = i - n * K;
  Wg[n * ldwg + k] = (T)((float)W[n * ldw + k] * (float)g[k]);
}

}  // namespace

hipError_t launch_fold_rms_weight(int dtype, const void* W, const void* g, void* Wg, int64_t N, int64_t K,
                                  int64_t ldw, int64_t ldwg, hipStream_t stream) {
  const int64_t blocks = (N * K + 255) / 256;
  if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(fold_rms_weight<__bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, (const __bf16*)W,
                       (const __bf16*)g, (__bf16*)Wg, N, K, ldw, ldwg);
  else
    hipLaunchKernelGGL(fold_rms_weight<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream, (const _Float16*)W,
                       (const _Float16*)g, (_Float16*)Wg, N, K, ldw, ldwg);
  return hipGetLastError();
}

}  // namespace hxmi
