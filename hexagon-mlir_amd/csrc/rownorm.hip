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
__global__ __launch_bounds__(128) void rmsnorm_vec(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 6);
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
__global__ __launch_bounds__(128) void rmsnorm_any(RArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 6);
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

// Larger of two raw values (smaller with MIN); fp16 compares in fp16.
template <bool MIN>
__device__ __forceinline__ _Float16 pick(_Float16 a, _Float16 b) {
  return MIN ? __builtin_fminf16(a, b) : __builtin_fmaxf16(a, b);
}
template <bool MIN>
__device__ __forceinline__ __bf16 pick(__bf16 a, __bf16 b) {
  return (MIN ? (float)b < (float)a : (float)b > (float)a) ? b : a;
}

// Row extremum over the G lanes of a row group: the largest raw value, or
// the smallest with MIN.
template <int G, bool MIN, typename T, int EPL>
__device__ __forceinline__ float row_extremum(const T (&h)[EPL]) {
  T m = h[0];
#pragma unroll
  for (int i = 1; i < EPL; ++i) m = pick<MIN>(m, h[i]);
  const float f = (float)m;
  return MIN ? -wave_reduce_dpp<G>(-f, [](float p, float q) { return fmaxf(p, q); })
             : wave_reduce_dpp<G>(f, [](float p, float q) { return fmaxf(p, q); });
}

// One row per group of G lanes (64 / G rows per wave), EPL = ceil(cols / G)
// elements per lane strided by G (coalesced 2-byte loads, any alignment):
// every slot but the last lies inside the row, so only the last is masked.
// The row extremum is taken on the raw values, since fp32 multiplication is
// monotonic: max(s*x) = s*max(x) for s >= 0 and s*min(x) for s < 0.  Each
// element then costs one fma for its exponent, 2^(x*s*log2e - m*s*log2e),
// one v_exp_f32, one add and one multiply by the reciprocal of the row sum.
// Softmax [18912, 197] on one MI355X: 3.97 us with 32 lanes per row (47 % of
// HBM; 4.62 us with 64, 4.25 us with 16), against 5.76 us for one row per
// wave with a scaled max and a divide; a plain 16-byte copy of the same
// bytes takes 2.93 us.  Staging spans of rows through LDS with 16-byte
// global accesses measured 6.4-9.3 us.
template <typename T, int G, int EPL>
__global__ __launch_bounds__(256) void softmax_rows(RArgs a) {
  constexpr int RW = 64 / G;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave * RW >= a.rows) return;
  const int64_t row = wave * RW + lane / G;
  const bool ok = row < a.rows;  // lanes past the last row read it again and store nothing
  const int c0 = lane % G;
  const T* x = (const T*)a.x + (ok ? row : a.rows - 1) * a.ldx + c0;
  const float sl2 = a.scale * 1.4426950408889634f;
  const bool neg = sl2 < 0.f;
  T h[EPL];
#pragma unroll
  for (int i = 0; i < EPL - 1; ++i) h[i] = x[G * i];
  const bool last = c0 + G * (EPL - 1) < a.cols;
  // a masked slot repeats slot 0 (inside the row when EPL > 1) or, alone,
  // holds a value that cannot win the extremum; it is left out of the sum
  const T far = (T)(neg ? INFINITY : -INFINITY);
  h[EPL - 1] = last ? x[G * (EPL - 1)] : (EPL > 1 ? h[0] : far);
  const float m = neg ? row_extremum<G, true>(h) : row_extremum<G, false>(h);
  const float nm = -(m * sl2);
  float t[EPL];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    t[i] = __builtin_amdgcn_exp2f(__builtin_fmaf((float)h[i], sl2, nm));
    if (i < EPL - 1 || last) sum += t[i];
  }
  sum = wave_reduce_dpp<G>(sum, [](float p, float q) { return p + q; });
  const float inv = __builtin_amdgcn_rcpf(sum);
  if (!ok) return;
  T* y = (T*)a.y + row * a.ldy + c0;
#pragma unroll
  for (int i = 0; i < EPL - 1; ++i) y[G * i] = (T)(t[i] * inv);
  if (last) y[G * (EPL - 1)] = (T)(t[EPL - 1] * inv);
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
  // two rows (waves) a workgroup: [512, 2048] then spans 256 workgroups, one
  // per CU (2.96 -> 2.88 us against four rows a workgroup; one row: 3.01)
  const dim3 grid((unsigned)((p.rows + 1) / 2)), block(128);
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

// softmax_rows<T, G, E> for E = epl (exactly), searched from E down to LO.
template <typename T, int G, int E, int LO>
bool softmax_rows_launch(const RArgs& a, int epl, hipStream_t stream) {
  if constexpr (E < LO) {
    return false;
  } else {
    if (epl != E) return softmax_rows_launch<T, G, E - 1, LO>(a, epl, stream);
    const int64_t waves = (a.rows + 64 / G - 1) / (64 / G);
    hipLaunchKernelGGL((softmax_rows<T, G, E>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, a);
    return true;
  }
}

template <typename T>
hipError_t softmax_launch(const RowProblem& p, hipStream_t stream) {
  const RArgs a = make_args(p);
  // 32 lanes a row up to 512 columns, 64 up to 1024, then three passes
  bool done = false;
  if (p.cols <= 512) done = softmax_rows_launch<T, 32, 16, 1>(a, (int)((p.cols + 31) / 32), stream);
  else if (p.cols <= 1024) done = softmax_rows_launch<T, 64, 16, 9>(a, (int)((p.cols + 63) / 64), stream);
  if (!done)
    hipLaunchKernelGGL((softmax_any<T>), dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, stream, a);
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

// ---- masked softmax: the attention scores' softmax with the mask operand --
// y[i][r] = softmax(scale * x[i][r] + M[i / mask_group][r] + causal(r, .)),
// one wave per row, three passes (max, sum, write) re-reading the row from
// cache.  It serves the composite attention path (any head dim, bf16),
// where the scores are already materialised by the batched GEMM; the fused
// kernel applies the same rule inside its key loop.
struct MArgs {
  const char* x;
  char* y;
  const _Float16* mask;
  int64_t slices;
  int sq, skv;
  int64_t ldx, sx, ldy, sy, ldm, sm, mgroup;
  int causal;
  float scale;
};

template <typename T>
__global__ __launch_bounds__(256) void softmax_masked(MArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.slices * a.sq) return;
  const int64_t i = row / a.sq;
  const int r = (int)(row - i * a.sq);
  const T* x = (const T*)a.x + i * a.sx + r * a.ldx;
  T* y = (T*)a.y + i * a.sy + r * a.ldy;
  const _Float16* m = a.mask ? a.mask + (i / a.mgroup) * a.sm + (int64_t)r * a.ldm : nullptr;
  // keys past `lim` are removed by the causal rule
  const int lim = a.causal == 1 ? r : a.causal == 2 ? r + a.skv - a.sq : a.skv;
  auto score = [&](int c) {
    float v = (float)x[c] * a.scale;
    if (m) v += (float)m[c];
    return c > lim ? -INFINITY : v;
  };
  float mx = -INFINITY;
  for (int c = lane; c < a.skv; c += 64) mx = fmaxf(mx, score(c));
  mx = wave_max_dpp(mx);
  // a row with every key removed has mx = -inf: exp(-inf - -inf) is NaN, and
  // so is the row, as the reference's max / exp / sum / div decomposition
  float sum = 0.f;
  for (int c = lane; c < a.skv; c += 64) sum += fast_exp(score(c) - mx);
  sum = wave_sum_dpp(sum);
  const float inv = 1.0f / sum;
  for (int c = lane; c < a.skv; c += 64) y[c] = (T)(fast_exp(score(c) - mx) * inv);
}

}  // namespace

hipError_t launch_softmax_masked(const MaskedSoftmaxProblem& p, hipStream_t stream) {
  const int64_t rows = p.slices * p.s_q;
  if (rows == 0 || p.s_kv == 0) return hipSuccess;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
  MArgs a;
  a.x = (const char*)p.x;
  a.y = (char*)p.y;
  a.mask = (const _Float16*)p.mask;
  a.slices = p.slices;
  a.sq = (int)p.s_q;
  a.skv = (int)p.s_kv;
  a.ldx = p.ldx;
  a.sx = p.stride_x;
  a.ldy = p.ldy;
  a.sy = p.stride_y;
  a.ldm = p.ldm;
  a.sm = p.stride_m;
  a.mgroup = p.mask_group;
  a.causal = p.causal;
  a.scale = p.scale;
  if (p.dtype == DT_BF16)
    hipLaunchKernelGGL(softmax_masked<__bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(softmax_masked<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
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
