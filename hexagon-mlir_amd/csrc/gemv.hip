// Decode-shaped y[M,N] = x[M,K] . W[N,K]^T (+bias) for M <= 16, HBM-bound.
//
// The reference has no dedicated GEMV: M = 1 matmuls go through its generic
// HVX matmul schedule (ScheduleMatmulForHVXPass.cpp:69-195, TilingPass.cpp
// :108-251).  Here W is streamed from HBM exactly once:
//   * a workgroup owns TPB tiles of 16 weight rows; its KS waves split K into
//     contiguous ranges so each wave streams long runs of every row;
//   * each lane loads 16 contiguous bytes of a row per step (16 rows x 64 B
//     per wave instruction) straight into the A operand of
//     v_mfma_f32_16x16x32_f16; x (M <= 16 rows, zero-padded by out-of-range
//     buffer loads) is the B operand, so M = 1..16 cost the same HBM bytes;
//   * int8 weights (weight-only quantisation) are converted to fp16 in
//     registers (exact for q in [-128,127]); the per-row scale multiplies the
//     fp32 sum once, after the K reduction;
//   * partial sums of the KS waves are reduced through LDS.
// The MFMA operand layout makes each wave instruction read 64 bytes of 16
// rows, half cache lines.  Three more kernels read whole lines (8 rows x 128
// bytes per wave instruction, non-temporal), which HBM serves faster:
//   * gemv_pair (fp16) / gemv_pair_i8 (int8): long weight matrices with
//     K <= 1024 (the lm_head, gate/up), still on the MFMA units (each row
//     read as two MFMA rows);
//   * gemv_pair_ks: K > 1024 on at most 2048 rows (down projections), the
//     same loads with K split over one workgroup's waves;
//   * gemv_valu: M <= 8 on other long matrices, on the vector ALUs.
#include <type_traits>

#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {

struct VArgs {
  const char* x;
  const char* W;
  const char* scale;
  const char* bias;
  char* y;
  int M, N, K;
  int64_t ldx, ldw, ldy;
  // K split over kg workgroups per row group (kg > 1): workspace with one
  // 64-bit arrival counter per 16-row tile, then kg fp32 partial tiles per
  // tile.  The counters are zero when the launch starts; the last K group of
  // a tile resets its counter to zero, so every launch leaves them zero.
  int kg;
  char* ws;
  int w_cached;  // GemvProblem::w_cached
};

typedef float float2v __attribute__((ext_vector_type(2)));

// 16x16x32 MFMA on fp16 or bf16 operands (T).
template <typename T>
__device__ __forceinline__ float4v mfma16(short8v a, short8v b, float4v c) {
  if constexpr (std::is_same_v<T, __bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, a), __builtin_bit_cast(half8v, b),
                                                  c, 0, 0, 0);
}

// Pairs of T for the vector-ALU dot products: v_dot2_f32_f16 / _bf16.
template <typename T>
struct Pair2 {
  typedef half2v type;
  static __device__ __forceinline__ float dot(type a, type b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};
template <>
struct Pair2<__bf16> {
  typedef bf16x2v type;
  static __device__ __forceinline__ float dot(type a, type b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};

// 8 int8 weights -> 8 exact fp16 (see the GEMM's dequant8 for the method).
__device__ __forceinline__ short8v dequant8v(uint32_t d0, uint32_t d1) {
  short8v out;
  half2v* o = (half2v*)&out;
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;
  o[0] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - bias;
  o[1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - bias;
  o[2] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - bias;
  o[3] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - bias;
  return out;
}

template <typename T, int TPB, int KS, bool I8, int UNR>
__global__ __launch_bounds__(KS * 64) void gemv_mfma(VArgs a) {
  // k covered by one lane-load step: fp16 -> 32 (one MFMA), int8 -> 64 (two)
  constexpr int KSTEP = I8 ? 64 : 32;
  __shared__ float4v red[KS][TPB][64];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = blockIdx.x / a.kg, kgi = blockIdx.x % a.kg;  // row group, K group
  const int n0 = rg * (TPB * 16);
  const int nsteps = (a.K + KSTEP - 1) / KSTEP;
  const int per_group = (nsteps + a.kg - 1) / a.kg;
  const int g_begin = min(nsteps, kgi * per_group);
  const int g_end = min(nsteps, g_begin + per_group);
  const int per_wave = (g_end - g_begin + KS - 1) / KS;
  const int s_begin = g_begin + w * per_wave;
  const int s_end = min(g_end, s_begin + per_wave);

  const int r16 = lane & 15, kq = lane >> 4;  // row within tile, k quarter
  const int esz = I8 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rW = make_rsrc(a.W + (int64_t)n0 * a.ldw * esz, 0x7fffffff);
  const __amdgpu_buffer_rsrc_t rX = make_rsrc(a.x, 0x7fffffff);
  bool rowok[TPB];
  uint32_t wbase[TPB];
#pragma unroll
  for (int t = 0; t < TPB; ++t) {
    rowok[t] = (n0 + t * 16 + r16) < a.N;
    wbase[t] = (uint32_t)((t * 16 + r16) * a.ldw * esz);
  }
  const bool mok = r16 < a.M;
  const uint32_t xbase = (uint32_t)(r16 * a.ldx * 2);

  float4v acc[TPB];
#pragma unroll
  for (int t = 0; t < TPB; ++t) acc[t] = float4v{0.f, 0.f, 0.f, 0.f};

  for (int s0 = s_begin; s0 < s_end; s0 += UNR) {
    int4v wv[UNR][TPB];
    int4v xv[UNR][I8 ? 2 : 1];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int s = s0 + u;
      const bool sok = s < s_end;
      if constexpr (I8) {
        const int k = s * 64 + kq * 16;  // 16 int8 weights per lane
        const bool kok = sok && k < a.K;
#pragma unroll
        for (int t = 0; t < TPB; ++t) wv[u][t] = load16(rW, (kok && rowok[t]) ? wbase[t] + k : kOOB);
        xv[u][0] = load16(rX, (kok && mok) ? xbase + k * 2 : kOOB);
        xv[u][1] = load16(rX, (kok && mok) ? xbase + k * 2 + 16 : kOOB);
      } else {
        const int k = s * 32 + kq * 8;
        const bool kok = sok && k < a.K;
#pragma unroll
        for (int t = 0; t < TPB; ++t) wv[u][t] = load16(rW, (kok && rowok[t]) ? wbase[t] + k * 2 : kOOB);
        xv[u][0] = load16(rX, (kok && mok) ? xbase + k * 2 : kOOB);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
#pragma unroll
      for (int t = 0; t < TPB; ++t) {
        if constexpr (I8) {
          const short8v w0 = dequant8v((uint32_t)wv[u][t][0], (uint32_t)wv[u][t][1]);
          const short8v w1 = dequant8v((uint32_t)wv[u][t][2], (uint32_t)wv[u][t][3]);
          acc[t] = mfma16<T>(w0, __builtin_bit_cast(short8v, xv[u][0]), acc[t]);
          acc[t] = mfma16<T>(w1, __builtin_bit_cast(short8v, xv[u][1]), acc[t]);
        } else {
          acc[t] = mfma16<T>(__builtin_bit_cast(short8v, wv[u][t]), __builtin_bit_cast(short8v, xv[u][0]), acc[t]);
        }
      }
    }
  }

  if constexpr (KS > 1) {
#pragma unroll
    for (int t = 0; t < TPB; ++t) red[w][t][lane] = acc[t];
    __syncthreads();
  }
  // wave w finalises tiles t = w, w + KS, ...
  for (int t = w; t < TPB; t += KS) {
    float4v sum = acc[t];
    if constexpr (KS > 1) {
      sum = red[0][t][lane];
#pragma unroll
      for (int q = 1; q < KS; ++q) sum += red[q][t][lane];
    }
    if (a.kg > 1) {
      // Split K: store this K group's partial tile (system-coherent stores,
      // visible to every XCD once vmcnt drains), arrive on the tile's
      // counter; the last K group adds all partials in K-group order and
      // finishes the tile.
      constexpr int kCoherent = 17;  // sc0 | sc1
      const int tile = rg * TPB + t;  // < kWsMaxTiles (the planner's check)
      unsigned long long* cnt = (unsigned long long*)a.ws + tile;
      float* part = (float*)(a.ws + kWsCounterBytes) + (int64_t)tile * a.kg * 256;
      const __amdgpu_buffer_rsrc_t rP = make_rsrc(part, a.kg * 1024);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4v, sum), rP, (uint32_t)(kgi * 1024 + lane * 16), 0,
                                             kCoherent);
      wait_vmcnt0();
      unsigned long long arrived = 0;
      if (lane == 0) arrived = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      arrived = __shfl(arrived, 0, 64);
      if (arrived + 1 != (unsigned long long)a.kg) continue;
      sum = float4v{0.f, 0.f, 0.f, 0.f};
      for (int g = 0; g < a.kg; ++g)
        sum += __builtin_bit_cast(float4v,
                                  __builtin_amdgcn_raw_buffer_load_b128(rP, (uint32_t)(g * 1024 + lane * 16), 0, kCoherent));
      if (lane == 0) __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // D[n][m]: lane holds m = lane % 16, n = 4*(lane / 16) + 0..3
    const int m = lane & 15;
    const int n = n0 + t * 16 + 4 * (lane >> 4);
    if (m < a.M && n < a.N) {
      float v[4] = {sum[0], sum[1], sum[2], sum[3]};
      if (I8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] *= (float)((const T*)a.scale)[n + q];
      }
      if (a.bias) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] += (float)((const T*)a.bias)[n + q];
      }
      T h[4] = {(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
      *(short4v*)(a.y + ((int64_t)m * a.ldy + n) * 2) = __builtin_bit_cast(short4v, h);
    }
  }
}

// Short-K GEMV on MFMA with whole-line weight loads, for M <= 16 and
// K <= 1024.  A wave owns 8-row weight tiles and walks K in 128-byte windows
// (fp16: 64 k, int8: 128 k); one wave load covers 8 rows x 128 contiguous
// bytes (8 lanes per row), the row-streaming access pattern, which HBM
// serves faster than the 16 rows x 64 bytes of the MFMA operand layout.
// The MFMA 16x16x32 still takes the loaded registers as its A operand by
// reading each weight row as two A rows: A row r' = 2 R + h holds half h of
// row R's window (lane l: r' = l % 16, k group l / 16, 16-byte chunk
// 4 h + l / 16 of the window).  One MFMA multiplies all 16 A rows by x's
// first-half fragments, a second by its second-half fragments; the first
// is right for the h = 0 rows, the second for h = 1, and a row's result is
// the sum of its two valid halves.  That doubles the MFMA work, which
// stays a few percent of the MFMA units at HBM speed.
// (launched for fp16 weights; int8 weights run gemv_pair_i8 below, which
// keeps this layout and overlaps the first tile's loads with x's staging)
template <typename T, bool I8, int NWIN, int U, int YKEEP, bool WNT = true>
__global__ __launch_bounds__(256) void gemv_pair(VArgs a) {
  constexpr int KW = I8 ? 128 : 64;   // k per 128-byte window
  constexpr int FPW = I8 ? 4 : 2;     // x fragments per window
  constexpr int CK = KW / 8;          // k per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rp = lane & 15, kq = lane >> 4;
  const int rr = rp >> 1, hh = rp & 1;
  const int esz = I8 ? 1 : 2;
  const int nwin = (a.K + KW - 1) / KW;
  const int tiles = (a.N + 7) / 8;

  // x fragments, staged once per workgroup: window j, fragment q (half
  // h = q / (FPW / 2), part p = q % (FPW / 2)) holds, for lane l, row l % 16
  // of x at k = KW j + (KW / 2) h + CK (l / 16) + 8 p + [0, 8)
  __shared__ __attribute__((aligned(16))) int4v xs[NWIN * FPW * 64];
  {
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(a.x, 0x7fffffff);
    const bool mok = rp < a.M;
    const uint32_t xbase = (uint32_t)(rp * a.ldx * 2);
#pragma unroll
    for (int f0 = 0; f0 < NWIN * FPW; f0 += 4) {
      const int f = f0 + w;
      const int j = f / FPW, q = f % FPW;
      const int k = KW * j + (KW / 2) * (q / (FPW / 2)) + CK * kq + 8 * (q % (FPW / 2));
      xs[f * 64 + lane] = load16(rX, (mok && k < a.K) ? xbase + (uint32_t)(k * 2) : kOOB);
    }
  }
  __syncthreads();

  const int chunk = hh * 4 + kq;  // this lane's 16-byte chunk of every window
  // The y pair of each of this wave's first YKEEP tiles waits in LDS and is
  // stored after the last tile, so y's scattered 16-byte pieces do not
  // interleave with the weight stream (lm_head M = 16 46.9 -> 44.6-45.2 us;
  // at M = 1, where y is 0.3 MB, deferring cost 0.6 us and YKEEP is 0).
  __shared__ uint32_t ykeep[4][YKEEP > 0 ? YKEEP : 1][64];
  const int m = lane & 15;
  auto store_pair = [&](int n, uint32_t bits) {
    T h2[2];
    __builtin_memcpy(h2, &bits, 4);
    T* yrow = (T*)(a.y + ((int64_t)m * a.ldy + n) * 2);
    if (n + 1 < a.N && ((a.ldy | n) & 1) == 0) {
      *(uint32_t*)yrow = bits;
    } else {
      if (n < a.N) yrow[0] = h2[0];
      if (n + 1 < a.N) yrow[1] = h2[1];
    }
  };
  int it = 0;
  for (int tile = blockIdx.x * 4 + w; tile < tiles; tile += gridDim.x * 4, ++it) {
    const int n0 = tile * 8;
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(a.W + (int64_t)n0 * a.ldw * esz, 0x7fffffff);
    const bool rowok = n0 + rr < a.N;
    const uint32_t wrow = (uint32_t)(rr * a.ldw * esz + chunk * 16);
    // this lane's two output rows: their scale and bias are fetched with the
    // weights, not after the MFMAs (a memory round trip per tile otherwise)
    const int n = n0 + 2 * kq;
    float sc[2] = {1.f, 1.f}, bi[2] = {0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (n + q < a.N) {
        if (I8) sc[q] = (float)((const T*)a.scale)[n + q];
        if (a.bias) bi[q] = (float)((const T*)a.bias)[n + q];
      }
    }
    float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j0 = 0; j0 < NWIN; j0 += U) {
      if (j0 >= nwin) break;
      int4v wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u;
        const bool ok = j < NWIN && rowok && (KW * j + CK * chunk) < a.K;
        const uint32_t off = ok ? wrow + (uint32_t)(j * 128) : kOOB;
        wv[u] = WNT ? load16_nt(rW, off) : load16(rW, off);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u;
        if (j < NWIN) {
          if constexpr (I8) {
            const short8v lo = dequant8v((uint32_t)wv[u][0], (uint32_t)wv[u][1]);
            const short8v hi = dequant8v((uint32_t)wv[u][2], (uint32_t)wv[u][3]);
            acc0 = mfma16<T>(lo, __builtin_bit_cast(short8v, xs[(j * 4 + 0) * 64 + lane]), acc0);
            acc0 = mfma16<T>(hi, __builtin_bit_cast(short8v, xs[(j * 4 + 1) * 64 + lane]), acc0);
            acc1 = mfma16<T>(lo, __builtin_bit_cast(short8v, xs[(j * 4 + 2) * 64 + lane]), acc1);
            acc1 = mfma16<T>(hi, __builtin_bit_cast(short8v, xs[(j * 4 + 3) * 64 + lane]), acc1);
          } else {
            const short8v wf = __builtin_bit_cast(short8v, wv[u]);
            acc0 = mfma16<T>(wf, __builtin_bit_cast(short8v, xs[(j * 2 + 0) * 64 + lane]), acc0);
            acc1 = mfma16<T>(wf, __builtin_bit_cast(short8v, xs[(j * 2 + 1) * 64 + lane]), acc1);
          }
        }
      }
    }
    // D[r'][m]: lane holds m = lane % 16 and A rows r' = 4 (lane / 16) + i,
    // i.e. halves 0, 1 of weight row n and of row n + 1
    {
      float v[2] = {acc0[0] + acc1[1], acc0[2] + acc1[3]};
#pragma unroll
      for (int q = 0; q < 2; ++q) v[q] = v[q] * sc[q] + bi[q];
      T h2[2] = {(T)v[0], (T)v[1]};
      const uint32_t bits = __builtin_bit_cast(uint32_t, h2);
      if (YKEEP > 0 && it < YKEEP) ykeep[w][it][lane] = bits;
      else if (m < a.M) store_pair(n, bits);
    }
  }
  if (YKEEP > 0 && m < a.M) {
    for (int i = 0; i < it && i < YKEEP; ++i)
      store_pair((blockIdx.x * 4 + w + i * gridDim.x * 4) * 8 + 2 * kq, ykeep[w][i][lane]);
  }
}

// gemv_pair for int8 weights, with the first tile's loads issued while x is
// staged: x's fragments are loaded into registers first and the first
// tile's weights right after, so the wait before storing x to LDS covers
// the x loads only and the weights' round trip overlaps the staging (int8
// lm_head at M = 16 29.0 -> 27.1 us on one MI355X).  Scale and bias are one
// 32-bit buffer load each per lane (rows n, n + 1; n is even, N % 4 == 0),
// out of range or absent reading as zero, kept as raw bits until the
// epilogue, so no branch makes the compiler drain the loads in flight.  The
// fp16 kernel keeps the plain order: its compiler schedule interleaves the
// weight loads with the MFMAs in fewer registers, and the same restructure
// measured slower there (lm_head M = 1 40.3 -> 42.1 us).
// YS (M > 4): a workgroup's four waves take four consecutive tiles per
// round; their y meets in LDS and leaves as 64-byte row pieces (16-byte
// stores from one wave) instead of 4-byte stores from every lane.  At M = 16
// the scattered stores cost ~3 us of the lm_head's 25 (a timing copy
// without y stores ran 22.6 us); staged, paired runs on two MI355Xs gained
// 0.25-0.5 us (25.45 -> 24.98, 25.66 -> 25.42).  Rounds of eight
// tiles (two per wave, 128-byte pieces) ran 27.8 us: twice the weight
// streams in flight per wave, as with more workgroups.
template <int NWIN, bool YS>
__global__ __launch_bounds__(256) void gemv_pair_i8(VArgs a) {
  using T = _Float16;
  constexpr bool I8 = true;
  constexpr int KW = I8 ? 128 : 64;   // k per 128-byte window
  constexpr int FPW = I8 ? 4 : 2;     // x fragments per window
  constexpr int CK = KW / 8;          // k per 16-byte chunk
  constexpr int NXF = NWIN * FPW / 4; // x fragments this lane stages
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rp = lane & 15, kq = lane >> 4;
  const int rr = rp >> 1, hh = rp & 1;
  const int esz = I8 ? 1 : 2;
  const int nwin = (a.K + KW - 1) / KW;
  const int tiles = (a.N + 7) / 8;
  const int stride = gridDim.x * 4;
  const int chunk = hh * 4 + kq;  // this lane's 16-byte chunk of every window

  // one tile's loads, all windows at once: weights, scale and bias
  const __amdgpu_buffer_rsrc_t rS = make_rsrc(a.scale, I8 ? (uint32_t)(a.N * 2) : 0u);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.bias, a.bias ? (uint32_t)(a.N * 2) : 0u);
  int4v wv[NWIN];
  uint32_t scb, bib;
  auto fetch = [&](int tile) {
    const int n0 = tile * 8;
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(a.W + (int64_t)n0 * a.ldw * esz, 0x7fffffff);
    const bool rowok = n0 + rr < a.N;
    const uint32_t wrow = (uint32_t)(rr * a.ldw * esz + chunk * 16);
#pragma unroll
    for (int j = 0; j < NWIN; ++j) {
      const bool ok = j < nwin && rowok && (KW * j + CK * chunk) < a.K;
      wv[j] = load16_nt(rW, ok ? wrow + (uint32_t)(j * 128) : kOOB);
    }
    const uint32_t off = (uint32_t)((n0 + 2 * kq) * 2);
    scb = I8 ? __builtin_amdgcn_raw_buffer_load_b32(rS, off, 0, 0) : 0u;
    bib = __builtin_amdgcn_raw_buffer_load_b32(rB, off, 0, 0);
  };

  // x fragments, staged once per workgroup (the layout gemv_pair uses)
  __shared__ __attribute__((aligned(16))) int4v xs[NWIN * FPW * 64];
  int4v xr[NXF];
  {
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(a.x, 0x7fffffff);
    const bool mok = rp < a.M;
    const uint32_t xbase = (uint32_t)(rp * a.ldx * 2);
#pragma unroll
    for (int i = 0; i < NXF; ++i) {
      const int f = 4 * i + w;
      const int j = f / FPW, q = f % FPW;
      const int k = KW * j + (KW / 2) * (q / (FPW / 2)) + CK * kq + 8 * (q % (FPW / 2));
      xr[i] = load16(rX, (mok && k < a.K) ? xbase + (uint32_t)(k * 2) : kOOB);
    }
  }
  // (unconditional: a wave without a tile reads past N, i.e. zeros, and a
  // branch here would make the compiler drain every load at the join)
  int tile = blockIdx.x * 4 + w;
  fetch(tile);
#pragma unroll
  for (int i = 0; i < NXF; ++i) xs[(4 * i + w) * 64 + lane] = xr[i];
  __syncthreads();

  // YS: the same number of rounds for every wave (tiles past the end read
  // zeros and store nothing); a round's first tile is tile - w.  Two LDS
  // buffers, so one barrier a round suffices.
  __shared__ __attribute__((aligned(16))) uint32_t ys[YS ? 2 : 1][16][16];
  const int last = YS ? tiles + w : tiles;
  int it = 0;
  for (bool first = true; tile < last; tile += stride, first = false, ++it) {
    if (!first) fetch(tile);
    {
      float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NWIN; ++j) {
        if (j < nwin) {
          const short8v lo = dequant8v((uint32_t)wv[j][0], (uint32_t)wv[j][1]);
          const short8v hi = dequant8v((uint32_t)wv[j][2], (uint32_t)wv[j][3]);
          acc0 = mfma16<T>(lo, __builtin_bit_cast(short8v, xs[(j * 4 + 0) * 64 + lane]), acc0);
          acc0 = mfma16<T>(hi, __builtin_bit_cast(short8v, xs[(j * 4 + 1) * 64 + lane]), acc0);
          acc1 = mfma16<T>(lo, __builtin_bit_cast(short8v, xs[(j * 4 + 2) * 64 + lane]), acc1);
          acc1 = mfma16<T>(hi, __builtin_bit_cast(short8v, xs[(j * 4 + 3) * 64 + lane]), acc1);
        }
      }
      // D[r'][m]: lane holds m = lane % 16 and A rows r' = 4 (lane / 16) + i,
      // i.e. halves 0, 1 of weight row n and of row n + 1
      const int n = tile * 8 + 2 * kq;
      const int m = lane & 15;
      const half2v s2 = __builtin_bit_cast(half2v, scb), b2 = __builtin_bit_cast(half2v, bib);
      const float sc0 = I8 ? (float)s2[0] : 1.f, sc1 = I8 ? (float)s2[1] : 1.f;
      const float v[2] = {(acc0[0] + acc1[1]) * sc0 + (float)b2[0], (acc0[2] + acc1[3]) * sc1 + (float)b2[1]};
      T h2[2] = {(T)v[0], (T)v[1]};
      const uint32_t bits = __builtin_bit_cast(uint32_t, h2);
      if constexpr (YS) {
        ys[it & 1][m][4 * w + kq] = bits;  // columns 8 w + 2 kq, + 1 of the round
      } else if (m < a.M) {
        T* yrow = (T*)(a.y + ((int64_t)m * a.ldy + n) * 2);
        if (n + 1 < a.N && ((a.ldy | n) & 1) == 0) {
          *(uint32_t*)yrow = bits;
        } else {
          if (n < a.N) yrow[0] = h2[0];
          if (n + 1 < a.N) yrow[1] = h2[1];
        }
      }
    }
    if constexpr (YS) {
      __syncthreads();
      // wave 0 stores the round: lane l takes row l / 4, columns 8 (l % 4) .. + 7
      if (w == 0) {
        const int mr = lane >> 2, c = lane & 3;
        const int n0 = tile * 8 + 8 * c;
        if (mr < a.M && n0 < a.N) {
          const int4v q = *(const int4v*)&ys[it & 1][mr][4 * c];
          T* yrow = (T*)(a.y + ((int64_t)mr * a.ldy + n0) * 2);
          if (n0 + 8 <= a.N && ((a.ldy | n0) & 7) == 0 && ((uintptr_t)a.y & 15) == 0) {
            *(int4v*)yrow = q;
          } else {
            T e[8];
            __builtin_memcpy(e, &q, 16);
            for (int i = 0; i < 8 && n0 + i < a.N; ++i) yrow[i] = e[i];
          }
        }
      }
    }
  }
}

// Long-K GEMV (K > 1024, few rows: down projections) with the same
// whole-line loads and row pairing: one workgroup per 8-row tile, its KS
// waves splitting K into contiguous runs of 128-byte windows, partial sums
// reduced through LDS.  Each wave loads its own x fragments (x is a few KB
// and stays in L2), so a tile costs one memory round trip plus the
// reduction, with no cross-workgroup fix-up.
template <typename T, bool I8, int KS, int U>
__global__ __launch_bounds__(KS * 64) void gemv_pair_ks(VArgs a) {
  constexpr int KW = I8 ? 128 : 64;
  constexpr int FPW = I8 ? 4 : 2;
  constexpr int CK = KW / 8;
  __shared__ float2v red[KS][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rp = lane & 15, kq = lane >> 4;
  const int rr = rp >> 1, hh = rp & 1;
  const int chunk = hh * 4 + kq;
  const int esz = I8 ? 1 : 2;
  const int n0 = blockIdx.x * 8;
  const int nwin = (a.K + KW - 1) / KW;
  const int per = (nwin + KS - 1) / KS;
  const int j_begin = min(nwin, w * per), j_end = min(nwin, j_begin + per);

  const __amdgpu_buffer_rsrc_t rW = make_rsrc(a.W + (int64_t)n0 * a.ldw * esz, 0x7fffffff);
  const __amdgpu_buffer_rsrc_t rX = make_rsrc(a.x, 0x7fffffff);
  const bool rowok = n0 + rr < a.N;
  const uint32_t wrow = (uint32_t)(rr * a.ldw * esz + chunk * 16);
  const bool mok = rp < a.M;
  const uint32_t xbase = (uint32_t)(rp * a.ldx * 2);
  // scale and bias of the lane's two output rows, fetched up front (wave 0
  // applies them after the reduction)
  const int n = n0 + 2 * kq;
  float sc[2] = {1.f, 1.f}, bi[2] = {0.f, 0.f};
  if (w == 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (n + q < a.N) {
        if (I8) sc[q] = (float)((const T*)a.scale)[n + q];
        if (a.bias) bi[q] = (float)((const T*)a.bias)[n + q];
      }
    }
  }

  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = j_begin; j0 < j_end; j0 += U) {
    int4v wv[U], xv[U][FPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u;
      const bool jok = j < j_end;
      wv[u] = load16_nt(rW, (jok && rowok && (KW * j + CK * chunk) < a.K) ? wrow + (uint32_t)(j * 128) : kOOB);
#pragma unroll
      for (int q = 0; q < FPW; ++q) {
        const int k = KW * j + (KW / 2) * (q / (FPW / 2)) + CK * kq + 8 * (q % (FPW / 2));
        xv[u][q] = load16(rX, (jok && mok && k < a.K) ? xbase + (uint32_t)(k * 2) : kOOB);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u < j_end) {
        if constexpr (I8) {
          const short8v lo = dequant8v((uint32_t)wv[u][0], (uint32_t)wv[u][1]);
          const short8v hi = dequant8v((uint32_t)wv[u][2], (uint32_t)wv[u][3]);
          acc0 = mfma16<T>(lo, __builtin_bit_cast(short8v, xv[u][0]), acc0);
          acc0 = mfma16<T>(hi, __builtin_bit_cast(short8v, xv[u][1]), acc0);
          acc1 = mfma16<T>(lo, __builtin_bit_cast(short8v, xv[u][2]), acc1);
          acc1 = mfma16<T>(hi, __builtin_bit_cast(short8v, xv[u][3]), acc1);
        } else {
          const short8v wf = __builtin_bit_cast(short8v, wv[u]);
          acc0 = mfma16<T>(wf, __builtin_bit_cast(short8v, xv[u][0]), acc0);
          acc1 = mfma16<T>(wf, __builtin_bit_cast(short8v, xv[u][1]), acc1);
        }
      }
    }
  }
  // lane: column m = lane % 16 of weight rows n0 + 2 (lane / 16) + {0, 1}
  red[w][lane] = float2v{acc0[0] + acc1[1], acc0[2] + acc1[3]};
  __syncthreads();
  if (w != 0) return;
  float2v s = red[0][lane];
#pragma unroll
  for (int q = 1; q < KS; ++q) s += red[q][lane];
  const int m = lane & 15;
  if (m < a.M) {
    float v[2] = {s[0], s[1]};
#pragma unroll
    for (int q = 0; q < 2; ++q) v[q] = v[q] * sc[q] + bi[q];
    T* yrow = (T*)(a.y + ((int64_t)m * a.ldy + n) * 2);
    if (n + 1 < a.N && ((a.ldy | n) & 1) == 0) {
      T h2[2] = {(T)v[0], (T)v[1]};
      *(uint32_t*)yrow = __builtin_bit_cast(uint32_t, h2);
    } else {
      if (n < a.N) yrow[0] = (T)v[0];
      if (n + 1 < a.N) yrow[1] = (T)v[1];
    }
  }
}

template <typename T, bool I8>
hipError_t launch_pair_ks(const VArgs& v, int ks, hipStream_t stream) {
  const int blocks = (v.N + 7) / 8;
  if (ks >= 16)
    hipLaunchKernelGGL((gemv_pair_ks<T, I8, 16, I8 ? 4 : 8>), dim3(blocks), dim3(1024), 0, stream, v);
  else
    hipLaunchKernelGGL((gemv_pair_ks<T, I8, 8, I8 ? 4 : 8>), dim3(blocks), dim3(512), 0, stream, v);
  return hipGetLastError();
}

template <typename T, bool I8>
hipError_t launch_pair(const VArgs& v, hipStream_t stream) {
  const int tiles = (v.N + 7) / 8;
  int blocks = (tiles + 3) / 4;
  // waves striding over the tiles, measured on the 896 -> 151936 lm_head
  // at M = 16: fp16 four workgroups per CU (512 / 768 / 1024 / 1280 / 2048
  // workgroups gave 49.3 / 47.7 / 46.5 / 55.4 / 48.5 us), int8 two (384 /
  // 448 / 512 / 576 / 640 / 1024 gave 28.0 / 26.7 / 25.3 / 31.4 / 29.1 /
  // 27.0 us: half the bytes per tile, and fewer concurrent row streams)
  int cap = I8 ? 512 : 1024;
  if (const int64_t e = knob(KNOB_GEMV_PAIR_WG); e != KNOB_UNSET && e > 0) cap = e < (1 << 20) ? (int)e : (1 << 20);
  if (blocks > cap) blocks = cap;
  if constexpr (I8) {
    if (v.M > 4)
      hipLaunchKernelGGL((gemv_pair_i8<8, true>), dim3(blocks), dim3(256), 0, stream, v);
    else
      hipLaunchKernelGGL((gemv_pair_i8<8, false>), dim3(blocks), dim3(256), 0, stream, v);
  }
  else if (v.M > 4)
    hipLaunchKernelGGL((gemv_pair<T, false, 16, 16, 6>), dim3(blocks), dim3(256), 0, stream, v);
  else if (v.w_cached)
    hipLaunchKernelGGL((gemv_pair<T, false, 16, 16, 0, false>), dim3(blocks), dim3(256), 0, stream, v);
  else
    hipLaunchKernelGGL((gemv_pair<T, false, 16, 16, 0>), dim3(blocks), dim3(256), 0, stream, v);
  return hipGetLastError();
}

// Row-streaming GEMV on the vector ALUs for M <= MM (MM <= 16).  A wave owns
// groups of 8 weight rows; lane l covers row l / 8 and the 16-byte chunk
// l % 8 of every 128-byte K-step (8 k for fp16 weights, 16 for int8), so one
// wave load is 8 rows x 128 contiguous bytes.  x (M x K, zero-padded to whole
// K-steps) is staged in LDS once per workgroup; the 8 partial dot products of
// a row are summed with lane shuffles at the end.  Workgroups stride over the
// row groups so each stages x once.
template <typename T, int MM, bool I8, int U>
__global__ __launch_bounds__(256) void gemv_valu(VArgs a, int kpad) {
  constexpr int WPB = 4;
  constexpr int KC = I8 ? 16 : 8;  // k per lane load
  constexpr int KSTEP = KC * 8;    // k per wave step
  extern __shared__ __attribute__((aligned(16))) char xs[];  // [M][kpad] fp16
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 3, c = lane & 7;
  const int esz = I8 ? 1 : 2;
  const int M = a.M;
  const int nsteps = kpad / KSTEP;
  const int groups = (a.N + 7) / 8;

  // stage x: 16-byte chunks, zero past K
  const int cpr = kpad / 8;
  const __amdgpu_buffer_rsrc_t rX = make_rsrc(a.x, 0x7fffffff);
  for (int i = threadIdx.x; i < M * cpr; i += WPB * 64) {
    const int m = i / cpr, k = (i % cpr) * 8;
    *(int4v*)(xs + ((int64_t)m * kpad + k) * 2) = load16(rX, k < a.K ? (uint32_t)((m * a.ldx + k) * 2) : kOOB);
  }
  __syncthreads();

  for (int g = blockIdx.x * WPB + w; g < groups; g += gridDim.x * WPB) {
    const int row = g * 8 + r;
    const bool rok = row < a.N;
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(a.W + (int64_t)g * 8 * a.ldw * esz, 0x7fffffff);
    const uint32_t wrow = (uint32_t)(r * a.ldw * esz);
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[m] = 0.f;
    for (int s0 = 0; s0 < nsteps; s0 += U) {
      int4v wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = (s0 + u) * KSTEP + c * KC;
        wv[u] = load16_nt(rW, (rok && k < a.K) ? wrow + (uint32_t)(k * esz) : kOOB);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (s0 + u < nsteps) {
          const int k = (s0 + u) * KSTEP + c * KC;
          typename Pair2<T>::type wh[KC / 2];
          if constexpr (I8) {
            const short8v lo = dequant8v((uint32_t)wv[u][0], (uint32_t)wv[u][1]);
            const short8v hi = dequant8v((uint32_t)wv[u][2], (uint32_t)wv[u][3]);
            __builtin_memcpy(&wh[0], &lo, 16);
            __builtin_memcpy(&wh[4], &hi, 16);
          } else {
            __builtin_memcpy(&wh[0], &wv[u], 16);
          }
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            if (m < M) {
              typename Pair2<T>::type xh[KC / 2];
              const char* xp = xs + ((int64_t)m * kpad + k) * 2;
              __builtin_memcpy(&xh[0], xp, 16);
              if constexpr (I8) __builtin_memcpy(&xh[4], xp + 16, 16);
#pragma unroll
              for (int q = 0; q < KC / 2; ++q) acc[m] = Pair2<T>::dot(wh[q], xh[q], acc[m]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      acc[m] += __shfl_xor(acc[m], 1, 64);
      acc[m] += __shfl_xor(acc[m], 2, 64);
      acc[m] += __shfl_xor(acc[m], 4, 64);
    }
    // lane c writes output rows m = c, c + 8
#pragma unroll
    for (int m0 = 0; m0 < MM; m0 += 8) {
      float v = 0.f;
#pragma unroll
      for (int m = m0; m < MM && m < m0 + 8; ++m)
        if (c == m - m0) v = acc[m];
      if (rok && m0 + c < M) {
        if (I8) v *= (float)((const T*)a.scale)[row];
        if (a.bias) v += (float)((const T*)a.bias)[row];
        ((T*)a.y)[(int64_t)(m0 + c) * a.ldy + row] = (T)v;
      }
    }
  }
}

template <typename T, int MM, bool I8>
hipError_t launch_valu(const VArgs& v, hipStream_t stream) {
  constexpr int KSTEP = I8 ? 128 : 64;
  const int kpad = (v.K + KSTEP - 1) / KSTEP * KSTEP;
  const int groups = (v.N + 7) / 8;
  int blocks = (groups + 3) / 4;
  const int cap = 256 * 8;  // enough workgroups to fill every CU several times over
  if (blocks > cap) blocks = cap;
  const size_t lds = (size_t)v.M * kpad * 2;
  hipLaunchKernelGGL((gemv_valu<T, MM, I8, 8>), dim3(blocks), dim3(256), lds, stream, v, kpad);
  return hipGetLastError();
}

template <typename T, bool I8>
hipError_t launch_valu_sel(const VArgs& v, hipStream_t stream) {
  if (v.M == 1) return launch_valu<T, 1, I8>(v, stream);
  if (v.M == 2) return launch_valu<T, 2, I8>(v, stream);
  if (v.M <= 4) return launch_valu<T, 4, I8>(v, stream);
  if (v.M <= 8) return launch_valu<T, 8, I8>(v, stream);
  return launch_valu<T, 16, I8>(v, stream);
}

template <typename T, int TPB, int KS, bool I8>
hipError_t launch_cfg(const VArgs& v, hipStream_t stream) {
  // loads in flight per wave: a wave whose K range is long (few tiles, large
  // K) issues 16 steps at a time; short ranges keep 4 (2 for 4-tile groups)
  const int kstep = I8 ? 64 : 32;
  const int per_wave = ((v.K + kstep - 1) / kstep + KS * v.kg - 1) / (KS * v.kg);
  const int blocks = (v.N + TPB * 16 - 1) / (TPB * 16) * v.kg;
  int unr = TPB >= 4 ? 2 : (per_wave >= 12 ? (TPB == 1 ? 16 : 8) : 4);
  if (const int64_t e = knob(KNOB_GEMV_UNR); e != KNOB_UNSET) unr = e >= 16 ? 16 : (e >= 8 ? 8 : (TPB >= 4 ? 2 : 4));
  if constexpr (TPB < 4) {
    if (unr == 16 && TPB == 1) {
      hipLaunchKernelGGL((gemv_mfma<T, 1, KS, I8, 16>), dim3(blocks), dim3(KS * 64), 0, stream, v);
      return hipGetLastError();
    }
    // (16 waves per workgroup leave 128 VGPRs: 8 steps of two tiles would spill)
    if constexpr (TPB == 1 || KS <= 8) {
      if (unr == 8) {
        hipLaunchKernelGGL((gemv_mfma<T, TPB, KS, I8, 8>), dim3(blocks), dim3(KS * 64), 0, stream, v);
        return hipGetLastError();
      }
    }
  }
  hipLaunchKernelGGL((gemv_mfma<T, TPB, KS, I8, (TPB >= 4 ? 2 : 4)>), dim3(blocks), dim3(KS * 64), 0, stream, v);
  return hipGetLastError();
}

template <typename T, bool I8>
hipError_t launch_sel(int tpb, int ks, const VArgs& v, hipStream_t stream) {
  if (tpb == 4) {
    if (ks == 4) return launch_cfg<T, 4, 4, I8>(v, stream);
    if (ks == 8) return launch_cfg<T, 4, 8, I8>(v, stream);
    return launch_cfg<T, 4, 16, I8>(v, stream);
  }
  if (tpb == 2) {
    if (ks == 4) return launch_cfg<T, 2, 4, I8>(v, stream);
    if (ks == 8) return launch_cfg<T, 2, 8, I8>(v, stream);
    return launch_cfg<T, 2, 16, I8>(v, stream);
  }
  if (ks == 4) return launch_cfg<T, 1, 4, I8>(v, stream);
  if (ks == 8) return launch_cfg<T, 1, 8, I8>(v, stream);
  return launch_cfg<T, 1, 16, I8>(v, stream);
}

}  // namespace

// Launch plan of a decode GEMV: rows per workgroup (TPB tiles of 16), waves
// splitting K inside a workgroup (KS), the row-streaming kernel (valu), and
// K groups across workgroups (kg).
struct GemvPlan {
  int tpb = 1, ks = 8, kg = 1;
  bool valu = false, pair = false, pair_ks = false;
};

static GemvPlan gemv_plan(const GemvProblem& p) {
  GemvPlan g;
  // TPB and KS from a sweep of every (TPB, KS) on the Qwen2.5-0.5B decode
  // shapes: one 16-row tile per workgroup keeps the most workgroups in flight
  // for M <= 4; for M > 4 the x fragments are shared by more rows (TPB 2-4)
  // once there are enough tiles; 8 waves per workgroup unless a wave would
  // get < 2 K-steps.
  const int64_t tiles16 = (p.N + 15) / 16;
  if (p.M > 4) g.tpb = tiles16 >= 600 ? 4 : (tiles16 >= 300 ? 2 : 1);
  if (p.w_int8 && p.M <= 4 && tiles16 >= 4096) g.tpb = 2;
  const int kstep = p.w_int8 ? 64 : 32;
  const int64_t nsteps = (p.K + kstep - 1) / kstep;
  while (g.ks > 4 && nsteps / g.ks < 2) g.ks /= 2;
  // tuning overrides (launch shape only; every shape computes the same sums)
  const int64_t ks_knob = knob(KNOB_GEMV_KS);
  if (const int64_t e = knob(KNOB_GEMV_TPB); e != KNOB_UNSET) g.tpb = e == 4 ? 4 : (e == 2 ? 2 : 1);
  if (ks_knob != KNOB_UNSET) g.ks = ks_knob >= 16 ? 16 : (ks_knob >= 8 ? 8 : 4);
  // Measured on the Qwen2.5-0.5B shapes (graph replays, weights rotating
  // past the Infinity Cache):
  //  * whole-line MFMA kernel (K <= 1024): long weight matrices -- lm_head
  //    M = 16 54.8 -> 46.3 us and M = 4 44.0 -> 41.2 us against the other
  //    two, gate/up 896 -> 9728 at M = 16 8.3 -> 7.0 us; even at fp16
  //    M = 1; int8 at every M once N >= 16384 fills its 512 workgroups
  //    (lm_head M = 1 / 4 21.9 / 22.1 us against 22.5 / 27.3 with row
  //    streaming; 896 -> 32000 at M = 1 / 4 7.1 / 7.3 against 8.2 / 9.1),
  //    int8 M <= 4 level with the other kernels below that; behind the
  //    16-row MFMA tiles below N ~ 8192 (too few 8-row tiles to fill the
  //    GPU);
  //  * vector-ALU row streaming: fp16 M = 1 from N = 4096, and M <= 8
  //    (int8 M <= 4) from N = 32768 where K is too long for the whole-line
  //    kernel;
  //  * whole-line kernel with K split over a workgroup's waves: K > 1024
  //    on at most 2048 rows (down projections; one workgroup per 8-row
  //    tile, so at most 256 workgroups): 4864 -> 896 at M = 1 8.1 -> 5.7 us,
  //    5632 -> 2048 9.6 -> 6.7 us, 2048 -> 896 at M = 16 6.3 -> 4.9 us; 16
  //    waves only where each still gets >= 4 windows (M > 4: 4864 -> 896 at
  //    M = 16 8.7 -> 8.5 us); behind the 16-row tiles from N = 2560;
  //  * the 16-row MFMA tiles elsewhere (K split across waves).
  const int kstep_v = p.w_int8 ? 128 : 64;
  const int64_t kpad = (p.K + kstep_v - 1) / kstep_v * kstep_v;
  const bool fits = p.M <= 16 && p.M * kpad * 2 <= 64 * 1024;
  const bool xfits = p.K <= 1024;
  g.pair = xfits && p.N >= 8192 && (!p.w_int8 || p.M > 4 || p.N >= 16384);
  g.pair_ks = !xfits && p.N <= 2048;
  if (g.pair_ks) {
    const int64_t nwin = (p.K + (p.w_int8 ? 127 : 63)) / (p.w_int8 ? 128 : 64);
    g.ks = (p.M > 4 && nwin >= 64) ? 16 : 8;
    if (ks_knob != KNOB_UNSET) g.ks = ks_knob >= 16 ? 16 : 8;
  }
  g.valu = !g.pair && !g.pair_ks && fits && p.M <= 8 &&
           (p.w_int8 ? (p.N >= 32768 && p.M <= 4) : ((p.N >= 32768) || (p.M == 1 && p.N >= 4096)));
  if (const int64_t e = knob(KNOB_GEMV_PATH); e != KNOB_UNSET) {
    g.valu = e == GEMV_PATH_VALU && fits;
    g.pair = e == GEMV_PATH_PAIR && xfits;
    g.pair_ks = e == GEMV_PATH_PAIR_KS;
    if (g.pair_ks && ks_knob == KNOB_UNSET) g.ks = 8;
  }
  if (g.valu || g.pair || g.pair_ks) return g;
  // few row groups, each streaming a long K (e.g. a down projection
  // 4864 -> 896): split K over 2-4 workgroups per row group.  Combining the
  // partial tiles costs ~2 us of round trips to memory, so (measured on the
  // Qwen2.5-0.5B and TinyLlama down projections, M 1-16) it pays from
  // ~144 KiB of weights per workgroup (M > 8 does twice the MFMA work per
  // byte: 72 KiB)
  const int64_t groups = (p.N + g.tpb * 16 - 1) / (g.tpb * 16);
  const int64_t wg_bytes = (int64_t)g.tpb * 16 * p.K * (p.w_int8 ? 1 : 2) * (p.M > 8 ? 2 : 1);
  if (groups < 192 && wg_bytes >= (144 << 10)) {
    int kg = (int)((192 + groups / 2) / groups);
    kg = kg < 2 ? 2 : (kg > 4 ? 4 : kg);
    while (kg > 1 && nsteps / kg < 2 * g.ks) --kg;
    g.kg = kg;
  }
  if (const int64_t e = knob(KNOB_GEMV_KG); e != KNOB_UNSET) g.kg = e < 1 ? 1 : (e > 16 ? 16 : (int)e);
  return g;
}

int64_t gemv_workspace_bytes(const GemvProblem& p) {
  const GemvPlan g = gemv_plan(p);
  if (g.valu || g.pair || g.pair_ks || g.kg <= 1) return 0;
  const int64_t tiles = (p.N + g.tpb * 16 - 1) / (g.tpb * 16) * g.tpb;  // 16-row tiles of whole row groups
  return tiles > kWsMaxTiles ? 0 : kWsCounterBytes + tiles * g.kg * 1024;
}

hipError_t launch_gemv(const GemvProblem& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  VArgs v;
  v.x = (const char*)p.x;
  v.W = (const char*)p.W;
  v.scale = (const char*)p.scale;
  v.bias = (const char*)p.bias;
  v.y = (char*)p.y;
  v.M = (int)p.M;
  v.N = (int)p.N;
  v.K = (int)p.K;
  v.ldx = p.ldx;
  v.ldw = p.ldw;
  v.ldy = p.ldy;
  v.kg = 1;
  v.ws = nullptr;
  v.w_cached = p.w_cached;
  const GemvPlan g = gemv_plan(p);
  const bool bf = p.dtype == DT_BF16;  // bf16 x, W, bias, y (fp16 weights otherwise; int8 takes fp16 x)
  if (g.valu)
    return p.w_int8 ? launch_valu_sel<_Float16, true>(v, stream)
                    : (bf ? launch_valu_sel<__bf16, false>(v, stream) : launch_valu_sel<_Float16, false>(v, stream));
  if (g.pair)
    return p.w_int8 ? launch_pair<_Float16, true>(v, stream)
                    : (bf ? launch_pair<__bf16, false>(v, stream) : launch_pair<_Float16, false>(v, stream));
  if (g.pair_ks)
    return p.w_int8 ? launch_pair_ks<_Float16, true>(v, g.ks, stream)
                    : (bf ? launch_pair_ks<__bf16, false>(v, g.ks, stream)
                          : launch_pair_ks<_Float16, false>(v, g.ks, stream));
  const int64_t need = g.kg > 1 ? gemv_workspace_bytes(p) : 0;
  if (need > 0 && p.ws && p.ws_bytes >= need && ((uintptr_t)p.ws % 256) == 0) {
    v.kg = g.kg;
    v.ws = (char*)p.ws;
  }
  return p.w_int8 ? launch_sel<_Float16, true>(g.tpb, g.ks, v, stream)
                  : (bf ? launch_sel<__bf16, false>(g.tpb, g.ks, v, stream)
                        : launch_sel<_Float16, false>(g.tpb, g.ks, v, stream));
}

}  // namespace hxmi
