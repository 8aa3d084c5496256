// GEMM dispatch: alignment checks, tile choice, and the element-wise kernel
// used for operands the MFMA fast path cannot take (odd strides, K or N not a
// multiple of 8, misaligned pointers).
#include <stdlib.h>

#include "gemm_impl.h"

namespace hxmi {
namespace gemm {
hipError_t launch_fast_f16(int tile, bool nn, int epi, bool out_f32, bool rms, const KArgs& k, hipStream_t s);
hipError_t launch_fast_bf16(int tile, bool nn, int epi, bool out_f32, const KArgs& k, hipStream_t s);
hipError_t launch_fast_w8(int tile, int epi, bool out_f32, const KArgs& k, hipStream_t s);

namespace {

struct GArgs {
  const char* A;
  const char* B;
  char* C;
  const char* bias;
  int64_t M, N, K, Nout;
  int64_t lda, ldb, ldc, sA, sB, sC, batch;
  float alpha;
  int nn, epi, out_f32;
  int rms;  // scale each output row by rsqrt(mean(A[m,:]^2) + rms_eps)
  float rms_eps;
};

template <typename T>
__device__ __forceinline__ float ld(const char* p, int64_t i) {
  return (float)((const T*)p)[i];
}

// One thread per output element; fp32 accumulation in k order.
template <typename T>
__global__ __launch_bounds__(256) void gemm_elementwise(GArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_batch = a.M * a.Nout;
  if (idx >= per_batch * a.batch) return;
  const int64_t b = idx / per_batch;
  const int64_t r = idx - b * per_batch;
  const int64_t m = r / a.Nout, o = r - m * a.Nout;
  const char* A = a.A + b * a.sA * (int64_t)sizeof(T);
  const char* B = a.B + b * a.sB * (int64_t)sizeof(T);
  // packed gate/up columns for SiLU-mul: output o reads packed columns
  // 32*(o/16) + o%16 (gate) and that + 16 (up)
  const int64_t c0 = (a.epi == EPI_SILU_MUL) ? 32 * (o / 16) + (o % 16) : o;
  const int64_t c1 = c0 + 16;
  float acc0 = 0.f, acc1 = 0.f;
  for (int64_t k = 0; k < a.K; ++k) {
    const float av = ld<T>(A, m * a.lda + k);
    const float b0 = a.nn ? ld<T>(B, k * a.ldb + c0) : ld<T>(B, c0 * a.ldb + k);
    acc0 += av * b0;
    if (a.epi == EPI_SILU_MUL) {
      const float b1 = a.nn ? ld<T>(B, k * a.ldb + c1) : ld<T>(B, c1 * a.ldb + k);
      acc1 += av * b1;
    }
  }
  if (a.rms) {
    float ss = 0.f;
    for (int64_t k = 0; k < a.K; ++k) {
      const float av = ld<T>(A, m * a.lda + k);
      ss += av * av;
    }
    const float r = rsqrtf(ss / (float)a.K + a.rms_eps);
    acc0 *= r;
    acc1 *= r;
  }
  float v = acc0 * a.alpha;
  if (a.epi == EPI_SILU_MUL) {
    v = silu(v) * (acc1 * a.alpha);
  } else {
    if (a.epi == EPI_BIAS || a.epi == EPI_BIAS_GELU_TANH) v += ld<T>(a.bias, o);
    if (a.epi == EPI_GELU_TANH || a.epi == EPI_BIAS_GELU_TANH) v = gelu_tanh(v);
  }
  if (a.out_f32)
    ((float*)a.C)[b * a.sC + m * a.ldc + o] = v;
  else
    ((T*)a.C)[b * a.sC + m * a.ldc + o] = (T)v;
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace
}  // namespace gemm

bool gemm_fast_path_ok(const GemmProblem& p) {
  const bool i8 = p.dtype == DT_W8A16;
  if (p.K % (i8 ? 16 : 8) || p.N % (p.epilogue == EPI_SILU_MUL ? 32 : 8)) return false;
  if (p.lda % 8 || p.ldb % (i8 ? 16 : 8) || p.ldc % 8) return false;
  if (p.batch > 1 && (p.sA % 8 || p.sB % (i8 ? 16 : 8) || p.sC % 8)) return false;
  if (!gemm::aligned(p.A, 16) || !gemm::aligned(p.B, 16) || !gemm::aligned(p.C, 16)) return false;
  if (p.bias && !gemm::aligned(p.bias, 8)) return false;
  // 32-bit buffer offsets inside one tile row-panel
  if ((int64_t)256 * p.lda * 2 >= (1ll << 31) || (int64_t)256 * p.ldb * 2 >= (1ll << 31)) return false;
  if (p.M >= (1ll << 31) || p.N >= (1ll << 31) || p.K >= (1ll << 31)) return false;
  if (p.b_nt == 0 && i8) return false;
  return true;
}

// Pick the tile that minimises an estimate of makespan: rounds of tiles over
// the 256 CUs (with the tiles a CU holds at once) times a per-tile cost that
// reflects each shape's MFMA efficiency.
int gemm_pick_tile(const GemmProblem& p) {
  struct Cand {
    int id, bm, bn, per_cu;
    float eff;
  };
  // (the 8-wave 128x128 tile at two per CU outruns one 256x128 per CU on the
  // 512-token LLaMA MLP GEMMs; measured on the block shapes)
  static const Cand cands[] = {
      {TILE_256x256_W8, 256, 256, 1, 1.00f}, {TILE_256x128_W8, 256, 128, 1, 0.85f},
      {TILE_128x256, 128, 256, 1, 0.80f},    {TILE_128x128_W8, 128, 128, 2, 0.90f},
      {TILE_64x128, 64, 128, 3, 0.50f},      {TILE_128x64, 128, 64, 3, 0.50f},
      {TILE_64x64, 64, 64, 4, 0.40f},
  };
  const int cus = 256;
  int best = TILE_64x64;
  double best_t = 1e300;
  for (const Cand& c : cands) {
    if (c.bn == 64 && p.epilogue == EPI_SILU_MUL) continue;
    const int64_t tm = (p.M + c.bm - 1) / c.bm, tn = (p.N + c.bn - 1) / c.bn;
    const int64_t tiles = tm * tn * p.batch;
    const int64_t slots = (int64_t)cus * c.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    const int64_t conc = tiles < slots ? (tiles + cus - 1) / cus : c.per_cu;  // tiles sharing a CU
    const double t = (double)rounds * c.bm * c.bn * (double)(conc > 0 ? conc : 1) / c.eff;
    if (t < best_t * 0.999) {
      best_t = t;
      best = c.id;
    }
  }
  return best;
}

namespace gemm {
namespace {

struct ReduceArgs {
  const float* W;  // [splits][M][N] fp32 partial sums
  char* C;
  const char* bias;
  int64_t M, N, Nout, ldc, splits;
  float alpha;
  int epi;
};

// Split-K reduction + epilogue: every thread produces 4 consecutive output
// columns from the fp32 partial sums (for SiLU-mul, 4 gate and the 4 up
// columns 16 further along in the packed layout).
template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce(ReduceArgs r) {
  const int64_t groups = r.Nout / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= r.M * groups) return;
  const int64_t m = idx / groups;
  const int64_t o = (idx - m * groups) * 4;
  const int64_t plane = r.M * r.N;
  float v[4];
  if (r.epi == EPI_SILU_MUL) {
    const int64_t pc = 32 * (o / 16) + (o % 16);
    float4v g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    for (int64_t s = 0; s < r.splits; ++s) {
      g += *(const float4v*)(r.W + s * plane + m * r.N + pc);
      u += *(const float4v*)(r.W + s * plane + m * r.N + pc + 16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = silu(g[q] * r.alpha) * (u[q] * r.alpha);
  } else {
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    for (int64_t s = 0; s < r.splits; ++s) acc += *(const float4v*)(r.W + s * plane + m * r.N + o);
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = acc[q] * r.alpha;
    if (r.epi == EPI_BIAS || r.epi == EPI_BIAS_GELU_TANH) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += (float)((const T*)r.bias)[o + q];
    }
    if (r.epi == EPI_GELU_TANH || r.epi == EPI_BIAS_GELU_TANH) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = gelu_tanh(v[q]);
    }
  }
  T t[4] = {(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
  *(short4v*)(r.C + (m * r.ldc + o) * (int64_t)sizeof(T)) = __builtin_bit_cast(short4v, t);
}

int tile_for(const GemmProblem& p) {
  int tile = p.tile >= 0 ? p.tile : env_int("HXMI_GEMM_TILE", -1);
  if (tile < 0 || tile >= TILE_COUNT) tile = gemm_pick_tile(p);
  if (p.epilogue == EPI_SILU_MUL && kTiles[tile].BN < 128) tile = TILE_64x128;
  return tile;
}

KArgs make_kargs(const GemmProblem& p, int tile) {
  const TileShape s = kTiles[tile];
  KArgs k{};
  k.A = (const char*)p.A;
  k.B = (const char*)p.B;
  k.C = (char*)p.C;
  k.bias = (const char*)p.bias;
  k.scale = (const char*)p.scale;
  k.M = (int)p.M;
  k.N = (int)p.N;
  k.K = (int)p.K;
  k.lda = p.lda;
  k.ldb = p.ldb;
  k.ldc = p.ldc;
  k.sA = p.sA;
  k.sB = p.sB;
  k.sC = p.sC;
  k.batch = (int)p.batch;
  k.alpha = p.alpha;
  k.tiles_m = (int)((p.M + s.BM - 1) / s.BM);
  k.tiles_n = (int)((p.N + s.BN - 1) / s.BN);
  const int gm = env_int("HXMI_GROUP_M", 4);
  k.group_m = gm < 1 ? 1 : (gm > k.tiles_m ? k.tiles_m : gm);
  k.k_last = 0;
  k.rms_eps = p.rms_eps;
  return k;
}

hipError_t launch_fast(const GemmProblem& p, int tile, const KArgs& k, hipStream_t stream) {
  if ((int64_t)k.tiles_m * k.tiles_n * k.batch >= (1ll << 31)) return hipErrorInvalidValue;
  if (p.rms && p.dtype != DT_F16) return hipErrorNotSupported;
  if (p.dtype == DT_W8A16) return launch_fast_w8(tile, p.epilogue, p.out_f32, k, stream);
  if (p.dtype == DT_BF16) return launch_fast_bf16(tile, !p.b_nt, p.epilogue, p.out_f32, k, stream);
  return launch_fast_f16(tile, !p.b_nt, p.epilogue, p.out_f32, p.rms != 0, k, stream);
}

}  // namespace
}  // namespace gemm

// Split K into slices when the output has too few tiles to occupy the 256
// CUs and K is long enough that each slice still runs many K-steps.
int gemm_splits(const GemmProblem& p) {
  if (p.batch != 1 || p.out_f32 || p.rms || p.K < 2048 || !gemm_fast_path_ok(p)) return 1;
  if (const char* e = getenv("HXMI_SPLITK")) return atoi(e) < 1 ? 1 : (atoi(e) > 16 ? 16 : atoi(e));
  // 128x128 output tiles are the unit of work split-K is judged by; below
  // K = 3072 the extra reduction pass costs more than the idle CUs
  const int64_t tiles = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (tiles >= 128 || p.K < 3072) return 1;
  int s = 1;
  while (s < 8 && tiles * s < 256 && p.K / (2 * s) >= 1024) s *= 2;
  return s;
}

int64_t gemm_workspace_bytes(const GemmProblem& p) {
  const int s = gemm_splits(p);
  return s > 1 ? (int64_t)s * p.M * p.N * 4 : 0;
}

hipError_t launch_gemm(const GemmProblem& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return hipSuccess;
  const bool i8 = p.dtype == DT_W8A16;
  if (!gemm_fast_path_ok(p)) {
    if (i8) return hipErrorNotSupported;
    gemm::GArgs g;
    g.A = (const char*)p.A;
    g.B = (const char*)p.B;
    g.C = (char*)p.C;
    g.bias = (const char*)p.bias;
    g.M = p.M;
    g.N = p.N;
    g.K = p.K;
    g.Nout = p.epilogue == EPI_SILU_MUL ? p.N / 2 : p.N;
    g.lda = p.lda;
    g.ldb = p.ldb;
    g.ldc = p.ldc;
    g.sA = p.sA;
    g.sB = p.sB;
    g.sC = p.sC;
    g.batch = p.batch;
    g.alpha = p.alpha;
    g.nn = !p.b_nt;
    g.epi = p.epilogue;
    g.out_f32 = p.out_f32;
    g.rms = p.rms;
    g.rms_eps = p.rms_eps;
    const int64_t total = p.batch * p.M * g.Nout;
    const int64_t blocks = (total + 255) / 256;
    if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
    if (p.dtype == DT_BF16)
      hipLaunchKernelGGL(gemm::gemm_elementwise<__bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, g);
    else
      hipLaunchKernelGGL(gemm::gemm_elementwise<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream, g);
    return hipGetLastError();
  }

  const int splits = gemm_splits(p);
  const int64_t need = splits > 1 ? (int64_t)splits * p.M * p.N * 4 : 0;
  if (splits > 1 && p.ws && p.ws_bytes >= need && ((uintptr_t)p.ws % 16) == 0) {
    // slices of kc (a multiple of the 64-deep K-step) as a batch of GEMMs
    // writing fp32 partial sums, then one reduction with the epilogue
    GemmProblem q = p;
    const int64_t kc = ((p.K + splits - 1) / splits + 63) / 64 * 64;
    const int64_t used = (p.K + kc - 1) / kc;
    q.K = kc;
    q.batch = used;
    q.sA = kc;
    q.sB = p.b_nt ? kc : kc * p.ldb;
    q.C = p.ws;
    q.ldc = p.N;
    q.sC = p.M * p.N;
    q.out_f32 = 1;
    q.epilogue = EPI_NONE;
    q.alpha = 1.f;
    q.bias = nullptr;
    q.tile = p.tile;
    const int tile = gemm::tile_for(q);
    gemm::KArgs k = gemm::make_kargs(q, tile);
    k.k_last = (int)(p.K - (used - 1) * kc);
    hipError_t e = gemm::launch_fast(q, tile, k, stream);
    if (e != hipSuccess) return e;
    gemm::ReduceArgs r;
    r.W = (const float*)p.ws;
    r.C = (char*)p.C;
    r.bias = (const char*)p.bias;
    r.M = p.M;
    r.N = p.N;
    r.Nout = p.epilogue == EPI_SILU_MUL ? p.N / 2 : p.N;
    r.ldc = p.ldc;
    r.splits = used;
    r.alpha = p.alpha;
    r.epi = p.epilogue;
    const int64_t blocks = (p.M * (r.Nout / 4) + 255) / 256;
    if (p.dtype == DT_BF16)
      hipLaunchKernelGGL(gemm::splitk_reduce<__bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, r);
    else
      hipLaunchKernelGGL(gemm::splitk_reduce<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream, r);
    return hipGetLastError();
  }

  const int tile = gemm::tile_for(p);
  return gemm::launch_fast(p, tile, gemm::make_kargs(p, tile), stream);
}

GemmProblem w8a16_as_gemm(const GemvProblem& p) {
  GemmProblem q{};
  q.A = p.x;
  q.B = p.W;
  q.C = p.y;
  q.bias = p.bias;
  q.scale = p.scale;
  q.M = p.M;
  q.N = p.N;
  q.K = p.K;
  q.lda = p.ldx;
  q.ldb = p.ldw;
  q.ldc = p.ldy;
  q.batch = 1;
  q.alpha = 1.f;
  q.dtype = DT_W8A16;
  q.b_nt = 1;
  q.epilogue = p.bias ? EPI_BIAS : EPI_NONE;
  q.tile = gemm::env_int("HXMI_W8_TILE", -1);
  return q;
}

hipError_t launch_w8a16_gemm(const GemvProblem& p, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  GemmProblem q = w8a16_as_gemm(p);
  q.ws = ws;
  q.ws_bytes = ws_bytes;
  if (!gemm_fast_path_ok(q) || ((uintptr_t)p.scale % 8) != 0) return hipErrorNotSupported;
  return launch_gemm(q, stream);
}

}  // namespace hxmi
