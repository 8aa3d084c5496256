// GEMM dispatch: alignment checks, tile choice, and the element-wise kernel
// used for operands the MFMA fast path cannot take (leading dimensions not a
// multiple of 8, misaligned pointers).  Ragged N and K (not multiples of 8)
// run on the MFMA path: ragged columns are stored element by element, and K
// not a multiple of 8 runs the instantiations that mask the last K-step.
#include "gemm_impl.h"

namespace hxmi {
namespace gemm {
hipError_t launch_fast_f16(int tile, bool nn, int epi, bool out_f32, bool rms, const KArgs& k, hipStream_t s);
hipError_t launch_fast_bf16(int tile, bool nn, int epi, bool out_f32, bool rms, const KArgs& k, hipStream_t s);
hipError_t launch_fast_w8(int tile, int epi, bool out_f32, const KArgs& k, hipStream_t s);
hipError_t launch_fast_ragged(int tile, bool bf16, bool nn, int epi, bool out_f32, const KArgs& k, hipStream_t s);

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
  float* rs_out;       // rms: the row scales, written by the column-0 threads
  const float* rs_in;  // !rms: given row scales
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
    if (a.rs_out && o == 0) a.rs_out[m] = r;
  } else if (a.rs_in) {
    acc0 *= a.rs_in[m];
    acc1 *= a.rs_in[m];
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

// a knob's value, or dflt when unset
int knob_or(Knob k, int dflt) {
  const int64_t v = knob(k);
  return v == KNOB_UNSET ? dflt : (int)v;
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace
}  // namespace gemm

bool gemm_fast_path_ok(const GemmProblem& p) {
  const bool i8 = p.dtype == DT_W8A16;
  if (i8 && (p.K % 16 || p.N % 8)) return false;
  if (p.epilogue == EPI_SILU_MUL && p.N % 32) return false;
  if (p.K % 8 && p.rms) return false;  // the RMS prologue sums whole fragments
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
  // 512-token LLaMA MLP GEMMs; 64x64 at two per CU outruns 64x128 on the
  // 512-token O projection; measured on the block shapes)
  static const Cand cands[] = {
      {TILE_256x256_W8, 256, 256, 1, 1.00f}, {TILE_256x128_W8, 256, 128, 1, 0.85f},
      {TILE_128x256, 128, 256, 1, 0.80f},    {TILE_128x128_W8, 128, 128, 2, 0.90f},
      {TILE_64x128, 64, 128, 3, 0.50f},      {TILE_128x64, 128, 64, 3, 0.50f},
      {TILE_64x64, 64, 64, 4, 0.52f},        {TILE_128x192_W8, 128, 192, 1, 0.80f},
  };
  const int cus = 256;
  int best = TILE_64x64;
  double best_t = 1e300;
  const bool i8 = p.dtype == DT_W8A16;
  for (const Cand& c : cands) {
    if (c.bn == 64 && p.epilogue == EPI_SILU_MUL) continue;
    // 128x192: k-contiguous fp16 / bf16 weights, one round of tiles (where
    // it was measured: TinyLlama gate/up, ViT-B/16 fc1)
    if (c.id == TILE_128x192_W8 && (p.dtype == DT_W8A16 || !p.b_nt ||
                                    ((p.M + 127) / 128) * ((p.N + 191) / 192) * p.batch > cus))
      continue;
    // int8 B converts every weight once per tile row: tall tiles amortise
    // it, and the latency-bound small shapes want the most workgroups
    // (measured on the Qwen2.5-0.5B int8 shapes at M = 256)
    float eff = c.eff;
    // the three-stage 8-wave 256x128 tile pays once K is long enough to keep
    // its deeper prefetch busy (TinyLlama gate/up, K = 2048: 33.1 -> 30.7 us
    // against 128x128 at two per CU; ViT fc1, K = 768: 19.4 -> 20.6 us)
    if (!i8 && c.id == TILE_256x128_W8 && p.K >= 1536) eff = 0.95f;
    if (i8 && (c.id == TILE_128x128_W8 || c.id == TILE_256x128_W8)) eff = 0.80f;
    if (i8 && c.id == TILE_64x64) eff = 0.60f;
    // (the int8 896 -> 4864 projection at M = 256: 152 tiles of 128x64 run
    // 11.5 us against 13.4 us for 304 tiles of 64x64)
    if (i8 && c.id == TILE_128x64) eff = 0.62f;
    // (the int8 lm_head 896 -> 151936 at M = 128: 1187 tiles of 128x128 at
    // two per CU run 56.0 us against 72.0 us for 594 tiles of 128x256)
    if (i8 && c.id == TILE_128x256) eff = 0.65f;
    // an RMSNorm-folded GEMM sums the squares of its A rows in every tile of
    // a row, so narrow tiles repeat that work more often (the 512-token QKV
    // projection, 512x2560x2048, in the block sequence: 64x128 1.3 us faster
    // than 64x64 once the K-step barriers kept the prefetch in flight)
    if (p.rms && c.id == TILE_64x64) eff = 0.45f;
    // long K with few tiles: 128x64 (4 waves, three per CU) over 64x64 and
    // 64x128 (ViT-B/16 fc2, 1576x768x3072: 156 tiles)
    if (!i8 && p.K >= 3072 && c.id == TILE_128x64) eff = 0.56f;
    const int64_t tm = (p.M + c.bm - 1) / c.bm, tn = (p.N + c.bn - 1) / c.bn;
    const int64_t tiles = tm * tn * p.batch;
    const int64_t slots = (int64_t)cus * c.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    const int64_t conc = tiles < slots ? (tiles + cus - 1) / cus : c.per_cu;  // tiles sharing a CU
    const double t = (double)rounds * c.bm * c.bn * (double)(conc > 0 ? conc : 1) / eff;
    if (t < best_t * 0.999) {
      best_t = t;
      best = c.id;
    }
  }
  // 64x64 tiles over K >= 2048: a fourth LDS stage (two workgroups still fit
  // a CU).  The 512-token O projection in the TinyLlama block sequence,
  // weights from HBM: block 75.46-75.90 -> 74.75-75.04 us (72.8-73.3 against
  // 74.3-74.6 on another MI355X); the 1024^3 GEMM, its operands in L2, ran
  // 6.42 -> 6.53 us with it and keeps three stages
  if (best == TILE_64x64 && !i8 && p.K >= 2048) best = TILE_64x64_S4;
  return best;
}

namespace gemm {
namespace {

int tile_for(const GemmProblem& p) {
  if (p.K % 8) {  // the ragged-K instantiations: 128x128 once its tiles cover the CUs
    const int64_t t128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.batch;
    return t128 >= 256 ? TILE_128x128 : TILE_64x64;
  }
  int tile = p.tile >= 0 ? p.tile : knob_or(KNOB_GEMM_TILE, -1);
  // (an override of 128x192 for a layout it does not take: the picker's tile)
  if (tile < 0 || tile >= TILE_COUNT || (tile == TILE_128x192_W8 && (!p.b_nt || p.dtype == DT_W8A16)))
    tile = gemm_pick_tile(p);
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
  const int gm = knob_or(KNOB_GROUP_M, 4);
  k.group_m = gm < 1 ? 1 : (gm > k.tiles_m ? k.tiles_m : gm);
  k.k_last = 0;
  k.rms_eps = p.rms_eps;
  k.rs_out = p.rs_out;
  k.rs_in = p.rs_in;
  return k;
}

hipError_t launch_fast(const GemmProblem& p, int tile, const KArgs& k, hipStream_t stream) {
  if ((int64_t)k.tiles_m * k.tiles_n * k.batch >= (1ll << 31)) return hipErrorInvalidValue;
  if (p.K % 8) return launch_fast_ragged(tile, p.dtype == DT_BF16, !p.b_nt, p.epilogue, p.out_f32, k, stream);
  if (p.rms && p.dtype == DT_W8A16) return hipErrorNotSupported;
  if (p.dtype == DT_W8A16) return launch_fast_w8(tile, p.epilogue, p.out_f32, k, stream);
  if (p.dtype == DT_BF16) return launch_fast_bf16(tile, !p.b_nt, p.epilogue, p.out_f32, p.rms != 0, k, stream);
  return launch_fast_f16(tile, !p.b_nt, p.epilogue, p.out_f32, p.rms != 0, k, stream);
}

}  // namespace
}  // namespace gemm

// Split K into slices when the output has too few tiles to occupy the 256
// CUs and K is long enough that each slice still runs many K-steps.  Split
// problems run 64x128 tiles (4 waves, two per CU at three LDS stages).
// Slices of >= 2048 of K that already give every CU a workgroup stop at
// two; otherwise the slice count aims at ~480 workgroups, each slice keeping
// >= 1024 of K.  With K below 4096 every split measured slower: the
// 512-token QKV and O projections, and ViT-B/16 fc2 (1576x768x3072) once
// the K-step barriers kept the prefetch in flight (whole on 128x64 tiles
// 0.9 us faster per ViT attention + MLP than 3 slices of 64x128).
// With int8 weights the slices run 64x64 tiles (Qwen2.5-0.5B down
// projection at M = 256: 105 -> 128 TFLOP/s).
int gemm_splits(const GemmProblem& p) {
  const bool i8 = p.dtype == DT_W8A16;
  if (p.batch != 1 || p.out_f32 || p.rms || p.K < (i8 ? 512 : 2048) || p.K % 8 || !gemm_fast_path_ok(p)) return 1;
  if (const int64_t e = knob(KNOB_SPLITK); e != KNOB_UNSET) return e < 1 ? 1 : (e > 16 ? 16 : (int)e);
  if (i8 && p.K < 2048) {
    // int8 weights at short K with few output tiles (the Qwen2.5-0.5B
    // 896 -> 896 projection at M = 256: 56 tiles of 64x64): each workgroup's
    // K-steps wait on memory, so slices of >= 256 of K put the same steps on
    // more CUs (10.7 -> 9.0 us with 3 slices; 7 slices of 128: 12.1 us)
    const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64);
    if (t64 >= 128) return 1;
    int s = (int)((240 + t64 / 2) / t64);
    s = s < 1 ? 1 : (s > 4 ? 4 : s);
    while (s > 1 && p.K / s < 256) --s;
    return s;
  }
  const int64_t tiles = ((p.M + 63) / 64) * ((p.N + 127) / 128);
  if (tiles >= 384 || p.K < 4096) return 1;
  // long slices: two of them once every CU has a workgroup (measured in the
  // TinyLlama block sequence, weights not resident in L2: the 512x2048x5632
  // down projection ran 80.9 us per block with 2 slices, 83.0 with 3, 83.3
  // with 4, where each slice's fix-up traffic outweighs the extra workgroups)
  if (p.dtype != DT_W8A16 && tiles * 2 >= 256 && p.K / 2 >= 2048) return 2;
  int s = (int)((480 + tiles / 2) / tiles);
  s = s < 1 ? 1 : (s > 4 ? 4 : s);
  while (s > 1 && p.K / s < 1024) --s;
  return s;
}

// The split-K launch of p: K slices of kc (a multiple of the 64-deep K-step)
// as a batch of GEMMs into the same output (sC = 0), the tile they run and
// the fix-up workspace they need.  False when p does not split.
static bool split_plan(const GemmProblem& p, GemmProblem& q, int& tile, int64_t& need) {
  const int splits = gemm_splits(p);
  if (splits <= 1) return false;
  q = p;
  const int64_t kc = ((p.K + splits - 1) / splits + 63) / 64 * 64;
  q.K = kc;
  q.batch = (p.K + kc - 1) / kc;
  q.sA = kc;
  q.sB = p.b_nt ? kc : kc * p.ldb;
  q.sC = 0;
  // (fp16: the two long slices of a down projection run 128x64 tiles, the
  // 512x2048x5632 one 0.65 us faster in the block sequence than 64x128;
  // ViT fc2's three slices of 1024 measured equal or slower with 128x64)
  if (q.tile < 0 && gemm::knob_or(KNOB_GEMM_TILE, -1) < 0)
    q.tile = p.dtype == DT_W8A16 ? TILE_64x64 : (splits == 2 && p.K / 2 >= 2048 ? TILE_128x64 : TILE_64x128);
  tile = gemm::tile_for(q);
  const gemm::TileShape s = gemm::kTiles[tile];
  const int64_t tiles = ((p.M + s.BM - 1) / s.BM) * ((p.N + s.BN - 1) / s.BN);
  need = kWsCounterBytes + tiles * q.batch * s.BM * s.BN * 4;
  return q.batch > 1 && tiles <= kWsMaxTiles;
}

int64_t gemm_workspace_bytes(const GemmProblem& p) {
  GemmProblem q;
  int tile;
  int64_t need;
  return split_plan(p, q, tile, need) ? need : 0;
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
    g.rs_out = p.rs_out;
    g.rs_in = p.rs_in;
    const int64_t total = p.batch * p.M * g.Nout;
    const int64_t blocks = (total + 255) / 256;
    if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
    if (p.dtype == DT_BF16)
      hipLaunchKernelGGL(gemm::gemm_elementwise<__bf16>, dim3((unsigned)blocks), dim3(256), 0, stream, g);
    else
      hipLaunchKernelGGL(gemm::gemm_elementwise<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream, g);
    return hipGetLastError();
  }

  GemmProblem q;
  int qtile;
  int64_t need;
  if (split_plan(p, q, qtile, need) && p.ws && p.ws_bytes >= need && ((uintptr_t)p.ws % 256) == 0) {
    // K slices as a batch into one output; the last slice to finish a tile
    // adds the fp32 partials (in the workspace) and runs the epilogue
    gemm::KArgs k = gemm::make_kargs(q, qtile);
    k.k_last = (int)(p.K - (q.batch - 1) * q.K);
    k.fix = (char*)p.ws;
    return gemm::launch_fast(q, qtile, k, stream);
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
  q.tile = gemm::knob_or(KNOB_W8_TILE, -1);
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
