// MFMA GEMM for gfx950: C = epilogue(alpha * A . op(B)), fp32 accumulate.
//
// Schedule (replaces the reference's VTCM tiling + DDR->TCM DMA ping-pong,
// VTCMTiling.cpp:231-266, HexmemCpyToDMA.cpp:120-271,
// DoubleBufferGenericS1.cpp:164-277 and the HVX matmul loop order of
// ScheduleMatmulForHVXPass.cpp:69-195):
//   * one workgroup owns a BM x BN tile of C and walks K in 64-deep steps;
//   * operand tiles move HBM -> LDS with buffer_load ... lds (no VGPR
//     staging), two LDS stages, so the copy of step k+1 overlaps the MFMAs of
//     step k (the ping-pong the reference only applies to elementwise loops);
//   * out-of-range rows / k-chunks use an offset past the buffer resource's
//     range, so the hardware returns zeros and no tail branches are needed;
//   * LDS rows are XOR-swizzled in 16-byte chunks so MFMA fragment reads are
//     free of conflicts on gfx950's 64 LDS banks; a [K,N] (NN) operand is read
//     with ds_read_b64_tr_b16;
//   * the MFMA is issued as D[n][m] = B^T . A^T so every lane owns four
//     consecutive output columns, which makes the fused epilogue (bias,
//     SiLU-mul, tanh-GELU) and the LDS-staged 16-byte stores cheap.
#pragma once

#include <type_traits>
#include <utility>

#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace gemm {

constexpr int BK = 64;

struct KArgs {
  const char* A;
  const char* B;
  char* C;
  const char* bias;
  const char* scale;  // per-column fp16 scale (int8 B only)
  int M, N, K;
  int64_t lda, ldb, ldc;  // elements
  int64_t sA, sB, sC;     // elements
  int batch;
  float alpha;
  int tiles_m, tiles_n;
  int group_m;
  int k_last;  // > 0: the last batch entry has this K (split-K: a ragged last slice)
  float rms_eps;  // RMS kernels: epsilon of the row RMSNorm folded into the GEMM
  // Split-K with in-kernel fix-up (fix != nullptr): the batch entries are K
  // slices of one output (sC = 0).  fix holds one 64-bit arrival counter per
  // output tile in its first kWsCounterBytes, then batch fp32 partial tiles
  // per output tile in fragment order.  The counters must be zero when the
  // launch starts; the last slice to arrive at a tile resets its counter to
  // zero, so every launch leaves them zero for the next one.
  char* fix;
  float* rs_out;       // RMS kernels: row scales rsqrt(mean + eps) written here (optional)
  const float* rs_in;  // other kernels: row scales applied before the epilogue (optional)
};


template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  static __device__ __forceinline__ float16v run(short8v a, short8v b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a),
                                                  __builtin_bit_cast(half8v, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  static __device__ __forceinline__ float16v run(short8v a, short8v b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                   __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
  }
};

// Workgroup id -> (batch, tile_m, tile_n).  Workgroups are dispatched
// round-robin over the 8 XCDs (id % 8); each XCD is given a contiguous run of
// tiles so the A/B panels it touches stay in its own L2.  Within the run,
// tiles are rastered in groups of group_m tile-rows.
__device__ __forceinline__ void map_tile(int bid, const KArgs& a, int& b, int& tm, int& tn) {
  const int tiles = a.tiles_m * a.tiles_n;
  const int total = tiles * a.batch;
  const int q = total >> 3, rem = total & 7;
  const int x = bid & 7, j = bid >> 3;
  const int r = x * q + (x < rem ? x : rem) + j;
  b = r / tiles;
  const int t = r - b * tiles;
  const int per_group = a.group_m * a.tiles_n;
  const int gid = t / per_group;
  const int first_m = gid * a.group_m;
  const int left = a.tiles_m - first_m;
  const int gsz = left < a.group_m ? left : a.group_m;
  const int wi = t - gid * per_group;
  tm = first_m + wi % gsz;
  tn = wi / gsz;
}

// A k-contiguous tile is stored as [rows][BK elements]: RB = 2*BK bytes per
// row (64 or 128), 256/RB rows per 256-byte line of the 64 4-byte LDS banks.
// A ds_read_b128 phase serves 16 lanes, which read the same 16-byte chunk of
// 16 consecutive rows; XOR-ing the chunk index with (row / (256/RB)) mod
// (RB/16) puts those 16 reads in 16 distinct bank groups.
template <int RB>
__device__ __forceinline__ int kc_swz(int r) {
  return (r / (256 / RB)) & (RB / 16 - 1);
}

// MFMA 32x32x16 operand layout: lane l holds row (l % 32), k = 8*(l / 32) .. +7
// of the 16-deep substep s.
template <int RB>
__device__ __forceinline__ short8v read_kc(const char* tile, int r_off, int s, int lane) {
  const int r = r_off + (lane & 31);
  const int c = (s << 1) + (lane >> 5);
  return *(const short8v*)(tile + r * RB + ((c ^ kc_swz<RB>(r)) << 4));
}

template <int BN>
__device__ __forceinline__ int nn_swz(int k) {
  return (BN / 8 >= 16) ? ((k & 3) << 2) : ((k & 3) << 1);
}

// Fragment of an n-contiguous [64][BN] tile (B in NN form) for the same MFMA
// operand layout, built from two transposing LDS reads.
template <int BN>
__device__ __forceinline__ short8v read_nn(const char* tile, int n_off, int s, int lane) {
  const int g = lane >> 4, li = lane & 15;
  const int n = n_off + ((g & 1) << 4) + ((li & 3) << 2);
  const int k = (s << 4) + ((g >> 1) << 3) + (li >> 2);
  const int sw = nn_swz<BN>(k);  // same for k and k+4
  const int col = ((((n >> 3) ^ sw)) << 4) + ((n & 7) << 1);
  short4v lo = lds_read_tr16(tile + k * (BN * 2) + col);
  short4v hi = lds_read_tr16(tile + (k + 4) * (BN * 2) + col);
  return short8v{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <typename T>
__device__ __forceinline__ void store4(char* p, float v0, float v1, float v2, float v3) {
  T t[4] = {(T)v0, (T)v1, (T)v2, (T)v3};
  *(short4v*)p = __builtin_bit_cast(short4v, t);
}

template <typename T>
__device__ __forceinline__ void load_bias4(const char* bias, int n, int N, float* out) {
  if (n + 4 > N) {  // ragged last columns
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = n + i < N ? (float)((const T*)bias)[n + i] : 0.f;
  } else if (n < N) {
    short4v raw = *(const short4v*)(bias + (int64_t)n * 2);
    T t[4];
    __builtin_memcpy(t, &raw, 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = (float)t[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = 0.f;
  }
}

// 8 int8 weights -> 8 fp16, exactly.  Each byte q is biased to u = q+128,
// placed in the mantissa of the fp16 value 1024 (0x6400 | u == 1024 + u,
// exact because fp16 has unit spacing on [1024, 2048)), and 1152 is
// subtracted, leaving q.
__device__ __forceinline__ short8v dequant8(int2v raw) {
  short8v out;
  half2v* o = (half2v*)&out;
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t u = (uint32_t)raw[d] ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    o[2 * d] = __builtin_bit_cast(half2v, lo) - bias;
    o[2 * d + 1] = __builtin_bit_cast(half2v, hi) - bias;
  }
  return out;
}

// ss + the sum of squares of 8 packed fp16 / bf16 values (v_dot2 on pairs).
template <typename T>
__device__ __forceinline__ float sumsq8(short8v v, float ss) {
  if constexpr (std::is_same_v<T, _Float16>) {
    const half8v h = __builtin_bit_cast(half8v, v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const half2v p2 = {h[2 * q], h[2 * q + 1]};
      ss = __builtin_amdgcn_fdot2(p2, p2, ss, false);
    }
  } else {
    const bf16x8v h = __builtin_bit_cast(bf16x8v, v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16x2v p2 = {h[2 * q], h[2 * q + 1]};
      ss = __builtin_amdgcn_fdot2_f32_bf16(p2, p2, ss, false);
    }
  }
  return ss;
}

// The first n (clamped to 0..8) of 8 packed 16-bit values, the rest zero.
__device__ __forceinline__ short8v keep_first(short8v v, int n) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = e < n ? v[e] : (short)0;
  return v;
}

// Instruction order inside one substep region (the compiler's scheduler
// otherwise bunches the LDS reads right before the MFMAs that consume them):
// the substep's NMF MFMAs with the NDS fragment reads of the next substep
// and NVM global->LDS loads slotted between them.
// NVA vector-ALU instructions (the RMSNorm sums of squares of this substep's
// fragments) go over the second half of the MFMAs, when every fragment has
// been consumed once and its LDS read has certainly returned.
template <int NMF, int NDS, int NVM, int NVA = 0>
__device__ __forceinline__ void schedule_substep() {
  static_assert(NMF > 0, "substep without MFMAs");
  constexpr int kVALU = 0x002, kMFMA = 0x008, kVMEMR = 0x020, kDSR = 0x100;
  // reads go one per MFMA from the start of the region (they feed the next
  // region); global loads are spread over the slots after them
  constexpr int FREE = NMF > NDS ? NMF - NDS : 1;
  constexpr int HALF = NMF - NMF / 2;
  static_for<NMF>([&](auto M) {
    constexpr int m = decltype(M)::value;
    __builtin_amdgcn_sched_group_barrier(kMFMA, 1, 0);
    constexpr int nds = m < NDS ? ((m + 1 == NMF) ? NDS - m : 1) : 0;
    if constexpr (nds > 0) __builtin_amdgcn_sched_group_barrier(kDSR, nds, 0);
    constexpr int mv = m - (NMF - FREE);
    constexpr int nv = mv >= 0 ? (mv + 1) * NVM / FREE - mv * NVM / FREE : 0;
    if constexpr (nv > 0) __builtin_amdgcn_sched_group_barrier(kVMEMR, nv, 0);
    constexpr int ma = m - (NMF - HALF);
    constexpr int na = (NVA > 0 && ma >= 0) ? (ma + 1) * NVA / HALF - ma * NVA / HALF : 0;
    if constexpr (na > 0) __builtin_amdgcn_sched_group_barrier(kVALU, na, 0);
  });
}

// Barrier of the ping-pong schedule: nothing is moved across it, and every
// LDS read of the wave has returned (so no stage is refilled under a reader).
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt / expcnt untouched
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// RMS = true: C = epilogue(rmsnorm(A) . B^T) for an NT GEMM whose B already
// holds the RMSNorm weight folded in (B[n][k] = g[k] * W[n][k]).  Every wave
// sums the squares of the A fragments it multiplies (its rows, all of K) and
// scales its accumulators by rsqrt(mean + eps) before the epilogue, so the
// normalised activations are never written.
//
// PP = true: ping-pong schedule for 8 waves in two groups of 4 (group =
// wave / 4 = the tile's upper or lower half of rows, one wave of each group
// per SIMD).  The groups run half a K-step apart, separated by workgroup
// barriers: while one group issues its MFMAs from registers, the other
// loads its next step's fragments from LDS and issues the global->LDS loads,
// so every SIMD's MFMA pipe alternates between its two waves.
template <int BM, int BN, int WM, int WN, int BK, int STAGES, bool NN, typename T, int EPI, bool OUTF32,
          bool BI8 = false, bool PP = false, bool RMS = false, bool RAGGED = false, int SB = 0, int FD = 1>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma(KArgs a) {
  constexpr int NWM = BM / WM, NWN = BN / WN, NW = NWM * NWN, NT = NW * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int RB = BK * 2;            // bytes per k-contiguous tile row
  constexpr int CH = RB / 16;           // 16-byte chunks per row
  constexpr int RPIK = 1024 / RB;       // k-contiguous rows per 1 KB wave instruction
  constexpr int A_BYTES = BM * RB;
  constexpr int B_BYTES = BI8 ? BN * BK : BN * RB;  // int8 B stays int8 in LDS
  // STAGES LDS stages of A, SBS of B (SB = 0: as many as A).  More B stages
  // than A ones prefetch B further ahead, for B streamed from HBM while A
  // stays in L2.  LDS holds the A stages, then the B stages.
  constexpr int SBS = SB ? SB : STAGES;
  constexpr int A_REGION = STAGES * A_BYTES;
  constexpr int BNO = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  constexpr int SROW = BNO * 2 + 16;
  constexpr int EPI_BYTES = OUTF32 ? 0 : BM * SROW;
  constexpr int SMEM_OPS = (A_REGION + SBS * B_BYTES > EPI_BYTES) ? A_REGION + SBS * B_BYTES : EPI_BYTES;
  // The epilogue's per-column vectors (bias, int8 scales) of the tile's BN
  // columns sit after that, 1 KB each: one direct load by wave 0 at the
  // start, so they cost no registers through the main loop and the
  // epilogue (the 8-wave 256x256 tile holds 256 accumulator VGPRs a lane).
  constexpr bool HAS_BIAS = EPI == EPI_BIAS || EPI == EPI_BIAS_GELU_TANH;
  constexpr int NCV = (HAS_BIAS ? 1 : 0) + (BI8 ? 1 : 0);
  constexpr int SMEM = SMEM_OPS + NCV * 1024;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(STAGES >= 2 && STAGES <= 4, "STAGES");
  static_assert(SBS >= STAGES && SBS <= 8 && (!PP || SBS == STAGES), "B stages");
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(BM % (RPIK * NW) == 0, "A tile rows per wave");
  static_assert(NN || BN % (RPIK * NW) == 0, "B tile rows per wave");
  static_assert(!BI8 || (!NN && BK == 64 && BN % (16 * NW) == 0), "int8 B: [N,K], BK 64, 16-row loads");
  static_assert(!PP || (NW == 8 && NWM == 2 && STAGES >= 3 && !BI8), "ping-pong: 2 x 4 waves, >= 3 stages");
  static_assert(!RMS || (!NN && !BI8 && !PP && !OUTF32), "RMSNorm prologue: NT, standard schedule");
  static_assert(!RAGGED || (!BI8 && !PP && !RMS), "ragged K: plain fp16 / bf16 operands, standard schedule");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];
  auto sa = [&](int i) { return smem + i * A_BYTES; };              // A stage i
  auto sb = [&](int i) { return smem + A_REGION + i * B_BYTES; };   // B stage i

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w / NWN, wn = w % NWN;

  int b, tm, tn;
  map_tile(blockIdx.x, a, b, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = (a.k_last > 0 && b == a.batch - 1) ? a.k_last : a.K;

  const char* Ab = a.A + (b * a.sA + (int64_t)m0 * a.lda) * 2;
  const char* Bb = NN    ? a.B + (b * a.sB + (int64_t)n0) * 2
                   : BI8 ? a.B + (b * a.sB + (int64_t)n0 * a.ldb)
                         : a.B + (b * a.sB + (int64_t)n0 * a.ldb) * 2;

  // column vectors -> LDS (N a multiple of 8: whole 16-byte chunks, columns
  // past N read as zero); the prologue's first wait covers these loads, as
  // they are issued before every operand load.  Other N read them from
  // global memory in the epilogue.
  static_assert(BN * 2 <= 1024, "column vector chunk");
  const bool cv_lds = NCV > 0 && (a.N % 8) == 0;
  char* const cv_bias = smem + SMEM_OPS;
  char* const cv_scale = smem + SMEM_OPS + (HAS_BIAS ? 1024 : 0);
  if (cv_lds && w == 0) {
    const uint32_t off = (uint32_t)(n0 + lane * 8) * 2u;
    if constexpr (HAS_BIAS) load_lds16(make_rsrc(a.bias, (uint32_t)a.N * 2u), (HXMI_LDS void*)to_lds(cv_bias), off);
    if constexpr (BI8) load_lds16(make_rsrc(a.scale, (uint32_t)a.N * 2u), (HXMI_LDS void*)to_lds(cv_scale), off);
  }
  // 4 consecutive column-vector values starting at tile column nl (n0 + nl
  // in the matrix)
  auto colvec4 = [&](const char* cv, const char* gv, int nl, float* out) {
    if (cv_lds) {
      const short4v raw = *(const short4v*)(cv + nl * 2);
      T t[4];
      __builtin_memcpy(t, &raw, 8);
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = (float)t[q];
    } else {
      load_bias4<T>(gv, n0 + nl, a.N, out);
    }
  };

  // ---- load plan --------------------------------------------------------------
  // Each wave instruction moves 1 KB (RPIK rows of a k-contiguous tile, or
  // 1024/(2*BN) rows of an NN tile).  One buffer resource per operand and
  // K-step starts at the step's first column and ends (num_records) at the
  // last valid row, so rows past M / N / K read as zero.  The only per-lane
  // state is one byte offset per operand; a chunk past K swaps it for kOOB.
  //
  // Lane l of a k-contiguous instruction fills slot (row l / CH, position
  // l % CH) of its RPIK-row block, so it loads logical chunk
  // position ^ kc_swz(row); the swizzle term does not depend on which of the
  // wave's instructions it is (checked below), so one offset serves them all.
  static_assert(((NW * RPIK) / (256 / RB)) % CH == 0, "swizzle period");
  constexpr int IA = BM / RPIK / NW;
  const int cA = (lane % CH) ^ ((((w * RPIK) / (256 / RB)) + (lane / CH) / (256 / RB)) % CH);
  const uint32_t voffA = (uint32_t)((w * RPIK + lane / CH) * a.lda * 2 + cA * 16);
  const uint32_t stepA = (uint32_t)(NW * RPIK * a.lda * 2);  // bytes between a wave's A instructions
  const uint32_t bytesA = (uint32_t)(min(BM, a.M - m0) * a.lda * 2);

  constexpr int CPR = BN / 8;                          // NN: 16-byte chunks per k-row
  constexpr int RPI = NN ? (1024 / (BN * 2)) : RPIK;   // rows per wave instruction
  // int8 B (BI8): 64-byte rows (BK int8 weights), four 16-byte chunks per
  // row, one 1 KB instruction per 16 rows; chunk c of row r is stored at
  // position c ^ ((r >> 2) & 3), which depends on the lane alone (rows of an
  // instruction start on multiples of 16).
  constexpr int IB = BI8 ? BN / 16 / NW : (NN ? (BK / RPI / NW) : (BN / RPIK / NW));
  static_assert(IB >= 1, "B load plan");
  static_assert(!NN || (NW * RPI) % 4 == 0, "NN swizzle period");
  uint32_t voffB, stepB, bytesB;
  int cB8 = 0;
  if constexpr (NN) {
    const int rowl = w * RPI + lane / CPR;  // (row & 3) is the same for every instruction
    const int c = (lane % CPR) ^ nn_swz<BN>(rowl);
    voffB = (n0 + c * 8) < a.N ? (uint32_t)(rowl * a.ldb * 2 + c * 16) : kOOB;
    stepB = (uint32_t)(NW * RPI * a.ldb * 2);
    bytesB = (uint32_t)(a.ldb * 2);  // per valid k-row
  } else if constexpr (BI8) {
    cB8 = (lane & 3) ^ ((lane >> 4) & 3);
    voffB = (uint32_t)((w * 16 + (lane >> 2)) * a.ldb + cB8 * 16);
    stepB = (uint32_t)(NW * 16 * a.ldb);
    bytesB = (uint32_t)(min(BN, a.N - n0) * a.ldb);
  } else {
    voffB = (uint32_t)((w * RPIK + lane / CH) * a.ldb * 2 + cA * 16);
    stepB = (uint32_t)(NW * RPIK * a.ldb * 2);
    bytesB = (uint32_t)(min(BN, a.N - n0) * a.ldb * 2);
  }
  const int nk = (K + BK - 1) / BK;

  // Loads of K-step kt into A / B stage `stage`; a step past the end issues
  // loads against an empty buffer (all zeros, nothing touched).
  auto issueA = [&](int kt, int stage) {
    const int k0 = kt * BK;
    const bool live = kt < nk;
    char* sA_ = sa(stage);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(Ab + (int64_t)k0 * 2, live ? bytesA - 2u * k0 : 0u);
    const uint32_t vA = (k0 + cA * 8) < K ? voffA : kOOB;
#pragma unroll
    for (int i = 0; i < IA; ++i)
      load_lds16(rA, (HXMI_LDS void*)to_lds(sA_ + (i * NW + w) * 1024), vA + i * stepA);
  };
  auto issueB = [&](int kt, int stage) {
    const int k0 = kt * BK;
    const bool live = kt < nk;
    char* sB_ = sb(stage);
    if constexpr (NN) {
      const uint32_t rows = (uint32_t)min(BK, K - k0);
      const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bb + (int64_t)k0 * a.ldb * 2, live ? rows * bytesB : 0u);
#pragma unroll
      for (int i = 0; i < IB; ++i)
        load_lds16(rB, (HXMI_LDS void*)to_lds(sB_ + (i * NW + w) * 1024), voffB + i * stepB);
    } else if constexpr (BI8) {
      const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bb + k0, live ? bytesB - (uint32_t)k0 : 0u);
      const uint32_t vB = (k0 + cB8 * 16) < K ? voffB : kOOB;
#pragma unroll
      for (int i = 0; i < IB; ++i)
        load_lds16(rB, (HXMI_LDS void*)to_lds(sB_ + (i * NW + w) * 1024), vB + i * stepB);
    } else {
      const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bb + (int64_t)k0 * 2, live ? bytesB - 2u * k0 : 0u);
      const uint32_t vB = (k0 + cA * 8) < K ? voffB : kOOB;
#pragma unroll
      for (int i = 0; i < IB; ++i)
        load_lds16(rB, (HXMI_LDS void*)to_lds(sB_ + (i * NW + w) * 1024), vB + i * stepB);
    }
  };
  auto issue = [&](int kt, int stage) {
    issueA(kt, stage);
    issueB(kt, stage);
  };

  // Byte offset of this lane's 16-byte chunk in a k-contiguous fragment of
  // substep s: the swizzle repeats every 16 rows and fragments start on
  // multiples of 32 rows, so it depends on the lane alone; the wave's first
  // row is folded in, leaving a constant per fragment (an immediate offset).
  //
  // Int8 B (BI8) is read 16 bytes (16 k) at a time, one chunk per pair of
  // substeps: in substeps 2p and 2p+1 lane l (h = l / 32) takes k = 32p +
  // 16h + 8(s & 1) .. +7 of its row, and its A fragment takes the same k
  // (chunk 4p + 2h + (s & 1) instead of 2s + h).  An MFMA sums over
  // whichever k its lanes hold as long as both operands agree, and the four
  // substeps still cover k = 0..63 once.  The 16-byte read matters: after an
  // 8-byte LDS read (the plain int8 fragment) the compiler waited for every
  // outstanding direct-to-LDS load (vmcnt(0)), which drained the prefetch in
  // every K-step.
  constexpr int SUBS_ = BK / 16;
  uint32_t lofA[SUBS_], lofB[SUBS_], lofB8[SUBS_];
#pragma unroll
  for (int s = 0; s < SUBS_; ++s) {
    const int l = lane & 31, h = lane >> 5;
    const int ca = BI8 ? ((s >> 1) << 2) + (h << 1) + (s & 1) : (s << 1) + h;
    lofA[s] = (uint32_t)(wm * WM * RB + l * RB + ((ca ^ kc_swz<RB>(l)) << 4));
    lofB[s] = (uint32_t)(wn * WN * RB + l * RB + ((((s << 1) + h) ^ kc_swz<RB>(l)) << 4));
    // int8 B rows (BK bytes) keep chunk c of row r at c ^ ((r >> 2) & 3)
    lofB8[s] = (uint32_t)((wn * WN + l) * BK + (((2 * (s >> 1) + h) ^ ((l >> 2) & 3)) << 4));
  }
  short8v fbo[BI8 ? TN : 1];  // BI8: the odd substep's B fragments, dequantised with the even one's
  // RAGGED (K % 8 != 0): the 16-byte chunk that straddles K brings in
  // elements past K (row padding, or the next row).  In the last K-step the
  // fragments keep only their elements below K; the NN B operand needs no
  // mask, its rows past K read as zero.
  auto read_frags = [&](short8v (&fa)[TM], short8v (&fb)[TN], const char* sA_, const char* sB_, int s,
                        int kstep) {
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      if constexpr (NN) {
        fb[i] = read_nn<BN>(sB_, wn * WN + i * 32, s, lane);
      } else if constexpr (BI8) {
        // 16 int8 weights of row wn WN + 32 i + lane % 32 -> 16 fp16,
        // exactly, in the even substep: its fragment takes the first 8, the
        // odd substep's the last 8
        if ((s & 1) == 0) {
          int4v q = __builtin_bit_cast(int4v, *(const short8v*)(sB_ + lofB8[s] + i * 32 * BK));
          asm("" : "+v"(q));  // one 16-byte read, not two 8-byte ones
          fb[i] = dequant8(int2v{q[0], q[1]});
          fbo[i] = dequant8(int2v{q[2], q[3]});
        } else {
          fb[i] = fbo[i];
        }
      } else {
        fb[i] = *(const short8v*)(sB_ + lofB[s] + i * 32 * RB);
      }
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) fa[j] = *(const short8v*)(sA_ + lofA[s] + j * 32 * RB);
    if constexpr (RAGGED) {
      if (kstep == nk - 1) {
        const int nv = K - (kstep * BK + s * 16 + (lane >> 5) * 8);
#pragma unroll
        for (int j = 0; j < TM; ++j) fa[j] = keep_first(fa[j], nv);
        if constexpr (!NN) {
#pragma unroll
          for (int i = 0; i < TN; ++i) fb[i] = keep_first(fb[i], nv);
        }
      }
    }
  };

  float16v acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = float16v{};
  float ss[TM];  // RMS: this lane's sum of squares of row (j*32 + lane%32), its k half
#pragma unroll
  for (int j = 0; j < TM; ++j) ss[j] = 0.f;

  // Software pipeline over K-steps: STAGES LDS stages (step kt lives in stage
  // kt % STAGES), fragments double buffered in registers.  Per K-step kt:
  //   substeps 0..SUBS-2: MFMAs of substep s, reads of substep s+1 between;
  //   then: wait until step kt+1 has landed (later steps may still be in
  //   flight), barrier (step kt+1 visible; every wave has read all of step
  //   kt), refill step kt's stage with step kt+STAGES;
  //   last substep: MFMAs, with step kt+1's first fragments and the new
  //   step's global loads in between.
  constexpr int SUBS = BK / 16;
  constexpr int NDS = (NN ? 2 * TN : TN) + TM;  // LDS read instructions per substep
  constexpr int NVM = IA + IB;                  // global->LDS loads per K-step per wave
  if constexpr (PP) {
    // Phases alternate memory / compute; group 0 runs phase 2k as the memory
    // phase of step k and 2k+1 as its compute phase, group 1 one phase later.
    // The memory phase of step k: issue the loads of step k+D (D = STAGES-1)
    // into the stage step k-1 used, read all of step k's fragments, wait
    // until this wave's loads of step k+1 have landed.  A stage is refilled
    // at phase 2k (group 0) or 2k+1 (group 1); its last reader, group 1's
    // memory phase of step k-1, ended at phase 2k-1 with its reads returned.
    // Step k+1 is first read at phase 2k+2, after both groups have waited
    // for their loads of it (at phases 2k and 2k+1).
    constexpr int D = STAGES - 1;
    const int grp = wm;
#pragma unroll
    for (int p = 0; p < D; ++p) issue(p, p);
    wait_vmcnt<(D - 1) * NVM>();
    barrier_after_lds_loads();
    if (grp == 1) pp_barrier();
    short8v fa[SUBS][TM], fb[SUBS][TN];
    int st = 0, stw = D;
    for (int kt = 0; kt < nk; ++kt) {
      issue(kt + D, stw);
      const char* sA_ = sa(st);
      const char* sB_ = sb(st);
      static_for<SUBS>([&](auto S) { read_frags(fa[decltype(S)::value], fb[decltype(S)::value], sA_, sB_, decltype(S)::value, kt); });
      wait_vmcnt<(D - 1) * NVM>();
      pp_barrier();
      static_for<SUBS>([&](auto S) {
        constexpr int s = decltype(S)::value;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j) acc[i][j] = Mfma<T>::run(fb[s][i], fa[s][j], acc[i][j]);
      });
      pp_barrier();
      st = (st + 1 == STAGES) ? 0 : st + 1;
      stw = (stw + 1 == STAGES) ? 0 : stw + 1;
    }
    if (grp == 0) pp_barrier();
  } else {
  // Issue order, step by step: step t issues A(t + STAGES), then
  // B(t + SBS); the prologue runs the virtual steps t = -SBS .. -1 (A only
  // where t + STAGES >= 0).  Step kt needs A(kt) and B(kt); with SBS >
  // STAGES, B(kt) was issued before A(kt), so waiting for A(kt) leaves in
  // flight the B issued just after it plus every later step's loads.
  constexpr int WB = SBS > STAGES ? IB : 0;
#pragma unroll
  for (int t = -SBS; t < 0; ++t) {
    if (t + STAGES >= 0) issueA(t + STAGES, t + STAGES);
    issueB(t + SBS, t + SBS);
  }
  wait_vmcnt<(STAGES - 1) * NVM + WB>();
  barrier_after_lds_loads();  // (__syncthreads() would wait for every stage)
  // Fragments are read FD substeps ahead of their MFMAs: FD = 1 double
  // buffers them; FD = 2 or 3 (64-deep K-steps) keeps one buffer per
  // substep, so a read has FD substeps of MFMAs to return.  The K-step's
  // wait and barrier come at the first substep that reads the next K-step
  // (SUBS - FD): by then this wave has issued every read of the current
  // step, and the barrier's wait for them lets the refill loads overwrite
  // its stage.
  static_assert(FD == 1 || (FD <= 3 && SUBS == 4 && !BI8), "fragment read distance");
  constexpr int NFB = FD == 1 ? 2 : 4;
  short8v fa[NFB][TM], fb[NFB][TN];
  static_for<FD>([&](auto P) {
    constexpr int p = decltype(P)::value;
    read_frags(fa[p], fb[p], sa(0), sb(0), p, 0);
  });
  int st = 0, stb = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int st1 = (st + 1 == STAGES) ? 0 : st + 1;
    const int stb1 = (stb + 1 == SBS) ? 0 : stb + 1;
    const char* sA_ = sa(st);
    const char* sB_ = sb(stb);
    static_for<SUBS>([&](auto S) {
      constexpr int s = decltype(S)::value;
      constexpr int t = s + FD;  // the substep whose fragments are read here
      constexpr int cur = s % NFB, nxt = t % NFB;
      if constexpr (t < SUBS) {
        read_frags(fa[nxt], fb[nxt], sA_, sB_, t, kt);
      } else if constexpr (t == SUBS) {
        wait_vmcnt<(STAGES - 2) * NVM + WB>();
        barrier_before_refill();
        // fragment reads first, then the refill loads: the same order as the
        // schedule below, so the loads can be spread between the MFMAs
        read_frags(fa[nxt], fb[nxt], sa(st1), sb(stb1), 0, kt + 1);
        issueA(kt + STAGES, st);
        issueB(kt + SBS, stb);
      } else {
        read_frags(fa[nxt], fb[nxt], sa(st1), sb(stb1), t - SUBS, kt + 1);
      }
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = Mfma<T>::run(fb[cur][i], fa[cur][j], acc[i][j]);
      if constexpr (RMS) {
#pragma unroll
        for (int j = 0; j < TM; ++j) ss[j] = sumsq8<T>(fa[cur][j], ss[j]);
      }
      schedule_substep<TN * TM, NDS, (t == SUBS) ? NVM : 0, RMS ? TM * 4 : 0>();
      __builtin_amdgcn_sched_barrier(0);
    });
    st = st1;
    stb = stb1;
  }
  }
  wait_vmcnt0();
  __syncthreads();

  if constexpr (RMS) {
    // lanes l and l+32 hold the two k halves of the same row
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const float tot = ss[j] + __shfl_xor(ss[j], 32, 64);
      const float r = rsqrtf(tot / (float)a.K + a.rms_eps);
#pragma unroll
      for (int i = 0; i < TN; ++i) acc[i][j] *= r;
      // the first column of tiles publishes the row scales for other
      // consumers of the same normalised rows
      const int m = m0 + wm * WM + j * 32 + lane;
      if (a.rs_out && tn == 0 && wn == 0 && lane < 32 && m < a.M) a.rs_out[m] = r;
    }
  }

  if constexpr (!OUTF32) {
    if (a.fix) {
      // Split-K fix-up: store this K slice's accumulators (system-coherent,
      // visible to every XCD once vmcnt drains), arrive on the output
      // tile's counter; the last slice to arrive adds all partial tiles in
      // slice order (deterministic) and runs the epilogue.
      constexpr int kCoherent = 17;  // sc0 | sc1
      constexpr int TILE_B = BM * BN * 4;
      const int tile = tm * a.tiles_n + tn;  // < kWsMaxTiles (the planner's check)
      unsigned long long* cnt = (unsigned long long*)a.fix + tile;
      const __amdgpu_buffer_rsrc_t rP =
          make_rsrc(a.fix + kWsCounterBytes + (int64_t)tile * a.batch * TILE_B, (uint32_t)(a.batch * TILE_B));
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4v v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
            const uint32_t off = (uint32_t)(b * TILE_B + (((i * TM + j) * 4 + g) * NT + threadIdx.x) * 16);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4v, v), rP, off, 0, kCoherent);
          }
      wait_vmcnt0();
      // The flag lives in the operand stages (all loads landed, no reads
      // left): a second __shared__ variable would make the compiler tag
      // every LDS access with per-variable alias scopes, and then wait for
      // every direct-to-LDS load before each transposing fragment read.
      int& is_last = *(int*)smem;
      __syncthreads();
      if (threadIdx.x == 0) {
        // every other slice of this tile has stored its partials once the
        // count reaches batch; that slice alone touches the counter again
        const unsigned long long before =
            __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = before + 1 == (unsigned long long)a.batch;
        if (is_last) __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!is_last) return;
      // GS slices' loads in flight at once (the small tiles, whose partial
      // fragments fit in spare registers), then added in slice order
      constexpr int GS = TN * TM == 1 ? 4 : (TN * TM == 2 ? 2 : 1);
      if constexpr (GS == 1) {
        for (int sl = 0; sl < a.batch; ++sl) {
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const uint32_t off = (uint32_t)(sl * TILE_B + (((i * TM + j) * 4 + g) * NT + threadIdx.x) * 16);
                const float4v v =
                    __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rP, off, 0, kCoherent));
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[i][j][4 * g + q] = sl == 0 ? v[q] : acc[i][j][4 * g + q] + v[q];
              }
        }
      } else for (int sl0 = 0; sl0 < a.batch; sl0 += GS) {
        float4v part[GS][TN][TM][4];
#pragma unroll
        for (int u = 0; u < GS; ++u)
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int sl = sl0 + u;
                const uint32_t off = (uint32_t)(sl * TILE_B + (((i * TM + j) * 4 + g) * NT + threadIdx.x) * 16);
                part[u][i][j][g] = __builtin_bit_cast(
                    float4v, __builtin_amdgcn_raw_buffer_load_b128(rP, sl < a.batch ? off : kOOB, 0, kCoherent));
              }
#pragma unroll
        for (int u = 0; u < GS; ++u) {
          if (sl0 + u >= a.batch) break;
#pragma unroll
          for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  acc[i][j][4 * g + q] = sl0 + u == 0 ? part[u][i][j][g][q] : acc[i][j][4 * g + q] + part[u][i][j][g][q];
        }
      }
    }
  }

  if constexpr (!RMS) {
    if (a.rs_in) {
      // rows normalised by scales another GEMM computed (B holds the folded
      // norm weight)
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int m = m0 + wm * WM + j * 32 + (lane & 31);
        const float r = m < a.M ? a.rs_in[m] : 0.f;
#pragma unroll
        for (int i = 0; i < TN; ++i) acc[i][j] *= r;
      }
    }
  }

  // ---- epilogue -------------------------------------------------------------
  const float alpha = a.alpha;
  const int hi = lane >> 5;
  if constexpr (OUTF32) {
    char* Cb = a.C + (b * a.sC) * 4;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int m = m0 + wm * WM + j * 32 + (lane & 31);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WN + i * 32 + 8 * g + 4 * hi;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[i][j][4 * g + q] * alpha;
          if constexpr (BI8) {
            float sv[4];
            colvec4(cv_scale, a.scale, n - n0, sv);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] *= sv[q];
          }
          if constexpr (HAS_BIAS) {
            float bv[4];
            colvec4(cv_bias, a.bias, n - n0, bv);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += bv[q];
          }
          if constexpr (EPI == EPI_GELU_TANH || EPI == EPI_BIAS_GELU_TANH) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = gelu_tanh(v[q]);
          }
          if (m < a.M && n + 4 <= a.N) {
            *(float4v*)(Cb + ((int64_t)m * a.ldc + n) * 4) = float4v{v[0], v[1], v[2], v[3]};
          } else if (m < a.M && n < a.N) {  // ragged last columns
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (n + q < a.N) ((float*)Cb)[(int64_t)m * a.ldc + n + q] = v[q];
          }
        }
      }
    return;
  } else {
    __syncthreads();  // every wave is done reading the operand stages
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int ml = wm * WM + j * 32 + (lane & 31);
        if constexpr (EPI == EPI_SILU_MUL) {
          // packed columns [32q, 32q+16) are gate, [32q+16, 32q+32) are up
          // for output columns [16q, 16q+16)
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float gate = acc[i][j][4 * g + q] * alpha;
              const float up = acc[i][j][4 * (g + 2) + q] * alpha;
              v[q] = silu(gate) * up;
            }
            const int ol = (wn * WN + i * 32) / 2 + 8 * g + 4 * hi;
            store4<T>(smem + ml * SROW + ol * 2, v[0], v[1], v[2], v[3]);
          }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int nl = wn * WN + i * 32 + 8 * g + 4 * hi;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc[i][j][4 * g + q] * alpha;
            if constexpr (BI8) {
              float sv[4];
              colvec4(cv_scale, a.scale, nl, sv);
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] *= sv[q];
            }
            if constexpr (HAS_BIAS) {
              float bv[4];
              colvec4(cv_bias, a.bias, nl, bv);
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] += bv[q];
            }
            if constexpr (EPI == EPI_GELU_TANH || EPI == EPI_BIAS_GELU_TANH) {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = gelu_tanh(v[q]);
            }
            store4<T>(smem + ml * SROW + nl * 2, v[0], v[1], v[2], v[3]);
          }
        }
      }
    __syncthreads();
    constexpr int CPRO = BNO / 8;
    const int Nout = (EPI == EPI_SILU_MUL) ? a.N / 2 : a.N;
    const int n0o = (EPI == EPI_SILU_MUL) ? n0 / 2 : n0;
    char* Cb = a.C + (b * a.sC) * 2;
#pragma unroll 4
    for (int t = threadIdx.x; t < BM * CPRO; t += NT) {
      const int row = t / CPRO, cc = t % CPRO;
      const int m = m0 + row, n = n0o + cc * 8;
      if (m < a.M && n + 8 <= Nout) {
        int4v v = *(const int4v*)(smem + row * SROW + cc * 16);
        *(int4v*)(Cb + ((int64_t)m * a.ldc + n) * 2) = v;
      } else if (m < a.M && n < Nout) {  // ragged last columns
        const short* src = (const short*)(smem + row * SROW + cc * 16);
        short* dst = (short*)(Cb + ((int64_t)m * a.ldc + n) * 2);
        for (int q = 0; q < Nout - n; ++q) dst[q] = src[q];
      }
    }
  }
}

struct TileShape {
  int BM, BN, WM, WN, BK, STAGES;
  bool PP = false;
  int SB = 0;  // B stages (0: as many as A)
  int FD = 1;  // substeps between a fragment's LDS read and its MFMAs
};

// The small tiles run three LDS stages: their K-steps are short (a 64x64x64
// step is ~130 MFMA cycles per wave), so with two stages every step waits a
// full memory round trip for the next; a third stage keeps two steps in
// flight while two or three workgroups still fit per CU.  Measured on the
// TinyLlama block in sequence (weights not resident in L2): 91.0 -> 79.3 us;
// four stages, at half the workgroups per CU, gave 87.1 us.
// The tiles of at most 128 rows read their fragments three substeps ahead
// (FD = 3): with one or two waves per SIMD and one to four MFMAs per wave
// and substep, an LDS read issued one substep ahead had not returned by its
// MFMA.  1024^3 NN on 64x64 tiles: 7.3 -> 6.3 us; the block's GEMMs and the
// 256-row tiles (two waves per SIMD, eight MFMAs a substep) did not change.
// The 384-row tiles (256x128 and 128x256, 48 KB per stage) hold one
// workgroup per CU with two stages already, so a third costs no occupancy:
// TinyLlama gate/up with SiLU-mul on the 8-wave 256x128 tile went 33.7 ->
// 30.7 us (the 8-wave 128x128 tile at two per CU: 33.1 us; with three or
// four stages, one per CU, 40.8 / 42.0 us).
// The 8-wave 128x192 tile (three 32-column MFMA blocks a wave, 40 KB a
// stage, one workgroup per CU) fills more CUs in one round where 128-row
// tiles would need two per CU: TinyLlama gate/up (512 x 11264) runs 236
// tiles on 236 CUs instead of 176 of 256x128, 28.4 -> 27.6 us and the block
// 76.6 -> 74.9-75.4 us; ViT-B/16 fc1 (1576 x 3072) 208 tiles instead of 312
// of 128x128 at two per CU, 17.3 -> 15.8 us.  Four waves of 64x96 on the same
// tile: 29.4 and 18.1 us.  It takes k-contiguous B ([N, K]) only: an NN
// B row of 192 columns (384 bytes) does not divide the 1 KB wave load, and
// 192 rows do not split into the int8 B loads' 16-row groups over 8 waves.
constexpr TileShape kTiles[TILE_COUNT] = {
    {256, 256, 128, 128, 64, 2},  // TILE_256x256
    {128, 256, 64, 128, 64, 3, false, 0, 3},   // TILE_128x256
    {256, 128, 128, 64, 64, 3},   // TILE_256x128
    {128, 128, 64, 64, 64, 2, false, 0, 3},    // TILE_128x128
    {64, 128, 32, 64, 64, 3, false, 0, 3},     // TILE_64x128
    {128, 64, 64, 32, 64, 3, false, 0, 3},     // TILE_128x64
    {64, 64, 32, 32, 64, 3, false, 0, 3},      // TILE_64x64
    {256, 256, 128, 128, 32, 4},  // TILE_256x256_K32S4
    {256, 256, 128, 64, 64, 2},   // TILE_256x256_W8
    {128, 128, 64, 64, 32, 4},    // TILE_128x128_K32S4
    {256, 128, 128, 64, 32, 4},   // TILE_256x128_K32S4
    {256, 256, 128, 64, 32, 3, true},  // TILE_256x256_PP
    {256, 128, 64, 64, 64, 3},         // TILE_256x128_W8
    {128, 128, 32, 64, 64, 2, false, 0, 3},    // TILE_128x128_W8
    {128, 192, 32, 96, 64, 3, false, 0, 3},    // TILE_128x192_W8
    {64, 64, 32, 32, 64, 4, false, 0, 3},      // TILE_64x64_S4
};

template <int TILE, bool NN, typename T, int EPI, bool OUTF32, bool BI8, bool RMS = false, bool RAGGED = false>
hipError_t launch_one(const KArgs& k, hipStream_t stream) {
  constexpr TileShape s = kTiles[TILE];
  constexpr int threads = (s.BM / s.WM) * (s.BN / s.WN) * 64;
  const int64_t blocks = (int64_t)k.tiles_m * k.tiles_n * k.batch;
  // int8 B: BK 64, two A stages (A is L2-resident) and up to six B stages
  // in the LDS that three stages of both took (same workgroups per CU): the
  // weights stream from HBM, so B is prefetched several K-steps ahead
  constexpr int W8_A = s.BM * 128, W8_B = s.BN * 64;
  constexpr int W8_SB = W8_A / W8_B + 3 > 6 ? 6 : W8_A / W8_B + 3;
  hipLaunchKernelGGL((gemm_mfma<s.BM, s.BN, s.WM, s.WN, (BI8 ? 64 : s.BK), (BI8 ? 2 : s.STAGES), NN, T, EPI, OUTF32, BI8,
                                (s.PP && !BI8 && !RMS), RMS, RAGGED, (BI8 ? W8_SB : s.SB), (BI8 || s.PP ? 1 : s.FD)>),
                     dim3((unsigned)blocks), dim3(threads), 0, stream, k);
  return hipGetLastError();
}

template <bool NN, typename T, int EPI, bool OUTF32, bool BI8 = false, bool RMS = false>
hipError_t launch_tile(int tile, const KArgs& k, hipStream_t stream) {
  switch (tile) {
    case TILE_256x256: return launch_one<TILE_256x256, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x256: return launch_one<TILE_128x256, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x128: return launch_one<TILE_256x128, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x128: return launch_one<TILE_128x128, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_64x128: return launch_one<TILE_64x128, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x64: return launch_one<TILE_128x64, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x256_K32S4: return launch_one<TILE_256x256_K32S4, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x256_W8: return launch_one<TILE_256x256_W8, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x128_K32S4: return launch_one<TILE_128x128_K32S4, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x128_K32S4: return launch_one<TILE_256x128_K32S4, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x256_PP: return launch_one<TILE_256x256_PP, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_256x128_W8: return launch_one<TILE_256x128_W8, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x128_W8: return launch_one<TILE_128x128_W8, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_128x192_W8:
      if constexpr (BI8 || NN) return hipErrorNotSupported;  // (k-contiguous fp16 / bf16 B only)
      else return launch_one<TILE_128x192_W8, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    case TILE_64x64_S4: return launch_one<TILE_64x64_S4, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
    default: return launch_one<TILE_64x64, NN, T, EPI, OUTF32, BI8, RMS>(k, stream);
  }
}

}  // namespace gemm
}  // namespace hxmi
