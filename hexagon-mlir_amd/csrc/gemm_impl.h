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
//     bank-conflict free; a [K,N] (NN) operand is read with ds_read_b64_tr_b16;
//   * the MFMA is issued as D[n][m] = B^T . A^T so every lane owns four
//     consecutive output columns, which makes the fused epilogue (bias,
//     SiLU-mul, tanh-GELU) and the LDS-staged 16-byte stores cheap.
#pragma once

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

// Fragment of a k-contiguous tile stored as [rows][64] with 16-byte chunks
// XOR-swizzled by (row & 7).  MFMA 32x32x16 operand layout: lane l holds row
// (l % 32), k = 8*(l / 32) .. +7 of the 16-deep step s.
__device__ __forceinline__ short8v read_kc(const char* tile, int r_off, int s, int lane) {
  const int r = r_off + (lane & 31);
  const int c = (s << 1) + (lane >> 5);
  return *(const short8v*)(tile + r * 128 + ((c ^ (r & 7)) << 4));
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
  if (n < N) {
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

template <int BM, int BN, int WM, int WN, bool NN, typename T, int EPI, bool OUTF32, bool BI8 = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma(KArgs a) {
  constexpr int NWM = BM / WM, NWN = BN / WN, NW = NWM * NWN, NT = NW * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int BNO = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  constexpr int SROW = BNO * 2 + 16;
  constexpr int EPI_BYTES = OUTF32 ? 0 : BM * SROW;
  constexpr int SMEM = (2 * STAGE > EPI_BYTES) ? 2 * STAGE : EPI_BYTES;
  static_assert(BM % (8 * NW) == 0, "A tile rows per wave");
  static_assert(NN || BN % (8 * NW) == 0, "B tile rows per wave");
  static_assert(!BI8 || (!NN && !OUTF32), "int8 B is [N,K] with fp16 output");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w / NWN, wn = w % NWN;

  int b, tm, tn;
  map_tile(blockIdx.x, a, b, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = a.K;

  const char* Ab = a.A + (b * a.sA + (int64_t)m0 * a.lda) * 2;
  const char* Bb = NN    ? a.B + (b * a.sB + (int64_t)n0) * 2
                   : BI8 ? a.B + (b * a.sB + (int64_t)n0 * a.ldb)
                         : a.B + (b * a.sB + (int64_t)n0 * a.ldb) * 2;

  // ---- per-lane load plan -------------------------------------------------
  constexpr int IA = BM / 8 / NW;
  uint32_t offA[IA];
  bool okA[IA];
  const int cA = (lane & 7) ^ (lane >> 3);
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int row = (i * NW + w) * 8 + (lane >> 3);
    okA[i] = (m0 + row) < a.M;
    offA[i] = (uint32_t)(row * a.lda * 2 + cA * 16);
  }

  constexpr int CPR = BN / 8;                              // NN: 16-byte chunks per k-row
  constexpr int RPI = NN ? (1024 / (BN * 2)) : 8;          // rows per wave instruction
  constexpr int IB = NN ? (BK / RPI / NW) : (BN / 8 / NW);
  static_assert(IB >= 1, "B load plan");
  uint32_t offB[IB];
  bool okB[IB];
  int rowB[IB];
  int cB = 0;
#pragma unroll
  for (int i = 0; i < IB; ++i) {
    if constexpr (NN) {
      const int row = (i * NW + w) * RPI + lane / CPR;
      const int c = (lane % CPR) ^ nn_swz<BN>(row);
      rowB[i] = row;
      okB[i] = (n0 + c * 8) < a.N;
      offB[i] = (uint32_t)(row * a.ldb * 2 + c * 16);
    } else {
      const int row = (i * NW + w) * 8 + (lane >> 3);
      cB = cA;
      rowB[i] = row;
      okB[i] = (n0 + row) < a.N;
      offB[i] = (uint32_t)(row * a.ldb * 2 + cA * 16);
    }
  }

  // int8 B: register-staged, 16 weights (one row, 16 k) per 16-byte load,
  // dequantised to fp16 on the way into the same swizzled LDS layout.
  constexpr int I8L = BI8 ? (BN * 4 + NT - 1) / NT : 1;
  uint32_t offQ[I8L];
  int rowQ[I8L], qQ[I8L];
  bool okQ[I8L];
  int4v regQ[I8L];
  if constexpr (BI8) {
#pragma unroll
    for (int i = 0; i < I8L; ++i) {
      const int idx = i * NT + threadIdx.x;
      rowQ[i] = idx >> 2;
      qQ[i] = idx & 3;
      okQ[i] = idx < BN * 4 && (n0 + rowQ[i]) < a.N;
      offQ[i] = (uint32_t)(rowQ[i] * a.ldb + qQ[i] * 16);
    }
  }
  auto load_q = [&](int kt) {
    const int k0 = kt * BK;
    const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Bb + k0, 0x7fffffff);
#pragma unroll
    for (int i = 0; i < I8L; ++i) {
      const bool ok = okQ[i] && (k0 + qQ[i] * 16) < K;
      regQ[i] = load16(rQ, ok ? offQ[i] : kOOB);
    }
  };
  auto store_q = [&](int stage) {
    char* sB_ = smem + stage * STAGE + A_BYTES;
#pragma unroll
    for (int i = 0; i < I8L; ++i) {
      if (BN * 4 % NT == 0 || i * NT + (int)threadIdx.x < BN * 4) {
        const int r = rowQ[i];
        const short8v lo = dequant8(int2v{regQ[i][0], regQ[i][1]});
        const short8v hi = dequant8(int2v{regQ[i][2], regQ[i][3]});
        *(short8v*)(sB_ + r * 128 + (((2 * qQ[i]) ^ (r & 7)) << 4)) = lo;
        *(short8v*)(sB_ + r * 128 + (((2 * qQ[i] + 1) ^ (r & 7)) << 4)) = hi;
      }
    }
  };

  auto issue = [&](int kt, int stage) {
    const int k0 = kt * BK;
    char* sA_ = smem + stage * STAGE;
    char* sB_ = sA_ + A_BYTES;
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(Ab + (int64_t)k0 * 2, 0x7fffffff);
    const bool kokA = (k0 + cA * 8) < K;
#pragma unroll
    for (int i = 0; i < IA; ++i) {
      const int rb = (i * NW + w) * 8;
      load_lds16(rA, (HXMI_LDS void*)to_lds(sA_ + rb * 128), (okA[i] && kokA) ? offA[i] : kOOB);
    }
    if constexpr (NN) {
      const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bb + (int64_t)k0 * a.ldb * 2, 0x7fffffff);
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int rb = (i * NW + w) * RPI;
        const bool ok = okB[i] && (k0 + rowB[i]) < K;
        load_lds16(rB, (HXMI_LDS void*)to_lds(sB_ + rb * (BN * 2)), ok ? offB[i] : kOOB);
      }
    } else if constexpr (!BI8) {
      const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bb + (int64_t)k0 * 2, 0x7fffffff);
      const bool kokB = (k0 + cB * 8) < K;
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int rb = (i * NW + w) * 8;
        load_lds16(rB, (HXMI_LDS void*)to_lds(sB_ + rb * 128), (okB[i] && kokB) ? offB[i] : kOOB);
      }
    }
  };

  float16v acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = float16v{};

  const int nk = (K + BK - 1) / BK;
  if (nk > 0) {
    issue(0, 0);
    if constexpr (BI8) {
      load_q(0);
      store_q(0);
    }
  }
  for (int kt = 0; kt < nk; ++kt) {
    wait_vmcnt0();
    __syncthreads();
    if (kt + 1 < nk) {
      issue(kt + 1, (kt + 1) & 1);
      if constexpr (BI8) load_q(kt + 1);
    }
    const char* sA_ = smem + (kt & 1) * STAGE;
    const char* sB_ = sA_ + A_BYTES;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      short8v bf[TN], af[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        if constexpr (NN)
          bf[i] = read_nn<BN>(sB_, wn * WN + i * 32, s, lane);
        else
          bf[i] = read_kc(sB_, wn * WN + i * 32, s, lane);
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) af[j] = read_kc(sA_, wm * WM + j * 32, s, lane);
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = Mfma<T>::run(bf[i], af[j], acc[i][j]);
    }
    if constexpr (BI8) {
      if (kt + 1 < nk) store_q((kt + 1) & 1);
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
          if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU_TANH) {
            float bv[4];
            load_bias4<T>(a.bias, n, a.N, bv);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += bv[q];
          }
          if constexpr (EPI == EPI_GELU_TANH || EPI == EPI_BIAS_GELU_TANH) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = gelu_tanh(v[q]);
          }
          if (m < a.M && n < a.N)
            *(float4v*)(Cb + ((int64_t)m * a.ldc + n) * 4) = float4v{v[0], v[1], v[2], v[3]};
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
              load_bias4<T>(a.scale, n0 + nl, a.N, sv);
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] *= sv[q];
            }
            if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU_TANH) {
              float bv[4];
              load_bias4<T>(a.bias, n0 + nl, a.N, bv);
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
      if (m < a.M && n < Nout) {
        int4v v = *(const int4v*)(smem + row * SROW + cc * 16);
        *(int4v*)(Cb + ((int64_t)m * a.ldc + n) * 2) = v;
      }
    }
  }
}

struct TileShape {
  int BM, BN, WM, WN;
};

constexpr TileShape kTiles[TILE_COUNT] = {
    {256, 256, 128, 128},  // TILE_256x256
    {128, 256, 64, 128},   // TILE_128x256
    {256, 128, 128, 64},   // TILE_256x128
    {128, 128, 64, 64},    // TILE_128x128
    {64, 128, 32, 64},     // TILE_64x128
    {128, 64, 64, 32},     // TILE_128x64
    {64, 64, 32, 32},      // TILE_64x64
};

template <int TILE, bool NN, typename T, int EPI, bool OUTF32, bool BI8>
hipError_t launch_one(const KArgs& k, hipStream_t stream) {
  constexpr TileShape s = kTiles[TILE];
  constexpr int threads = (s.BM / s.WM) * (s.BN / s.WN) * 64;
  const int64_t blocks = (int64_t)k.tiles_m * k.tiles_n * k.batch;
  hipLaunchKernelGGL((gemm_mfma<s.BM, s.BN, s.WM, s.WN, NN, T, EPI, OUTF32, BI8>),
                     dim3((unsigned)blocks), dim3(threads), 0, stream, k);
  return hipGetLastError();
}

template <bool NN, typename T, int EPI, bool OUTF32, bool BI8 = false>
hipError_t launch_tile(int tile, const KArgs& k, hipStream_t stream) {
  switch (tile) {
    case TILE_256x256: return launch_one<TILE_256x256, NN, T, EPI, OUTF32, BI8>(k, stream);
    case TILE_128x256: return launch_one<TILE_128x256, NN, T, EPI, OUTF32, BI8>(k, stream);
    case TILE_256x128: return launch_one<TILE_256x128, NN, T, EPI, OUTF32, BI8>(k, stream);
    case TILE_128x128: return launch_one<TILE_128x128, NN, T, EPI, OUTF32, BI8>(k, stream);
    case TILE_64x128: return launch_one<TILE_64x128, NN, T, EPI, OUTF32, BI8>(k, stream);
    case TILE_128x64: return launch_one<TILE_128x64, NN, T, EPI, OUTF32, BI8>(k, stream);
    default: return launch_one<TILE_64x64, NN, T, EPI, OUTF32, BI8>(k, stream);
  }
}

}  // namespace gemm
}  // namespace hxmi
