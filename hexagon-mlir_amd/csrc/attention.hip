// Fused attention O = softmax(scale * Q.K^T + mask) . V for head dims 64 and
// 128, with an optional additive fp16 mask, a causal rule and grouped K/V
// heads.
//
// The reference lowers tm_tensor.attention to batch_matmul(Q, K^T), a scale,
// the mask add, a row softmax and batch_matmul(P, V) (LowerTmTensor.cpp:91-250,
// mask at :158-163), each a separate pass over HBM.  Here one kernel streams
// K and V once per query block and keeps S and P in registers (online
// softmax, Milakov & Gimelshein 2018, the blockwise form the reference's
// test/python/triton/test_online_softmax.py:30-81 exercises):
//   * a workgroup owns QG x 32 queries of one (batch, head) slice and runs
//     QG x KS waves: wave (qg, kh) takes the 32 queries of group qg against
//     every KS-th block of 32 keys, and the KS partial (max, sum, O) of a
//     query group are merged through LDS at the end;
//   * K and V pass through LDS in chunks of 256 keys (D = 64; 128 for
//     D = 128: 64 KB either way) with direct global->LDS buffer loads, whose
//     out-of-range rows read as zeros;
//   * S is computed as D[key][query] = K . Q^T with v_mfma_f32_32x32x16_f16,
//     so every lane owns one query's scores: the row max / sum are in-lane
//     plus one exchange with the lane 32 away;
//   * the running max is only raised when a block's max exceeds it by more
//     than 8 (in log2 units), so most blocks skip the rescale of O; the
//     unnormalised weights then stay below 2^8, well inside fp16;
//   * the fp16 probabilities of a 32-key block are exactly the B operand of
//     the P.V MFMA for two 16-key steps (the k order inside an MFMA is free as
//     long as both operands use the same one); the matching V^T operand comes
//     from LDS with ds_read_b64_tr_b16, so P never leaves registers;
//   * O = D[d][query] accumulates in registers and is divided by the sum of
//     the same fp16 weights once at the end.  A query whose every key is
//     masked divides 0 by 0 (NaN), as the reference's decomposition does.
#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct AArgs {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  const char* mask;
  int bh, sq, skv;
  int nqb;         // query blocks per slice
  int kv_group;    // query slices per K/V slice
  int mask_group;  // query slices per mask slice
  int causal_off;  // key > query + causal_off is masked (skv: no causal rule)
  int mask_vec;    // mask rows allow aligned 8-byte loads
  uint32_t kbytes, vbytes;  // extent of one K / V slice
  int64_t ldq, ldk, ldv, ldo, ldm;  // row strides, elements
  int64_t bq, bk, bv, bo, bm;       // slice strides, elements
  float c;                          // scale * log2(e)
};

// Combine a value with the one of the lane 32 away (v_permlane32_swap: one
// VALU op instead of a round trip through LDS).
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float16v mfma32(short8v a, short8v b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a), __builtin_bit_cast(half8v, b), c, 0,
                                                0, 0);
}

// K chunk: [KC][D] fp16, rows of 2*D bytes, 16-byte chunks XOR-swizzled as
// the GEMM's k-contiguous tiles; V chunk: [KC][D], 16-byte chunks XOR-ed with
// a multiple of (key & 3) chosen so the 8 row segments (2 lane groups x 4
// keys x 32 bytes) of one transposing read phase cover all 64 banks.  Both
// are involutions on the chunk index, so the loader inverts them the same way.
template <int D>
__device__ __forceinline__ int k_swz(int r) {
  constexpr int RB = 2 * D;
  return (r / (256 / RB)) & (RB / 16 - 1);
}
template <int D>
__device__ __forceinline__ int v_swz(int r) {
  return (r & 3) << (D == 64 ? 1 : 2);  // 32-byte steps for 128-byte rows, 64-byte for 256
}
template <int D>
__device__ __forceinline__ int k_off(int r, int c) {
  return r * (2 * D) + ((c ^ k_swz<D>(r)) << 4);
}
template <int D>
__device__ __forceinline__ int v_off(int r, int c) {
  return r * (2 * D) + ((c ^ v_swz<D>(r)) << 4);
}

template <int D, int QG, int KS>
struct AttnShape {
  static constexpr int NT = 64 * QG * KS;
  static constexpr int KC = D == 64 ? 256 : 128;  // keys per LDS chunk
  static constexpr int CHUNK = KC * 2 * D;        // bytes of K (and of V) per chunk: 32 KB
  static constexpr int NV = D / 32 * 16 + 2;      // floats per lane in the key-split merge
  static constexpr bool ok = NT <= 1024 && (KS - 1) * QG * NV * 64 * 4 <= 2 * CHUNK;
};

// PIPE: the key blocks of a chunk start load index by load index (below);
// chosen at launch for sequences of at least one chunk.
template <int D, int QG, int KS, bool MASK, bool PIPE>
__global__ __launch_bounds__(64 * QG * KS) void attention_fwd(AArgs a) {
  using Sh = AttnShape<D, QG, KS>;
  static_assert(Sh::ok, "attention shape");
  constexpr int NW = QG * KS;
  constexpr int KC = Sh::KC;
  constexpr int CHUNK = Sh::CHUNK;
  constexpr int RB = 2 * D;     // bytes per K / V row
  constexpr int DS = D / 16;    // 16-deep MFMA steps over the head dim
  constexpr int DT = D / 32;    // 32-wide output tiles over the head dim
  constexpr int LPW = CHUNK / 1024 / NW;  // 1 KB direct loads of K (and of V) per wave per chunk
  static_assert(LPW * NW * 1024 == CHUNK, "chunk split");
  __shared__ __attribute__((aligned(1024))) char lds[2 * CHUNK];
  char* const ks = lds;
  char* const vs = lds + CHUNK;

  const int lane = threadIdx.x & 63;
  // wave-uniform values live in scalar registers, so branches on them are
  // scalar branches rather than exec-masked paths
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qg = w % QG, kh = w / QG;
  const int h = lane >> 5;

  // workgroup -> (slice, query block).  Workgroups go round-robin over the
  // 8 XCDs; each XCD takes a contiguous run, so the query blocks of a slice
  // (and slices sharing a K/V head) read K and V through one L2.
  const int total = a.bh * a.nqb;
  const int per = total >> 3, rem = total & 7;
  const int xcd = blockIdx.x & 7;
  const int r = xcd * per + (xcd < rem ? xcd : rem) + (int)(blockIdx.x >> 3);
  const int bh = r / a.nqb;
  const int qb0 = (r - bh * a.nqb) * (32 * QG);
  const int q0 = qb0 + qg * 32;
  const int qme = q0 + (lane & 31);
  const int kvbh = bh / a.kv_group;
  const char* Q = a.q + (int64_t)bh * a.bq * 2;
  const char* Kp = a.k + (int64_t)kvbh * a.bk * 2;
  const char* Vp = a.v + (int64_t)kvbh * a.bv * 2;

  // keys this workgroup / this wave needs (the causal rule cuts both)
  const int wg_qlast = min(qb0 + 32 * QG, a.sq) - 1;
  const int kend = min(a.skv, wg_qlast + a.causal_off + 1);
  const int wkend = q0 < a.sq ? max(0, min(a.skv, min(q0 + 31, a.sq - 1) + a.causal_off + 1)) : 0;

  const _Float16* mrow = nullptr;
  if (MASK && qme < a.sq)
    mrow = (const _Float16*)a.mask + ((int64_t)(bh / a.mask_group) * a.bm + (int64_t)qme * a.ldm);

  // direct loads: wave w's load i fills LDS bytes [(i*NW + w) KB, +1 KB) of
  // the chunk; lane l's 16 bytes there are row (i*NW + w) * (1024/RB) + lr,
  // stored chunk cs, which holds the row's chunk cs ^ swizzle(row)
  const int lr = lane / (RB / 16), cs = lane % (RB / 16);
  const __amdgpu_buffer_rsrc_t rK = make_rsrc(Kp, a.kbytes);
  const __amdgpu_buffer_rsrc_t rV = make_rsrc(Vp, a.vbytes);

  float16v oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = float16v{};
  float m_run = -INFINITY, l_run = 0.f;
  // This lane's V^T fragment reads for output tile dt sit at vbase[dt] plus
  // a multiple of 4 rows: the chunk's V swizzle depends on (row & 3) only,
  // so rows 4h + L/4 + 32b + 16t (+ 8) share one column offset.
  int vbase[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int g = lane >> 4, L = lane & 15;
    const int d = dt * 32 + ((g & 1) << 4) + ((L & 3) << 2);
    vbase[dt] = v_off<D>(4 * h + (L >> 2), d >> 3) + (d & 7) * 2;
  }

  auto issue_chunk = [&](int c0) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int row = (i * NW + w) * (1024 / RB) + lr;
      const int key = c0 + row;
      const bool live = key < kend;
      const uint32_t ko = live ? (uint32_t)(key * a.ldk * 2 + ((cs ^ k_swz<D>(row)) << 4)) : kOOB;
      const uint32_t vo = live ? (uint32_t)(key * a.ldv * 2 + ((cs ^ v_swz<D>(row)) << 4)) : kOOB;
      load_lds16(rK, (HXMI_LDS void*)to_lds(ks + (i * NW + w) * 1024), ko);
      load_lds16(rV, (HXMI_LDS void*)to_lds(vs + (i * NW + w) * 1024), vo);
    }
  };
  // Q fragments of this wave's 32 queries (zero past the sequence), then
  // the first chunk's K / V: the chunk's loads are waited for load index by
  // load index (below), which leaves the later ones in flight only when Q
  // was issued before them.  The Q loads take no branch (an offset past the
  // buffer reads zeros), so the compiler does not wait for them early.
  short8v qf[DS];
  {
    const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q, 0x7fffffffu);
#pragma unroll
    for (int s = 0; s < DS; ++s)
      qf[s] = __builtin_bit_cast(
          short8v, load16(rQ, qme < a.sq ? (uint32_t)(((int64_t)qme * a.ldq + s * 16 + h * 8) * 2) : kOOB));
  }
  if (kend > 0) issue_chunk(0);

  // Keys [c0, c0 + KC) of one chunk, its loads issued: load index i of every
  // wave brings keys [i KPL, (i + 1) KPL) of K and V.  PIPE: before the key
  // blocks of round j (block kh + j KS of wave kh) every wave waits for its
  // loads up to the last index the round reads (the next round's K for the
  // scores computed ahead), then one barrier, so the first blocks start when
  // their keys have landed rather than the whole chunk.  That pays on full
  // chunks (2 x 12 x 1024: 17.2 -> 16.85 us; head dim 128, 16 x 512 causal:
  // 10.47 -> 10.15 us) but not on a short one, where the extra barriers
  // cost more than the overlap gives (ViT-B/16, 197 keys: 7.47 -> 7.56 us),
  // so the launch takes PIPE only for sequences of at least KC keys; the
  // other instance waits for the first half of the chunk, then for the
  // rest (ViT-B/16 7.35-7.41 -> 7.31-7.32 us against one wait for all).  (One kernel with both
  // paths, chosen per chunk, took 30-60 more VGPRs, and the head-dim-128
  // instances then held one wave per SIMD instead of two.)
  constexpr int KPL = NW * (1024 / RB);
  constexpr int JMAX = KC / 32 / KS;
  constexpr auto li_end = [](int b) constexpr {
    const int i = ((b + 1) * 32 - 1) / KPL;  // the load index of block b's last key, within the chunk
    return i < LPW - 1 ? i : LPW - 1;
  };
  auto run_chunk = [&](int c0) {
    const int cn = min(KC, wkend - c0);
    const int nblk = cn > 0 ? (cn + 31) >> 5 : 0;
    // S block b: D[key][query], lane holds query lane%32, keys 8g + 4h + j
    auto scores = [&](int b) {
      float16v sb = {};
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const short8v kf = *(const short8v*)(ks + k_off<D>(b * 32 + (lane & 31), st * 2 + h));
        sb = mfma32(kf, qf[st], sb);
      }
      return sb;
    };
    // mask entries of block b's 16 scores of this lane: keys kb + 8g + 4h + j
    auto mask_vals = [&](int b, _Float16 (&mk)[16]) {
      const int kb = c0 + b * 32;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int kk = kb + 8 * g + 4 * h;
        if (mrow && a.mask_vec && kk + 4 <= a.skv) {
          const half4v m4 = *(const half4v*)(mrow + kk);
#pragma unroll
          for (int j = 0; j < 4; ++j) mk[4 * g + j] = m4[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) mk[4 * g + j] = (mrow && kk + j < a.skv) ? mrow[kk + j] : (_Float16)0.f;
        }
      }
    };
    // Block b: its scores s (and mask entries mk) are in registers; the MFMAs
    // of the next block's scores (and its mask loads) go out into s_nx / mk_nx
    // first, so they run while this block's softmax occupies the vector
    // ALUs.
    auto block = [&](int b, float16v& s, float16v& s_nx, _Float16 (&mk)[16], _Float16 (&mk_nx)[16]) {
      const int kb = c0 + b * 32;
      if (MASK && b + KS < nblk) mask_vals(b + KS, mk_nx);
      if (b + KS < nblk) s_nx = scores(b + KS);
      // ragged keys and the causal rule only reach the blocks at their edges
      const bool edge = kb + 32 > a.skv || kb + 31 > q0 + a.causal_off;
      const bool scaled = MASK || edge;
      float mx = -INFINITY;
      if (scaled) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float t = s[i] * a.c;
          if constexpr (MASK) t = fmaf((float)mk[i], kLog2e, t);
          if (edge) {
            const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
            if (key >= a.skv || key > qme + a.causal_off) t = -INFINITY;
          }
          s[i] = t;
          mx = fmaxf(mx, t);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
        mx *= a.c;  // scale > 0
      }
      mx = xor32_max(mx);
      const bool upd = mx > m_run + 8.0f;
      if (__any(upd)) {
        const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;  // 0 on a first block
        if (upd) m_run = mx;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;  // every key so far masked: weights 0
      const float cs = scaled ? 1.0f : a.c;                    // s already scaled on the edge path
      half2v p2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        p2[i] = half2v{(_Float16)__builtin_amdgcn_exp2f(fmaf(s[2 * i], cs, -m_use)),
                       (_Float16)__builtin_amdgcn_exp2f(fmaf(s[2 * i + 1], cs, -m_use))};
      // the row sum uses the fp16 weights P.V sees, so O is their exact
      // weighted average (a constant V comes back unchanged)
      float psum = 0.f;
      const half2v one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
      for (int i = 0; i < 8; ++i) psum = __builtin_amdgcn_fdot2(p2[i], one2, psum, false);
      l_run += psum;
      // two 16-key MFMA steps: step t uses keys {16t + 4h + j, 16t + 8 + 4h + j},
      // at rows 32 b + 16 t (+ 8) past this lane's V base
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const short8v pf = __builtin_bit_cast(
            short8v, half8v{p2[4 * t][0], p2[4 * t][1], p2[4 * t + 1][0], p2[4 * t + 1][1], p2[4 * t + 2][0],
                            p2[4 * t + 2][1], p2[4 * t + 3][0], p2[4 * t + 3][1]});
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const char* vb = vs + vbase[dt] + (b * 32 + 16 * t) * RB;
          const short4v lo = lds_read_tr16(vb);
          const short4v hi = lds_read_tr16(vb + 8 * RB);
          const short8v vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          oacc[dt] = mfma32(vf, pf, oacc[dt]);
        }
      }
    };
    constexpr bool pipe = PIPE;
    // (the other instance: the first half of the chunk, then the rest)
    constexpr int L0 = pipe ? li_end(KS - 1) : (li_end(KS - 1) > LPW / 2 - 1 ? li_end(KS - 1) : LPW / 2 - 1);
    wait_vmcnt<2 * (LPW - 1 - L0)>();
    barrier_after_lds_loads();
    float16v s_next = kh < nblk ? scores(kh) : float16v{};
    _Float16 mk_next[16];
    if (MASK && kh < nblk) mask_vals(kh, mk_next);
    static_for<JMAX>([&](auto J) {
      constexpr int j = decltype(J)::value;
      constexpr int need = li_end(KS - 1 + (j + 1) * KS), prev = li_end(KS - 1 + j * KS);
      constexpr int wn = pipe ? need : (need <= L0 ? L0 : LPW - 1);
      constexpr int wp = pipe ? prev : (prev <= L0 ? L0 : LPW - 1);
      if constexpr (wn > wp) {
        wait_vmcnt<2 * (LPW - 1 - wn)>();
        barrier_after_lds_loads();
      }
      const int b = kh + j * KS;
      if (b < nblk) {
        float16v s = s_next;
        _Float16 mk[16];
        if constexpr (MASK) {
#pragma unroll
          for (int i = 0; i < 16; ++i) mk[i] = mk_next[i];
        }
        block(b, s, s_next, mk, mk_next);
      }
    });
  };
  // the first chunk outside the loop: the compiler waits for every
  // outstanding load before a loop that reads registers loaded before it (Q)
  if (kend > 0) run_chunk(0);
  for (int c0 = KC; c0 < kend; c0 += KC) {
    __syncthreads();  // previous chunk fully consumed
    issue_chunk(c0);
    run_chunk(c0);
  }

  // merge the key-split partials of each query group into wave kh = 0
  if constexpr (KS > 1) {
    constexpr int NV = Sh::NV;
    __syncthreads();  // every wave is done with the K / V chunk
    float* red = (float*)lds;
    if (kh > 0) {
      float* dst = red + ((kh - 1) * QG + qg) * NV * 64 + lane;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) dst[(t * 16 + i) * 64] = oacc[t][i];
      dst[DT * 16 * 64] = m_run;
      dst[(DT * 16 + 1) * 64] = l_run;
    }
    __syncthreads();
    if (kh > 0) return;
#pragma unroll
    for (int o = 1; o < KS; ++o) {
      const float* src = red + ((o - 1) * QG + qg) * NV * 64 + lane;
      const float m2 = src[DT * 16 * 64], l2 = src[(DT * 16 + 1) * 64];
      const float mn = fmaxf(m_run, m2);
      const float a1 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
      const float a2 = m2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - mn);
      l_run = l_run * a1 + l2 * a2;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[t][i] = oacc[t][i] * a1 + src[(t * 16 + i) * 64] * a2;
      m_run = mn;
    }
  }

  // O = D[d][query]: lane holds query lane%32, d = 32 dt + 8 g + 4 h + j
  const float l_tot = xor32_sum(l_run);
  const float inv = 1.0f / l_tot;
  if (qme < a.sq) {
    char* O = a.o + ((int64_t)bh * a.bo + (int64_t)qme * a.ldo) * 2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        _Float16 o4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o4[j] = (_Float16)(oacc[dt][4 * g + j] * inv);
        *(short4v*)(O + (dt * 32 + 8 * g + 4 * h) * 2) = __builtin_bit_cast(short4v, o4);
      }
  }
}

template <int D, int QG, int KS>
hipError_t launch_cfg(AArgs a, const AttnProblem& p, bool mask, hipStream_t stream) {
  if constexpr (!AttnShape<D, QG, KS>::ok) {
    return hipErrorNotSupported;
  } else {
    a.nqb = (int)((p.s + 32 * QG - 1) / (32 * QG));
    const int64_t blocks = p.bh * a.nqb;
    if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(64 * QG * KS);
    const bool pipe = p.skv >= AttnShape<D, QG, KS>::KC;
    if (mask && pipe)
      hipLaunchKernelGGL((attention_fwd<D, QG, KS, true, true>), grid, block, 0, stream, a);
    else if (mask)
      hipLaunchKernelGGL((attention_fwd<D, QG, KS, true, false>), grid, block, 0, stream, a);
    else if (pipe)
      hipLaunchKernelGGL((attention_fwd<D, QG, KS, false, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attention_fwd<D, QG, KS, false, false>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
}

template <int D>
hipError_t launch_d(const AArgs& a, const AttnProblem& p, int cfg, hipStream_t stream) {
  const bool m = p.mask != nullptr;
  switch (cfg) {
    case 41: return launch_cfg<D, 4, 1>(a, p, m, stream);
    case 22: return launch_cfg<D, 2, 2>(a, p, m, stream);
    case 14: return launch_cfg<D, 1, 4>(a, p, m, stream);
    case 21: return launch_cfg<D, 2, 1>(a, p, m, stream);
    case 12: return launch_cfg<D, 1, 2>(a, p, m, stream);
    case 42: return launch_cfg<D, 4, 2>(a, p, m, stream);
    case 24: return launch_cfg<D, 2, 4>(a, p, m, stream);
    default: return hipErrorNotSupported;
  }
}

// Launch shape: query waves x key-split waves per workgroup.
int pick_cfg(const AttnProblem& p) {
  const int64_t forced = knob(KNOB_ATTN_CFG);
  if (forced != KNOB_UNSET) return (int)forced;
  // Enough 128-query workgroups to cover most CUs: 4 query waves (x2 key
  // splits at D = 64, where the merge fits in LDS); otherwise one query group
  // per workgroup with the keys split over 4 waves (ViT-B/16 batch 8: 7.3 us
  // against 7.6 / 10.8; a 32-head 512-token causal prefill: 8.3 us against
  // 10.9 / 11.3, measured on MI355X)
  const int64_t wg4 = p.bh * ((p.s + 127) / 128);
  if (wg4 >= 192) return p.d == 64 ? 42 : 41;
  return 14;
}

}  // namespace

hipError_t launch_attention(const AttnProblem& p, hipStream_t stream) {
  if (p.bh == 0 || p.s == 0) return hipSuccess;
  AArgs a{};
  a.q = (const char*)p.q;
  a.k = (const char*)p.k;
  a.v = (const char*)p.v;
  a.o = (char*)p.o;
  a.mask = (const char*)p.mask;
  a.bh = (int)p.bh;
  a.sq = (int)p.s;
  a.skv = (int)p.skv;
  a.kv_group = (int)p.kv_group;
  a.mask_group = (int)(p.mask_group > 0 ? p.mask_group : 1);
  a.causal_off = p.causal == 1 ? 0 : p.causal == 2 ? (int)(p.skv - p.s) : (int)p.skv;
  a.mask_vec = p.mask && p.ldm % 4 == 0 && p.sm % 4 == 0 && ((uintptr_t)p.mask & 7) == 0;
  a.kbytes = (uint32_t)(((p.skv - 1) * p.ldk + p.d) * 2);
  a.vbytes = (uint32_t)(((p.skv - 1) * p.ldv + p.d) * 2);
  a.ldq = p.ldq;
  a.ldk = p.ldk;
  a.ldv = p.ldv;
  a.ldo = p.ldo;
  a.ldm = p.ldm;
  a.bq = p.sq;
  a.bk = p.sk;
  a.bv = p.sv;
  a.bo = p.so;
  a.bm = p.sm;
  a.c = p.scale * kLog2e;
  const int cfg = pick_cfg(p);
  if (p.d == 64) return launch_d<64>(a, p, cfg, stream);
  if (p.d == 128) return launch_d<128>(a, p, cfg, stream);
  return hipErrorNotSupported;
}

}  // namespace hxmi
