// Fused attention O = softmax(scale * Q.K^T) . V for head dims 64 and 128.
//
// The reference lowers tm_tensor.attention to batch_matmul(Q, K^T), a scale,
// a row softmax and batch_matmul(P, V) (LowerTmTensor.cpp:91-250), each a
// separate pass over HBM.  Here one kernel streams K and V once per query
// block and keeps S and P in registers (online softmax, Milakov &
// Gimelshein 2018, the blockwise form the reference's
// test/python/triton/test_online_softmax.py:30-81 exercises):
//   * a workgroup is 4 waves x 32 queries of one (batch, head); K and V pass
//     through LDS in chunks of 256 keys (D = 64; 128 for D = 128: 64 KB
//     either way) shared by the 4 waves, so a ViT sequence (197 tokens) is
//     one chunk, loaded with every global load in flight at once;
//   * S is computed as D[key][query] = K . Q^T with v_mfma_f32_32x32x16_f16,
//     so every lane owns one query's scores: the row max / sum are in-lane
//     plus one exchange with the lane 32 away;
//   * the fp16 probabilities of a 32-key block are exactly the B operand of
//     the P.V MFMA for two 16-key steps (the k order inside an MFMA is free as
//     long as both operands use the same one); the matching V^T operand comes
//     from LDS with ds_read_b64_tr_b16, so P never leaves registers;
//   * O = D[d][query] accumulates in registers, is rescaled when the running
//     max grows, and is divided by the row sum once at the end.
#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {


struct AArgs {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  int bh, sq, skv;
  int64_t ldq, ldk, ldv, ldo;  // row strides, elements
  int64_t bq, bk, bv, bo;      // (batch*head) strides, elements
  float scale_log2e;
};

__device__ __forceinline__ float16v mfma32(short8v a, short8v b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a), __builtin_bit_cast(half8v, b), c, 0,
                                                0, 0);
}

// K chunk: [KC][D] fp16, rows of 2*D bytes, 16-byte chunks XOR-swizzled as
// the GEMM's k-contiguous tiles; V chunk: [KC][D], 16-byte chunks XOR-ed with
// a multiple of (key & 3) chosen so the 8 row segments (2 lane groups x 4
// keys x 32 bytes) of one transposing read phase cover all 64 banks.
template <int D>
__device__ __forceinline__ int k_off(int r, int c) {
  constexpr int RB = 2 * D;
  return r * RB + ((c ^ ((r / (256 / RB)) & (RB / 16 - 1))) << 4);
}
template <int D>
__device__ __forceinline__ int v_off(int r, int c) {
  constexpr int SH = D == 64 ? 1 : 2;  // 32-byte steps for 128-byte rows, 64-byte for 256
  return r * (2 * D) + ((c ^ ((r & 3) << SH)) << 4);
}

template <int D>
__global__ __launch_bounds__(256) void attention_fwd(AArgs a) {
  constexpr int KC = D == 64 ? 256 : 128;  // keys per LDS chunk (32 KB of K, 32 KB of V)
  constexpr int DC = D / 8;   // 16-byte chunks per row
  constexpr int DS = D / 16;  // 16-deep MFMA steps over the head dim
  constexpr int DT = D / 32;  // 32-wide output tiles over the head dim
  constexpr int PER = KC * DC / 256;  // 16-byte chunks of K (and of V) per thread
  __shared__ __attribute__((aligned(1024))) char ks[KC * 2 * D];
  __shared__ __attribute__((aligned(1024))) char vs[KC * 2 * D];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int h = lane >> 5;
  const int qblocks = (a.sq + 127) / 128;
  const int bh = blockIdx.x / qblocks;
  const int q0 = (blockIdx.x % qblocks) * 128 + w * 32;
  const char* Q = a.q + (int64_t)bh * a.bq * 2;
  const char* Kp = a.k + (int64_t)bh * a.bk * 2;
  const char* Vp = a.v + (int64_t)bh * a.bv * 2;

  // Q fragments of this wave's 32 queries (zero past the sequence)
  short8v qf[DS];
  {
    const int q = q0 + (lane & 31);
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      qf[s] = short8v{};
      if (q < a.sq) qf[s] = *(const short8v*)(Q + ((int64_t)q * a.ldq + s * 16 + h * 8) * 2);
    }
  }

  float16v oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = float16v{};
  float m_run = -INFINITY, l_run = 0.f;

  for (int c0 = 0; c0 < a.skv; c0 += KC) {
    // every load of the chunk in flight before the first LDS store
    int4v kv[PER], vv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = i * 256 + threadIdx.x;
      const int r = idx / DC, c = idx % DC;
      const int key = c0 + r;
      kv[i] = int4v{0, 0, 0, 0};
      vv[i] = int4v{0, 0, 0, 0};
      if (key < a.skv) {
        kv[i] = *(const int4v*)(Kp + ((int64_t)key * a.ldk + c * 8) * 2);
        vv[i] = *(const int4v*)(Vp + ((int64_t)key * a.ldv + c * 8) * 2);
      }
    }
    __syncthreads();  // previous chunk fully consumed
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = i * 256 + threadIdx.x;
      const int r = idx / DC, c = idx % DC;
      *(int4v*)(ks + k_off<D>(r, c)) = kv[i];
      *(int4v*)(vs + v_off<D>(r, c)) = vv[i];
    }
    __syncthreads();

    const int nblk = min(KC, a.skv - c0 + 31) / 32;
    for (int b = 0; b < nblk; ++b) {
      // S block: D[key][query], lane holds query lane%32, keys 8g + 4h + j
      float16v s = {};
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const int r = b * 32 + (lane & 31);
        const short8v kf = *(const short8v*)(ks + k_off<D>(r, st * 2 + h));
        s = mfma32(kf, qf[st], s);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = c0 + b * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        s[i] = key < a.skv ? s[i] * a.scale_log2e : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first block
      m_run = m_new;
      float psum = 0.f;
      _Float16 p16[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // the row sum uses the fp16 weights P.V sees, so O is their exact
        // weighted average (a constant V comes back unchanged)
        p16[i] = (_Float16)__builtin_amdgcn_exp2f(s[i] - m_new);
        psum += (float)p16[i];
      }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
      // two 16-key MFMA steps: step t uses keys {16t + 4h + j, 16t + 8 + 4h + j}
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        short8v pf;
        __builtin_memcpy(&pf, &p16[8 * t], 16);
        const int g = lane >> 4, L = lane & 15;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = dt * 32 + ((g & 1) << 4) + ((L & 3) << 2);
          const int r1 = b * 32 + 16 * t + 4 * h + (L >> 2);
          const short4v lo = lds_read_tr16(vs + v_off<D>(r1, d >> 3) + (d & 7) * 2);
          const short4v hi = lds_read_tr16(vs + v_off<D>(r1 + 8, d >> 3) + (d & 7) * 2);
          const short8v vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          oacc[dt] = mfma32(vf, pf, oacc[dt]);
        }
      }
    }
  }

  // O = D[d][query]: lane holds query lane%32, d = 32 dt + 8 g + 4 h + j
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l_tot;
  const int q = q0 + (lane & 31);
  if (q < a.sq) {
    char* O = a.o + ((int64_t)bh * a.bo + (int64_t)q * a.ldo) * 2;
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

}  // namespace

hipError_t launch_attention(const AttnProblem& p, hipStream_t stream) {
  if (p.bh == 0 || p.s == 0) return hipSuccess;
  AArgs a;
  a.q = (const char*)p.q;
  a.k = (const char*)p.k;
  a.v = (const char*)p.v;
  a.o = (char*)p.o;
  a.bh = (int)p.bh;
  a.sq = (int)p.s;
  a.skv = (int)p.skv;
  a.ldq = p.ldq;
  a.ldk = p.ldk;
  a.ldv = p.ldv;
  a.ldo = p.ldo;
  a.bq = p.sq;
  a.bk = p.sk;
  a.bv = p.sv;
  a.bo = p.so;
  a.scale_log2e = p.scale * 1.4426950408889634f;
  const int64_t blocks = p.bh * ((p.s + 127) / 128);
  if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
  if (p.d == 64)
    hipLaunchKernelGGL(attention_fwd<64>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else if (p.d == 128)
    hipLaunchKernelGGL(attention_fwd<128>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    return hipErrorNotSupported;
  return hipGetLastError();
}

}  // namespace hxmi
