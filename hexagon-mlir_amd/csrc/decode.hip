// Persistent one-token decoder step (M = 1) of a Llama / Qwen2 stack.
//
// The reference runs Qwen2.5-0.5B as one whole-model forward of a one-token
// prompt at position 0 with the KV cache off
// (benchmark_models/run_qwen2.5-0.5b.py:171-173,224-233): embedding row ->
// L x [RMSNorm, q|k|v projection (+bias), attention, o projection +
// residual, RMSNorm, gate|up projection, SiLU-mul, down projection +
// residual] -> final RMSNorm -> lm_head.  With a single key the softmax
// weight is exactly 1 and RoPE at position 0 is the identity, so the
// attention output of query head h is v of its key/value head
// h / (heads / kv_heads).  Every projection is an M = 1 GEMV whose weights
// do not depend on the data: the step is a chain of 4L dependent,
// latency-bound phases over 0.7 GB of weights (Qwen2.5-0.5B).
//
// One launch keeps one workgroup per CU (at most) for the whole chain.
//   * Loader waves stream the workgroup's rows of every layer's weights, in
//     phase order, through a 128 KiB LDS ring with direct global->LDS loads,
//     up to the ring's size ahead of the data dependencies.  A loader issues
//     a batch of 4 KiB, waits for it, and publishes a batch count in LDS;
//     kNL = 4 loaders interleave batches, one loader and one compute wave
//     per SIMD.  Small batches hand each phase its first rows sooner:
//     loaders x KiB per batch measured 2 x 16: 535 us a forward (with the
//     lm_head), 3 x 8: 528, 4 x 8: 524, 4 x 4: 521; 2 x 8: 591 (too little
//     in flight) and 5 or more loaders 700+ (two loaders on a SIMD).
//   * Compute waves take each phase's input vector from the workspace into
//     LDS (one poller per workgroup), stage their K-part of the normalised
//     (or expanded) input, and multiply 16-row tiles of the ring by it on
//     v_mfma_f32_16x16x32_f16, each wave a quarter of K (one wave alone
//     reads LDS at ~1 KiB per 25 cycles); the parts meet in LDS once per
//     phase.
//   * Each phase output element is published as one 32-bit word, fp16 value
//     in the low half and a 16-bit tag of (launch, layer) in the high half,
//     with agent-scope stores into 2 copies.  Consumers load the words they
//     need with agent-scope loads until every tag matches: a phase boundary
//     costs one memory round trip (no grid barrier: arrive, release, read).
// Measured on one MI355X (Qwen2.5-0.5B, 24 layers): ~480 us for the layers,
// 5.0 us per phase.  A bare all-to-all chain of this kind (256 workgroups
// publish 4 words, every workgroup polls the 896) costs ~2 us per phase on
// its own; streaming the weights at the same time slows the polls by
// another ~0.7 us, and the MFMA work and its rendezvous are on the chain.
// fp16 rounding follows the HF fp16 forward: RMSNorm normalises in fp32,
// rounds, then multiplies by the weight; every projection output, the SiLU,
// the product and both residual sums are rounded to fp16.
// Tags: the workspace keeps a running tag base B (mod 65535); a launch of L
// layers tags layer l's outputs 1 + (B + l) mod 65535 (the final state
// B + L) and its last wave to leave sets B += L + 1, so no tag of a launch
// equals one of the launch before it, whatever L was.  With one stack shape
// per workspace every published word is rewritten by every launch, so the
// words a consumer can find are from this launch or the previous one.
// Every wait is bounded by the caller's timeout: an expired wait sets the
// workspace's sticky error word and an abort word that every other wait
// also checks, so all waves leave.  The last wave to leave resets the abort
// word and advances the tag base.
#include <algorithm>

#include "hxmi_common.h"
#include "hxmi_internal.h"

namespace hxmi {
namespace {

constexpr int kNC = 4;                   // compute waves per workgroup
constexpr int kNL = 4;                   // loader waves per workgroup
constexpr int kRing = 128 * 1024;        // LDS weight ring, bytes (power of two)
constexpr int kChunk = 1024;             // one wave's direct-to-LDS load: 64 lanes x 16 B
constexpr int kRingChunks = kRing / kChunk;
constexpr int kBatch = 4;                // chunks per loader batch
constexpr int kPH = 4;                   // 8-element pieces per lane for K = hidden (<= 2048)
constexpr int kPI = 12;                  // for K = intermediate (<= 6144)
constexpr int kPoll = 8;                 // 16-byte poll groups per lane (vectors <= 8192)
constexpr int kMaxKV = 512;              // kv_heads * head_dim
constexpr int kThreads = (kNC + kNL) * 64;
constexpr int kMaxTiles = 8;             // 16-row tiles of a phase run concurrently

// workspace words: control block, then the published vectors
constexpr int kTagBase = 0, kDone = 1, kAbort = 2, kError = DECODE_WS_ERROR_WORD, kCtrlWords = 64;
constexpr uint32_t kSC1 = 16;  // buffer cache policy: agent-scope coherent
// Each published vector is written in kCopies copies and workgroup b polls
// copy b % kCopies: every polled line has 1/kCopies of the grid's pollers.
// Forwards with the lm_head measured 528 us with one copy, 514 with two,
// 518 with four and 519 with eight (one writer and one poller see each
// other in 0.55 us; more copies cost the producers more stores).
constexpr int kCopies = 2;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct DArgs {
  const char* x;
  const char* w_qkv;
  const char* b_qkv;
  const char* w_o;
  const char* w_ov;  // o projection folded onto the normalised input (fold: w_o unused)
  const char* b_ov;
  const char* w_gu;
  const char* w_down;
  const char* g_attn;
  const char* g_mlp;
  const char* g_final;
  char* qkv_out;
  char* x_out;
  char* h_out;
  uint32_t* ws;
  int L, H, NKV, I, HD, grp;
  int fold;  // 1: the o rows run in phase 0 on w_ov (no phase 1)
  int offXB, offX1B, offVB, offAB;  // word offsets of the published vectors (copy 0)
  int strXB, strVB, strAB;         // words between copies
  int swzH, swzI;                  // ring piece swizzle masks for rows of H / I elements
  float eps;
  uint64_t timeout;  // s_memrealtime ticks (100 MHz)
};

struct Shared {
  char ring[kRing];
  _Float16 xin[kPH * 512];  // X or X1 of the current layer
  _Float16 ain[kPI * 512];  // SiLU-mul output
  _Float16 vin[kMaxKV];     // v
  _Float16 hin[kPH * 512];  // B operand: normalised X / X1, or the attention output
  // K-split partial row sums, one set per phase parity: a wave writes the
  // set of phase p + 2 only after the rendezvous of phase p + 1, which every
  // wave reaches after it has read its tiles of phase p
  float red[2][kMaxTiles * kNC][16];
  int prog[kNC];            // per compute wave: every row it owns that starts below this byte is done
  int filled[kNL];          // per loader: batches completed
  int sync_cnt;
  int abort;
};

// Bytes of each phase of one layer in this workgroup's weight stream.  Phase
// 0: q|k|v rows, 1: o rows, 2: gate/up rows (pairs x 2), 3: down rows.  With
// the o projection folded (fold), phase 0 streams the workgroup's o rows of
// w_ov and then its q|k|v rows, and phase 1 is empty.  The o rows come first
// so that they are all in tile 0: the finish of tile 0 runs on compute wave
// 0, which also polls the next phase's input into s.xin, and the o rows'
// residual reads x from s.xin (the host keeps a workgroup's o rows <= 16).
// Named fields, not arrays: an array indexed by a run-time phase would live
// in scratch memory.
struct Geo {
  int ro;                          // fold: o rows of this workgroup (the first rows of phase 0), else 0
  int rows0, rows1, rows2, rows3;  // rows in the stream (phase 2: 2 per pair)
  int row00, row01, row02, row03;  // first global row (phase 2: first pair)
  int bytes0, bytes1, bytes2, bytes3;
  int pre1, pre2, pre3, pre4;  // padded prefix sums; pre4 = bytes of one layer
};

__device__ __forceinline__ int pad_chunk(int b) { return (b + kChunk - 1) / kChunk * kChunk; }

__device__ __forceinline__ Geo make_geo(const DArgs& a, int w, int G) {
  auto lo = [&](int n) { return (int)((int64_t)n * w / G); };
  auto cnt = [&](int n) { return (int)((int64_t)n * (w + 1) / G) - lo(n); };
  Geo g;
  g.row00 = lo(a.H + 2 * a.NKV);
  g.row01 = lo(a.H);
  g.ro = a.fold ? cnt(a.H) : 0;
  g.rows0 = g.ro + cnt(a.H + 2 * a.NKV);
  g.rows1 = a.fold ? 0 : cnt(a.H);
  g.row02 = lo(a.I);
  g.rows2 = 2 * cnt(a.I);
  g.row03 = lo(a.H);
  g.rows3 = cnt(a.H);
  g.bytes0 = g.rows0 * a.H * 2;
  g.bytes1 = g.rows1 * a.H * 2;
  g.bytes2 = g.rows2 * a.H * 2;
  g.bytes3 = g.rows3 * a.I * 2;
  g.pre1 = pad_chunk(g.bytes0);
  g.pre2 = g.pre1 + pad_chunk(g.bytes1);
  g.pre3 = g.pre2 + pad_chunk(g.bytes2);
  g.pre4 = g.pre3 + pad_chunk(g.bytes3);
  return g;
}

__device__ __forceinline__ uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int lds_ld(int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void cfence() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }

__device__ __forceinline__ uint32_t bits16(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ _Float16 lo16(uint32_t w) { return __builtin_bit_cast(_Float16, (uint16_t)(w & 0xffff)); }
__device__ __forceinline__ _Float16 hi16(uint32_t w) { return __builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }
__device__ __forceinline__ uint32_t pack2(_Float16 lo, _Float16 hi) { return bits16(lo) | (bits16(hi) << 16); }
// Word -> half2 through a by-value argument: hipcc miscompiles
// __builtin_bit_cast applied directly to an ext-vector element (v[e]),
// returning element 0 for every e.
__device__ __forceinline__ half2v as_half2(uint32_t w) { return __builtin_bit_cast(half2v, w); }

// Bounded-wait bookkeeping of one wave.
struct Guard {
  uint32_t* ws;
  uint64_t timeout;
  Shared* s;
  int lane;
  // Records an expired wait: sticky error word, abort word, LDS abort flag.
  __device__ void raise() const {
    lds_st(&s->abort, 1);
    if (lane == 0) {
      st_agent(ws + kError, 1);
      st_agent(ws + kAbort, 1);
    }
  }
  // false: give up (this wave expired, or another wave did).  The clock is
  // read every 16th iteration of a wait loop.
  __device__ bool ok(uint64_t t0, int it) const {
    if (lds_ld(&s->abort)) return false;
    if ((it & 15) == 0 && now() - t0 > timeout) {
      raise();
      return false;
    }
    return true;
  }
};

// ---- loader waves ------------------------------------------------------------

// Issues one chunk of phase P of layer l (byte `off` of the phase's rows)
// into ring slot `slot`.  The 16-byte pieces of each stream row are stored
// XOR-swizzled by the row's index m in the phase: piece q of row m sits in
// piece slot q ^ (m & swz) of the row's ring bytes.  An MFMA tile reads one
// piece of 16 consecutive rows at once, and rows are a multiple of 256
// bytes apart, so unswizzled the 16 lanes would hit the same LDS banks.
// swz + 1 divides the row's piece count.
template <int P>
__device__ __forceinline__ void issue_chunk(const DArgs& a, Shared& s, const Geo& g, int bytes, int l, int off,
                                            int slot, int lane) {
  const int o = off + lane * 16;
  if (o >= bytes) return;
  const int rb = (P == 3 ? a.I : a.H) * 2;
  const int swz = P == 3 ? a.swzI : a.swzH;
  const int m = o / rb, pd = (o - m * rb) >> 4;
  const int col = (pd ^ (m & swz)) << 4;
  const char* base;
  int row;
  if constexpr (P == 0) {
    if (m < g.ro) {  // fold: the o rows of w_ov before the q|k|v rows
      base = a.w_ov + (int64_t)l * a.H * rb;
      row = g.row01 + m;
    } else {
      base = a.w_qkv + (int64_t)l * (a.H + 2 * a.NKV) * rb;
      row = g.row00 + (m - g.ro);
    }
  } else if constexpr (P == 1) {
    base = a.w_o + (int64_t)l * a.H * rb;
    row = g.row01 + m;
  } else if constexpr (P == 2) {
    // rows of the stream alternate gate row i, up row i of this workgroup's pairs
    base = a.w_gu + (int64_t)l * 2 * a.I * rb;
    row = ((m & 1) ? a.I : 0) + g.row02 + (m >> 1);
  } else {
    base = a.w_down + (int64_t)l * a.H * rb;
    row = g.row03 + m;
  }
  // non-temporal (cache policy nt): each weight byte is read once a step
  // (Qwen2.5-0.5B forward with the lm_head 450.7-451.3 -> 449.3-449.5 us)
  __builtin_amdgcn_global_load_lds((const void*)(base + (int64_t)row * rb + col),
                                   (HXMI_LDS void*)(s.ring + slot * kChunk), 16, 0, 2);
}

// Loader j owns batches j, j + kNL, ... of kBatch chunks.  It walks the
// stream in phase order (the phase is a compile-time constant at each issue,
// so the loop touches no memory but the loads themselves: any other vector
// memory or LDS access here would wait for the batch in flight), waits for
// the ring slots of a batch to be released before its first chunk, and
// after its last chunk waits for the batch and publishes it.
__device__ __forceinline__ void loader(const DArgs& a, Shared& s, const Geo& g, int j, const Guard& gd) {
  const int total = a.L * (g.pre4 / kChunk);
  int c = 0;  // stream chunk index
  for (int l = 0; l < a.L; ++l) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int pc = (p == 0 ? g.pre1 : p == 1 ? g.pre2 - g.pre1 : p == 2 ? g.pre3 - g.pre2 : g.pre4 - g.pre3) / kChunk;
      const int bytes = p == 0 ? g.bytes0 : p == 1 ? g.bytes1 : p == 2 ? g.bytes2 : g.bytes3;
      for (int k = 0; k < pc; ++k, ++c) {
        const int b = c / kBatch;
        if (b % kNL != j) {  // another loader's batch: skip to its end (or the phase's)
          const int skip = min(pc - k, (b + 1) * kBatch - c) - 1;
          k += skip;
          c += skip;
          continue;
        }
        if (c % kBatch == 0) {
          const uint64_t t0 = now();
          for (int it = 1;; ++it) {
            int rel = lds_ld(&s.prog[0]);
#pragma unroll
            for (int w = 1; w < kNC; ++w) rel = min(rel, lds_ld(&s.prog[w]));
            if ((b + 1) * kBatch <= rel / kChunk + kRingChunks) break;
            if (!gd.ok(t0, it)) return;
            __builtin_amdgcn_s_sleep(1);
          }
          cfence();
        }
        const int off = k * kChunk, slot = c % kRingChunks;
        if (p == 0) issue_chunk<0>(a, s, g, bytes, l, off, slot, gd.lane);
        else if (p == 1) issue_chunk<1>(a, s, g, bytes, l, off, slot, gd.lane);
        else if (p == 2) issue_chunk<2>(a, s, g, bytes, l, off, slot, gd.lane);
        else issue_chunk<3>(a, s, g, bytes, l, off, slot, gd.lane);
        if (c % kBatch == kBatch - 1 || c == total - 1) {
          wait_vmcnt0();
          cfence();
          lds_st(&s.filled[j], b / kNL + 1);
        }
      }
    }
  }
}

// ---- compute waves -----------------------------------------------------------
// Compute-side waits spin without sleeping: each is on the critical path.

// Waits until the ring holds every stream byte below `end`.
__device__ __forceinline__ bool wait_fill(Shared& s, int end, const Guard& gd) {
  const int bl = (end - 1) / kChunk / kBatch;  // last batch needed
  int need[kNL];
#pragma unroll
  for (int j = 0; j < kNL; ++j) need[j] = bl >= j ? (bl - j) / kNL + 1 : 0;
  uint64_t t0 = 0;
  for (int it = 0;; ++it) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < kNL; ++j) ready &= lds_ld(&s.filled[j]) >= need[j];
    if (ready) break;
    if (it == 0) t0 = now();
    else if (!gd.ok(t0, it)) return false;
  }
  cfence();
  return true;
}

// Rendezvous of the compute waves after each has written its share of a
// phase input into LDS.
__device__ __forceinline__ bool sync_compute(Shared& s, int& nsync, const Guard& gd) {
  ++nsync;
  cfence();
  if (gd.lane == 0) __hip_atomic_fetch_add(&s.sync_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  uint64_t t0 = 0;
  for (int it = 0; lds_ld(&s.sync_cnt) < kNC * nsync; ++it) {
    if (it == 0) t0 = now();
    else if (!gd.ok(t0, it)) return false;
  }
  cfence();
  return true;
}

// Groups [g0, g1) of 4 words of a published n-word vector: polls the words
// until every tag equals `tag`, then stores the fp16 values to dst.
// Each round issues the loads of every group still pending and checks them
// when they return; the abort word rides along every 8th round.
__device__ __forceinline__ bool poll_vector(const DArgs& a, const uint32_t* src, int n, int g0, int g1, uint32_t tag,
                                            _Float16* dst, const Guard& gd) {
  const int lane = gd.lane;
  uint32_t pend = 0;
#pragma unroll
  for (int t = 0; t < kPoll; ++t)
    if (g0 + lane + 64 * t < g1) pend |= 1u << t;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)n * 4);
  const uint64_t t0 = now();
  for (int it = 1;; ++it) {
    u32x4 v[kPoll];
#pragma unroll
    for (int t = 0; t < kPoll; ++t)
      if (pend >> t & 1)
        v[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, (uint32_t)(g0 + lane + 64 * t) * 16, 0, kSC1));
    uint32_t ab = 0;
    if (lane == 0 && (it & 7) == 0) ab = ld_agent(a.ws + kAbort);
#pragma unroll
    for (int t = 0; t < kPoll; ++t) {
      if (pend >> t & 1) {
        const u32x4 x = v[t];
        if ((x[0] >> 16) == tag && (x[1] >> 16) == tag && (x[2] >> 16) == tag && (x[3] >> 16) == tag) {
          const u32x2 h = {__builtin_amdgcn_perm(x[1], x[0], 0x05040100u), __builtin_amdgcn_perm(x[3], x[2], 0x05040100u)};
          *(u32x2*)(dst + (g0 + lane + 64 * t) * 4) = h;
          pend &= ~(1u << t);
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(pend != 0) == 0) return true;
    if (__builtin_amdgcn_readfirstlane(ab)) {
      lds_st(&gd.s->abort, 1);
      return false;
    }
    if (!gd.ok(t0, it)) return false;
  }
}

// A plain fp16 vector (the caller's input row), all of it.
__device__ __forceinline__ void copy_vector(const char* src, int n, _Float16* dst, int lane) {
  for (int gi = lane; gi < (n >> 2); gi += 64) *(u32x2*)(dst + gi * 4) = *(const u32x2*)(src + (int64_t)gi * 8);
}

// A whole published vector into LDS for every compute wave: wave 0 polls it
// and then releases the others through the rendezvous counter (one poller
// per workgroup measured ~0.5 us a phase faster than four).  Its own input
// row instead of a published vector when src is null (the first layer).
__device__ __forceinline__ bool poll_shared(const DArgs& a, const uint32_t* src, const char* plain, int n, uint32_t tag,
                                            _Float16* dst, int w, Shared& s, int& nsync, const Guard& gd) {
  ++nsync;
  if (w == 0) {
    if (plain) copy_vector(plain, n, dst, gd.lane);
    else if (!poll_vector(a, src, n, 0, n >> 2, tag, dst, gd)) return false;
    cfence();
    if (gd.lane == 0) __hip_atomic_fetch_add(&s.sync_cnt, kNC, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  uint64_t t0 = 0;
  for (int it = 0; lds_ld(&s.sync_cnt) < kNC * nsync; ++it) {
    if (it == 0) t0 = now();
    else if (!gd.ok(t0, it)) return false;
  }
  cfence();
  return true;
}

__device__ __forceinline__ void unpack8(u32x4 w, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = (float)lo16(w[e]);
    f[2 * e + 1] = (float)hi16(w[e]);
  }
}

// This lane's pieces of a K-vector in memory (piece q = lane + 64j holds
// elements 8q..8q+7): the norm weights, loaded before a phase's input is.
template <int P>
__device__ __forceinline__ void load_pieces(const void* v, int K, int lane, u32x4 (&h)[P]) {
  const int np = K >> 3;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int q = lane + 64 * j;
    if (q < np) h[j] = *(const u32x4*)((const char*)v + q * 16);
  }
}

// Pieces are 8 consecutive elements (16 bytes).  Compute wave w handles
// K-steps [w * steps / kp, (w + 1) * steps / kp) of every tile of a phase
// (32 elements, 4 pieces per step), so it stages only the B-operand pieces
// of that K-part, itself: no other wave reads them.
constexpr int kGP = 2;  // norm-weight pieces per lane of one K-part (<= 128 pieces)

struct KPart {
  int k0, k1;  // K-steps
  int q0, q1;  // pieces (q1 clipped to the vector)
};
__device__ __forceinline__ KPart k_part(int K, int kp, int w) {
  const int steps = (K + 31) / 32;
  KPart p;
  p.k0 = w < kp ? w * steps / kp : steps;
  p.k1 = w < kp ? (w + 1) * steps / kp : steps;
  p.q0 = min(4 * p.k0, K >> 3);
  p.q1 = min(4 * p.k1, K >> 3);
  return p;
}

// This lane's norm-weight pieces of a K-part (loaded before the phase input
// is polled): pieces q0 + lane + 64 j.
__device__ __forceinline__ void weight_pieces(const char* g, const KPart& kp, int lane, u32x4 (&gw)[kGP]) {
#pragma unroll
  for (int j = 0; j < kGP; ++j) {
    const int q = kp.q0 + lane + 64 * j;
    if (q < kp.q1) gw[j] = *(const u32x4*)(g + q * 16);
  }
}

// RMSNorm of the K-vector in s.xin into s.hin over the pieces of a K-part:
// h = fp16(g * fp16(x * rsqrt(mean(x^2) + eps))); the wave sums all of x.
__device__ __forceinline__ void norm_part(Shared& s, int K, float eps, const KPart& kp, int lane,
                                          const u32x4 (&gw)[kGP]) {
  float ss = 0.f;
  for (int q = lane; q < (K >> 3); q += 64) {
    float f[8];
    unpack8(*(const u32x4*)(s.xin + q * 8), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
  }
  ss = wave_sum_dpp(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)K + eps);
#pragma unroll
  for (int j = 0; j < kGP; ++j) {
    const int q = kp.q0 + lane + 64 * j;
    if (q < kp.q1) {
      float f[8], gf[8];
      unpack8(*(const u32x4*)(s.xin + q * 8), f);
      unpack8(gw[j], gf);
      u32x4 h;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h[e] = pack2((_Float16)(gf[2 * e] * (float)(_Float16)(f[2 * e] * r)),
                     (_Float16)(gf[2 * e + 1] * (float)(_Float16)(f[2 * e + 1] * r)));
      *(u32x4*)(s.hin + q * 8) = h;
    }
  }
}

// Attention output at position 0 into s.hin over the pieces of a K-part:
// element k of query head k / hd is v of its key/value head,
// (k / hd / grp) * hd + k % hd.
__device__ __forceinline__ void attn_part(Shared& s, int hd, int grp, const KPart& kp, int lane) {
  for (int q = kp.q0 + lane; q < kp.q1; q += 64) {
    const int k = q * 8, head = k / hd;
    *(u32x4*)(s.hin + k) = *(const u32x4*)(s.vin + (head / grp) * hd + (k - head * hd));
  }
}

// Partial dot products of stream rows m0 + r (r < nr <= 16; the phase's
// rows start at stream byte sp, rb bytes each) with the K-vector hsrc in
// LDS, over K-steps [k0, k1) of 32, on v_mfma_f32_16x16x32_f16: lane l
// supplies row l % 16, elements 8 * (l / 16) .. + 7 of each step as A and
// the same elements of hsrc as B (every B column equal), and receives rows
// 4 * (l / 16) + i in acc[i].
__device__ __forceinline__ float4v tile_dot(const Shared& s, int sp, int rb, int swz, int m0, int nr, int np, int k0,
                                            int k1, const _Float16* hsrc, int lane) {
  const int r16 = lane & 15, kq = lane >> 4;
  // Rows past the tile's end (r16 >= nr) read whatever ring bytes follow:
  // an MFMA output row depends only on its own A row, and those rows are
  // never stored.
  (void)nr;
  const int rowst = sp + (m0 + r16) * rb;
  const int key = (m0 + r16) & swz;
  const half8v zero = {};
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  const int kfull = min(k1, np >> 2);  // steps whose 4 pieces all exist
  auto ld = [&](int t, half8v& av, half8v& bv) {
    const int q = t * 4 + kq;
    bv = *(const half8v*)(hsrc + q * 8);
    av = *(const half8v*)(s.ring + ((rowst + ((q ^ key) << 4)) & (kRing - 1)));
  };
  // Groups of eight steps; the next group's operands are loaded before the
  // current group's MFMAs, which alternate between two accumulators.  (Left
  // to itself the compiler reuses one register pair and waits out the LDS
  // latency at every step; the MFMA builtin is convergent, so a loop of
  // unknown trip count is not unrolled for us.)
  int t = k0;
  if (t + 8 <= kfull) {
    half8v av[8], bv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ld(t + i, av[i], bv[i]);
    for (; t + 16 <= kfull; t += 8) {
      half8v an[8], bn[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) ld(t + 8 + i, an[i], bn[i]);
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[i], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i + 1], bv[i + 1], acc1, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        av[i] = an[i];
        bv[i] = bn[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[i], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i + 1], bv[i + 1], acc1, 0, 0, 0);
    }
    t += 8;
  }
  if (t < kfull) {
    // the last (or only) 1..7 steps (a K-part of K = 896 over four waves
    // is 7): every load first, then the MFMAs, so the steps wait out one
    // LDS latency between them, not one each.  Slots past kfull reload the
    // last step and feed no MFMA.
    half8v av[8], bv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ld(min(t + i, kfull - 1), av[i], bv[i]);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      if (t + i < kfull) acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[i], acc0, 0, 0, 0);
      if (t + i + 1 < kfull) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i + 1], bv[i + 1], acc1, 0, 0, 0);
    }
  }
  if (kfull < k1) {  // the last, partial step (np % 4 != 0)
    const int q = kfull * 4 + kq;
    half8v av = zero, bv = zero;
    if (q < np) {
      bv = *(const half8v*)(hsrc + q * 8);
      av = *(const half8v*)(s.ring + ((rowst + ((q ^ key) << 4)) & (kRing - 1)));
    }
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc0, 0, 0, 0);
  }
  return acc0 + acc1;
}

// How a phase's rows are spread over the compute waves.  Every 16-row tile
// is split into kp <= kNC K-parts, part p going to wave p: one wave reads
// LDS at about 1 KiB per 25 cycles, so a tile read by one wave would take
// four times as long.  The parts meet in s.red.  A phase whose rows fit the
// ring (with a loader batch to spare) and have at most kMaxTiles tiles runs
// all its tiles before the parts meet and releases its ring bytes when it
// ends; a larger phase (a wide gate|up) meets once per tile, releasing the
// ring tile by tile.
struct Plan {
  int tiles, kp, steps;
  bool seq;
};
__device__ __forceinline__ Plan make_plan(int nr, int K) {
  Plan p;
  p.tiles = (nr + 15) / 16;
  p.steps = (K + 31) / 32;
  p.seq = nr * K * 2 > kRing - (kBatch + 1) * kChunk || p.tiles > kMaxTiles;
  p.kp = min(kNC, p.steps);
  return p;
}

// Rows 4 * (l / 16) + i of a tile are in acc[i] of lane l: lanes with
// l % 16 < 4 hold row 4 * (l / 16) + l % 16 in acc[l % 16].
__device__ __forceinline__ float own_row(float4v acc, int c) {
  return c == 0 ? acc[0] : c == 1 ? acc[1] : c == 2 ? acc[2] : acc[3];
}

// Sum of the K-parts of tile row r in red[par] (parts 0..kp-1 at unit base..),
// in part order.  The reads go out together (a loop over the run-time part
// count would wait out one LDS round trip per part).
__device__ __forceinline__ float part_sum(const Shared& s, int par, int base, int kp, int r) {
  float u[kNC];
#pragma unroll
  for (int p = 0; p < kNC; ++p) u[p] = s.red[par][base + min(p, kp - 1)][r];
  float v = 0.f;
#pragma unroll
  for (int p = 0; p < kNC; ++p)
    if (p < kp) v += u[p];
  return v;
}

// Runs a phase for wave w and hands each finished row to out(m, v, 0)
// (stream row m, fp32 sum) on one lane; with pairs, out(i, gate, up) gets
// pair i (stream rows 2i, 2i+1).  Waits for the ring data of each tile and
// releases ring bytes as described at Plan.  The K-parts meet in
// s.red[par] (par: the phase's parity); a large phase alternates two groups
// of kNC units tile by tile.  false: gave up.
template <bool PAIRS, typename Out>
__device__ __forceinline__ bool run_phase(Shared& s, const Plan& pl, int par, int sp, int end, int nr, int rb, int swz,
                                          int K, const _Float16* hsrc, int w, int lane, int& nsync, const Guard& gd,
                                          Out out) {
  const int c = lane & 15, g4 = lane >> 4;
  const int k0 = w * pl.steps / pl.kp, k1 = (w + 1) * pl.steps / pl.kp;  // this wave's K-part
  // finishes a tile (rows m0.., n of them) from the K-parts in red[par][base..]
  auto finish = [&](int base, int m0, int n) {
    if (PAIRS) {
      if (2 * lane + 1 < n)
        out(m0 / 2 + lane, part_sum(s, par, base, pl.kp, 2 * lane), part_sum(s, par, base, pl.kp, 2 * lane + 1));
    } else if (lane < n) {
      out(m0 + lane, part_sum(s, par, base, pl.kp, lane), 0.f);
    }
  };
  for (int tile = 0; tile < pl.tiles; ++tile) {
    const int m0 = tile * 16, n = min(16, nr - m0);
    if (w < pl.kp) {
      if (!wait_fill(s, sp + (m0 + n) * rb, gd)) return false;
      const float4v acc = tile_dot(s, sp, rb, swz, m0, n, K >> 3, k0, k1, hsrc, lane);
      if (c < 4) s.red[par][(pl.seq ? (tile & 1) * kNC : tile * pl.kp) + w][4 * g4 + c] = own_row(acc, c);
    }
    if (pl.seq) {
      cfence();
      if (lane == 0) lds_st(&s.prog[w], tile + 1 < pl.tiles ? sp + (m0 + 16) * rb : end);
      if (!sync_compute(s, nsync, gd)) return false;
      if (tile % kNC == w) finish((tile & 1) * kNC, m0, n);
    }
  }
  if (pl.seq) return true;
  cfence();
  if (lane == 0) lds_st(&s.prog[w], end);
  if (!sync_compute(s, nsync, gd)) return false;
  for (int tile = w; tile < pl.tiles; tile += kNC) finish(tile * pl.kp, tile * 16, min(16, nr - tile * 16));
  return true;
}

__device__ __forceinline__ void compute(const DArgs& a, Shared& s, const Geo& g, int w, uint32_t base, const Guard& gd) {
  const int lane = gd.lane;
  const int H = a.H, I = a.I, NKV = a.NKV, NQKV = H + 2 * NKV;
  uint32_t* XB = a.ws + a.offXB;
  uint32_t* X1B = a.ws + a.offX1B;
  uint32_t* VB = a.ws + a.offVB;
  uint32_t* AB = a.ws + a.offAB;
  // copy this workgroup polls; publish() writes every copy
  const int cp = blockIdx.x % kCopies;
  const uint32_t* XBc = XB + cp * a.strXB;
  const uint32_t* X1Bc = X1B + cp * a.strXB;
  const uint32_t* VBc = VB + cp * a.strVB;
  const uint32_t* ABc = AB + cp * a.strAB;
  auto publish = [](uint32_t* v, int stride, int i, uint32_t word) {
#pragma unroll
    for (int c = 0; c < kCopies; ++c) st_agent(v + c * stride + i, word);
  };
  int nsync = 0;
  const int rbH = H * 2, rbI = I * 2;
  const Plan p0 = make_plan(g.rows0, H), p1 = make_plan(g.rows1, H), p2 = make_plan(g.rows2, H),
             p3 = make_plan(g.rows3, I);
  // every phase with K = H splits K the same way (kp depends on K only)
  const KPart kh = k_part(H, p0.kp, w), ki = k_part(I, p3.kp, w);
  u32x4 gw[kGP];

  int ph = 0;  // phases run so far: consecutive phases use the two partial-sum sets in turn
  for (int l = 0; l < a.L; ++l) {
    const uint32_t tag = 1 + (base + l) % 65535u, tagn = 1 + (base + l + 1) % 65535u;
    const int sl = l * g.pre4;

    // phase 0: RMSNorm, q|k|v projection (+bias); v is published.  With the
    // o projection folded, the o rows come first (x1 = x + h . w_ov^T +
    // b_ov, published for phase 2) and v is not published
    {
      // the biases of the first 16 rows, loaded before the poll (the finish
      // of tile 0 adds lane m's to row m)
      float bq = 0.f;
      if (lane < min(16, g.rows0)) {
        if (lane < g.ro) {
          if (a.b_ov) bq = (float)((const _Float16*)a.b_ov)[(int64_t)l * H + g.row01 + lane];
        } else if (a.b_qkv) {
          bq = (float)((const _Float16*)a.b_qkv)[(int64_t)l * NQKV + g.row00 + lane - g.ro];
        }
      }
      weight_pieces(a.g_attn + (int64_t)l * rbH, kh, lane, gw);
      if (!poll_shared(a, XBc, l == 0 ? a.x : nullptr, H, tag, s.xin, w, s, nsync, gd)) return;
      norm_part(s, H, a.eps, kh, lane, gw);
      const bool ok = run_phase<false>(s, p0, ph++ & 1, sl, sl + g.pre1, g.rows0, rbH, a.swzH, H, s.hin, w, lane,
                                       nsync, gd, [&](int m, float v, float) {
        if (m < g.ro) {  // (tile 0: wave 0)
          const int row = g.row01 + m;
          if (a.b_ov) v += bq;
          const _Float16 x1 = (_Float16)((float)s.xin[row] + (float)(_Float16)v);
          publish(X1B, a.strXB, row, tag << 16 | bits16(x1));
        } else {
          const int row = g.row00 + (m - g.ro);
          if (a.b_qkv) v += m < 16 ? bq : (float)((const _Float16*)a.b_qkv)[(int64_t)l * NQKV + row];
          const _Float16 y = (_Float16)v;
          if (a.qkv_out) ((_Float16*)a.qkv_out)[(int64_t)l * NQKV + row] = y;
          if (!a.fold && row >= H + NKV) publish(VB, a.strVB, row - H - NKV, tag << 16 | bits16(y));
        }
      });
      if (!ok) return;
    }

    // phase 1: o projection of the attention output, + residual
    if (!a.fold) {
      if (!poll_shared(a, VBc, nullptr, NKV, tag, s.vin, w, s, nsync, gd)) return;
      attn_part(s, a.HD, a.grp, kh, lane);
      const bool ok = run_phase<false>(s, p1, ph++ & 1, sl + g.pre1, sl + g.pre2, g.rows1, rbH, a.swzH, H, s.hin, w,
                                       lane, nsync, gd, [&](int m, float v, float) {
        const int row = g.row01 + m;
        const _Float16 x1 = (_Float16)((float)s.xin[row] + (float)(_Float16)v);
        publish(X1B, a.strXB, row, tag << 16 | bits16(x1));
      });
      if (!ok) return;
    }

    // phase 2: RMSNorm, gate|up projection, SiLU-mul
    {
      weight_pieces(a.g_mlp + (int64_t)l * rbH, kh, lane, gw);
      if (!poll_shared(a, X1Bc, nullptr, H, tag, s.xin, w, s, nsync, gd)) return;
      norm_part(s, H, a.eps, kh, lane, gw);
      const bool ok = run_phase<true>(s, p2, ph++ & 1, sl + g.pre2, sl + g.pre3, g.rows2, rbH, a.swzH, H, s.hin, w,
                                      lane, nsync, gd, [&](int i, float gv, float uv) {
        const _Float16 gh = (_Float16)gv, uh = (_Float16)uv;
        const _Float16 sh = (_Float16)silu((float)gh);
        const _Float16 ah = (_Float16)((float)sh * (float)uh);
        publish(AB, a.strAB, g.row02 + i, tag << 16 | bits16(ah));
      });
      if (!ok) return;
    }

    // phase 3: down projection, + residual -> next layer's input
    {
      // only this wave's K-part of the SiLU-mul output (pieces are 2 groups of 4 words)
      if (!poll_vector(a, ABc, I, 2 * ki.q0, 2 * ki.q1, tag, s.ain, gd)) return;
      const bool ok = run_phase<false>(s, p3, ph++ & 1, sl + g.pre3, sl + g.pre4, g.rows3, rbI, a.swzI, I, s.ain, w,
                                       lane, nsync, gd, [&](int m, float v, float) {
        const int row = g.row03 + m;
        const _Float16 xn = (_Float16)((float)s.xin[row] + (float)(_Float16)v);
        publish(XB, a.strXB, row, tagn << 16 | bits16(xn));
      });
      if (!ok) return;
    }
  }

  // final RMSNorm (workgroup 0): each wave writes its K-part of h
  if (blockIdx.x != 0) return;
  const uint32_t tagL = 1 + (base + a.L) % 65535u;
  weight_pieces(a.g_final, kh, lane, gw);
  if (!poll_shared(a, XBc, nullptr, H, tagL, s.xin, w, s, nsync, gd)) return;
  norm_part(s, H, a.eps, kh, lane, gw);
  for (int q = kh.q0 + lane; q < kh.q1; q += 64) {
    *(u32x4*)(a.h_out + q * 16) = *(const u32x4*)(s.hin + q * 8);
    if (a.x_out) *(u32x4*)(a.x_out + q * 16) = *(const u32x4*)(s.xin + q * 8);
  }
}

// FOLD: the o projection folded into phase 0 (a.fold), as a compile-time
// constant in each instance
template <bool FOLD>
__global__ __launch_bounds__(kThreads, 1) void decode_step_persistent(DArgs a) {
  a.fold = FOLD;
  __shared__ __attribute__((aligned(16))) Shared s;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x < kNC) s.prog[threadIdx.x] = 0;
  if (threadIdx.x < kNL) s.filled[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    s.sync_cnt = 0;
    s.abort = 0;
  }
  __syncthreads();
  const uint32_t base = __builtin_amdgcn_readfirstlane(ld_agent(a.ws + kTagBase)) % 65535u;
  const Geo g = make_geo(a, blockIdx.x, gridDim.x);
  const Guard gd{a.ws, a.timeout, &s, lane};
  if (wv < kNC) compute(a, s, g, wv, base, gd);
  else loader(a, s, g, wv - kNC, gd);
  // leave: the last wave of the grid resets the abort word and advances the tag base
  if (lane == 0) {
    const uint32_t total = gridDim.x * (kNC + kNL);
    const uint32_t old = __hip_atomic_fetch_add(a.ws + kDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == total - 1) {
      st_agent(a.ws + kDone, 0);
      st_agent(a.ws + kAbort, 0);
      st_agent(a.ws + kTagBase, (base + (uint32_t)a.L + 1) % 65535u);
    }
  }
}

int rup64(int64_t n) { return (int)((n + 63) / 64 * 64); }

}  // namespace

bool decode_shape_ok(int64_t H, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t I) {
  const int64_t kv = kv_heads * head_dim;
  return H > 0 && I > 0 && heads > 0 && kv_heads > 0 && head_dim > 0 && H % 8 == 0 && I % 8 == 0 &&
         head_dim % 8 == 0 && heads * head_dim == H && heads % kv_heads == 0 && H <= 512 * kPH &&
         I <= 512 * kPI && kv <= kMaxKV && kv % 4 == 0 && 2 * I + kChunk <= kRing &&
         I <= 4 * kNC * 64 * kPoll && H <= 4 * kNC * 64 * kPoll;
}

// Whether a grid of G workgroups can stream an L-layer stack.  A phase too
// large for the ring runs tile by tile and frees a tile's bytes only after
// the tile is consumed, while a loader batch is issued only once its end is
// at most one ring past the freed bytes: one 16-row tile (or the whole
// phase, when a workgroup has fewer rows) must therefore fit the ring less
// a batch and a chunk.  Row counts are the largest share of a workgroup
// (ceil(rows / G)).  The stream offset of a layer is an int.  The rows whose
// finish adds the residual from s.xin (o and down rows, H / G of them) must
// fit one 16-row tile, which compute wave 0 finishes before it polls the
// next phase's input into s.xin.
static bool decode_grid_ok(int64_t H, int64_t kv, int64_t I, int64_t L, int64_t G, bool fold) {
  const int64_t room = kRing - (int64_t)(kBatch + 1) * kChunk;
  auto share = [&](int64_t n) { return (n + G - 1) / G; };
  auto tile_fits = [&](int64_t rows, int64_t K) { return std::min<int64_t>(rows, 16) * K * 2 <= room; };
  if (share(H) > 16) return false;
  const int64_t r0 = share(H + 2 * kv) + (fold ? share(H) : 0), r1 = fold ? 0 : share(H), r2 = 2 * share(I),
                r3 = share(H);
  if (!tile_fits(r0, H) || !tile_fits(r1, H) || !tile_fits(r2, H) || !tile_fits(r3, I)) return false;
  auto pad = [](int64_t b) { return (b + kChunk - 1) / kChunk * kChunk; };
  const int64_t layer = pad(r0 * H * 2) + pad(r1 * H * 2) + pad(r2 * H * 2) + pad(r3 * I * 2);
  return L * layer < ((int64_t)1 << 31) - layer;
}

int64_t decode_workspace_bytes(int64_t H, int64_t kv_dim, int64_t I) {
  return 4 * ((int64_t)kCtrlWords + kCopies * (2 * (int64_t)rup64(H) + rup64(kv_dim) + rup64(I)));
}

hipError_t launch_decode_step(const DecodeProblem& p, hipStream_t stream) {
  if (!decode_shape_ok(p.H, p.heads, p.kv_heads, p.head_dim, p.I)) return hipErrorNotSupported;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int cus = 0;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
  int per_cu = 0;
  if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_persistent<true>, kThreads, 0)) !=
      hipSuccess)
    return e;
  int per_cu2 = 0;
  if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu2, decode_step_persistent<false>, kThreads, 0)) !=
      hipSuccess)
    return e;
  per_cu = std::min(per_cu, per_cu2);
  if (per_cu < 1 || cus < 1) return hipErrorNotSupported;
  // At most one workgroup per CU, and no more than H or I: then every
  // workgroup owns rows in every phase, so every phase's output needs every
  // workgroup, and no workgroup can run a phase ahead of one still polling
  // the vector it would overwrite (a published vector is rewritten one
  // layer later, after a phase that waited for that poller's own rows).
  const int G = (int)std::min<int64_t>(cus, std::min(p.H, p.I));
  if (!decode_grid_ok(p.H, p.kv_heads * p.head_dim, p.I, p.L, G, p.w_ov != nullptr)) return hipErrorNotSupported;

  DArgs a{};
  a.x = (const char*)p.x;
  a.w_qkv = (const char*)p.w_qkv;
  a.b_qkv = (const char*)p.b_qkv;
  a.w_o = (const char*)p.w_o;
  a.w_ov = (const char*)p.w_ov;
  a.b_ov = (const char*)p.b_ov;
  a.fold = p.w_ov != nullptr;
  a.w_gu = (const char*)p.w_gu;
  a.w_down = (const char*)p.w_down;
  a.g_attn = (const char*)p.g_attn;
  a.g_mlp = (const char*)p.g_mlp;
  a.g_final = (const char*)p.g_final;
  a.qkv_out = (char*)p.qkv_out;
  a.x_out = (char*)p.x_out;
  a.h_out = (char*)p.h_out;
  a.ws = p.ws;
  a.L = (int)p.L;
  a.H = (int)p.H;
  a.NKV = (int)(p.kv_heads * p.head_dim);
  a.I = (int)p.I;
  a.HD = (int)p.head_dim;
  a.grp = (int)(p.heads / p.kv_heads);
  a.strXB = rup64(p.H);
  a.strVB = rup64(a.NKV);
  a.strAB = rup64(p.I);
  a.offXB = kCtrlWords;
  a.offX1B = a.offXB + kCopies * a.strXB;
  a.offVB = a.offX1B + kCopies * a.strXB;
  a.offAB = a.offVB + kCopies * a.strVB;
  a.eps = p.eps;
  auto swz = [](int64_t K) {
    const int64_t np = K / 8;
    return np % 16 == 0 ? 15 : np % 8 == 0 ? 7 : np % 4 == 0 ? 3 : np % 2 == 0 ? 1 : 0;
  };
  a.swzH = swz(p.H);
  a.swzI = swz(p.I);
  a.timeout = (uint64_t)(p.timeout_us > 0 ? p.timeout_us : 1000000) * 100;  // 100 MHz clock
  // An ordinary launch: G <= the CU count workgroups, each of which fits a
  // CU on its own, are all resident at once on a device with nothing else
  // running.  Should some not be (another stream's kernel holding CUs), the
  // resident ones wait for them with bounded waits, so the launch ends with
  // the error word set rather than hanging.
  if (a.fold)
    hipLaunchKernelGGL(decode_step_persistent<true>, dim3(G), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(decode_step_persistent<false>, dim3(G), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace hxmi
