// Host-side launch interface between the C ABI (capi.hip) and the kernel
// translation units. Nothing here crosses the library boundary.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hxmi {

enum Dtype { DT_F16 = 0, DT_BF16 = 1, DT_W8A16 = 2 /* fp16 A, int8 B */ };

enum Epilogue {
  EPI_NONE = 0,
  EPI_BIAS = 1,
  EPI_SILU_MUL = 2,
  EPI_GELU_TANH = 3,
  EPI_BIAS_GELU_TANH = 4,
};

enum OutType { OUT_SAME = 0, OUT_F32 = 1 };

// Layout of a split-K workspace (GEMM and GEMV alike): a fixed region of
// 64-bit arrival counters at the head, one per output tile of the call,
// then the fp32 partial tiles.  Fixing the counter region for every shape
// lets one zero-filled workspace serve calls of different shapes: a call
// writes partials only past the region and leaves its counters zero.
// A problem whose split would need more tiles than counters runs unsplit.
constexpr int64_t kWsCounterBytes = 16384;
constexpr int64_t kWsMaxTiles = kWsCounterBytes / 8;

// Launch-shape tuning knobs (tuning.hip): the environment value HXMI_<NAME>
// read once at load, overridden per thread by hxmi_set_tuning.
enum Knob {
  KNOB_GEMM_TILE = 0,  // forced GEMM TileId
  KNOB_GROUP_M,        // tile-rows per raster group
  KNOB_SPLITK,         // forced K slice count
  KNOB_W8_TILE,        // forced tile of the int8-weight GEMM
  KNOB_GEMV_PATH,      // GemvPath
  KNOB_GEMV_TPB,       // 16-row tiles per workgroup of the MFMA GEMV
  KNOB_GEMV_KS,        // waves splitting K inside a GEMV workgroup
  KNOB_GEMV_KG,        // workgroups splitting K per GEMV row group
  KNOB_GEMV_UNR,       // K-steps in flight per GEMV wave
  KNOB_GEMV_PAIR_WG,   // workgroup cap of the whole-line GEMV
  KNOB_ATTN_CFG,       // fused attention: 10 * query waves + key-split waves per workgroup
  KNOB_COUNT
};
enum GemvPath { GEMV_PATH_MFMA = 0, GEMV_PATH_VALU = 1, GEMV_PATH_PAIR = 2, GEMV_PATH_PAIR_KS = 3 };
constexpr int64_t KNOB_UNSET = INT64_MIN;
int64_t knob(Knob k);  // KNOB_UNSET: the library's own choice
int knob_index(const char* name);
// Sets this thread's override of knob k (value < 0 clears it); returns the
// previous override, -1 if there was none.
int64_t set_knob_override(int k, int64_t value);

// One (optionally batched) GEMM  C[b] = epilogue(alpha * A[b] . op(B[b])).
// A is [M,K] row-major with leading dimension lda.  B is [K,N] (b_nt = 0) or
// [N,K] (b_nt = 1).  For EPI_SILU_MUL, N counts the packed gate/up columns of
// B and C receives N/2 columns.
struct GemmProblem {
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC;  // batch strides, elements
  int64_t batch;
  float alpha;
  int dtype;     // Dtype of A, B and (unless out_f32) C
  int b_nt;      // 1: B is [N,K]
  int epilogue;  // Epilogue
  int out_f32;   // 1: C is fp32
  int tile;      // forced tile id (< 0: heuristic)
  void* ws;      // split-K workspace (fp32 partial sums) or null
  int64_t ws_bytes;
  const void* scale;  // int8 B only: per-column fp16 scale
  int rms;            // 1: C = epilogue(rmsnorm(A) . B^T), B holds the folded norm weight
  float rms_eps;
  float* rs_out;       // rms: also write each row's rsqrt(mean(A[m,:]^2) + eps) here
  const float* rs_in;  // !rms: scale row m of A . B^T by rs_in[m] before the epilogue
};

// Wg[n][k] = fp16(W[n][k] * g[k]): folds an RMSNorm weight into the linear
// layer that consumes the normalised activations.
hipError_t launch_fold_rms_weight(int dtype, const void* W, const void* g, void* Wg, int64_t N, int64_t K, int64_t ldw,
                                  int64_t ldwg, hipStream_t stream);

// s[n] = fp16 scale covering max_k |W[n][k]| / 127, q[n][k] = rint(W[n][k] / s[n]):
// per-row symmetric int8 codes for the weight-only int8 path.  K, ldw, ldq
// multiples of 8, W 16-byte and q 8-byte aligned (checked by the caller).
hipError_t launch_quantize_int8_rows(const void* W, int8_t* q, void* s, int64_t N, int64_t K, int64_t ldw,
                                     int64_t ldq, hipStream_t stream);

// Split-K factor the dispatcher uses for p (1 = none) and the workspace bytes
// it needs; both depend only on shapes and epilogue.
int gemm_splits(const GemmProblem& p);
int64_t gemm_workspace_bytes(const GemmProblem& p);

// Tile shapes the fast kernel is instantiated for.
enum TileId {
  TILE_256x256 = 0,
  TILE_128x256,
  TILE_256x128,
  TILE_128x128,
  TILE_64x128,
  TILE_128x64,
  TILE_64x64,
  TILE_256x256_K32S4,
  TILE_256x256_W8,
  TILE_128x128_K32S4,
  TILE_256x128_K32S4,
  TILE_256x256_PP,  // 8 waves, ping-pong schedule, 32-deep K-steps, 3 stages
  TILE_256x128_W8,  // 8 waves of 64x64, 3 stages
  TILE_128x128_W8,  // 8 waves of 32x64
  TILE_128x192_W8,  // 8 waves of 32x96, 3 stages; k-contiguous fp16 / bf16 B only (not NN, not int8)
  TILE_64x64_S4,    // TILE_64x64 with 4 LDS stages
  TILE_COUNT
};

hipError_t launch_gemm(const GemmProblem& p, hipStream_t stream);
// Whether p satisfies the alignment rules of the MFMA fast path.
bool gemm_fast_path_ok(const GemmProblem& p);
int gemm_pick_tile(const GemmProblem& p);

struct GemvProblem {
  const void* x;      // [M,K] fp16 (bf16 with dtype DT_BF16)
  const void* W;      // [N,K] fp16 / bf16, or int8
  const void* scale;  // [N] fp16 (int8 weights only)
  const void* bias;   // [N] x's type, or null
  void* y;            // [M,N] x's type
  int64_t M, N, K;
  int64_t ldx, ldw, ldy;
  int w_int8;
  int dtype = DT_F16;  // DT_F16 or DT_BF16 (int8 weights: fp16 activations)
  // 1: the whole-line fp16 / bf16 kernel loads W with the ordinary cache
  // policy instead of non-temporal (the decode forward's lm_head, which runs
  // after a non-temporal stream of the layer weights)
  int w_cached = 0;
  void* ws;  // optional workspace for K split over workgroups
  int64_t ws_bytes;
};

hipError_t launch_gemv(const GemvProblem& p, hipStream_t stream);
// Workspace bytes launch_gemv can use for p (0: it never splits K).
int64_t gemv_workspace_bytes(const GemvProblem& p);

// W8A16 GEMM for larger M (MFMA, int8 weights dequantised in registers).
hipError_t launch_w8a16_gemm(const GemvProblem& p, void* ws, int64_t ws_bytes, hipStream_t stream);
GemmProblem w8a16_as_gemm(const GemvProblem& p);

struct RowProblem {
  const void* x;
  const void* g;  // RMSNorm weight or null
  void* y;
  int64_t rows, cols, ldx, ldy;
  float eps;    // RMSNorm
  float scale;  // softmax: y = softmax(scale * x)
  int dtype;
};

hipError_t launch_rmsnorm(const RowProblem& p, hipStream_t stream);
hipError_t launch_softmax(const RowProblem& p, hipStream_t stream);

// Softmax of attention scores with the mask operand and the causal rule:
// slices of s_q rows of s_kv columns, slice i reads mask slice
// i / mask_group (mask fp16 or null; stride_m 0 broadcasts).
struct MaskedSoftmaxProblem {
  const void* x;
  void* y;
  const void* mask;
  int64_t slices, s_q, s_kv;
  int64_t ldx, stride_x, ldy, stride_y, ldm, stride_m, mask_group;
  int causal;  // 0 none, 1 key j > query r removed, 2 j > r + s_kv - s_q
  float scale;
  int dtype;
};
hipError_t launch_softmax_masked(const MaskedSoftmaxProblem& p, hipStream_t stream);

struct AttnProblem {
  const void* q;  // [B*H, S, D]
  const void* k;  // [B*H / kv_group, SKV, D]
  const void* v;
  void* o;
  const void* mask;  // fp16 additive [B*H / mask_group, S, SKV] or null
  int64_t bh, s, skv, d;
  int64_t sq, sk, sv, so, sm;  // per-slice strides, elements
  int64_t ldq, ldk, ldv, ldo, ldm;
  int64_t kv_group;    // query heads per key/value head
  int64_t mask_group;  // (batch, head) slices sharing one mask slice
  int causal;          // 0 none, 1 key <= query, 2 key <= query + skv - s
  float scale;
};

hipError_t launch_attention(const AttnProblem& p, hipStream_t stream);

// One-token decoder step of a Llama / Qwen2 stack (persistent kernel).
struct DecodeProblem {
  const void* x;        // [H] fp16: the token's embedding row
  const void* w_qkv;    // [L, H + 2*kv_dim, H]: q rows, k rows, v rows
  const void* b_qkv;    // [L, H + 2*kv_dim] or null
  const void* w_o;      // [L, H, H] (unused with w_ov)
  const void* w_ov;     // [L, H, H] o projection folded onto the normalised input, or null
  const void* b_ov;     // [L, H] its bias, or null
  const void* w_gu;     // [L, 2*I, H]: gate rows, then up rows
  const void* w_down;   // [L, H, I]
  const void* g_attn;   // [L, H] RMSNorm weights before attention
  const void* g_mlp;    // [L, H] RMSNorm weights before the MLP
  const void* g_final;  // [H]
  void* qkv_out;        // [L, H + 2*kv_dim] or null
  void* x_out;          // [H] final hidden state before the last norm, or null
  void* h_out;          // [H] normalised final hidden state
  uint32_t* ws;         // decode_workspace_bytes(), zero-filled before first use
  int64_t L, H, heads, kv_heads, head_dim, I;
  float eps;
  int64_t timeout_us;  // bound of every wait inside the kernel
};

int64_t decode_workspace_bytes(int64_t H, int64_t kv_dim, int64_t I);
// Word of the decode workspace that records an expired wait (sticky).
constexpr int DECODE_WS_ERROR_WORD = 3;
// hipErrorNotSupported: shape outside the kernel's limits (the caller falls
// back to per-GEMV launches).
hipError_t launch_decode_step(const DecodeProblem& p, hipStream_t stream);
bool decode_shape_ok(int64_t H, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t I);

// Region profiling: record `slot` of `records` (3 words each) = {id, wall
// clock low word, high word}, taken when the marker runs on `stream`.
hipError_t launch_lwp_mark(uint32_t* records, int64_t slot, uint32_t id, hipStream_t stream);

}  // namespace hxmi
