/*
 * hxmi — C ABI of the MI355X (gfx950) hot-path kernels.
 *
 * Replaces, for one GPU, what Hexagon-MLIR's qcom_hexagon_backend generates
 * and links for the matmul / GEMV / RMSNorm / softmax path: the compiled
 * kernel entry `_mlir_ciface_<func>` that the Python launcher builds and runs
 * (qcom_hexagon_backend/lib/Conversion/LinalgToLLVM/LinalgToLLVMPass.cpp:156-189,
 * qcom_hexagon_backend/backend/torch_mlir_hexagon_launcher.py:258-306) and the
 * runtime it calls (qcom_hexagon_backend/bin/runtime/include/HexagonCAPI.h:19-25,
 * bin/runtime/UserDMA/RuntimeDMA.cc:48-96, bin/runtime/include/HexKLAPI.h:17-20).
 *
 * Conventions for every entry point:
 *   - all tensor pointers are device pointers owned by the caller; nothing is
 *     allocated or freed on these calls;
 *   - matrices are row-major with explicit leading dimensions in elements;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is
 *     stream-ordered and the call returns after the launch;
 *   - return value: HXMI_OK, or an error code with a message available from
 *     hxmi_last_error() (thread-local); invalid arguments are rejected before
 *     anything is launched;
 *   - a size of 0 in any output dimension is a no-op that returns HXMI_OK.
 */
#ifndef HXMI_H
#define HXMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 element type for the HexKL-compatible entry (ABI: a 2-byte value). */
#if defined(__clang__) || (defined(__GNUC__) && __GNUC__ >= 12)
typedef _Float16 hxmi_f16_t;
#else
typedef uint16_t hxmi_f16_t;
#endif

#define HXMI_OK 0
#define HXMI_ERR_INVALID_ARGUMENT 1
#define HXMI_ERR_UNSUPPORTED 2
#define HXMI_ERR_HIP 3

/* Bytes of arrival counters at the head of every split-K workspace. */
#define HXMI_WORKSPACE_COUNTER_BYTES 16384

/* GEMM epilogues, applied to alpha * (A . op(B)) in fp32 before the store. */
#define HXMI_EPI_NONE 0
#define HXMI_EPI_BIAS 1           /* + bias[n]                                  */
#define HXMI_EPI_SILU_MUL 2       /* silu(gate) * up over packed gate/up columns */
#define HXMI_EPI_GELU_TANH 3      /* tanh-approximate GELU                       */
#define HXMI_EPI_BIAS_GELU_TANH 4 /* GELU(x + bias[n])                           */

/* Message describing the last failed call on this thread ("" if none). */
const char* hxmi_last_error(void);

/* Library version, major * 10000 + minor * 100 + patch. */
int hxmi_version(void);

/*
 * Launch-shape tuning override for the calls this thread makes afterwards
 * (value < 0 removes it).  Knobs: "gemm_tile" (forced GEMM tile id),
 * "group_m", "splitk", "w8_tile", "gemv_path" (0 16-row MFMA, 1 vector-ALU
 * rows, 2 whole-line pairs, 3 whole-line pairs with K split), "gemv_tpb",
 * "gemv_ks", "gemv_kg", "gemv_unr", "gemv_pair_wg", "attn_cfg" (fused
 * attention: 10 * query waves + key-split waves).  A knob without a thread
 * override takes the value of the environment variable HXMI_<NAME> read once
 * when the library loaded, else the library's own choice.  Knobs change how a
 * result is computed (tile, K split, kernel), not what it is.  *previous
 * (optional) receives the thread's previous override, -1 if none, so a caller
 * can restore it.
 * Replaces: the compile options that steer the reference's tiling for one
 * compilation (tileSizes, hexagon_options.py:17-88), scoped here to a thread.
 */
int hxmi_set_tuning(const char* name, int64_t value, int64_t* previous);

/*
 * C[M,N] = epilogue(alpha * A[M,K] . op(B)), fp32 accumulation, fp16 output.
 *   b_is_nt = 0: B is [K,N] (linalg.matmul; reference config "C = A . B")
 *   b_is_nt = 1: B is [N,K] (linalg.matmul_transpose_b; every nn.Linear)
 * For HXMI_EPI_SILU_MUL, B holds N packed columns (N % 32 == 0): packed
 * columns [32q, 32q+16) are gate rows 16q..16q+15 and [32q+16, 32q+32) the
 * matching up rows; C receives N/2 columns, C[:, 16q+i] = silu(g_i) * u_i.
 * bias (fp16, N entries) is required for the BIAS epilogues, else ignored.
 * workspace / workspace_bytes: optional caller-owned device scratch (256-byte
 * aligned).  When the output has too few tiles to occupy the GPU and K is
 * long, the GEMM splits K into slices that write fp32 partial tiles there;
 * the last slice to finish an output tile adds them in slice order and
 * applies the epilogue (one launch).  It needs hxmi_gemm_workspace_bytes()
 * bytes.  NULL / 0 (or a smaller or misaligned buffer) runs the GEMM
 * unsplit.  Workspace contract (every entry point that takes one): the
 * first HXMI_WORKSPACE_COUNTER_BYTES bytes hold per-tile arrival counters,
 * which must be zero when a call that uses the workspace starts; partial
 * tiles go after them.  Zero the whole buffer once after allocating it:
 * every call leaves its counters zero again and writes nothing else into
 * that region, so one buffer serves later calls of any shape (and graph
 * replays) on the same stream without being cleared.  A counter region
 * holding anything else gives wrong results.  Two calls must not use one
 * workspace concurrently.
 * Replaces: the linalg.matmul / matmul_transpose_b lowering scheduled by
 * ScheduleMatmulForHVXPass.cpp:69-195 and tiled by VTCMTiling.cpp:231-266
 * (with HexmemCpyToDMA.cpp:120-271 DMA staging), plus the elementwise
 * generics HexagonFusionPass leaves after it (FusionPass.cpp:161-179).
 */
int hxmi_gemm_f16(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                  int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* Same contract as hxmi_gemm_f16 with bf16 operands, bias and output. */
int hxmi_gemm_bf16(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* Workspace bytes a contiguous hxmi_gemm_f16/bf16 call of this shape can use
 * (0: it never splits K).  Depends on shapes and epilogue only. */
int64_t hxmi_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int b_is_nt, int epilogue);

/* Bytes of the per-GPU device scratch array hxmi_gemm_f16_noalloc uses. */
#define HXMI_NOALLOC_SCRATCH_BYTES 33554432

/*
 * hxmi_gemm_f16 without a workspace argument and without any allocation:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and epilogues as hxmi_gemm_f16; where that call would
 * split K, the fp32 partial tiles go to a library-owned array of
 * HXMI_NOALLOC_SCRATCH_BYTES in each GPU's memory (held until the process
 * ends) instead of a caller workspace.  A shape whose partials need more is
 * rejected with HXMI_ERR_INVALID_ARGUMENT before anything is launched.  The
 * array's arrival counters start zero and every call leaves them zero.  All
 * calls on one GPU share its array: two calls whose executions overlap on
 * one GPU (different streams, or concurrent graph replays) race and give
 * wrong results; calls ordered on one stream are safe.  `stream` must
 * belong to the current device.
 * No counterpart in the reference (its kernels allocate VTCM from a runtime
 * pool, VTCMPool.cpp:62-106); it exists for the callers named above.
 */
int hxmi_gemm_f16_noalloc(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                          int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha,
                          void* stream);

/*
 * Strided batched GEMM: for b in [0,batch): C + b*strideC = epilogue(alpha *
 * (A + b*strideA) . op(B + b*strideB)).  Strides in elements.
 * Replaces: linalg.batch_matmul(_transpose_b) scheduling
 * (ScheduleMatmulForHVXPass.cpp:105-167), used by the attention lowering
 * LowerTmTensor.cpp:91-250 (Q.K^T scaled, then P.V).
 */
int hxmi_bgemm_f16(const void* A, const void* B, void* C, const void* bias, int64_t batch, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t strideA, int64_t strideB,
                   int64_t strideC, int b_is_nt, int epilogue, float alpha, void* stream);
int hxmi_bgemm_bf16(const void* A, const void* B, void* C, const void* bias, int64_t batch, int64_t M, int64_t N,
                    int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t strideA, int64_t strideB,
                    int64_t strideC, int b_is_nt, int epilogue, float alpha, void* stream);

/*
 * Decode GEMV/skinny GEMM: y[M,N] = x[M,K] . W[N,K]^T (+ bias[N]), fp16,
 * fp32 accumulation, any M (M <= 16 streams W once through the GEMV kernel,
 * larger M goes to the GEMM).  bias may be NULL.
 * workspace / workspace_bytes: optional caller-owned device scratch
 * (256-byte aligned).  With few output rows and a long K (a down
 * projection) the GEMV splits K over workgroups, which combine their fp32
 * partial tiles there; it needs hxmi_gemv_workspace_bytes() bytes.  NULL / 0
 * runs unsplit.  Same workspace contract as hxmi_gemm_f16 (zeroed once after
 * allocation, left zeroed by every call, one call at a time).
 * Replaces: the M = 1 matmul_transpose_b that the reference sends through
 * the same generic HVX schedule (TilingPass.cpp:108-251); it has no GEMV.
 */
int hxmi_gemv_f16(const void* x, const void* W, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                  int64_t ldx, int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, void* stream);

/* Same contract as hxmi_gemv_f16 with bf16 x, W, bias and y (fp32
 * accumulation; the same kernels and launch plans on bf16 MFMA / dot). */
int hxmi_gemv_bf16(const void* x, const void* W, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                   int64_t ldx, int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes a contiguous hxmi_gemv_f16 call of this shape can use (0: never split). */
int64_t hxmi_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Weight-only int8 linear: y[m,n] = scale[n] * sum_k x[m,k] * Wq[n,k] (+ bias[n]).
 * x, scale, bias, y fp16; Wq int8 [N,K] (symmetric, per-output-channel
 * scale).  Weights are converted to fp16 exactly in registers; the scale
 * multiplies the fp32 sum.  Requires K % 16 == 0, ldw % 16 == 0, N % 4 == 0.
 * M <= 16 streams Wq once (GEMV kernel); larger M runs the MFMA GEMM with
 * the int8 operand.  Either may split K into the optional workspace (see
 * hxmi_gemv_f16 / hxmi_gemm_f16; size from hxmi_w8a16_workspace_bytes).
 * Replaces: no reference kernel (only quant.qcast/dcast lowering to arith,
 * LinalgToLLVMPass.cpp:203-209); defined by the weight-only int8 configs.
 */
int hxmi_gemv_w8a16(const void* x, const int8_t* Wq, const void* scale, const void* bias, void* y, int64_t M,
                    int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* Workspace bytes a contiguous hxmi_gemv_w8a16 call of this shape can use
 * (M <= 16: the GEMV's K split, as hxmi_gemv_f16; larger M: the GEMM's). */
int64_t hxmi_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * RMSNorm per row: y = g * T(x * rsqrt(mean(x^2) + eps)), fp32 math, T = fp16
 * (or bf16).  Replaces the HVX split-reduction lowering of the RMSNorm
 * generic chain (SplitReductionUtils.cpp, TilingPass.cpp:261-289) whose
 * semantics are test/python/triton/test_rms_norm.py:37-63 and HF LlamaRMSNorm.
 */
int hxmi_rmsnorm_f16(const void* x, const void* g, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                     float eps, void* stream);
int hxmi_rmsnorm_bf16(const void* x, const void* g, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                      float eps, void* stream);

/*
 * Row softmax of scale * x: y = exp(s*x - max) / sum(exp(s*x - max)), fp32
 * math.  Replaces the max/sub/exp/sum/div generic chain
 * (qcom_hexagon_backend/test/Conversion/LinalgToLLVM/fusion_softmax_2D.mlir:8-57,
 * LowerTmTensor.cpp:165-229) with its scale from the SDPA lowering.
 */
int hxmi_softmax_f16(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float scale,
                     void* stream);
int hxmi_softmax_bf16(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float scale,
                      void* stream);

/*
 * The softmax step of attention with the reference's mask operand and the
 * causal rule, over `slices` slices of s_q rows of s_kv scores (fp16 or
 * bf16 x / y, in place allowed):
 *   y[i][r][j] = softmax_j(scale * x[i][r][j] + M[i / mask_group][r][j] + C[r][j])
 * C[r][j] = -inf when causal = 1 and j > r, or causal = 2 and j > r + s_kv - s_q
 * (torch's is_causal and the bottom-right rule), else 0.  x / y: row stride
 * ldx / ldy, slice stride stride_x / stride_y (elements).  mask: fp16
 * additive, row stride ldm >= s_kv, slice stride stride_m (0 broadcasts one
 * slice), mask_group consecutive slices per mask slice; NULL for none.  A
 * row whose every score is -inf comes out NaN, as the reference's
 * max / exp / sum / div decomposition gives.  With hxmi_bgemm_* before and
 * after it, this is attention for any head dimension, bf16, grouped K/V
 * heads (query heads of one K/V head as one batch entry of group * s_q rows)
 * and masks, where the fused kernel does not apply.
 * Replaces: the mask addition and softmax of the tm_tensor.attention lowering
 * (LowerTmTensor.cpp:158-163 adds the mask to the scaled scores, :165-229
 * the max / exp / sum / div over each row).
 */
int hxmi_softmax_masked_f16(const void* x, void* y, int64_t slices, int64_t s_q, int64_t s_kv, int64_t ldx,
                            int64_t stride_x, int64_t ldy, int64_t stride_y, const void* mask, int64_t ldm,
                            int64_t stride_m, int64_t mask_group, int causal, float scale, void* stream);
int hxmi_softmax_masked_bf16(const void* x, void* y, int64_t slices, int64_t s_q, int64_t s_kv, int64_t ldx,
                             int64_t stride_x, int64_t ldy, int64_t stride_y, const void* mask, int64_t ldm,
                             int64_t stride_m, int64_t mask_group, int causal, float scale, void* stream);

/*
 * RMSNorm folded into the linear layer that consumes it (LLaMA QKV and
 * gate/up projections):
 *   C[M,N'] = epilogue(rmsnorm(x) . W^T),  rmsnorm(x)[m,k] = x[m,k] * g[k] / sqrt(mean_k x[m,k]^2 + eps)
 * with Wg[N,K] = g (.) W prepared once by hxmi_fold_rmsnorm_weight_f16.  The
 * row statistics are taken inside the GEMM from the x tiles it multiplies,
 * so the normalised activations never go to memory.  epilogue: HXMI_EPI_NONE,
 * HXMI_EPI_BIAS (bias: fp16, N entries, added after the normalisation, as
 * Qwen2's q/k/v projections) or HXMI_EPI_SILU_MUL (packed gate/up Wg, as
 * hxmi_gemm_f16; N' = N/2).
 * fp32 statistics and accumulation; differs from normalise-round-multiply
 * (HF LlamaRMSNorm) by the fp16 rounding of the normalised activations.
 * rscale_out (optional, M floats): also receives each row's
 * rsqrt(mean_k x[m,k]^2 + eps).  rscale_in (optional, M floats): row scales
 * a previous call computed for the same x; the statistics are then not
 * recomputed (eps is ignored) and C = epilogue(diag(rscale_in) . x . Wg^T),
 * so a second consumer of the same normalised rows (the gate/up projection
 * beside QKV) costs a plain GEMM.  The two are exclusive.
 * Replaces: the RMSNorm generic chain (SplitReductionUtils.cpp,
 * TilingPass.cpp:261-289; semantics test/python/triton/test_rms_norm.py:37-63)
 * plus the matmul_transpose_b after it (ScheduleMatmulForHVXPass.cpp:69-195),
 * which the reference runs as separate passes over HBM.
 */
int hxmi_rmsnorm_linear_f16(const void* x, const void* Wg, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                            int64_t ldx, int64_t ldw, int64_t ldc, int epilogue, float eps, float* rscale_out,
                            const float* rscale_in, void* stream);

/* Same contract as hxmi_rmsnorm_linear_f16 with bf16 x, Wg, bias and C
 * (statistics and accumulation in fp32). */
int hxmi_rmsnorm_linear_bf16(const void* x, const void* Wg, void* C, const void* bias, int64_t M, int64_t N,
                             int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int epilogue, float eps,
                             float* rscale_out, const float* rscale_in, void* stream);

/* Wg[n,k] = fp16(W[n,k] * g[k]) (fp32 product, one rounding): the weight
 * hxmi_rmsnorm_linear_f16 takes.  W, Wg [N,K] (leading dims ldw, ldwg), g [K]. */
int hxmi_fold_rmsnorm_weight_f16(const void* W, const void* g, void* Wg, int64_t N, int64_t K, int64_t ldw,
                                 int64_t ldwg, void* stream);

/* The bf16 form of hxmi_fold_rmsnorm_weight_f16 (bf16 W, g, Wg), for
 * hxmi_rmsnorm_linear_bf16. */
int hxmi_fold_rmsnorm_weight_bf16(const void* W, const void* g, void* Wg, int64_t N, int64_t K, int64_t ldw,
                                  int64_t ldwg, void* stream);

/*
 * Per-output-channel symmetric int8 quantisation, the weight layout
 * hxmi_gemv_w8a16 reads:
 *   s[n]   = fp16(max_k |W[n,k]| / 127), moved one fp16 step up if
 *            127 * s[n] < max_k |W[n,k]| (so no code clips); 1 for a zero row
 *   q[n,k] = rint(W[n,k] / s[n]) (round half to even), in [-127, 127]
 * so |W[n,k] - q[n,k] * s[n]| <= s[n] / 2.  W [N,K] fp16 (ldw), q [N,K] int8
 * (ldq), s [N] fp16; K, ldw and ldq multiples of 8, W 16-byte and q 8-byte
 * aligned; W finite.
 * Replaces: the int8 weights the reference can only take through MLIR's
 * quant.qcast lowering (createLowerQuantOps, LinalgToLLVMPass.cpp:203-205);
 * it has no weight quantiser of its own.
 */
int hxmi_quantize_int8_rows_f16(const void* W, int8_t* q, void* s, int64_t N, int64_t K, int64_t ldw, int64_t ldq,
                                void* stream);

/*
 * Fused attention, fp16: for each of bh (batch x head) slices,
 *   O[i] = softmax(scale * Q[i] . K^T) . V  over s_kv keys,
 * Q/O [s_q, d], K/V [s_kv, d] row-major (leading dims ld*, slice strides
 * stride_*, elements), d = 64 or 128, scale > 0, fp32 softmax and accumulation,
 * no mask.
 * Replaces: tm_tensor.attention as LowerTmTensor.cpp:52-250 lowers it
 * (batch_matmul(Q, K^T) -> scale -> softmax -> batch_matmul(P, V), semantics
 * of qcom_hexagon_backend/test/Conversion/TmTensorToLinalg/SDPA.mlir:18-59)
 * in one kernel; the same three steps remain available as hxmi_bgemm_f16 +
 * hxmi_softmax_f16.
 */
int hxmi_attention_f16(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t s_q, int64_t s_kv,
                       int64_t d, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, int64_t stride_q,
                       int64_t stride_k, int64_t stride_v, int64_t stride_o, float scale, void* stream);

/*
 * Fused attention with the reference's mask operand, fp16:
 *   O[i] = softmax(scale * Q[i] . K[i / kv_group]^T + M[i / mask_group]) . V[i / kv_group]
 * with, when causal != 0, every key j of query r with j > r (causal = 1, the
 * top-left rule of torch's is_causal) or j > r + s_kv - s_q (causal = 2,
 * bottom-right) masked to -inf.
 *  - mask: fp16 additive [s_q, s_kv] per slice (row stride ldm >= s_kv, slice
 *    stride stride_m, 0 broadcasts one slice to all), or NULL for none; -inf
 *    entries remove a key.  mask_group consecutive (batch, head) slices share
 *    one mask slice (e.g. the heads of one batch row for a [B, 1, S, S_kv]
 *    mask).
 *  - kv_group consecutive query slices share one K/V slice (grouped-query
 *    attention: q heads per kv head; 1 = one K/V slice per query slice);
 *    stride_k / stride_v step between K/V slices.
 *  - scale > 0.  A query whose every key is masked yields NaN (0/0), as the
 *    reference's decomposition does.
 * Other arguments as hxmi_attention_f16, which equals kv_group = 1, no mask,
 * causal = 0.
 * Replaces: tm_tensor.attention with its mask operand
 * (LowerTmTensor.cpp:81-88 reads it, :158-163 adds it to the scaled Q.K^T
 * before the softmax).
 */
int hxmi_attention_ex_f16(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t s_q,
                          int64_t s_kv, int64_t d, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                          int64_t stride_q, int64_t stride_k, int64_t stride_v, int64_t stride_o, int64_t kv_group,
                          const void* mask, int64_t ldm, int64_t stride_m, int64_t mask_group, int causal,
                          float scale, void* stream);

/*
 * One-token decoder step of a Llama / Qwen2 stack of `layers` layers at
 * position 0 (empty KV cache), fp16 in and out, fp32 accumulation, as ONE
 * persistent launch (plus the lm_head GEMV when w_lm is given):
 *   x_0 = x; for each layer l:
 *     h   = rmsnorm(x_l, g_attn[l]);   qkv = h . w_qkv[l]^T (+ b_qkv[l])
 *     att = attention of the single token: query head i gets v of key/value
 *           head i / (heads / kv_heads)  (softmax over one key is 1; RoPE at
 *           position 0 is the identity)
 *     x1  = x_l + att . w_o[l]^T
 *     h2  = rmsnorm(x1, g_mlp[l]);     [g | u] = h2 . w_gu[l]^T
 *     x_{l+1} = x1 + (silu(g) * u) . w_down[l]^T
 *   h_out = rmsnorm(x_L, g_final);     logits = h_out . w_lm^T
 * rmsnorm(x, g) = g * fp16(x * rsqrt(mean(x^2) + eps)) with the mean in
 * fp32; each projection output, the SiLU, the product and each residual sum
 * is rounded to fp16, as in the HF fp16 forward.
 * Layouts (device, contiguous; kv_dim = kv_heads * head_dim): x [H] (the
 * token's embedding row); w_qkv [L, H + 2*kv_dim, H] (q rows, k rows, v
 * rows); b_qkv [L, H + 2*kv_dim] or NULL; w_o [L, H, H]; w_gu [L, 2*I, H]
 * (gate rows, then up rows); w_down [L, H, I]; g_attn, g_mlp [L, H];
 * g_final [H]; w_lm [vocab, H] or NULL.
 * Outputs: h_out [H]; logits [vocab] when w_lm is given; qkv_out
 * [L, H + 2*kv_dim] (its k and v rows are what a KV cache appends) or NULL;
 * x_out [H] = x_L or NULL.
 * Limits: heads * head_dim == H, H % 8 == 0, H <= 2048, I % 8 == 0,
 * I <= 6144, head_dim % 8 == 0, kv_dim <= 512; x, the weights and the
 * outputs 16-byte aligned.  Other shapes: HXMI_ERR_UNSUPPORTED.
 * workspace: hxmi_decode_workspace_bytes(H, kv_dim, I) bytes of device
 * memory, zero-filled once after allocation.  It carries the published
 * phase outputs and a running tag from call to call: one call at a time
 * per workspace, and one stack shape (H, kv_dim, I) per workspace -- zero
 * it again before using it for another shape.
 * timeout_us: bound of every wait inside the kernel (0: one second).  A
 * wait that expires ends the launch early with the workspace's error word
 * set (hxmi_decode_status) and the outputs undefined.
 * Replaces: the reference's Qwen2.5-0.5B forward of a one-token prompt at
 * position 0 with the cache off (benchmark_models/run_qwen2.5-0.5b.py:
 * 171-173, 224-233), which it compiles into one generic matmul per
 * projection (TilingPass.cpp:108-251) and separate elementwise kernels.
 */
int hxmi_decode_step_f16(const void* x, const void* w_qkv, const void* b_qkv, const void* w_o, const void* w_gu,
                         const void* w_down, const void* g_attn, const void* g_mlp, const void* g_final,
                         const void* w_lm, void* qkv_out, void* x_out, void* h_out, void* logits, int64_t layers,
                         int64_t hidden, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t intermediate,
                         int64_t vocab, float eps, int64_t timeout_us, void* workspace, int64_t workspace_bytes,
                         void* stream);

/*
 * hxmi_decode_step_f16 with each layer's o projection folded onto the
 * normalised input h of the same layer: at position 0 the attention output
 * is att = E (h . w_v^T + b_v) (E copies key/value head j's head_dim
 * elements to every query head of its group), so
 *   att . w_o^T = h . w_ov^T + b_ov,  w_ov = w_o E w_v,  b_ov = w_o E b_v
 * (w_v, b_v: the v rows of w_qkv, b_qkv).  The step then runs the o
 * projection with q|k|v from the same input and has three dependent phases
 * a layer instead of four.  w_ov [L, H, H]; b_ov [L, H] or NULL (b_qkv
 * NULL).  Per layer, with Ev = E w_v ([H, H], row i = v row (i / head_dim /
 * (heads / kv_heads)) * head_dim + i % head_dim) and Eb = E b_v:
 * w_ov = hxmi_gemm_f16 NN of w_o and Ev, b_ov = hxmi_gemv_f16 of Eb and
 * w_o (fp32 accumulation, one fp16 rounding).  Everything else, the
 * outputs and the workspace are as for hxmi_decode_step_f16; x1 differs
 * from that step's by the rounding of w_ov and of the un-rounded v (fp16
 * v is never formed).
 * No counterpart in the reference: it serves the same one-token forward
 * (benchmark_models/run_qwen2.5-0.5b.py:171-173, 224-233), for callers that
 * keep the folded weights beside the stack.
 */
int hxmi_decode_step_ov_f16(const void* x, const void* w_qkv, const void* b_qkv, const void* w_ov, const void* b_ov,
                            const void* w_gu, const void* w_down, const void* g_attn, const void* g_mlp,
                            const void* g_final, const void* w_lm, void* qkv_out, void* x_out, void* h_out,
                            void* logits, int64_t layers, int64_t hidden, int64_t heads, int64_t kv_heads,
                            int64_t head_dim, int64_t intermediate, int64_t vocab, float eps, int64_t timeout_us,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of hxmi_decode_step_f16 for these sizes. */
int64_t hxmi_decode_workspace_bytes(int64_t hidden, int64_t kv_dim, int64_t intermediate);

/* Waits for `stream`, then reads the error word of a decode workspace into
 * *status (0: every launch so far finished its waits; 1: a wait expired)
 * and, with clear != 0, resets it. */
int hxmi_decode_status(void* workspace, int clear, int* status, void* stream);

/*
 * Region profiling hook: enqueues on `stream` a one-wave marker that, when it
 * runs (after every kernel enqueued before it on that stream has finished),
 * writes record `slot` of `records` -- three uint32 words {id, t low word,
 * t high word}, t the GPU's constant-rate wall clock -- so a begin and an end
 * record with the same id bracket the kernels enqueued between them.  The
 * buffer is device memory of at least 3 * (slot + 1) words, owned by the
 * caller; slots are the caller's to assign (no two in-flight records may
 * share one).  Written out as {"entries": [{"id": id, "cyc": t}, ...]} in
 * record order, the records are what the reference's region tooling reads.
 * Replaces: the LWP instrumentation hooks and record buffer
 * (test/utils/dsp/include/prof_utils.cc:37-60, bin/runtime/profiler/
 * lwp_handler.S), whose JSON test/python/process_lwp.py:20-60 folds.
 */
int hxmi_lwp_record(uint32_t* records, int64_t slot, uint32_t id, void* stream);

/* Ticks per second of the clock hxmi_lwp_record reads, for the current
 * device (0 if it cannot be queried). */
int64_t hxmi_lwp_clock_hz(void);

/*
 * HexKL-compatible matmul: outM[n_row, n_col] (fp32) = inAct[n_row, n_inner]
 * . inW[n_inner, n_col] (both fp16, row-major, contiguous), device pointers,
 * default stream, synchronous like the reference.  Returns 0 on success.
 * Replaces: hexkl_matmul_f16f16_f32 (bin/runtime/include/HexKLAPI.h:17-20,
 * bin/runtime/src/HexKLAPI.cpp:15-141), whose accumulator is read back as
 * fp16; here it stays fp32.
 */
int hexkl_matmul_f16f16_f32(int64_t n_row, int64_t n_col, int64_t n_inner, float* outM, const hxmi_f16_t* inAct,
                            const hxmi_f16_t* inW);

#ifdef __cplusplus
}
#endif

#endif /* HXMI_H */
