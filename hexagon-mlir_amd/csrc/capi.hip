// extern "C" entry points declared in include/hxmi.h: argument validation,
// error reporting, dispatch to the kernel launchers.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/hxmi.h"
#include "hxmi_internal.h"

// Split-K scratch of hxmi_gemm_f16_noalloc: one array per GPU, in the code
// object's zero-filled data, so its arrival counters start at zero and every
// call leaves them zero.  In host code `scratch` names a host-side stand-in,
// not the device array: kernels get the address from hipGetSymbolAddress.
static __device__ __align__(256) char scratch[HXMI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];

// Device address of the current device's scratch array, looked up once per
// device (with that device current).
hipError_t scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess) return g_scratch_err[dev];
  *out = g_scratch_ptr[dev];
  return *out ? hipSuccess : hipErrorInvalidSymbol;
}

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return HXMI_OK;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  if (e == hipErrorNotSupported) return fail(HXMI_ERR_UNSUPPORTED, "%s: unsupported shape/alignment", what);
  return fail(HXMI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define REQUIRE(cond, ...)                                   \
  do {                                                       \
    if (!(cond)) return fail(HXMI_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

int gemm_common(int dtype, const void* A, const void* B, void* C, const void* bias, int64_t batch, int64_t M,
                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB, int64_t sC,
                int b_is_nt, int epilogue, float alpha, int out_f32, void* ws, int64_t ws_bytes, void* stream,
                const char* name, int rms = 0, float rms_eps = 0.f, float* rs_out = nullptr,
                const float* rs_in = nullptr, bool noalloc = false) {
  REQUIRE(batch >= 0 && M >= 0 && N >= 0 && K >= 0, "%s: negative size (batch=%lld M=%lld N=%lld K=%lld)", name,
          (long long)batch, (long long)M, (long long)N, (long long)K);
  REQUIRE(b_is_nt == 0 || b_is_nt == 1, "%s: b_is_nt must be 0 or 1", name);
  REQUIRE(epilogue >= HXMI_EPI_NONE && epilogue <= HXMI_EPI_BIAS_GELU_TANH, "%s: unknown epilogue %d", name,
          epilogue);
  const int64_t nout = epilogue == HXMI_EPI_SILU_MUL ? N / 2 : N;
  if (batch == 0 || M == 0 || nout == 0) return ok();
  REQUIRE(epilogue != HXMI_EPI_SILU_MUL || N % 32 == 0, "%s: SiLU-mul needs N %% 32 == 0 (packed gate/up), got %lld",
          name, (long long)N);
  REQUIRE(C && ((A && B) || K == 0), "%s: null operand pointer", name);
  REQUIRE(bias || (epilogue != HXMI_EPI_BIAS && epilogue != HXMI_EPI_BIAS_GELU_TANH),
          "%s: epilogue %d needs a bias pointer", name, epilogue);
  REQUIRE(lda >= K && ldb >= (b_is_nt ? K : N) && ldc >= nout, "%s: leading dimension too small (lda=%lld ldb=%lld ldc=%lld)",
          name, (long long)lda, (long long)ldb, (long long)ldc);
  REQUIRE(sA >= 0 && sB >= 0 && sC >= 0, "%s: negative batch stride", name);
  hxmi::GemmProblem p{};
  p.A = A;
  p.B = B;
  p.C = C;
  p.bias = bias;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = ldc;
  p.sA = sA;
  p.sB = sB;
  p.sC = sC;
  p.batch = batch;
  p.alpha = alpha;
  p.dtype = dtype;
  p.b_nt = b_is_nt;
  p.epilogue = epilogue;
  p.out_f32 = out_f32;
  p.tile = -1;
  p.ws = ws_bytes > 0 ? ws : nullptr;
  p.ws_bytes = ws_bytes > 0 ? ws_bytes : 0;
  p.rms = rms;
  p.rms_eps = rms_eps;
  p.rs_out = rs_out;
  p.rs_in = rs_in;
  if (noalloc) {
    // the split-K partials go to this device's scratch array
    const int64_t need = hxmi::gemm_workspace_bytes(p);
    REQUIRE(need <= (int64_t)HXMI_NOALLOC_SCRATCH_BYTES,
            "%s: this shape's split-K partials need %lld bytes, more than the %lld-byte device scratch (call "
            "hxmi_gemm_f16 with a workspace instead)",
            name, (long long)need, (long long)HXMI_NOALLOC_SCRATCH_BYTES);
    if (need > 0) {
      void* s = nullptr;
      const hipError_t e = scratch_ptr(&s);
      if (e != hipSuccess) return from_hip(e, name);
      p.ws = s;
      p.ws_bytes = HXMI_NOALLOC_SCRATCH_BYTES;
    }
  }
  return from_hip(hxmi::launch_gemm(p, (hipStream_t)stream), name);
}

int row_common(bool rms, int dtype, const void* x, const void* g, void* y, int64_t rows, int64_t cols, int64_t ldx,
               int64_t ldy, float eps, float scale, void* stream, const char* name) {
  REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", name);
  if (rows == 0 || cols == 0) return ok();
  REQUIRE(x && y && (g || !rms), "%s: null pointer", name);
  REQUIRE(ldx >= cols && ldy >= cols, "%s: leading dimension smaller than cols", name);
  REQUIRE(cols < (1ll << 31), "%s: cols too large", name);
  hxmi::RowProblem p{};
  p.x = x;
  p.g = g;
  p.y = y;
  p.rows = rows;
  p.cols = cols;
  p.ldx = ldx;
  p.ldy = ldy;
  p.eps = eps;
  p.scale = scale;
  p.dtype = dtype;
  return from_hip(rms ? hxmi::launch_rmsnorm(p, (hipStream_t)stream) : hxmi::launch_softmax(p, (hipStream_t)stream),
                  name);
}

bool al(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" {

const char* hxmi_last_error(void) { return g_err; }

int hxmi_version(void) { return 200; }

int hxmi_set_tuning(const char* name, int64_t value, int64_t* previous) {
  const int k = hxmi::knob_index(name);
  REQUIRE(k >= 0, "hxmi_set_tuning: unknown knob %s", name ? name : "(null)");
  const int64_t prev = hxmi::set_knob_override(k, value);
  if (previous) *previous = prev;
  return ok();
}

int hxmi_gemm_f16(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                  int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha, void* workspace,
                  int64_t workspace_bytes, void* stream) {
  return gemm_common(hxmi::DT_F16, A, B, C, bias, 1, M, N, K, lda, ldb, ldc, 0, 0, 0, b_is_nt, epilogue, alpha, 0,
                     workspace, workspace_bytes, stream, "hxmi_gemm_f16");
}

int hxmi_gemm_bf16(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  return gemm_common(hxmi::DT_BF16, A, B, C, bias, 1, M, N, K, lda, ldb, ldc, 0, 0, 0, b_is_nt, epilogue, alpha, 0,
                     workspace, workspace_bytes, stream, "hxmi_gemm_bf16");
}

int hxmi_gemm_f16_noalloc(const void* A, const void* B, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                          int64_t lda, int64_t ldb, int64_t ldc, int b_is_nt, int epilogue, float alpha,
                          void* stream) {
  return gemm_common(hxmi::DT_F16, A, B, C, bias, 1, M, N, K, lda, ldb, ldc, 0, 0, 0, b_is_nt, epilogue, alpha, 0,
                     nullptr, 0, stream, "hxmi_gemm_f16_noalloc", 0, 0.f, nullptr, nullptr, true);
}

int64_t hxmi_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int b_is_nt, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  hxmi::GemmProblem p{};
  p.M = M;
  p.N = N;
  p.K = K;
  // a contiguous, 16-byte aligned stand-in: the split decision depends on
  // shapes only, the fast-path check needs some aligned address
  p.A = p.B = p.C = (void*)(uintptr_t)256;
  p.lda = K;
  p.ldb = b_is_nt ? K : N;
  p.ldc = epilogue == HXMI_EPI_SILU_MUL ? N / 2 : N;
  p.batch = 1;
  p.b_nt = b_is_nt;
  p.epilogue = epilogue;
  p.dtype = hxmi::DT_F16;
  p.tile = -1;
  return hxmi::gemm_workspace_bytes(p);
}

int hxmi_bgemm_f16(const void* A, const void* B, void* C, const void* bias, int64_t batch, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t strideA, int64_t strideB,
                   int64_t strideC, int b_is_nt, int epilogue, float alpha, void* stream) {
  return gemm_common(hxmi::DT_F16, A, B, C, bias, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC, b_is_nt,
                     epilogue, alpha, 0, nullptr, 0, stream, "hxmi_bgemm_f16");
}

int hxmi_bgemm_bf16(const void* A, const void* B, void* C, const void* bias, int64_t batch, int64_t M, int64_t N,
                    int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t strideA, int64_t strideB,
                    int64_t strideC, int b_is_nt, int epilogue, float alpha, void* stream) {
  return gemm_common(hxmi::DT_BF16, A, B, C, bias, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC, b_is_nt,
                     epilogue, alpha, 0, nullptr, 0, stream, "hxmi_bgemm_bf16");
}

namespace {
int gemv_common(int dtype, const char* name, const void* x, const void* W, const void* bias, void* y, int64_t M,
                int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, void* workspace,
                int64_t workspace_bytes, void* stream, int w_cached = 0) {
  REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", name);
  if (M == 0 || N == 0) return ok();
  REQUIRE(x && W && y, "%s: null pointer", name);
  REQUIRE(ldx >= K && ldw >= K && ldy >= N, "%s: leading dimension too small", name);
  const bool gemv_ok = M <= 16 && K % 8 == 0 && N % 4 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldy % 4 == 0 &&
                       al(x, 16) && al(W, 16) && al(y, 8) && (!bias || al(bias, 8)) && 64 * ldw * 2 < (1ll << 31) &&
                       16 * ldx * 2 < (1ll << 31);
  if (!gemv_ok)
    return gemm_common(dtype, x, W, y, bias, 1, M, N, K, ldx, ldw, ldy, 0, 0, 0, 1,
                       bias ? HXMI_EPI_BIAS : HXMI_EPI_NONE, 1.f, 0, nullptr, 0, stream, name);
  hxmi::GemvProblem p{};
  p.x = x;
  p.W = W;
  p.bias = bias;
  p.y = y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.w_int8 = 0;
  p.dtype = dtype;
  p.ws = workspace_bytes > 0 ? workspace : nullptr;
  p.ws_bytes = workspace_bytes > 0 ? workspace_bytes : 0;
  p.w_cached = w_cached;
  return from_hip(hxmi::launch_gemv(p, (hipStream_t)stream), name);
}
}  // namespace

int hxmi_gemv_f16(const void* x, const void* W, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                  int64_t ldx, int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemv_common(hxmi::DT_F16, "hxmi_gemv_f16", x, W, bias, y, M, N, K, ldx, ldw, ldy, workspace,
                     workspace_bytes, stream);
}

int hxmi_gemv_bf16(const void* x, const void* W, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                   int64_t ldx, int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemv_common(hxmi::DT_BF16, "hxmi_gemv_bf16", x, W, bias, y, M, N, K, ldx, ldw, ldy, workspace,
                     workspace_bytes, stream);
}

int64_t hxmi_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || M > 16 || N <= 0 || K <= 0 || K % 8 || N % 4) return 0;
  hxmi::GemvProblem g{};
  g.M = M;
  g.N = N;
  g.K = K;
  g.ldx = K;
  g.ldw = K;
  g.ldy = N;
  g.w_int8 = 0;
  return hxmi::gemv_workspace_bytes(g);
}

int hxmi_gemv_w8a16(const void* x, const int8_t* Wq, const void* scale, const void* bias, void* y, int64_t M,
                    int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  const char* name = "hxmi_gemv_w8a16";
  REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", name);
  if (M == 0 || N == 0) return ok();
  REQUIRE(x && Wq && scale && y, "%s: null pointer", name);
  REQUIRE(ldx >= K && ldw >= K && ldy >= N, "%s: leading dimension too small", name);
  REQUIRE(K % 16 == 0 && ldw % 16 == 0 && N % 4 == 0 && ldx % 8 == 0 && ldy % 8 == 0,
          "%s: needs K %% 16 == 0, ldw %% 16 == 0, N %% 4 == 0, ldx %% 8 == 0, ldy %% 8 == 0", name);
  REQUIRE(al(x, 16) && al(Wq, 16) && al(y, 16) && al(scale, 8) && (!bias || al(bias, 8)),
          "%s: x, Wq, y need 16-byte and scale/bias 8-byte alignment", name);
  REQUIRE(256 * ldw < (1ll << 31) && 256 * ldx * 2 < (1ll << 31), "%s: leading dimension too large", name);
  hxmi::GemvProblem p{};
  p.x = x;
  p.W = Wq;
  p.scale = scale;
  p.bias = bias;
  p.y = y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.w_int8 = 1;
  p.ws = workspace_bytes > 0 ? workspace : nullptr;
  p.ws_bytes = workspace_bytes > 0 ? workspace_bytes : 0;
  if (M <= 16) return from_hip(hxmi::launch_gemv(p, (hipStream_t)stream), name);
  REQUIRE(N % 8 == 0, "%s: M > 16 needs N %% 8 == 0", name);
  return from_hip(hxmi::launch_w8a16_gemm(p, workspace_bytes > 0 ? workspace : nullptr,
                                          workspace_bytes > 0 ? workspace_bytes : 0, (hipStream_t)stream),
                  name);
}

int64_t hxmi_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  hxmi::GemvProblem g{};
  g.M = M;
  g.N = N;
  g.K = K;
  g.ldx = K;
  g.ldw = K;
  g.ldy = N;
  g.x = g.W = g.y = (void*)(uintptr_t)256;
  g.w_int8 = 1;
  if (M <= 16) return K % 16 || N % 4 ? 0 : hxmi::gemv_workspace_bytes(g);
  return hxmi::gemm_workspace_bytes(hxmi::w8a16_as_gemm(g));
}

int hxmi_rmsnorm_f16(const void* x, const void* g, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                     float eps, void* stream) {
  return row_common(true, hxmi::DT_F16, x, g, y, rows, cols, ldx, ldy, eps, 1.f, stream, "hxmi_rmsnorm_f16");
}

int hxmi_rmsnorm_bf16(const void* x, const void* g, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                      float eps, void* stream) {
  return row_common(true, hxmi::DT_BF16, x, g, y, rows, cols, ldx, ldy, eps, 1.f, stream, "hxmi_rmsnorm_bf16");
}

int hxmi_softmax_f16(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float scale,
                     void* stream) {
  return row_common(false, hxmi::DT_F16, x, nullptr, y, rows, cols, ldx, ldy, 0.f, scale, stream, "hxmi_softmax_f16");
}

int hxmi_softmax_bf16(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float scale,
                      void* stream) {
  return row_common(false, hxmi::DT_BF16, x, nullptr, y, rows, cols, ldx, ldy, 0.f, scale, stream,
                    "hxmi_softmax_bf16");
}

namespace {
int softmax_masked_common(int dtype, const void* x, void* y, int64_t slices, int64_t s_q, int64_t s_kv, int64_t ldx,
                          int64_t stride_x, int64_t ldy, int64_t stride_y, const void* mask, int64_t ldm,
                          int64_t stride_m, int64_t mask_group, int causal, float scale, void* stream,
                          const char* name) {
  REQUIRE(slices >= 0 && s_q >= 0 && s_kv >= 0, "%s: negative size", name);
  if (slices == 0 || s_q == 0 || s_kv == 0) return ok();
  REQUIRE(x && y, "%s: null pointer", name);
  REQUIRE(ldx >= s_kv && ldy >= s_kv, "%s: row stride smaller than s_kv", name);
  REQUIRE(stride_x >= 0 && stride_y >= 0, "%s: negative slice stride", name);
  REQUIRE(slices == 1 || (stride_x >= s_q * ldx && stride_y >= s_q * ldy), "%s: slices overlap", name);
  REQUIRE(causal >= 0 && causal <= 2, "%s: causal must be 0, 1 or 2", name);
  REQUIRE(s_q < (1ll << 31) && s_kv < (1ll << 31), "%s: s_q or s_kv too large", name);
  if (mask) {
    REQUIRE(ldm >= s_kv && stride_m >= 0 && mask_group >= 1, "%s: bad mask strides or group", name);
    REQUIRE(al(mask, 2), "%s: mask must be 2-byte aligned", name);
  }
  hxmi::MaskedSoftmaxProblem p{};
  p.x = x;
  p.y = y;
  p.mask = mask;
  p.slices = slices;
  p.s_q = s_q;
  p.s_kv = s_kv;
  p.ldx = ldx;
  p.stride_x = stride_x;
  p.ldy = ldy;
  p.stride_y = stride_y;
  p.ldm = mask ? ldm : 0;
  p.stride_m = mask ? stride_m : 0;
  p.mask_group = mask ? mask_group : 1;
  p.causal = causal;
  p.scale = scale;
  p.dtype = dtype;
  return from_hip(hxmi::launch_softmax_masked(p, (hipStream_t)stream), name);
}
}  // namespace

int hxmi_softmax_masked_f16(const void* x, void* y, int64_t slices, int64_t s_q, int64_t s_kv, int64_t ldx,
                            int64_t stride_x, int64_t ldy, int64_t stride_y, const void* mask, int64_t ldm,
                            int64_t stride_m, int64_t mask_group, int causal, float scale, void* stream) {
  return softmax_masked_common(hxmi::DT_F16, x, y, slices, s_q, s_kv, ldx, stride_x, ldy, stride_y, mask, ldm,
                               stride_m, mask_group, causal, scale, stream, "hxmi_softmax_masked_f16");
}

int hxmi_softmax_masked_bf16(const void* x, void* y, int64_t slices, int64_t s_q, int64_t s_kv, int64_t ldx,
                             int64_t stride_x, int64_t ldy, int64_t stride_y, const void* mask, int64_t ldm,
                             int64_t stride_m, int64_t mask_group, int causal, float scale, void* stream) {
  return softmax_masked_common(hxmi::DT_BF16, x, y, slices, s_q, s_kv, ldx, stride_x, ldy, stride_y, mask, ldm,
                               stride_m, mask_group, causal, scale, stream, "hxmi_softmax_masked_bf16");
}

namespace {
int attention_common(const char* name, const void* q, const void* k, const void* v, void* o, int64_t bh,
                     int64_t s_q, int64_t s_kv, int64_t d, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                     int64_t stride_q, int64_t stride_k, int64_t stride_v, int64_t stride_o, int64_t kv_group,
                     const void* mask, int64_t ldm, int64_t stride_m, int64_t mask_group, int causal, float scale,
                     void* stream) {
  REQUIRE(bh >= 0 && s_q >= 0 && s_kv >= 0 && d >= 0, "%s: negative size", name);
  if (bh == 0 || s_q == 0) return ok();
  REQUIRE(s_kv > 0, "%s: softmax over zero keys", name);
  REQUIRE(d == 64 || d == 128, "%s: head dim %lld unsupported (64 or 128)", name, (long long)d);
  REQUIRE(q && k && v && o, "%s: null pointer", name);
  REQUIRE(scale > 0.f && scale < INFINITY, "%s: scale must be positive and finite", name);
  REQUIRE(kv_group >= 1 && bh % kv_group == 0, "%s: kv_group %lld must divide bh %lld", name, (long long)kv_group,
          (long long)bh);
  REQUIRE(causal >= 0 && causal <= 2, "%s: causal %d (0 none, 1 top-left, 2 bottom-right)", name, causal);
  REQUIRE(ldq >= d && ldk >= d && ldv >= d && ldo >= d, "%s: leading dimension smaller than head dim", name);
  REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 4 == 0 && stride_q % 8 == 0 && stride_k % 8 == 0 &&
              stride_v % 8 == 0 && stride_o % 4 == 0,
          "%s: strides must keep 16-byte aligned rows", name);
  REQUIRE(al(q, 16) && al(k, 16) && al(v, 16) && al(o, 8), "%s: q, k, v need 16-byte, o 8-byte alignment", name);
  REQUIRE(s_q < (1ll << 30) && s_kv < (1ll << 30), "%s: sequence too long", name);
  REQUIRE(((s_kv - 1) * ldk + d) * 2 <= (1ll << 31) && ((s_kv - 1) * ldv + d) * 2 <= (1ll << 31),
          "%s: one K or V slice must span at most 2 GiB", name);
  if (mask) {
    REQUIRE(ldm >= s_kv && stride_m >= 0, "%s: mask row stride %lld below s_kv", name, (long long)ldm);
    REQUIRE(mask_group >= 1 && bh % mask_group == 0, "%s: mask_group %lld must divide bh", name,
            (long long)mask_group);
    REQUIRE(al(mask, 2), "%s: mask needs 2-byte alignment", name);
  }
  hxmi::AttnProblem p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.mask = mask;
  p.bh = bh;
  p.s = s_q;
  p.skv = s_kv;
  p.d = d;
  p.ldq = ldq;
  p.ldk = ldk;
  p.ldv = ldv;
  p.ldo = ldo;
  p.ldm = ldm;
  p.sq = stride_q;
  p.sk = stride_k;
  p.sv = stride_v;
  p.so = stride_o;
  p.sm = stride_m;
  p.kv_group = kv_group;
  p.mask_group = mask ? mask_group : 1;
  p.causal = causal;
  p.scale = scale;
  return from_hip(hxmi::launch_attention(p, (hipStream_t)stream), name);
}
}  // namespace

int hxmi_attention_ex_f16(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t s_q,
                          int64_t s_kv, int64_t d, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                          int64_t stride_q, int64_t stride_k, int64_t stride_v, int64_t stride_o, int64_t kv_group,
                          const void* mask, int64_t ldm, int64_t stride_m, int64_t mask_group, int causal,
                          float scale, void* stream) {
  return attention_common("hxmi_attention_ex_f16", q, k, v, o, bh, s_q, s_kv, d, ldq, ldk, ldv, ldo, stride_q,
                          stride_k, stride_v, stride_o, kv_group, mask, ldm, stride_m, mask_group, causal, scale,
                          stream);
}

int hxmi_attention_f16(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t s_q, int64_t s_kv,
                       int64_t d, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, int64_t stride_q,
                       int64_t stride_k, int64_t stride_v, int64_t stride_o, float scale, void* stream) {
  return attention_common("hxmi_attention_f16", q, k, v, o, bh, s_q, s_kv, d, ldq, ldk, ldv, ldo, stride_q, stride_k,
                          stride_v, stride_o, 1, nullptr, 0, 0, 1, 0, scale, stream);
}

namespace {
int rms_linear_common(int dtype, const char* name, const void* x, const void* Wg, void* C, const void* bias, int64_t M,
                      int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int epilogue, float eps,
                      float* rscale_out, const float* rscale_in, void* stream) {
  REQUIRE(epilogue == HXMI_EPI_NONE || epilogue == HXMI_EPI_BIAS || epilogue == HXMI_EPI_SILU_MUL,
          "%s: epilogue %d unsupported (none, bias or silu_mul)", name, epilogue);
  REQUIRE(K > 0 || M <= 0 || N <= 0, "%s: RMSNorm over zero columns", name);
  REQUIRE(eps >= 0.f, "%s: negative eps", name);
  REQUIRE(!(rscale_out && rscale_in), "%s: rscale_out and rscale_in are exclusive", name);
  if (rscale_in)  // statistics given: a plain GEMM with a row scale before the epilogue
    return gemm_common(dtype, x, Wg, C, bias, 1, M, N, K, ldx, ldw, ldc, 0, 0, 0, 1, epilogue, 1.f, 0, nullptr, 0,
                       stream, name, 0, 0.f, nullptr, rscale_in);
  return gemm_common(dtype, x, Wg, C, bias, 1, M, N, K, ldx, ldw, ldc, 0, 0, 0, 1, epilogue, 1.f, 0, nullptr, 0,
                     stream, name, 1, eps, rscale_out, nullptr);
}

int fold_common(int dtype, const char* name, const void* W, const void* g, void* Wg, int64_t N, int64_t K,
                int64_t ldw, int64_t ldwg, void* stream) {
  REQUIRE(N >= 0 && K >= 0, "%s: negative size", name);
  if (N == 0 || K == 0) return ok();
  REQUIRE(W && g && Wg, "%s: null pointer", name);
  REQUIRE(ldw >= K && ldwg >= K, "%s: leading dimension smaller than K", name);
  return from_hip(hxmi::launch_fold_rms_weight(dtype, W, g, Wg, N, K, ldw, ldwg, (hipStream_t)stream), name);
}
}  // namespace

int hxmi_rmsnorm_linear_f16(const void* x, const void* Wg, void* C, const void* bias, int64_t M, int64_t N, int64_t K,
                            int64_t ldx, int64_t ldw, int64_t ldc, int epilogue, float eps, float* rscale_out,
                            const float* rscale_in, void* stream) {
  return rms_linear_common(hxmi::DT_F16, "hxmi_rmsnorm_linear_f16", x, Wg, C, bias, M, N, K, ldx, ldw, ldc, epilogue,
                           eps, rscale_out, rscale_in, stream);
}

int hxmi_rmsnorm_linear_bf16(const void* x, const void* Wg, void* C, const void* bias, int64_t M, int64_t N,
                             int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int epilogue, float eps,
                             float* rscale_out, const float* rscale_in, void* stream) {
  return rms_linear_common(hxmi::DT_BF16, "hxmi_rmsnorm_linear_bf16", x, Wg, C, bias, M, N, K, ldx, ldw, ldc,
                           epilogue, eps, rscale_out, rscale_in, stream);
}

int hxmi_fold_rmsnorm_weight_f16(const void* W, const void* g, void* Wg, int64_t N, int64_t K, int64_t ldw,
                                 int64_t ldwg, void* stream) {
  return fold_common(hxmi::DT_F16, "hxmi_fold_rmsnorm_weight_f16", W, g, Wg, N, K, ldw, ldwg, stream);
}

int hxmi_fold_rmsnorm_weight_bf16(const void* W, const void* g, void* Wg, int64_t N, int64_t K, int64_t ldw,
                                  int64_t ldwg, void* stream) {
  return fold_common(hxmi::DT_BF16, "hxmi_fold_rmsnorm_weight_bf16", W, g, Wg, N, K, ldw, ldwg, stream);
}

int hxmi_quantize_int8_rows_f16(const void* W, int8_t* q, void* s, int64_t N, int64_t K, int64_t ldw, int64_t ldq,
                                void* stream) {
  const char* name = "hxmi_quantize_int8_rows_f16";
  REQUIRE(N >= 0 && K >= 0, "%s: negative size", name);
  if (N == 0 || K == 0) return ok();
  REQUIRE(W && q && s, "%s: null pointer", name);
  REQUIRE(ldw >= K && ldq >= K, "%s: leading dimension smaller than K", name);
  REQUIRE(K % 8 == 0 && ldw % 8 == 0 && ldq % 8 == 0, "%s: K, ldw and ldq must be multiples of 8", name);
  REQUIRE((uintptr_t)W % 16 == 0 && (uintptr_t)q % 8 == 0 && (uintptr_t)s % 2 == 0,
          "%s: W must be 16-byte, q 8-byte aligned", name);
  return from_hip(hxmi::launch_quantize_int8_rows(W, q, s, N, K, ldw, ldq, (hipStream_t)stream), name);
}

int64_t hxmi_decode_workspace_bytes(int64_t hidden, int64_t kv_dim, int64_t intermediate) {
  if (hidden <= 0 || kv_dim <= 0 || intermediate <= 0) return 0;
  return hxmi::decode_workspace_bytes(hidden, kv_dim, intermediate);
}

// The decode step with the o projection as w_o (w_ov null) or folded onto
// the normalised input as w_ov, b_ov.
static int decode_common(const char* name, const void* x, const void* w_qkv, const void* b_qkv, const void* w_o,
                         const void* w_ov, const void* b_ov, const void* w_gu, const void* w_down, const void* g_attn,
                         const void* g_mlp, const void* g_final, const void* w_lm, void* qkv_out, void* x_out,
                         void* h_out, void* logits, int64_t layers, int64_t hidden, int64_t heads, int64_t kv_heads,
                         int64_t head_dim, int64_t intermediate, int64_t vocab, float eps, int64_t timeout_us,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  REQUIRE(layers > 0 && hidden > 0 && heads > 0 && kv_heads > 0 && head_dim > 0 && intermediate > 0,
          "%s: sizes must be positive", name);
  REQUIRE(layers <= 4096, "%s: at most 4096 layers, got %lld", name, (long long)layers);
  REQUIRE(x && w_qkv && (w_o || w_ov) && w_gu && w_down && g_attn && g_mlp && g_final && h_out && workspace,
          "%s: null pointer", name);
  REQUIRE(!b_ov || al(b_ov, 2), "%s: b_ov must be 2-byte aligned", name);
  REQUIRE(!w_lm || (logits && vocab > 0), "%s: w_lm needs logits and vocab > 0", name);
  REQUIRE(eps >= 0.f, "%s: eps must be >= 0", name);
  const int64_t kv_dim = kv_heads * head_dim;
  REQUIRE(workspace_bytes >= hxmi::decode_workspace_bytes(hidden, kv_dim, intermediate),
          "%s: workspace of %lld bytes, needs hxmi_decode_workspace_bytes() = %lld", name,
          (long long)workspace_bytes, (long long)hxmi::decode_workspace_bytes(hidden, kv_dim, intermediate));
  REQUIRE(al(workspace, 256), "%s: workspace must be 256-byte aligned", name);
  if (!hxmi::decode_shape_ok(hidden, heads, kv_heads, head_dim, intermediate))
    return fail(HXMI_ERR_UNSUPPORTED,
                "%s: unsupported shape (hidden %lld, heads %lld, kv_heads %lld, head_dim %lld, intermediate %lld)",
                name, (long long)hidden, (long long)heads, (long long)kv_heads, (long long)head_dim,
                (long long)intermediate);
  for (const void* p : {x, w_qkv, w_o ? w_o : w_ov, w_gu, w_down, g_attn, g_mlp, g_final, (const void*)h_out})
    REQUIRE(al(p, 16), "%s: x, weights and outputs must be 16-byte aligned", name);
  REQUIRE(!x_out || al(x_out, 16), "%s: x_out must be 16-byte aligned", name);
  REQUIRE(!qkv_out || al(qkv_out, 2), "%s: qkv_out must be 2-byte aligned", name);
  hxmi::DecodeProblem p{};
  p.x = x;
  p.w_qkv = w_qkv;
  p.b_qkv = b_qkv;
  p.w_o = w_o;
  p.w_ov = w_ov;
  p.b_ov = b_ov;
  p.w_gu = w_gu;
  p.w_down = w_down;
  p.g_attn = g_attn;
  p.g_mlp = g_mlp;
  p.g_final = g_final;
  p.qkv_out = qkv_out;
  p.x_out = x_out;
  p.h_out = h_out;
  p.ws = (uint32_t*)workspace;
  p.L = layers;
  p.H = hidden;
  p.heads = heads;
  p.kv_heads = kv_heads;
  p.head_dim = head_dim;
  p.I = intermediate;
  p.eps = eps;
  p.timeout_us = timeout_us;
  const hipError_t e = hxmi::launch_decode_step(p, (hipStream_t)stream);
  if (e != hipSuccess) return from_hip(e, name);
  if (!w_lm) return ok();
  // the lm_head after the non-temporal layer-weight stream: its own weight
  // loads with the ordinary cache policy (Qwen2.5-0.5B folded forward
  // 449.3-449.5 -> 447.7-448.2 us; the same loads were 3 us slower after a
  // layer stream with the ordinary policy)
  return gemv_common(hxmi::DT_F16, name, h_out, w_lm, nullptr, logits, 1, vocab, hidden, hidden, hidden, vocab,
                     nullptr, 0, stream, 1);
}

int hxmi_decode_step_f16(const void* x, const void* w_qkv, const void* b_qkv, const void* w_o, const void* w_gu,
                         const void* w_down, const void* g_attn, const void* g_mlp, const void* g_final,
                         const void* w_lm, void* qkv_out, void* x_out, void* h_out, void* logits, int64_t layers,
                         int64_t hidden, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t intermediate,
                         int64_t vocab, float eps, int64_t timeout_us, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  REQUIRE(w_o, "hxmi_decode_step_f16: null pointer");
  return decode_common("hxmi_decode_step_f16", x, w_qkv, b_qkv, w_o, nullptr, nullptr, w_gu, w_down, g_attn, g_mlp,
                       g_final, w_lm, qkv_out, x_out, h_out, logits, layers, hidden, heads, kv_heads, head_dim,
                       intermediate, vocab, eps, timeout_us, workspace, workspace_bytes, stream);
}

int hxmi_decode_step_ov_f16(const void* x, const void* w_qkv, const void* b_qkv, const void* w_ov, const void* b_ov,
                            const void* w_gu, const void* w_down, const void* g_attn, const void* g_mlp,
                            const void* g_final, const void* w_lm, void* qkv_out, void* x_out, void* h_out,
                            void* logits, int64_t layers, int64_t hidden, int64_t heads, int64_t kv_heads,
                            int64_t head_dim, int64_t intermediate, int64_t vocab, float eps, int64_t timeout_us,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  REQUIRE(w_ov, "hxmi_decode_step_ov_f16: null pointer");
  return decode_common("hxmi_decode_step_ov_f16", x, w_qkv, b_qkv, nullptr, w_ov, b_ov, w_gu, w_down, g_attn, g_mlp,
                       g_final, w_lm, qkv_out, x_out, h_out, logits, layers, hidden, heads, kv_heads, head_dim,
                       intermediate, vocab, eps, timeout_us, workspace, workspace_bytes, stream);
}

int hxmi_decode_status(void* workspace, int clear, int* status, void* stream) {
  REQUIRE(workspace && status, "hxmi_decode_status: null pointer");
  uint32_t word = 0;
  const uint32_t* err = (const uint32_t*)workspace + hxmi::DECODE_WS_ERROR_WORD;
  hipError_t e = hipMemcpyAsync(&word, err, sizeof(word), hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e == hipSuccess && clear && word) {
    static const uint32_t zero = 0;
    e = hipMemcpyAsync((uint32_t*)err, &zero, sizeof(zero), hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  }
  *status = (int)word;
  return from_hip(e, "hxmi_decode_status");
}

int hxmi_lwp_record(uint32_t* records, int64_t slot, uint32_t id, void* stream) {
  const char* name = "hxmi_lwp_record";
  REQUIRE(records, "%s: null record buffer", name);
  REQUIRE(slot >= 0, "%s: negative slot", name);
  REQUIRE((uintptr_t)records % 4 == 0, "%s: record buffer must be 4-byte aligned", name);
  return from_hip(hxmi::launch_lwp_mark(records, slot, id, (hipStream_t)stream), name);
}

int64_t hxmi_lwp_clock_hz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return 0;
  return (int64_t)khz * 1000;
}

int hexkl_matmul_f16f16_f32(int64_t n_row, int64_t n_col, int64_t n_inner, float* outM, const hxmi_f16_t* inAct,
                            const hxmi_f16_t* inW) {
  const int rc = gemm_common(hxmi::DT_F16, inAct, inW, outM, nullptr, 1, n_row, n_col, n_inner, n_inner, n_col, n_col,
                             0, 0, 0, 0, HXMI_EPI_NONE, 1.f, 1, nullptr, 0, nullptr, "hexkl_matmul_f16f16_f32");
  if (rc != HXMI_OK) return rc;
  return from_hip(hipStreamSynchronize(nullptr), "hexkl_matmul_f16f16_f32");
}

}  // extern "C"
