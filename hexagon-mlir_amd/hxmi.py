"""ctypes binding of libhxmi.so and the torch-tensor ops built on it.

PyTorch-ROCm supplies device memory and the current HIP stream; every
computation runs in the hand-written HIP kernels of ``csrc/``.  There is no
fallback: if the library is missing, or a tensor is not on the GPU, the call
raises.
"""
from __future__ import annotations

import collections
import dataclasses
import contextlib
import ctypes
import pathlib
from typing import Optional

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libhxmi.so"

EPILOGUES = {
    None: 0,
    "none": 0,
    "bias": 1,
    "silu_mul": 2,
    "gelu_tanh": 3,
    "bias_gelu_tanh": 4,
}

# Every symbol include/hxmi.h declares, with its ctypes signature.
_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_F = ctypes.c_float
_I = ctypes.c_int
SIGNATURES = {
    "hxmi_last_error": ([], ctypes.c_char_p),
    "hxmi_version": ([], _I),
    "hxmi_set_tuning": ([ctypes.c_char_p, _I64, ctypes.POINTER(_I64)], _I),
    "hxmi_gemm_f16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _F, _P, _I64, _P], _I),
    "hxmi_gemm_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _F, _P, _I64, _P], _I),
    "hxmi_gemm_workspace_bytes": ([_I64, _I64, _I64, _I, _I], _I64),
    "hxmi_gemm_f16_noalloc": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _F, _P], _I),
    "hxmi_bgemm_f16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _F, _P], _I),
    "hxmi_bgemm_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _F, _P], _I),
    "hxmi_gemv_f16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "hxmi_gemv_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "hxmi_gemv_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "hxmi_gemv_w8a16": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "hxmi_w8a16_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "hxmi_rmsnorm_f16": ([_P, _P, _P, _I64, _I64, _I64, _I64, _F, _P], _I),
    "hxmi_rmsnorm_bf16": ([_P, _P, _P, _I64, _I64, _I64, _I64, _F, _P], _I),
    "hxmi_softmax_f16": ([_P, _P, _I64, _I64, _I64, _I64, _F, _P], _I),
    "hxmi_softmax_bf16": ([_P, _P, _I64, _I64, _I64, _I64, _F, _P], _I),
    "hxmi_softmax_masked_f16": ([_P, _P] + [_I64] * 7 + [_P, _I64, _I64, _I64, _I, _F, _P], _I),
    "hxmi_softmax_masked_bf16": ([_P, _P] + [_I64] * 7 + [_P, _I64, _I64, _I64, _I, _F, _P], _I),
    "hxmi_attention_f16": ([_P, _P, _P, _P] + [_I64] * 12 + [_F, _P], _I),
    "hxmi_attention_ex_f16": ([_P, _P, _P, _P] + [_I64] * 13 + [_P, _I64, _I64, _I64, _I, _F, _P], _I),
    "hxmi_rmsnorm_linear_f16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _F, _P, _P, _P], _I),
    "hxmi_rmsnorm_linear_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _F, _P, _P, _P], _I),
    "hxmi_fold_rmsnorm_weight_f16": ([_P, _P, _P, _I64, _I64, _I64, _I64, _P], _I),
    "hxmi_fold_rmsnorm_weight_bf16": ([_P, _P, _P, _I64, _I64, _I64, _I64, _P], _I),
    "hxmi_quantize_int8_rows_f16": ([_P, _P, _P, _I64, _I64, _I64, _I64, _P], _I),
    "hxmi_decode_step_f16": ([_P] * 14 + [_I64] * 7 + [_F, _I64, _P, _I64, _P], _I),
    "hxmi_decode_step_ov_f16": ([_P] * 15 + [_I64] * 7 + [_F, _I64, _P, _I64, _P], _I),
    "hxmi_decode_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "hxmi_decode_status": ([_P, _I, ctypes.POINTER(_I), _P], _I),
    "hxmi_lwp_record": ([_P, _I64, ctypes.c_uint32, _P], _I),
    "hxmi_lwp_clock_hz": ([], _I64),
    "hexkl_matmul_f16f16_f32": ([_I64, _I64, _I64, _P, _P, _P], _I),
}


class HxmiError(RuntimeError):
    """A kernel call was rejected or failed."""


class HxmiNotBuiltError(HxmiError):
    """libhxmi.so has not been built (run hexagon-mlir_amd/build.py)."""


_lib: Optional[ctypes.CDLL] = None


def load_library() -> ctypes.CDLL:
    """Load libhxmi.so (once) and bind the signatures of every entry point."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HxmiNotBuiltError(f"{LIB_PATH} is missing; build it with hexagon-mlir_amd/build.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        msg = load_library().hxmi_last_error().decode(errors="replace")
        raise HxmiError(f"hxmi error {rc}: {msg}")


TUNING_KNOBS = ("gemm_tile", "group_m", "splitk", "w8_tile", "gemv_path", "gemv_tpb", "gemv_ks", "gemv_kg",
                "gemv_unr", "gemv_pair_wg", "attn_cfg")


def set_tuning(name: str, value) -> Optional[int]:
    """Set (or with None clear) this thread's override of a launch-shape knob;
    returns the previous override (None if there was none).  gemv_path also
    takes a kernel name, read by its first letter as HXMI_GEMV_PATH is:
    "valu", "pair", "ksplit" (whole-line pairs, K split), else the 16-row
    MFMA kernel."""
    if isinstance(value, str):
        value = {"v": 1, "p": 2, "k": 3}.get(value[:1], 0) if name == "gemv_path" else int(value)
    prev = ctypes.c_int64(-1)
    _check(load_library().hxmi_set_tuning(name.encode(), -1 if value is None else int(value), ctypes.byref(prev)))
    return None if prev.value < 0 else prev.value


@contextlib.contextmanager
def tuning(**knobs):
    """Launch-shape overrides for the calls made inside the block on this
    thread, restored afterwards, e.g. ``with tuning(gemm_tile=3): ...``."""
    saved = {}
    try:
        for name, value in knobs.items():
            saved[name] = set_tuning(name, value)
        yield
    finally:
        for name, prev in saved.items():
            set_tuning(name, prev)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """Handle of torch's current HIP stream on t's device (where it launches)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(*ts: Optional[torch.Tensor]) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise HxmiError("hxmi ops take GPU tensors; got a tensor on " + str(t.device))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise HxmiError(f"tensors on different devices: {dev} and {t.device}")


def _rowmajor(t: torch.Tensor, name: str) -> int:
    """Leading dimension of a 2-D view with unit stride in the last dim."""
    if t.dim() != 2:
        raise HxmiError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.size(1) > 1:
        raise HxmiError(f"{name} must have unit stride in its last dimension")
    return max(t.stride(0), t.size(1), 1)


def _vec(t: Optional[torch.Tensor], n: int, dtype: torch.dtype, name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.dtype != dtype or t.dim() != 1 or t.numel() != n:
        raise HxmiError(f"{name} must be a 1-D {dtype} tensor of {n} elements")
    return t.contiguous()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_WS_CACHE: "collections.OrderedDict[tuple, torch.Tensor]" = collections.OrderedDict()
_WS_KEEP = 16  # workspaces kept (one per device and stream or capture, least recently used dropped)
# Counter head of a split-K workspace (kWsCounterBytes in csrc/hxmi_internal.h):
# the only part that must be zero when a call starts.
_WS_COUNTER_BYTES = 16 * 1024

_hip_rt: Optional[ctypes.CDLL] = None


def _hip_runtime() -> Optional[ctypes.CDLL]:
    """The HIP runtime torch has loaded (for hipStreamGetCaptureInfo), or None."""
    global _hip_rt
    if _hip_rt is None:
        for cand in (pathlib.Path(torch.__file__).parent / "lib" / "libamdhip64.so", "libamdhip64.so"):
            try:
                rt = ctypes.CDLL(str(cand))
            except OSError:
                continue
            fn = rt.hipStreamGetCaptureInfo
            fn.argtypes = [_P, ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_ulonglong)]
            fn.restype = _I
            _hip_rt = rt
            break
    return _hip_rt


def _capture_key(device: torch.device) -> Optional[tuple]:
    """None when the current stream of `device` is not capturing a HIP graph;
    else a key unique to the capture under way (its capture id), or a fresh
    object when the id cannot be read (nothing is then shared between calls)."""
    if not torch.cuda.is_current_stream_capturing():
        return None
    rt = _hip_runtime()
    if rt is not None:
        status, cid = _I(0), ctypes.c_ulonglong(0)
        stream = torch.cuda.current_stream(device).cuda_stream
        if rt.hipStreamGetCaptureInfo(stream, ctypes.byref(status), ctypes.byref(cid)) == 0 and status.value == 1:
            return ("capture", cid.value)
    return ("capture", object())


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _workspace(nbytes: int, device: torch.device) -> Optional[torch.Tensor]:
    """Split-K scratch for the calls launched on the current stream of `device`.

    The C ABI wants the arrival counters at the workspace's head zero when a
    call starts and leaves them zero afterwards, so one buffer whose counters
    were cleared before its first call serves every later call in the same
    stream order.  Eager calls share one buffer per (device, stream),
    replaced by a larger one when a call needs more; allocated on that
    stream, a dropped buffer is handed out again by torch's caching allocator
    only in that stream's order.

    Inside a HIP graph capture nothing is run, only recorded, so the clearing
    fill of a buffer belongs to the graph that captured it.  Each capture
    therefore gets buffers of its own (keyed by its capture id, from the
    graph's memory pool), cleared by a fill node recorded before their first
    use: every replay of that graph clears them again, and no other graph or
    eager call ever sees them.  Two graphs replayed concurrently thus never
    share counters, whatever order they are captured or replayed in."""
    if nbytes <= 0:
        return None
    cap = _capture_key(device)
    stream = (_raw_stream(device.index) if _raw_stream is not None
              else torch.cuda.current_stream(device).cuda_stream)
    key = (_device_index(device), stream if cap is None else cap)
    ws = _WS_CACHE.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        ws = torch.empty((nbytes + 15) // 16 * 4, dtype=torch.float32, device=device)
        # a fill kernel (recorded as a kernel node under capture), counters only
        ws[: min(ws.numel(), _WS_COUNTER_BYTES // 4)].zero_()
        _WS_CACHE[key] = ws
    _WS_CACHE.move_to_end(key)
    while len(_WS_CACHE) > _WS_KEEP:
        _WS_CACHE.popitem(last=False)
    return ws


def gemm(
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    b_layout: str = "nn",
    epilogue: Optional[str] = None,
    bias: Optional[torch.Tensor] = None,
    alpha: float = 1.0,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """C = epilogue(alpha * a @ op(b)).  b_layout "nn": b is [K,N]; "nt": b is [N,K].

    For epilogue "silu_mul", b holds packed gate/up columns (see pack_gate_up)
    and the result has N/2 columns.
    """
    _require_gpu(a, b, bias, out)
    if a.dtype not in (torch.float16, torch.bfloat16) or b.dtype != a.dtype:
        raise HxmiError(f"gemm takes fp16 or bf16 operands of one dtype, got {a.dtype} and {b.dtype}")
    if b_layout not in ("nn", "nt"):
        raise HxmiError(f"b_layout must be 'nn' or 'nt', got {b_layout!r}")
    if epilogue not in EPILOGUES:
        raise HxmiError(f"unknown epilogue {epilogue!r}")
    lda, ldb = _rowmajor(a, "a"), _rowmajor(b, "b")
    M, K = a.shape
    nt = b_layout == "nt"
    N = b.shape[0] if nt else b.shape[1]
    if (b.shape[1] if nt else b.shape[0]) != K:
        raise HxmiError(f"inner dimensions differ: a {tuple(a.shape)}, b {tuple(b.shape)} ({b_layout})")
    nout = N // 2 if epilogue == "silu_mul" else N
    if epilogue in ("bias", "bias_gelu_tanh"):
        bias = _vec(bias, N, a.dtype, "bias")
        if bias is None:
            raise HxmiError(f"epilogue {epilogue} needs a bias")
    else:
        bias = None
    if out is None:
        out = torch.empty((M, nout), dtype=a.dtype, device=a.device)
    elif out.shape != (M, nout) or out.dtype != a.dtype:
        raise HxmiError(f"out must be {a.dtype} {(M, nout)}")
    ldc = _rowmajor(out, "out")
    lib = load_library()
    ws = _workspace(lib.hxmi_gemm_workspace_bytes(M, N, K, int(nt), EPILOGUES[epilogue]), a.device)
    fn = lib.hxmi_gemm_f16 if a.dtype == torch.float16 else lib.hxmi_gemm_bf16
    _check(fn(a.data_ptr(), b.data_ptr(), out.data_ptr(), _ptr(bias), M, N, K, lda, ldb, ldc, int(nt),
              EPILOGUES[epilogue], float(alpha), _ptr(ws), 0 if ws is None else ws.numel() * 4, _stream(a)))
    return out


def _batched(t: torch.Tensor, name: str) -> tuple[int, int]:
    if t.dim() != 3:
        raise HxmiError(f"{name} must be 3-D, got shape {tuple(t.shape)}")
    if t.stride(2) != 1 and t.size(2) > 1:
        raise HxmiError(f"{name} must have unit stride in its last dimension")
    return max(t.stride(1), t.size(2), 1), t.stride(0)


def bgemm(
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    b_layout: str = "nn",
    epilogue: Optional[str] = None,
    bias: Optional[torch.Tensor] = None,
    alpha: float = 1.0,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Batched C[i] = epilogue(alpha * a[i] @ op(b[i])) over 3-D strided tensors."""
    _require_gpu(a, b, bias, out)
    if a.dtype not in (torch.float16, torch.bfloat16) or b.dtype != a.dtype:
        raise HxmiError("bgemm takes fp16 or bf16 operands of one dtype")
    if epilogue not in EPILOGUES:
        raise HxmiError(f"unknown epilogue {epilogue!r}")
    lda, sa = _batched(a, "a")
    ldb, sb = _batched(b, "b")
    batch, M, K = a.shape
    nt = b_layout == "nt"
    N = b.shape[1] if nt else b.shape[2]
    if b.shape[0] != batch or (b.shape[2] if nt else b.shape[1]) != K:
        raise HxmiError(f"shapes do not match: a {tuple(a.shape)}, b {tuple(b.shape)} ({b_layout})")
    nout = N // 2 if epilogue == "silu_mul" else N
    if epilogue in ("bias", "bias_gelu_tanh"):
        bias = _vec(bias, N, a.dtype, "bias")
        if bias is None:
            raise HxmiError(f"epilogue {epilogue} needs a bias")
    else:
        bias = None
    if out is None:
        out = torch.empty((batch, M, nout), dtype=a.dtype, device=a.device)
    ldc, sc = _batched(out, "out")
    fn = load_library().hxmi_bgemm_f16 if a.dtype == torch.float16 else load_library().hxmi_bgemm_bf16
    _check(fn(a.data_ptr(), b.data_ptr(), out.data_ptr(), _ptr(bias), batch, M, N, K, lda, ldb, ldc, sa, sb, sc,
              int(nt), EPILOGUES[epilogue], float(alpha), _stream(a)))
    return out


def linear(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
           epilogue: Optional[str] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """nn.Linear forward, y = x @ w.T (+ bias), with an optional fused activation.

    epilogue: None, "gelu_tanh" or "silu_mul" (w then packed by pack_gate_up).
    out: optional 2-D destination [rows of x, output features].
    """
    if epilogue is None:
        epi = "bias" if bias is not None else None
    elif epilogue == "gelu_tanh":
        epi = "bias_gelu_tanh" if bias is not None else "gelu_tanh"
    elif epilogue == "silu_mul":
        if bias is not None:
            raise HxmiError("silu_mul epilogue takes no bias")
        epi = "silu_mul"
    else:
        raise HxmiError(f"unknown activation {epilogue!r}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    y = gemm(x2, w, b_layout="nt", epilogue=epi, bias=bias, out=out)
    return y if out is not None else y.reshape(*lead, y.shape[-1])


def fold_rms_weight(w: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """w [N,K] with the RMSNorm weight g [K] folded in: T(w[n,k] * g[k]) (T = fp16 or bf16), the
    weight rms_norm_linear takes (fold a packed gate/up weight after packing)."""
    _require_gpu(w, g)
    if w.dtype not in (torch.float16, torch.bfloat16) or g.dtype != w.dtype:
        raise HxmiError("fold_rms_weight takes fp16 or bf16 tensors of one dtype")
    if w.dim() != 2:
        raise HxmiError("fold_rms_weight takes a 2-D weight")
    N, K = w.shape
    ldw = _rowmajor(w, "w")
    g = _vec(g, K, w.dtype, "g")
    out = torch.empty((N, K), dtype=w.dtype, device=w.device)
    lib = load_library()
    fn = lib.hxmi_fold_rmsnorm_weight_f16 if w.dtype == torch.float16 else lib.hxmi_fold_rmsnorm_weight_bf16
    _check(fn(w.data_ptr(), g.data_ptr(), out.data_ptr(), N, K, ldw, K, _stream(w)))
    return out


def quantize_int8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 codes of an fp16 weight [N, K]:
    returns (q [N, K] int8, s [N] fp16) with s[n] the smallest fp16 step at or
    above max|w[n]| / 127 and q = rint(w / s), so |w - q * s| <= s / 2; the
    layout w8a16_linear takes.  K must be a multiple of 8."""
    _require_gpu(w)
    if w.dtype != torch.float16 or w.dim() != 2:
        raise HxmiError("quantize_int8 takes a 2-D fp16 weight")
    N, K = w.shape
    ldw = _rowmajor(w, "w")
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float16, device=w.device)
    _check(load_library().hxmi_quantize_int8_rows_f16(w.data_ptr(), q.data_ptr(), s.data_ptr(), N, K, ldw, K,
                                                      _stream(w)))
    return q, s


def rms_norm_linear(x: torch.Tensor, w_folded: torch.Tensor, eps: float = 1e-5, epilogue: Optional[str] = None,
                    out: Optional[torch.Tensor] = None, rscale_out: Optional[torch.Tensor] = None,
                    rscale_in: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """linear(rms_norm(x, g, eps), w, bias) in one GEMM, with w_folded = fold_rms_weight(w, g);
    epilogue None or "silu_mul" (w packed by pack_gate_up before folding; no bias).

    rscale_out (fp32, one per row of x) also receives the row scales
    rsqrt(mean(x^2) + eps); a later call on the same x can pass them as
    rscale_in and skip the statistics (eps is then ignored)."""
    _require_gpu(x, w_folded, out, rscale_out, rscale_in, bias)
    if rscale_out is not None and rscale_in is not None:
        raise HxmiError("rscale_out and rscale_in are exclusive")
    if rscale_out is not None and not rscale_out.is_contiguous():
        raise HxmiError("rscale_out must be contiguous")
    if x.dtype not in (torch.float16, torch.bfloat16) or w_folded.dtype != x.dtype:
        raise HxmiError("rms_norm_linear takes fp16 or bf16 tensors of one dtype")
    if epilogue not in (None, "silu_mul"):
        raise HxmiError(f"rms_norm_linear epilogue must be None or 'silu_mul', got {epilogue!r}")
    if bias is not None and epilogue is not None:
        raise HxmiError("rms_norm_linear takes a bias only without an epilogue")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    N = w_folded.shape[0]
    if w_folded.dim() != 2 or w_folded.shape[1] != K:
        raise HxmiError(f"weight {tuple(w_folded.shape)} does not match x {tuple(x.shape)}")
    nout = N // 2 if epilogue == "silu_mul" else N
    if out is None:
        out = torch.empty((M, nout), dtype=x.dtype, device=x.device)
    out2 = out.reshape(M, nout)
    rs_out = _vec(rscale_out, M, torch.float32, "rscale_out")
    rs_in = _vec(rscale_in, M, torch.float32, "rscale_in")
    bias = _vec(bias, N, x.dtype, "bias")
    epi = EPILOGUES["bias"] if bias is not None else EPILOGUES[epilogue]
    lib = load_library()
    fn = lib.hxmi_rmsnorm_linear_f16 if x.dtype == torch.float16 else lib.hxmi_rmsnorm_linear_bf16
    _check(fn(x2.data_ptr(), w_folded.data_ptr(), out2.data_ptr(), _ptr(bias),
              M, N, K, _rowmajor(x2, "x"), _rowmajor(w_folded, "w"), _rowmajor(out2, "out"), epi, float(eps),
              _ptr(rs_out), _ptr(rs_in), _stream(x)))
    return out2.reshape(*lead, nout)


def gemv(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode linear y[M,N] = x[M,K] @ w[N,K].T (+ bias); HBM-streaming for M <= 16.  fp16 or bf16."""
    _require_gpu(x, w, bias, out)
    if x.dtype not in (torch.float16, torch.bfloat16) or w.dtype != x.dtype:
        raise HxmiError("gemv takes fp16 or bf16 x and w of one dtype")
    ldx, ldw = _rowmajor(x, "x"), _rowmajor(w, "w")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise HxmiError(f"x {tuple(x.shape)} and w {tuple(w.shape)} disagree on K")
    bias = _vec(bias, N, x.dtype, "bias")
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ldy = _rowmajor(out, "out")
    lib = load_library()
    ws = _workspace(lib.hxmi_gemv_workspace_bytes(M, N, K), x.device)
    fn = lib.hxmi_gemv_f16 if x.dtype == torch.float16 else lib.hxmi_gemv_bf16
    _check(fn(x.data_ptr(), w.data_ptr(), _ptr(bias), out.data_ptr(), M, N, K, ldx, ldw, ldy,
              _ptr(ws), 0 if ws is None else ws.numel() * 4, _stream(x)))
    return out


def w8a16_linear(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Weight-only int8 linear: y = (x @ wq.T) * scale (+ bias); wq int8 [N,K], scale fp16 [N]."""
    _require_gpu(x, wq, scale, bias, out)
    if x.dtype != torch.float16 or wq.dtype != torch.int8:
        raise HxmiError("w8a16_linear takes fp16 x and int8 wq")
    ldx, ldw = _rowmajor(x, "x"), _rowmajor(wq, "wq")
    M, K = x.shape
    N = wq.shape[0]
    if wq.shape[1] != K:
        raise HxmiError(f"x {tuple(x.shape)} and wq {tuple(wq.shape)} disagree on K")
    scale = _vec(scale, N, torch.float16, "scale")
    bias = _vec(bias, N, torch.float16, "bias")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    ldy = _rowmajor(out, "out")
    lib = load_library()
    ws = _workspace(lib.hxmi_w8a16_workspace_bytes(M, N, K), x.device)
    _check(lib.hxmi_gemv_w8a16(x.data_ptr(), wq.data_ptr(), scale.data_ptr(), _ptr(bias), out.data_ptr(),
                               M, N, K, ldx, ldw, ldy, _ptr(ws), 0 if ws is None else ws.numel() * 4, _stream(x)))
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm over the last dim: weight * T(x * rsqrt(mean(x^2) + eps))."""
    _require_gpu(x, weight, out)
    if x.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != x.dtype:
        raise HxmiError("rms_norm takes fp16 or bf16 x and weight of the same dtype")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    ldx = _rowmajor(x2, "x")
    rows, cols = x2.shape
    weight = _vec(weight, cols, x.dtype, "weight")
    if out is None:
        out = torch.empty_like(x2)
    out2 = out.reshape(rows, cols)
    ldy = _rowmajor(out2, "out")
    fn = load_library().hxmi_rmsnorm_f16 if x.dtype == torch.float16 else load_library().hxmi_rmsnorm_bf16
    _check(fn(x2.data_ptr(), weight.data_ptr(), out2.data_ptr(), rows, cols, ldx, ldy, float(eps), _stream(x)))
    return out2.reshape(*lead, cols)


def softmax(x: torch.Tensor, scale: float = 1.0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(scale * x) over the last dim, fp32 math."""
    _require_gpu(x, out)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise HxmiError("softmax takes fp16 or bf16 input")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    ldx = _rowmajor(x2, "x")
    rows, cols = x2.shape
    if out is None:
        out = torch.empty_like(x2)
    out2 = out.reshape(rows, cols)
    ldy = _rowmajor(out2, "out")
    fn = load_library().hxmi_softmax_f16 if x.dtype == torch.float16 else load_library().hxmi_softmax_bf16
    _check(fn(x2.data_ptr(), out2.data_ptr(), rows, cols, ldx, ldy, float(scale), _stream(x)))
    return out2.reshape(*lead, cols)


def _mask_slices(mask: torch.Tensor, lead: tuple, S: int, Skv: int) -> tuple[torch.Tensor, int, int, int]:
    """An additive fp16 mask broadcast over the leading dims as (tensor, ldm,
    slice stride, slices per mask slice).  A boolean mask keeps the True
    entries (0) and removes the others (-inf), as torch's SDPA reads it."""
    if mask.dtype == torch.bool:
        mask = torch.zeros(mask.shape, dtype=torch.float16, device=mask.device).masked_fill_(~mask, float("-inf"))
    elif mask.dtype != torch.float16:
        mask = mask.to(torch.float16)
    try:
        m = mask.expand(*lead, S, Skv)
    except RuntimeError:
        raise HxmiError(f"mask of shape {tuple(mask.shape)} does not broadcast to {(*lead, S, Skv)}") from None
    if m.stride(-1) != 1 or m.data_ptr() % 2:
        m = m.contiguous()
    st = m.stride()[:-2]
    if all(x == 0 for x in st):
        return m, m.stride(-2), 0, 1
    if len(lead) >= 2 and st[-1] == 0 and all(st[i] == st[i + 1] * lead[i + 1] for i in range(len(lead) - 2)):
        return m, m.stride(-2), st[-2], lead[-1]  # [..., B, 1, S, Skv]: one slice per row of heads
    if all(st[i] == st[i + 1] * lead[i + 1] for i in range(len(lead) - 1)):
        return m, m.stride(-2), st[-1], 1
    m = m.contiguous()
    return m, Skv, S * Skv, 1


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
              out: Optional[torch.Tensor] = None, *, mask: Optional[torch.Tensor] = None,
              causal: int = 0) -> torch.Tensor:
    """SDPA as the reference lowers it (LowerTmTensor.cpp:91-250): softmax(scale * Q.K^T + mask) . V over
    q [..., S, D], k and v [..., S_kv, D].  K/V may have fewer slices than q in their last leading dim
    (grouped-query attention: that many q heads per kv head).  mask: additive (or boolean keep) mask
    broadcastable to [..., S, S_kv]; causal: 1 masks keys after the query (torch's is_causal), 2 after
    query + S_kv - S.  fp16 with D in {64, 128} and scale > 0 runs the fused kernel (hxmi_attention_ex_f16);
    every other case (bf16, other head dims) runs the reference's three steps as bmm(Q, K^T) -> softmax
    (with the mask and causal rule: hxmi_softmax_masked_*) -> bmm(P, V)."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    S, D = q.shape[-2:]
    Skv = k.shape[-2]
    lead = tuple(q.shape[:-2])
    if q.dim() < 3 or k.dim() != q.dim() or v.dim() != q.dim() or k.shape[-1] != D or v.shape[-2] != Skv \
            or k.shape[:-3] != q.shape[:-3] or v.shape[:-2] != k.shape[:-2] or q.shape[-3] % max(k.shape[-3], 1):
        raise HxmiError(f"attention shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    group = q.shape[-3] // k.shape[-3] if k.shape[-3] else 1
    if causal not in (0, 1, 2, False, True):
        raise HxmiError(f"causal must be 0, 1 or 2, got {causal}")
    q3 = q.reshape(-1, S, D)
    k3 = k.reshape(-1, Skv, D)
    v3 = v.reshape(-1, Skv, v.shape[-1])
    if q.dtype == torch.float16 and D in (64, 128) and v.shape[-1] == D and k.dtype == v.dtype == q.dtype \
            and scale > 0:
        _require_gpu(q3, k3, v3)
        q3, k3, v3 = (t if t.stride(-1) == 1 and t.stride(1) % 8 == 0 and t.stride(0) % 8 == 0
                      and t.data_ptr() % 16 == 0 else t.contiguous() for t in (q3, k3, v3))
        if out is None:
            o = torch.empty((q3.shape[0], S, D), dtype=q.dtype, device=q.device)
        else:
            if out.shape != (*lead, S, D) or out.dtype != q.dtype:
                raise HxmiError(f"out must be {q.dtype} {(*lead, S, D)}")
            o = out.reshape(-1, S, D)
            if o.data_ptr() != out.data_ptr() or o.stride(-1) != 1 or o.data_ptr() % 8 or o.stride(1) % 4 \
                    or o.stride(0) % 4:
                raise HxmiError("out must be a view with unit last stride and 8-byte aligned rows")
        _require_gpu(o)
        ldq, bq = _batched(q3, "q")
        ldk, bk = _batched(k3, "k")
        ldv, bv = _batched(v3, "v")
        ldo, bo = _batched(o, "out")
        mp, ldm, sm, mg = 0, 0, 0, 1
        if mask is not None:
            _require_gpu(mask)
            m, ldm, sm, mg = _mask_slices(mask, lead, S, Skv)
            mp = m.data_ptr()
        _check(load_library().hxmi_attention_ex_f16(q3.data_ptr(), k3.data_ptr(), v3.data_ptr(), o.data_ptr(),
                                                    q3.shape[0], S, Skv, D, ldq, ldk, ldv, ldo, bq, bk, bv, bo,
                                                    group, mp, ldm, sm, mg, int(causal), float(scale), _stream(q)))
        return out if out is not None else o.reshape(*lead, S, D)
    # The reference's three steps: bmm(Q, K^T) * scale -> (+ mask, causal)
    # softmax -> bmm(P, V).  The query heads of one K/V head form one batch
    # entry of group * S rows (q slices i = hkv * group + g are consecutive),
    # so each K/V slice is read by one GEMM batch entry.  S and P rows are
    # padded to a multiple of 8 keys, so both GEMMs (ragged N for Q.K^T,
    # ragged K for P.V) run on the MFMA path; the softmax runs in place.
    _require_gpu(q3, k3, v3, mask)
    if q3.dtype not in (torch.float16, torch.bfloat16) or k3.dtype != q3.dtype or v3.dtype != q3.dtype:
        raise HxmiError("attention takes fp16 or bf16 q, k, v of one dtype")
    nq, dv = q3.shape[0], v.shape[-1]
    if group > 1:
        q3 = q3.contiguous().view(nq // group, group * S, D)
    skv8 = (Skv + 7) // 8 * 8
    sbuf = torch.empty((nq, S, skv8), dtype=q.dtype, device=q.device)
    s = bgemm(q3, k3, b_layout="nt", alpha=scale, out=sbuf.view(q3.shape[0], q3.shape[1], skv8)[..., :Skv])
    if mask is None and not causal:
        p = softmax(s, out=s)
    else:
        mp, ldm, sm, mg = 0, 0, 0, 1
        if mask is not None:
            m, ldm, sm, mg = _mask_slices(mask, lead, S, Skv)
            mp = m.data_ptr()
        fn = (load_library().hxmi_softmax_masked_f16 if q.dtype == torch.float16
              else load_library().hxmi_softmax_masked_bf16)
        _check(fn(sbuf.data_ptr(), sbuf.data_ptr(), nq, S, Skv, skv8, S * skv8, skv8, S * skv8, mp or None, ldm,
                  sm, mg, int(causal), 1.0, _stream(q)))
        p = s
    if out is not None:
        if out.shape != (*lead, S, dv) or out.dtype != q.dtype:
            raise HxmiError(f"out must be {q.dtype} {(*lead, S, dv)}")
        bgemm(p, v3, b_layout="nn", out=out.view(q3.shape[0], q3.shape[1], dv))
        return out
    o = bgemm(p, v3, b_layout="nn")
    return o.reshape(*lead, S, dv)


def hexkl_matmul(act: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """hexkl_matmul_f16f16_f32 contract: fp32 out[n_row, n_col] = act[n_row, n_inner] @ w[n_inner, n_col]."""
    _require_gpu(act, w)
    if act.dtype != torch.float16 or w.dtype != torch.float16:
        raise HxmiError("hexkl_matmul takes fp16 operands")
    act = act.contiguous()
    w = w.contiguous()
    n_row, n_inner = act.shape
    n_col = w.shape[1]
    if w.shape[0] != n_inner:
        raise HxmiError("inner dimensions differ")
    out = torch.empty((n_row, n_col), dtype=torch.float32, device=act.device)
    torch.cuda.current_stream(act.device).synchronize()
    _check(load_library().hexkl_matmul_f16f16_f32(n_row, n_col, n_inner, out.data_ptr(), act.data_ptr(),
                                                  w.data_ptr()))
    return out


@dataclasses.dataclass
class DecoderStack:
    """fp16 weights of a Llama / Qwen2 decoder stack, stacked per layer, on one
    GPU (H hidden, I intermediate, kv_dim = kv_heads * head_dim, head_dim =
    H / heads):

    w_qkv [L, H + 2*kv_dim, H] (q rows, k rows, v rows), b_qkv [L, H + 2*kv_dim]
    or None, w_o [L, H, H], w_gu [L, 2*I, H] (gate rows, then up rows), w_down
    [L, H, I], g_attn and g_mlp [L, H] (RMSNorm weights), g_final [H], w_lm
    [vocab, H] or None (no logits).  w_ov [L, H, H] and b_ov [L, H] (None
    without b_qkv): the o projection folded onto the normalised layer input,
    set by fold_o(); decode_step then runs three dependent phases a layer."""
    w_qkv: torch.Tensor
    b_qkv: Optional[torch.Tensor]
    w_o: torch.Tensor
    w_gu: torch.Tensor
    w_down: torch.Tensor
    g_attn: torch.Tensor
    g_mlp: torch.Tensor
    g_final: torch.Tensor
    heads: int
    kv_heads: int
    eps: float
    w_lm: Optional[torch.Tensor] = None
    w_ov: Optional[torch.Tensor] = None
    b_ov: Optional[torch.Tensor] = None

    @property
    def dims(self) -> tuple[int, int, int, int]:
        """(layers, hidden, intermediate, kv_dim)"""
        L, nqkv, H = self.w_qkv.shape
        return L, H, self.w_gu.shape[1] // 2, (nqkv - H) // 2

    def fold_o(self) -> "DecoderStack":
        """Sets w_ov = w_o E w_v and b_ov = w_o E b_v per layer, E copying key /
        value head j's head_dim rows to every query head of its group: at
        position 0 the attention output is E (h . w_v^T + b_v), so the o
        projection becomes h . w_ov^T + b_ov on the layer's normalised input
        h.  Computed with this library's NN GEMM and GEMV (fp32 accumulation,
        one fp16 rounding).  Returns self."""
        L, H, _, kv_dim = self.dims
        hd = H // self.heads
        grp = self.heads // self.kv_heads
        i = torch.arange(H, device=self.w_qkv.device)
        vrow = H + kv_dim + (i // hd // grp) * hd + i % hd  # the v row each o input element reads
        w_ov = torch.empty((L, H, H), dtype=torch.float16, device=self.w_qkv.device)
        b_ov = None if self.b_qkv is None else torch.empty((L, H), dtype=torch.float16, device=self.w_qkv.device)
        for layer in range(L):
            ev = self.w_qkv[layer].index_select(0, vrow).contiguous()
            gemm(self.w_o[layer], ev, b_layout="nn", out=w_ov[layer])
            if b_ov is not None:
                eb = self.b_qkv[layer].index_select(0, vrow).reshape(1, H).contiguous()
                gemv(eb, self.w_o[layer], out=b_ov[layer].view(1, H))
        self.w_ov, self.b_ov = w_ov, b_ov
        return self


_DECODE_WS: "collections.OrderedDict[tuple, torch.Tensor]" = collections.OrderedDict()
_DECODE_KEEP_CAPTURED = 32  # workspaces of captured graphs kept for decode_status (oldest dropped)


def _decode_workspace(device: torch.device, shape: tuple, nbytes: int) -> torch.Tensor:
    """The decode workspace for one stack shape (hidden, kv_dim, intermediate)
    of the calls launched on the current stream of `device`: it carries the
    step's published vectors and running tag from call to call, so it is
    kept, zero-filled when created, and shared neither between streams nor
    between shapes.  Inside a HIP graph capture each capture gets its own
    (keyed by its capture id), zero-filled by a fill node recorded before its
    first use, so every replay starts from the zero state and no other graph
    or eager call touches it."""
    cap = _capture_key(device)
    key = (_device_index(device), torch.cuda.current_stream(device).cuda_stream if cap is None else cap, shape)
    ws = _DECODE_WS.get(key)
    if ws is None:
        ws = torch.zeros((nbytes + 255) // 256 * 64, dtype=torch.int32, device=device)
        _DECODE_WS[key] = ws
        captured = [k for k in _DECODE_WS if isinstance(k[1], tuple)]
        for k in captured[: max(0, len(captured) - _DECODE_KEEP_CAPTURED)]:
            del _DECODE_WS[k]
    return ws


def decode_step(x: torch.Tensor, stack: DecoderStack, *, out_qkv: bool = False,
                timeout_us: int = 0) -> dict:
    """One-token forward of the decoder stack at position 0 (empty KV cache)
    from the token's embedding row x [H] (fp16), as one persistent kernel
    (plus the lm_head GEMV when stack.w_lm is set).  Returns {"h": final
    normalised hidden state [H], "x": hidden state before the final norm [H],
    "logits": [vocab] or None, "qkv": [L, H + 2*kv_dim] or None}.  A wait
    inside the kernel longer than timeout_us (0: one second) ends the launch
    early; decode_status() reports it."""
    L, H, inter, kv_dim = stack.dims
    ts = [x, stack.w_qkv, stack.b_qkv, stack.w_o, stack.w_gu, stack.w_down, stack.g_attn, stack.g_mlp,
          stack.g_final, stack.w_lm, stack.w_ov, stack.b_ov]
    _require_gpu(*ts)
    for t in ts:
        if t is not None and (t.dtype != torch.float16 or not t.is_contiguous()):
            raise HxmiError("decode_step takes contiguous fp16 tensors")
    head_dim = H // stack.heads
    want = {"w_o": (L, H, H), "w_gu": (L, 2 * inter, H), "w_down": (L, H, inter), "g_attn": (L, H),
            "g_mlp": (L, H), "g_final": (H,)}
    for name, shape in want.items():
        if tuple(getattr(stack, name).shape) != shape:
            raise HxmiError(f"{name} is {tuple(getattr(stack, name).shape)}, expected {shape}")
    if stack.b_qkv is not None and tuple(stack.b_qkv.shape) != (L, H + 2 * kv_dim):
        raise HxmiError("b_qkv must be [L, H + 2*kv_dim]")
    if stack.w_ov is not None and tuple(stack.w_ov.shape) != (L, H, H):
        raise HxmiError("w_ov must be [L, H, H]")
    if (stack.b_ov is not None) != (stack.w_ov is not None and stack.b_qkv is not None) or (
            stack.b_ov is not None and tuple(stack.b_ov.shape) != (L, H)):
        raise HxmiError("b_ov must be [L, H] with w_ov and b_qkv, else None")
    if x.numel() != H:
        raise HxmiError(f"x has {x.numel()} elements, expected {H}")
    if stack.kv_heads * head_dim != kv_dim or stack.heads * head_dim != H:
        raise HxmiError("w_qkv rows do not match heads / kv_heads")
    dev = x.device
    h = torch.empty(H, dtype=torch.float16, device=dev)
    xo = torch.empty(H, dtype=torch.float16, device=dev)
    qkv = torch.empty((L, H + 2 * kv_dim), dtype=torch.float16, device=dev) if out_qkv else None
    vocab = 0 if stack.w_lm is None else stack.w_lm.shape[0]
    if stack.w_lm is not None and tuple(stack.w_lm.shape) != (vocab, H):
        raise HxmiError("w_lm must be [vocab, H]")
    logits = torch.empty(vocab, dtype=torch.float16, device=dev) if vocab else None
    lib = load_library()
    nbytes = lib.hxmi_decode_workspace_bytes(H, kv_dim, inter)
    ws = _decode_workspace(dev, (H, kv_dim, inter), nbytes)
    tail = (stack.w_gu.data_ptr(), stack.w_down.data_ptr(), stack.g_attn.data_ptr(), stack.g_mlp.data_ptr(),
            stack.g_final.data_ptr(), _ptr(stack.w_lm), _ptr(qkv), xo.data_ptr(), h.data_ptr(), _ptr(logits), L, H,
            stack.heads, stack.kv_heads, head_dim, inter, vocab, float(stack.eps), int(timeout_us), ws.data_ptr(),
            ws.numel() * 4, _stream(x))
    if stack.w_ov is not None:
        _check(lib.hxmi_decode_step_ov_f16(x.data_ptr(), stack.w_qkv.data_ptr(), _ptr(stack.b_qkv),
                                           stack.w_ov.data_ptr(), _ptr(stack.b_ov), *tail))
    else:
        _check(lib.hxmi_decode_step_f16(x.data_ptr(), stack.w_qkv.data_ptr(), _ptr(stack.b_qkv),
                                        stack.w_o.data_ptr(), *tail))
    return {"h": h, "x": xo, "logits": logits, "qkv": qkv}


def decode_status(device: Optional[torch.device] = None, clear: bool = True) -> int:
    """Error words of the decode workspaces after their work has finished: 0 =
    every decode_step so far completed its waits, 1 = a wait expired (that
    launch's outputs are undefined).  It reads the workspaces of the current
    stream's eager calls and those of every HIP graph captured on the device
    (a graph's replays may run on any stream; its workspace holds the last
    replay's word).  clear resets them."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    stream = torch.cuda.current_stream(device).cuda_stream
    dev_index = _device_index(device)
    status = 0
    for (d, s, _), ws in list(_DECODE_WS.items()):
        if d == dev_index and (s == stream or isinstance(s, tuple)):
            st = ctypes.c_int(0)
            _check(load_library().hxmi_decode_status(ws.data_ptr(), int(clear), ctypes.byref(st), stream))
            status |= st.value
    return status


def release_workspaces() -> None:
    """Drop every cached split-K and decode workspace (after the work that
    used them has finished), e.g. before the process tears the GPU state down."""
    _WS_CACHE.clear()
    _DECODE_WS.clear()


def pack_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """Interleave gate and up projections [I,K] into the packed [2I,K] layout the
    SiLU-mul epilogue reads: rows [32q, 32q+16) = gate[16q:16q+16],
    rows [32q+16, 32q+32) = up[16q:16q+16].  I must be a multiple of 16."""
    if w_gate.shape != w_up.shape or w_gate.dim() != 2 or w_gate.shape[0] % 16:
        raise HxmiError("gate and up must be [I, K] with I % 16 == 0")
    inter, k = w_gate.shape
    packed = torch.stack((w_gate.reshape(inter // 16, 16, k), w_up.reshape(inter // 16, 16, k)), dim=1)
    return packed.reshape(2 * inter, k).contiguous()
