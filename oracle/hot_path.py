"""Oracle: CPU restatement of the reference's hot-path op semantics.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the reference the kernels are
compared with or as the timed CPU baseline, never as the product path (the
product is libhxmi.so).

Everything here is numpy, computed in float32 (float64 where an exact answer
is wanted), following the reference files cited on each function.  The
reference's own correctness oracle is PyTorch on x86
(test/python/triton/test_matmul.py:90, test_rms_norm.py:85-87,
test_softmax.py:91, test_silu.py:63, test_gelu.py:72,
benchmark_models/micro_bench/test_matmul_benchmark.py:91-92); tests/ pin each
function here against those torch CPU functions, against closed forms and
against exact integer arithmetic.

Parity status per function (how each is pinned, see tests/test_oracle.py):
  matmul, linear, bmm         exact-integer known answers (golden fixtures
                              from pure-Python integer loops), torch.matmul
  gelu_tanh, silu, silu_mul   closed forms / special values, torch F.gelu
                              (approximate="tanh") and F.silu
  rms_norm, rms_norm_hf       closed forms (constant row, scale invariance),
                              torch F.rms_norm
  softmax                     row sums, shift invariance, uniform row,
                              torch F.softmax
  w8a16_linear, dequant_int8  exact integer one-hot known answers, scale
                              linearity
  quantize_int8_rows          exact known answers (w = integer * 2^-7),
                              round-half-even ties vs Python's round(), the
                              scale against a brute-force search over every
                              fp16 value, sign symmetry and power-of-two
                              equivariance
  sdpa                        torch F.scaled_dot_product_attention (fp32 CPU)
                              with and without an additive / boolean mask,
                              is_causal, enable_gqa and torch's lower-right
                              causal bias; one-hot and fully-masked closed
                              forms; mask shift invariance
  decode_step                 transformers' Qwen2ForCausalLM on one token at
                              position 0 (fp32, and its fp16 forward with
                              fp16 rounding on); closed forms: zero o/down
                              projections, kv-head routing of each query head
                              (tests/test_decode_oracle.py)
  vtcm_tile_sizes             the reference's lit expectation
                              (vtcm_tiling_static.mlir:80-88) and the
                              footprint rule it encodes
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def _f32(x) -> np.ndarray:
    return np.asarray(x).astype(F32)


# ---- matmul family -----------------------------------------------------------


def matmul(a, b, b_layout: str = "nn") -> np.ndarray:
    """C = A . op(B) with fp16 inputs widened to fp32 and fp32 accumulation.

    Follows the generic matmul body the reference tiles for HVX
    (qcom_hexagon_backend/test/Conversion/LinalgToLLVM/vtcm_tiling_static.mlir
    :62-68: extf f16->f32, mulf, addf) and the f32 CPU check of config 1
    (benchmark_models/micro_bench/test_matmul_benchmark.py:22-31, 91-92).
    b_layout "nt" is linalg.matmul_transpose_b
    (lib/Transforms/ScheduleMatmulForHVXPass.cpp:78-139).
    """
    a32, b32 = _f32(a), _f32(b)
    if b_layout == "nt":
        b32 = b32.T
    return a32 @ b32


def linear(x, w, bias=None) -> np.ndarray:
    """nn.Linear: x . w^T (+ bias), fp32."""
    y = matmul(x, w, "nt")
    if bias is not None:
        y = y + _f32(bias)
    return y


def bmm(a, b, b_layout: str = "nn") -> np.ndarray:
    """Batched matmul over the leading dim (linalg.batch_matmul[_transpose_b])."""
    a32, b32 = _f32(a), _f32(b)
    if b_layout == "nt":
        b32 = np.swapaxes(b32, -1, -2)
    return np.matmul(a32, b32)


# ---- elementwise epilogues -----------------------------------------------------


def silu(x) -> np.ndarray:
    """x / (1 + exp(-x)) (test/python/triton/test_silu.py:35-45)."""
    x = _f32(x)
    return x / (F32(1) + np.exp(-x))


def gelu_tanh(x) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))): the tanh form of
    test/python/triton/test_gelu.py:25-53 and benchmark_models/run_vit.py:125
    ("gelu_new"), checked against F.gelu(approximate="tanh") (test_gelu.py:72)."""
    x = _f32(x)
    k0 = F32(math.sqrt(2.0 / math.pi))
    return F32(0.5) * x * (F32(1) + np.tanh(k0 * (x + F32(0.044715) * x * x * x)))


def silu_mul_linear(x, w_gate, w_up) -> np.ndarray:
    """HF LlamaMLP front half: silu(x . Wg^T) * (x . Wu^T)."""
    return silu(linear(x, w_gate)) * linear(x, w_up)


def gemm_epilogue(a, b, b_layout="nt", epilogue=None, bias=None, alpha=1.0) -> np.ndarray:
    """alpha * A . op(B) followed by the fused epilogue, all fp32.

    For "silu_mul", B holds packed gate/up columns (pack_gate_up)."""
    y = matmul(a, b, b_layout) * F32(alpha)
    if epilogue in (None, "none"):
        return y
    if epilogue == "bias":
        return y + _f32(bias)
    if epilogue == "gelu_tanh":
        return gelu_tanh(y)
    if epilogue == "bias_gelu_tanh":
        return gelu_tanh(y + _f32(bias))
    if epilogue == "silu_mul":
        n = y.shape[-1]
        g, u = unpack_gate_up_cols(y, n)
        return silu(g) * u
    raise ValueError(epilogue)


def pack_gate_up(w_gate, w_up) -> np.ndarray:
    """Packed [2I,K] layout: rows [32q,32q+16) = gate[16q:16q+16],
    rows [32q+16,32q+32) = up[16q:16q+16]."""
    wg, wu = np.asarray(w_gate), np.asarray(w_up)
    i, k = wg.shape
    return np.stack((wg.reshape(i // 16, 16, k), wu.reshape(i // 16, 16, k)), axis=1).reshape(2 * i, k)


def unpack_gate_up_cols(y, n):
    """Split packed output columns back into (gate, up), each n/2 wide."""
    y = np.asarray(y)
    lead = y.shape[:-1]
    yy = y.reshape(*lead, n // 32, 2, 16)
    return yy[..., 0, :].reshape(*lead, n // 2), yy[..., 1, :].reshape(*lead, n // 2)


# ---- row reductions -----------------------------------------------------------------


def rms_norm(x, g, eps: float = 1e-5) -> np.ndarray:
    """fp32 reference RMSNorm, y = x / sqrt(mean(x^2) + eps) * g
    (test/python/triton/test_rms_norm.py:52-60, checked there against
    F.rms_norm at :85-87)."""
    x32 = _f32(x)
    ms = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=np.float64).astype(F32)
    return x32 / np.sqrt(ms + F32(eps)) * _f32(g)


def rms_norm_hf(x, g, eps: float = 1e-5) -> np.ndarray:
    """HF LlamaRMSNorm order (what benchmark_models/run_tinyllama.py runs):
    normalise in fp32, round to fp16, multiply by the fp16 weight in fp16.
    Returns the fp16 result."""
    x32 = _f32(x)
    ms = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=np.float64).astype(F32)
    n16 = (x32 / np.sqrt(ms + F32(eps))).astype(np.float16)
    return (n16.astype(F32) * _f32(g)).astype(np.float16)


def softmax(x, scale: float = 1.0) -> np.ndarray:
    """Row softmax of scale*x with max subtraction: max, sub, exp, sum, div
    (qcom_hexagon_backend/test/Conversion/LinalgToLLVM/fusion_softmax_2D.mlir
    :8-57; test/python/triton/test_softmax.py:60-66)."""
    z = _f32(x) * F32(scale)
    z = z - np.max(z, axis=-1, keepdims=True)
    e = np.exp(z)
    return e / np.sum(e, axis=-1, keepdims=True)


def sdpa(q, k, v, scale=None, mask=None, causal: int = 0, kv_group: int = 1) -> np.ndarray:
    """Attention as lib/Transforms/LowerTmTensor.cpp:91-250 lowers
    tm_tensor.attention: bmm(Q, K^T) * scale (:130-145) + mask (:158-163) ->
    softmax (max, exp(x - max), sum, div: :165-229) -> bmm(P, V)
    (scale 1/sqrt(d), qcom_hexagon_backend/test/Conversion/TmTensorToLinalg/
    SDPA.mlir:18-31).  q [..., S, D], k and v [..., S_kv, D]; mask is added
    to the scaled scores (broadcast over the leading dims); causal = 1 masks
    key j of query i when j > i (torch's is_causal), causal = 2 when
    j > i + S_kv - S; kv_group consecutive query slices of the leading
    dims' last axis share one K/V slice.  A row whose every entry is -inf
    comes out NaN, as exp(x - max) over it does in the decomposition."""
    q32, k32, v32 = _f32(q), _f32(k), _f32(v)
    if scale is None:
        scale = 1.0 / math.sqrt(q32.shape[-1])
    if kv_group > 1:
        k32 = np.repeat(k32, kv_group, axis=-3)
        v32 = np.repeat(v32, kv_group, axis=-3)
    z = bmm(q32, k32, "nt") * F32(scale)
    if mask is not None:
        z = z + _f32(mask)
    if causal:
        sq, skv = z.shape[-2:]
        off = 0 if causal == 1 else skv - sq
        z = np.where(np.arange(skv)[None, :] > np.arange(sq)[:, None] + off, F32(-np.inf), z)
    with np.errstate(invalid="ignore"):
        z = z - np.max(z, axis=-1, keepdims=True)
        e = np.exp(z)
        p = e / np.sum(e, axis=-1, keepdims=True)
    return np.matmul(p, v32)


# ---- one-token decoder step --------------------------------------------------------------


def decode_step(x, w_qkv, b_qkv, w_o, w_gu, w_down, g_attn, g_mlp, g_final, heads: int, kv_heads: int,
                eps: float, w_lm=None, fp16: bool = True) -> dict:
    """Forward of a Llama / Qwen2 decoder stack on ONE token at position 0
    with an empty KV cache -- what benchmark_models/run_qwen2.5-0.5b.py
    :171-173,224-233 runs through the reference (prompt "Hi", use_cache off,
    position_ids [0]).  Per layer (HF Qwen2DecoderLayer order):
      h = RMSNorm(x) ; qkv = h W_qkv^T + b ; att[head i] = v[kv head i // (heads/kv_heads)]
      x = x + att W_o^T ; h = RMSNorm(x) ; [g|u] = h W_gu^T ; x = x + (silu(g)*u) W_down^T
    then h = RMSNorm(x, g_final), logits = h W_lm^T.  With one key the
    softmax weight is exactly 1 and RoPE at position 0 is the identity
    (cos 1, sin 0), so the attention output is v.  w_qkv [L, H + 2*kv, H]
    (q, k, v rows), w_gu [L, 2I, H] (gate rows, then up rows).
    fp16=True rounds to fp16 where the HF fp16 forward does (RMSNorm as
    rms_norm_hf, each projection output, SiLU, the product, each residual
    sum); fp16=False is the plain fp32 forward."""
    L, nqkv, H = np.shape(w_qkv)
    kv = (nqkv - H) // 2
    hd = H // heads
    grp = heads // kv_heads
    r16 = (lambda a: a.astype(np.float16).astype(F32)) if fp16 else (lambda a: a)

    def norm(v, g):
        if fp16:
            return rms_norm_hf(v, g, eps).astype(F32)
        return rms_norm(v, g, eps)

    xs = _f32(x).reshape(H)
    qkv_all = []
    for l in range(L):
        h = norm(xs, g_attn[l])
        qkv = h @ _f32(w_qkv[l]).T
        if b_qkv is not None:
            qkv = qkv + _f32(b_qkv[l])
        qkv = r16(qkv)
        qkv_all.append(qkv)
        v = qkv[H + kv:].reshape(kv_heads, hd)
        att = v[np.arange(heads) // grp].reshape(H)
        xs = r16(xs + r16(att @ _f32(w_o[l]).T))
        h = norm(xs, g_mlp[l])
        gu = r16(h @ _f32(w_gu[l]).T)
        inter = gu.shape[0] // 2
        a = r16(r16(silu(gu[:inter])) * gu[inter:])
        xs = r16(xs + r16(a @ _f32(w_down[l]).T))
    h = norm(xs, g_final)
    logits = None if w_lm is None else r16(h @ _f32(w_lm).T)
    return {"h": h, "x": xs, "logits": logits, "qkv": np.stack(qkv_all)}


# ---- weight-only int8 ----------------------------------------------------------------


def dequant_int8(q) -> np.ndarray:
    """Integer weights as floats; exact for every int8 code."""
    return np.asarray(q).astype(np.int32).astype(F32)


def quantize_int8_rows(w) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8 codes of fp16 weights [N, K]:
    s[n] = the smallest fp16 value with 127 * s[n] >= max_k |w[n,k]| (fp16
    round-to-nearest of max/127, one step up where that fell below; 1 for a
    zero row), q = rint(w / s) (half to even).  The reference has no weight
    quantiser (int8 enters only through MLIR's quant.qcast lowering,
    lib/Conversion/LinalgToLLVM/LinalgToLLVMPass.cpp:203-205); this states
    the rule the int8 path's loader uses."""
    wf = np.asarray(w, dtype=np.float16).astype(F32)
    amax = np.abs(wf).max(axis=1)
    s = (amax / F32(127)).astype(np.float16)
    low = s.astype(F32) * F32(127) < amax
    s = np.where(low, np.nextafter(s, np.float16(np.inf)), s)
    s = np.where(amax == 0, np.float16(1), s).astype(np.float16)
    q = np.clip(np.rint(wf / s.astype(F32)[:, None]), -127, 127).astype(np.int8)
    return q, s


def w8a16_linear(x, q, s, bias=None) -> np.ndarray:
    """y = x . (q * s[:,None])^T (+ bias), fp32: the weight-only int8 config
    (no reference kernel exists; only quant.qcast/dcast lowering,
    lib/Conversion/LinalgToLLVM/LinalgToLLVMPass.cpp:203-209)."""
    w = dequant_int8(q) * _f32(s)[:, None]
    y = _f32(x) @ w.T
    if bias is not None:
        y = y + _f32(bias)
    return y


# ---- VTCM tile-size model ------------------------------------------------------------

VTCM_BYTES = 2 * 1024 * 1024  # include/hexagon/Conversion/LinalgToLLVM/Common.h:26
HVX_VECTOR_BYTES = 128  # lib/Conversion/LinalgToLLVM/Common.cpp:80-85 (native vector width)


def _footprint(tile, operand_dims, elem_bytes) -> int:
    # Sum over operands of (element size x product of the tile extents its
    # indexing map reads); a constant-0 map result counts as extent 1
    # (VTCMTilingOptions.cpp:98-117, 125-134).
    return sum(eb * math.prod(tile[d] for d in od) for od, eb in zip(operand_dims, elem_bytes))


def _reduction_factor(size: int, budget: int) -> int:
    # Next power of two of size/budget, 1 when it already fits
    # (VTCMTilingOptions.cpp:169-184).
    if size < budget:
        return 1
    return 1 << math.ceil(math.log2(size / budget))


def vtcm_tile_sizes(loop_ranges, operand_dims, elem_bytes, iterator_types, budget=VTCM_BYTES):
    """Restatement of the reference's VTCM tile-size search, determineTileSizes
    (lib/Conversion/LinalgToLLVM/VTCMTilingOptions.cpp:374-432).

    loop_ranges:    static loop extents of the linalg op
    operand_dims:   per operand (inputs then outputs), the loop indices its
                    indexing map reads
    elem_bytes:     per operand element size in bytes
    iterator_types: per loop, "parallel" or "reduction"

    Returns the tile sizes, or None when even unit tiles do not fit.
    """
    ranges = list(loop_ranges)
    size = _footprint(ranges, operand_dims, elem_bytes)
    if size <= budget:
        return ranges
    # priority: parallel dims, then reduction dims, each ordered by the
    # footprint left after halving that dim alone (:190-243)
    order = []
    for kind in ("parallel", "reduction"):
        cand = []
        for d, it in enumerate(iterator_types):
            if it != kind:
                continue
            t = list(ranges)
            t[d] //= 2
            cand.append((_footprint(t, operand_dims, elem_bytes), d))
        order += [d for _, d in sorted(cand)]
    # lower bounds: outermost dim >= 4 (parallelisation factor), innermost dim
    # >= one HVX vector of the smallest operand type (:283-313)
    lower = [1] * len(ranges)
    if ranges[0] >= 4:
        lower[0] = 4
    vec = HVX_VECTOR_BYTES // min(elem_bytes)
    if ranges[-1] >= vec:
        lower[-1] = vec
    tile = list(ranges)
    rf = _reduction_factor(size, budget)
    for first_pass in (True, False):
        for d in order:
            lb = lower[d] if first_pass else 1
            tile[d] = max(tile[d] // rf, lb)
            updated = _footprint(tile, operand_dims, elem_bytes)
            if updated <= budget:
                return tile
            rf = _reduction_factor(updated, budget)
    return None


def matmul_tile_sizes(m: int, n: int, k: int, in_bytes: int = 2, out_bytes: int = 4):
    """determineTileSizes for linalg.matmul after ScheduleMatmulForHVX's
    interchange to loop order (m, k, n) (lib/Transforms/LinalgUtils.cpp:67-83):
    A reads (m,k), B reads (k,n), C reads (m,n)."""
    return vtcm_tile_sizes([m, k, n], [(0, 1), (1, 2), (0, 2)], [in_bytes, in_bytes, out_bytes],
                           ["parallel", "reduction", "parallel"])


# ---- tolerance metric --------------------------------------------------------------


def max_rel_err(out, ref, floor_frac: float = 1e-3) -> float:
    """max_i |out_i - ref_i| / max(|ref_i|, floor), floor = floor_frac * rms(ref).

    The floor keeps entries whose exact value is (near) zero from dividing by
    ~0; it is 1e-3 of the output's RMS, far below any fp16 rounding of a
    typical entry."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    if o.shape != r.shape:
        raise ValueError(f"shape mismatch {o.shape} vs {r.shape}")
    if r.size == 0:
        return 0.0
    if not np.all(np.isfinite(o)):
        return float("inf")
    rms = float(np.sqrt(np.mean(r * r)))
    floor = max(floor_frac * rms, 1e-30)
    return float(np.max(np.abs(o - r) / np.maximum(np.abs(r), floor)))


def max_err_vs_scale(out, ref) -> float:
    """max_i |out_i - ref_i| / max_i |ref_i|: the error relative to the
    output's scale.  Used for multi-kernel pipelines whose fp16
    intermediates (as the reference's own decomposed lowering materialises
    them, e.g. S and P of attention) leave ~1e-4 absolute noise that an
    elementwise ratio would magnify at outputs that cancel to ~0."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    if o.shape != r.shape:
        raise ValueError(f"shape mismatch {o.shape} vs {r.shape}")
    if r.size == 0:
        return 0.0
    if not np.all(np.isfinite(o)):
        return float("inf")
    return float(np.max(np.abs(o - r)) / max(float(np.max(np.abs(r))), 1e-30))
