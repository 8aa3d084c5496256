"""Pin the oracle (oracle/hot_path.py) before trusting it as the GPU checker.

Each oracle function is checked against (a) the torch CPU function the
reference's own tests compare with, (b) closed forms / invariants, and (c) the
exact-integer golden fixtures in tests/golden/.  A planted mistake (dropped
term, wrong sign, transposed operand) fails at least one of these.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN
from oracle import hot_path as ref


def rng(seed=0):
    return np.random.default_rng(seed)


# ---- matmul family ------------------------------------------------------------------


@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_matmul_exact_integer_golden(layout):
    d = np.load(GOLDEN / f"gemm_int_{layout}.npz")
    out = ref.matmul(d["a"].astype(np.float16), d["b"].astype(np.float16), layout)
    assert np.array_equal(out.astype(np.int64), d["c"])


def test_matmul_matches_torch_matmul():
    r = rng(1)
    a = r.uniform(-1, 1, (64, 96)).astype(np.float16)
    b = r.uniform(-1, 1, (96, 40)).astype(np.float16)
    t = torch.matmul(torch.from_numpy(a).float(), torch.from_numpy(b).float()).numpy()
    # fp32 summation order differs between BLAS builds: allow order noise only
    assert ref.max_rel_err(ref.matmul(a, b), t) < 1e-4
    assert ref.max_rel_err(ref.matmul(a, np.ascontiguousarray(b.T), "nt"), t) < 1e-4


def test_matmul_identity_zero_outer():
    r = rng(2)
    a = r.uniform(-1, 1, (16, 16)).astype(np.float16)
    assert np.array_equal(ref.matmul(a, np.eye(16, dtype=np.float16)), a.astype(np.float32))
    assert not np.any(ref.matmul(a, np.zeros((16, 8), np.float16)))
    u = r.uniform(-1, 1, (7, 1)).astype(np.float32)
    v = r.uniform(-1, 1, (1, 5)).astype(np.float32)
    assert np.allclose(ref.matmul(u, v), u * v)


def test_bmm_is_per_batch_matmul():
    r = rng(3)
    a = r.standard_normal((3, 5, 8)).astype(np.float32)
    b = r.standard_normal((3, 6, 8)).astype(np.float32)
    out = ref.bmm(a, b, "nt")
    for i in range(3):
        assert np.allclose(out[i], a[i] @ b[i].T, atol=1e-6)


def test_linear_bias_golden():
    d = np.load(GOLDEN / "gemm_int_epi.npz")
    out = ref.linear(d["a"].astype(np.float16), d["b"].astype(np.float16), d["bias"].astype(np.float16))
    assert np.array_equal(out.astype(np.int64), d["c"])


# ---- epilogues ----------------------------------------------------------------------


def test_silu_against_torch_and_closed_form():
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    assert np.allclose(ref.silu(x), F.silu(torch.from_numpy(x)).numpy(), rtol=1e-6, atol=1e-7)
    assert ref.silu(np.float32(0)) == 0
    assert abs(ref.silu(np.float32(30)) - 30) < 1e-5  # x * sigmoid(x) -> x
    assert abs(ref.silu(np.float32(-30))) < 1e-10


def test_gelu_tanh_against_torch_and_closed_form():
    x = np.linspace(-10, 10, 2001, dtype=np.float32)
    t = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.allclose(ref.gelu_tanh(x), t, rtol=1e-5, atol=1e-6)
    # not the erf form: they differ by more than 1e-4 somewhere
    e = F.gelu(torch.from_numpy(x)).numpy()
    assert np.max(np.abs(ref.gelu_tanh(x) - e)) > 1e-4
    assert ref.gelu_tanh(np.float32(0)) == 0
    # the test_gelu.py:53 form with its rounded constants agrees to ~1e-4
    k = 0.5 * x * (1 + np.tanh(0.797885 * x + 0.035677 * x * x * x))
    assert np.max(np.abs(k - ref.gelu_tanh(x))) < 1e-3


def test_pack_gate_up_round_trip():
    r = rng(4)
    wg = r.standard_normal((64, 8)).astype(np.float32)
    wu = r.standard_normal((64, 8)).astype(np.float32)
    p = ref.pack_gate_up(wg, wu)
    assert p.shape == (128, 8)
    assert np.array_equal(p[0:16], wg[0:16]) and np.array_equal(p[16:32], wu[0:16])
    assert np.array_equal(p[32:48], wg[16:32])
    x = r.standard_normal((5, 8)).astype(np.float32)
    y = ref.gemm_epilogue(x, p, "nt", "silu_mul")
    assert np.allclose(y, ref.silu_mul_linear(x, wg, wu), rtol=1e-5, atol=1e-6)


def test_pack_gate_up_matches_package(pkg):
    wg = torch.randn(32, 8)
    wu = torch.randn(32, 8)
    assert np.array_equal(pkg.pack_gate_up(wg, wu).numpy(), ref.pack_gate_up(wg.numpy(), wu.numpy()))


def test_gemm_epilogue_bias_gelu_order():
    # bias is added before GELU (GELU(x + b)), not after
    x = np.ones((1, 4), np.float32)
    w = np.eye(4, dtype=np.float32)
    b = np.full(4, -1.0, np.float32)
    assert np.allclose(ref.gemm_epilogue(x, w, "nt", "bias_gelu_tanh", b), 0.0)


# ---- row reductions -----------------------------------------------------------------


def test_rms_norm_against_torch():
    r = rng(5)
    x = r.standard_normal((127, 513)).astype(np.float32)
    g = r.uniform(0, 1, 513).astype(np.float32)
    t = F.rms_norm(torch.from_numpy(x), (513,), weight=torch.from_numpy(g), eps=1e-5).numpy()
    assert ref.max_rel_err(ref.rms_norm(x, g, 1e-5), t) < 1e-5


def test_rms_norm_closed_forms():
    c = np.float32(3.0)
    row = np.full((1, 64), c, np.float32)
    g = np.linspace(0.5, 1.5, 64).astype(np.float32)
    exp = c / np.sqrt(c * c + np.float32(1e-5)) * g
    assert np.allclose(ref.rms_norm(row, g, 1e-5), exp, rtol=1e-6)
    x = rng(6).standard_normal((4, 64)).astype(np.float32)
    assert np.allclose(ref.rms_norm(7 * x, g, 0.0), ref.rms_norm(x, g, 0.0), rtol=1e-5)
    assert not np.any(ref.rms_norm(np.zeros((2, 8), np.float32), np.ones(8, np.float32), 1e-5))


def test_rms_norm_hf_matches_torch_hf_order():
    r = rng(7)
    x = torch.from_numpy(r.standard_normal((8, 2048)).astype(np.float16))
    g = torch.from_numpy((1 + 0.02 * r.standard_normal(2048)).astype(np.float16))
    xf = x.float()
    hf = g * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.float16)
    out = ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5)
    assert np.max(np.abs(out.astype(np.float32) - hf.float().numpy())) <= 2e-3


def test_softmax_against_torch_and_invariants():
    r = rng(8)
    x = r.standard_normal((128, 197)).astype(np.float32)
    t = F.softmax(torch.from_numpy(x) * 0.125, dim=-1).numpy()
    out = ref.softmax(x, 0.125)
    assert ref.max_rel_err(out, t) < 1e-5
    assert np.allclose(out.sum(-1), 1.0, atol=1e-6)
    assert np.allclose(ref.softmax(x + 5.0), ref.softmax(x), atol=1e-7)  # shift invariance
    assert np.allclose(ref.softmax(np.zeros((1, 197), np.float32)), 1 / 197)
    big = np.zeros((1, 10), np.float32)
    big[0, 3] = 100
    assert ref.softmax(big)[0, 3] > 0.999999


def test_sdpa_against_torch():
    r = rng(9)
    q, k, v = (r.standard_normal((2, 3, 17, 8)).astype(np.float32) for _ in range(3))
    t = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v)).numpy()
    assert np.allclose(ref.sdpa(q, k, v), t, atol=1e-5)
    assert np.allclose(ref.sdpa(q, k, v, 0.125), ref.sdpa(q, k, v, 1 / math.sqrt(64)))


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


def test_sdpa_mask_causal_gqa_against_torch():
    """The mask operand (LowerTmTensor.cpp:158-163), the causal rules and
    grouped K/V heads against torch's own SDPA on the CPU in fp32."""
    r = rng(10)
    b, hq, hkv, s, skv, d = 2, 6, 2, 13, 21, 8
    q = r.standard_normal((b, hq, s, d)).astype(np.float32)
    k, v = (r.standard_normal((b, hkv, skv, d)).astype(np.float32) for _ in range(2))
    m = r.standard_normal((b, 1, s, skv)).astype(np.float32)
    m[0, 0, 3, 5:9] = -np.inf
    t = F.scaled_dot_product_attention(_t(q), _t(k), _t(v), attn_mask=_t(m), scale=0.3, enable_gqa=True).numpy()
    assert np.allclose(ref.sdpa(q, k, v, 0.3, mask=m, kv_group=3), t, atol=1e-5)
    # boolean mask (True = keep) is the additive mask with 0 / -inf
    keep = r.random((s, skv)) > 0.3
    keep[:, 0] = True
    t = F.scaled_dot_product_attention(_t(q[:, :2]), _t(k), _t(v), attn_mask=_t(keep)).numpy()
    add = np.where(keep, 0.0, -np.inf).astype(np.float32)
    assert np.allclose(ref.sdpa(q[:, :2], k, v, mask=add), t, atol=1e-5)
    # causal, top-left (is_causal) and bottom-right (torch's causal_lower_right bias)
    kq = r.standard_normal((b, hkv, skv, d)).astype(np.float32)
    t = F.scaled_dot_product_attention(_t(kq), _t(k), _t(v), is_causal=True).numpy()
    assert np.allclose(ref.sdpa(kq, k, v, causal=1), t, atol=1e-5)
    from torch.nn.attention.bias import causal_lower_right

    qs = r.standard_normal((b, hkv, 5, d)).astype(np.float32)
    t = F.scaled_dot_product_attention(_t(qs), _t(k), _t(v), attn_mask=causal_lower_right(5, skv)).numpy()
    assert np.allclose(ref.sdpa(qs, k, v, causal=2), t, atol=1e-5)


def test_sdpa_mask_closed_forms():
    r = rng(11)
    q, k, v = (r.standard_normal((3, 9, 4)).astype(np.float32) for _ in range(3))
    base = ref.sdpa(q, k, v)
    assert np.allclose(ref.sdpa(q, k, v, mask=np.zeros((9, 9), np.float32)), base, atol=1e-7)
    # a constant added along a whole row changes nothing (shift invariance)
    assert np.allclose(ref.sdpa(q, k, v, mask=np.full((9, 9), 7.5, np.float32)), base, atol=1e-5)
    # only key 4 left: the output is V[4]
    m = np.full((9, 9), -np.inf, np.float32)
    m[:, 4] = 0
    assert np.allclose(ref.sdpa(q, k, v, mask=m), np.broadcast_to(v[:, 4:5], (3, 9, 4)), atol=1e-7)
    # causal: query 0 sees key 0 only
    assert np.allclose(ref.sdpa(q, k, v, causal=1)[:, 0], v[:, 0], atol=1e-7)
    # a row with every key masked is NaN; the other rows are untouched
    m = np.zeros((9, 9), np.float32)
    m[2] = -np.inf
    out = ref.sdpa(q, k, v, mask=m)
    assert np.isnan(out[:, 2]).all() and np.allclose(np.delete(out, 2, 1), np.delete(base, 2, 1), atol=1e-7)


# ---- int8 -------------------------------------------------------------------------------


def test_dequant_exact_for_all_codes():
    codes = np.arange(-128, 128, dtype=np.int8)
    assert np.array_equal(ref.dequant_int8(codes), np.arange(-128, 128, dtype=np.float32))
    # and exact through fp16
    assert np.array_equal(codes.astype(np.float16).astype(np.int32), codes.astype(np.int32))


def test_w8a16_onehot_golden():
    d = np.load(GOLDEN / "w8_onehot.npz")
    q, cols = d["q"], d["cols"]
    x = np.zeros((len(cols), q.shape[1]), np.float16)
    x[np.arange(len(cols)), cols] = 1
    out = ref.w8a16_linear(x, q, np.ones(q.shape[0], np.float16))
    assert np.array_equal(out.astype(np.int32), d["y"])


def test_w8a16_scale_linearity():
    r = rng(10)
    q = r.integers(-127, 128, (32, 64)).astype(np.int8)
    x = r.standard_normal((3, 64)).astype(np.float16)
    s = r.uniform(1e-3, 1e-2, 32).astype(np.float16)
    y1 = ref.w8a16_linear(x, q, np.ones(32, np.float16))
    # scaling the fp32 sum vs scaling the weights differs by fp32 rounding only
    assert ref.max_rel_err(ref.w8a16_linear(x, q, s), y1 * s.astype(np.float32)) < 1e-4
    t = torch.from_numpy(x).float() @ (torch.from_numpy(q).float() * torch.from_numpy(s).float()[:, None]).T
    assert ref.max_rel_err(ref.w8a16_linear(x, q, s), t.numpy()) < 1e-4


# ---- VTCM tile model -----------------------------------------------------------------------


def test_vtcm_tile_model_matches_reference_lit():
    d = np.load(GOLDEN / "tile_model.npz")
    m, k, n = (int(v) for v in d["dims"])
    assert ref.matmul_tile_sizes(m, n, k, 2, 4) == [int(v) for v in d["tile"]]


def test_vtcm_tile_model_fits_and_respects_bounds():
    # config 1 (f16 outs, loop order m,k,n): 6 MiB -> factor 4 -> [256,1024,1024]
    # (3 MiB) -> factor 2 on n -> [256,1024,512] (1.75 MiB)
    t = ref.matmul_tile_sizes(1024, 1024, 1024, 2, 2)
    assert t == [256, 1024, 512]
    fp = lambda t, o: 2 * t[0] * t[1] + 2 * t[1] * t[2] + o * t[0] * t[2]  # noqa: E731
    assert fp(t, 2) <= ref.VTCM_BYTES
    for m, n, k in [(512, 2560, 2048), (512, 11264, 2048), (4096, 4096, 4096), (1576, 3072, 768)]:
        t = ref.matmul_tile_sizes(m, n, k, 2, 2)
        assert fp(t, 2) <= ref.VTCM_BYTES
        assert t[0] >= 4 and t[2] >= 64
    # already fitting: untouched
    assert ref.matmul_tile_sizes(64, 64, 64) == [64, 64, 64]


# ---- tolerance metric ------------------------------------------------------------------------


def test_max_rel_err_catches_planted_mistakes():
    r = rng(11)
    a = r.uniform(-1, 1, (32, 48)).astype(np.float16)
    b = r.uniform(-1, 1, (48, 24)).astype(np.float16)
    good = ref.matmul(a, b)
    assert ref.max_rel_err(good.astype(np.float16), good) < 1e-3
    # transposed operand, dropped k-term, wrong sign of one entry
    assert ref.max_rel_err(ref.matmul(a[:, :24], b[:24]), good) > 1e-2
    bad = good.copy()
    bad[3, 4] = -bad[3, 4]
    assert ref.max_rel_err(bad, good) > 1e-2
    assert ref.max_rel_err(np.full_like(good, np.nan), good) == float("inf")
