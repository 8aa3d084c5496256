"""GPU parity of RMSNorm folded into the following linear layer
(hxmi_rmsnorm_linear_f16 + hxmi_fold_rmsnorm_weight_f16).

The fused op computes linear(x / rms(x), Wg) in fp32 with Wg = fp16(g * W):
the fold is checked bit-exact, the GEMM against the oracle's fp32 RMSNorm
(test/python/triton/test_rms_norm.py:37-63) applied with the folded weight
(elementwise max relative error), and the whole against the unfused HF order
(HF LlamaRMSNorm rounds the normalised activations to fp16 before the
weight and the linear layer) relative to the output scale: the two differ by
that fp16 rounding, ~1e-4 absolute."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import TOL, normal, np32
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

TILES = list(range(16))  # every GEMM tile shape (TileId)


def check(y, x, wf_cpu, exp_hf, eps, epi=None):
    """y against the fp32 oracle on the folded weight (elementwise) and against
    the unfused HF-order oracle (relative to the output scale)."""
    xn = ref.rms_norm(x.numpy(), np.ones(x.shape[-1], np.float32), eps)
    if epi == "silu_mul":
        wfu = ref.unpack_gate_up_cols(np32(wf_cpu).T, wf_cpu.shape[0])  # gate [K, I], up [K, I]
        exact = ref.silu_mul_linear(xn, wfu[0].T, wfu[1].T)
    else:
        exact = ref.linear(xn, np32(wf_cpu))
    assert ref.max_rel_err(np32(y), exact) <= TOL
    assert ref.max_err_vs_scale(np32(y), exp_hf) <= TOL


def _norm_weight(K, seed):
    return (1 + 0.02 * torch.randn(K, generator=torch.Generator().manual_seed(seed))).half()


def test_fold_weight_is_one_fp16_rounding(pkg, dev):
    w = normal((300, 520), 1, 0.02)
    g = _norm_weight(520, 2)
    wf = pkg.fold_rms_weight(w.to(dev), g.to(dev)).cpu()
    exp = (np32(w) * np32(g)[None, :]).astype(np.float16)
    assert np.array_equal(wf.numpy(), exp)


@pytest.mark.parametrize("N,K", [(2560, 2048), (2048, 2048)])  # TinyLlama QKV and O-sized
def test_rms_norm_linear_tinyllama(pkg, dev, N, K):
    x = normal((512, K), 3)
    g = _norm_weight(K, 4)
    w = normal((N, K), 5, 0.02)
    wf = pkg.fold_rms_weight(w.to(dev), g.to(dev))
    y = pkg.rms_norm_linear(x.to(dev), wf, 1e-5).cpu()
    check(y, x, wf.cpu(), ref.linear(ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5), w.numpy()), 1e-5)


def test_rms_norm_gate_up_silu_mul(pkg, dev):
    M, I, K = 512, 1408, 2048
    x = normal((M, K), 6)
    g = _norm_weight(K, 7)
    wg = normal((I, K), 8, 0.02)
    wu = normal((I, K), 9, 0.02)
    wf = pkg.fold_rms_weight(pkg.pack_gate_up(wg.to(dev), wu.to(dev)), g.to(dev))
    h = pkg.rms_norm_linear(x.to(dev), wf, 1e-5, epilogue="silu_mul").cpu()
    xn = ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5)
    check(h, x, wf.cpu(), ref.silu_mul_linear(xn, wg.numpy(), wu.numpy()), 1e-5, "silu_mul")


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("epi", [None, "silu_mul"])
def test_rms_norm_linear_every_tile(pkg, dev, force_tile, tile, epi):
    force_tile(tile)
    M, N, K = 200, 320, 264
    x = normal((M, K), 10)
    g = _norm_weight(K, 11)
    if epi is None:
        w = normal((N, K), 12, 0.05)
        exp_fn = lambda xn: ref.linear(xn, w.numpy())  # noqa: E731
        wp = w.to(dev)
    else:
        wg, wu = normal((N // 2, K), 13, 0.05), normal((N // 2, K), 14, 0.05)
        exp_fn = lambda xn: ref.silu_mul_linear(xn, wg.numpy(), wu.numpy())  # noqa: E731
        wp = pkg.pack_gate_up(wg.to(dev), wu.to(dev))
    wf = pkg.fold_rms_weight(wp, g.to(dev))
    y = pkg.rms_norm_linear(x.to(dev), wf, 1e-5, epilogue=epi).cpu()
    check(y, x, wf.cpu(), exp_fn(ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5)), 1e-5, epi)


@pytest.mark.parametrize("M,N,K", [(3, 40, 45), (33, 72, 1000), (1, 8, 8)])
def test_rms_norm_linear_ragged_and_unaligned(pkg, dev, M, N, K):
    # K % 8 != 0 runs the element-wise kernel, which applies the same row scale
    x = normal((M, K), 15)
    g = _norm_weight(K, 16)
    w = normal((N, K), 17, 0.05)
    wf = pkg.fold_rms_weight(w.to(dev), g.to(dev))
    y = pkg.rms_norm_linear(x.to(dev), wf, 1e-6).cpu()
    check(y, x, wf.cpu(), ref.linear(ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-6), w.numpy()), 1e-6)


def test_rms_norm_linear_zero_row_and_scale_invariance(pkg, dev):
    """A zero row stays zero; scaling a row by 4 (exact in fp16) leaves its
    output unchanged up to eps: the normalisation really is per row."""
    M, N, K = 64, 256, 512
    x = normal((M, K), 18)
    x[5] = 0
    x4 = x.clone()
    x4[7] *= 4
    g = _norm_weight(K, 19)
    wf = pkg.fold_rms_weight(normal((N, K), 20, 0.05).to(dev), g.to(dev))
    y = pkg.rms_norm_linear(x.to(dev), wf, 1e-12).cpu()
    y4 = pkg.rms_norm_linear(x4.to(dev), wf, 1e-12).cpu()
    assert torch.count_nonzero(y[5]) == 0
    assert ref.max_rel_err(np32(y4[7]), np32(y[7])) <= 1e-3
    assert torch.equal(y4[:7], y[:7])


def test_rms_norm_linear_rejects_gelu_epilogue(pkg, dev):
    lib = pkg.load_library()
    t = torch.zeros(64, 64, dtype=torch.float16, device=dev)
    rc = lib.hxmi_rmsnorm_linear_f16(t.data_ptr(), t.data_ptr(), t.data_ptr(), None, 64, 64, 64, 64, 64, 64, 3,
                                     ctypes.c_float(1e-5), None, None, None)
    assert rc == 1 and b"epilogue" in lib.hxmi_last_error()
    r = torch.zeros(64, dtype=torch.float32, device=dev)
    rc = lib.hxmi_rmsnorm_linear_f16(t.data_ptr(), t.data_ptr(), t.data_ptr(), None, 64, 64, 64, 64, 64, 64, 0,
                                     ctypes.c_float(1e-5), r.data_ptr(), r.data_ptr(), None)
    assert rc == 1 and b"exclusive" in lib.hxmi_last_error()


def _rscale(x, eps):
    xf = np32(x).astype(np.float64)
    return (1.0 / np.sqrt((xf * xf).mean(axis=1) + eps)).astype(np.float32)


@pytest.mark.parametrize("tile", TILES)
def test_rscale_out_every_tile(pkg, dev, force_tile, tile):
    # the first column of tiles writes each row's rsqrt(mean(x^2) + eps)
    force_tile(tile)
    M, N, K = 300, 256, 520
    x = normal((M, K), 21)
    wf = pkg.fold_rms_weight(normal((N, K), 22, 0.05).to(dev), _norm_weight(K, 23).to(dev))
    rs = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    pkg.rms_norm_linear(x.to(dev), wf, 1e-5, rscale_out=rs)
    assert np.allclose(rs.cpu().numpy(), _rscale(x, 1e-5), rtol=1e-5, atol=0)


def test_rscale_out_elementwise_path(pkg, dev):
    M, N, K = 33, 72, 1000 + 3  # K % 8 != 0: element-wise kernel
    x = normal((M, K), 24)
    wf = pkg.fold_rms_weight(normal((N, K), 25, 0.05).to(dev), _norm_weight(K, 26).to(dev))
    rs = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    pkg.rms_norm_linear(x.to(dev), wf, 1e-6, rscale_out=rs)
    assert np.allclose(rs.cpu().numpy(), _rscale(x, 1e-6), rtol=1e-5, atol=0)


@pytest.mark.parametrize("tile", [None, 4, 11, 13])
@pytest.mark.parametrize("M,K", [(512, 2048), (200, 264), (7, 1003)])
def test_rscale_in_second_consumer(pkg, dev, force_tile, tile, M, K):
    """QKV computes the row scales, gate/up (SiLU-mul) reuses them: same
    result as recomputing the statistics, against the exact oracle."""
    if tile is not None:
        force_tile(tile)
    I = 160
    x = normal((M, K), 27)
    g = _norm_weight(K, 28)
    wq = normal((96, K), 29, 0.05)
    wg, wu = normal((I, K), 30, 0.05), normal((I, K), 31, 0.05)
    xd = x.to(dev)
    wqf = pkg.fold_rms_weight(wq.to(dev), g.to(dev))
    wguf = pkg.fold_rms_weight(pkg.pack_gate_up(wg.to(dev), wu.to(dev)), g.to(dev))
    rs = torch.empty(M, dtype=torch.float32, device=dev)
    q = pkg.rms_norm_linear(xd, wqf, 1e-5, rscale_out=rs).cpu()
    h = pkg.rms_norm_linear(xd, wguf, 1e-5, epilogue="silu_mul", rscale_in=rs).cpu()
    h_rms = pkg.rms_norm_linear(xd, wguf, 1e-5, epilogue="silu_mul").cpu()
    xn = ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5)
    check(q, x, wqf.cpu(), ref.linear(xn, wq.numpy()), 1e-5)
    check(h, x, wguf.cpu(), ref.silu_mul_linear(xn, wg.numpy(), wu.numpy()), 1e-5, "silu_mul")
    assert ref.max_rel_err(np32(h), np32(h_rms)) <= 1e-3


@pytest.mark.parametrize("tile", TILES)
def test_rms_norm_linear_bias_every_tile(pkg, dev, force_tile, tile):
    """Qwen2-style q/k/v: RMSNorm, then a projection with bias; the first
    projection takes the statistics, the next reuses its row scales."""
    force_tile(tile)
    M, K = 200, 264
    x = normal((M, K), 32)
    g = _norm_weight(K, 33)
    wq, wk = normal((128, K), 34, 0.05), normal((64, K), 35, 0.05)
    bq, bk = normal((128,), 36, 0.5), normal((64,), 37, 0.5)
    xd = x.to(dev)
    wqf = pkg.fold_rms_weight(wq.to(dev), g.to(dev))
    wkf = pkg.fold_rms_weight(wk.to(dev), g.to(dev))
    rs = torch.empty(M, dtype=torch.float32, device=dev)
    q = pkg.rms_norm_linear(xd, wqf, 1e-6, bias=bq.to(dev), rscale_out=rs).cpu()
    k = pkg.rms_norm_linear(xd, wkf, 1e-6, bias=bk.to(dev), rscale_in=rs).cpu()
    xn = ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-6)
    xn_exact = ref.rms_norm(x.numpy(), np.ones(K, np.float32), 1e-6)
    for y, wf, w, b in ((q, wqf, wq, bq), (k, wkf, wk, bk)):
        assert ref.max_rel_err(np32(y), ref.linear(xn_exact, np32(wf.cpu()), b.numpy())) <= TOL
        assert ref.max_err_vs_scale(np32(y), ref.linear(xn, w.numpy(), b.numpy())) <= TOL


# ---- bf16 -------------------------------------------------------------------------------------------


def test_fold_weight_bf16_is_one_rounding(pkg, dev):
    w = normal((300, 520), 21, 0.02, dtype=torch.bfloat16)
    g = (1 + 0.02 * torch.randn(520, generator=torch.Generator().manual_seed(22))).to(torch.bfloat16)
    wf = pkg.fold_rms_weight(w.to(dev), g.to(dev)).cpu()
    exp = (w.float() * g.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(wf, exp)


def test_rms_norm_linear_bf16_block_pair(pkg, dev):
    """The TinyLlama QKV call (statistics in the GEMM, row scales published)
    and gate/up with SiLU-mul reusing them, in bf16."""
    M, K, N, I = 512, 2048, 2560, 1408
    bf = torch.bfloat16
    x = normal((M, K), 23, dtype=bf)
    g = (1 + 0.02 * torch.randn(K, generator=torch.Generator().manual_seed(24))).to(bf)
    w = normal((N, K), 25, 0.02, dtype=bf)
    wg, wu = normal((I, K), 26, 0.02, dtype=bf), normal((I, K), 27, 0.02, dtype=bf)
    wf = pkg.fold_rms_weight(w.to(dev), g.to(dev))
    wguf = pkg.fold_rms_weight(pkg.pack_gate_up(wg.to(dev), wu.to(dev)), g.to(dev))
    rs = torch.empty(M, dtype=torch.float32, device=dev)
    y = pkg.rms_norm_linear(x.to(dev), wf, 1e-5, rscale_out=rs)
    h = pkg.rms_norm_linear(x.to(dev), wguf, 1e-5, epilogue="silu_mul", rscale_in=rs)
    torch.cuda.synchronize()
    assert y.dtype == bf and h.dtype == bf
    xf = np32(x)
    r = 1.0 / np.sqrt((xf * xf).mean(-1) + 1e-5)
    assert np.allclose(rs.cpu().numpy(), r, rtol=1e-5)
    xn = ref.rms_norm(xf, np.ones(K, np.float32), 1e-5)
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(xn, np32(wf.cpu()))) <= TOL
    wfu = ref.unpack_gate_up_cols(np32(wguf.cpu()).T, wguf.shape[0])
    assert ref.max_rel_err(np32(h.cpu()), ref.silu_mul_linear(xn, wfu[0].T, wfu[1].T)) <= TOL
