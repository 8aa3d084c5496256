"""GPU parity of the decode GEMV and the weight-only int8 linear."""
import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import TOL, normal, np32
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

# Qwen2.5-0.5B decode shapes (K, N): q/o, k/v, gate/up, down, lm_head
QWEN = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936)]


@pytest.mark.parametrize("K,N", QWEN)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_qwen_shapes(pkg, dev, M, K, N):
    x = normal((M, K), 100 + M)
    w = normal((N, K), 200 + K % 7, 0.02)
    y = pkg.gemv(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy())) <= TOL


@pytest.mark.parametrize("M,N,K", [(3, 100, 64), (16, 52, 136), (7, 1000, 4104), (1, 4, 8)])
def test_gemv_ragged(pkg, dev, M, N, K):
    x = normal((M, K), 1)
    w = normal((N, K), 2, 0.05)
    b = normal((N,), 3)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


def test_gemv_unaligned_falls_back(pkg, dev):
    x = normal((2, 45), 4)
    w = normal((30, 45), 5, 0.05)
    y = pkg.gemv(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy())) <= TOL


def test_gemv_large_m_uses_gemm(pkg, dev):
    x = normal((40, 896), 6)
    w = normal((256, 896), 7, 0.02)
    y = pkg.gemv(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy())) <= TOL


def int8_weights(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 9e-3 + 1e-3).half()
    return q, s


@pytest.mark.parametrize("K,N", QWEN)
@pytest.mark.parametrize("M", [1, 16, 256])
def test_w8a16_qwen_shapes(pkg, dev, M, K, N):
    x = normal((M, K), 300 + M)
    q, s = int8_weights(N, K, 400 + K % 5)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy())) <= TOL


@pytest.fixture
def gemv_path(monkeypatch):
    """Force the decode kernel: "mfma" (16-row MFMA tiles) or "valu" (row streaming)."""

    def force(path):
        monkeypatch.setenv("HXMI_GEMV_PATH", path)

    return force


@pytest.mark.parametrize("path", ["mfma", "valu"])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("N,K", [(4100, 904), (1028, 136), (8, 64)])
def test_gemv_both_paths(pkg, dev, gemv_path, path, M, N, K):
    gemv_path(path)
    x = normal((M, K), 11 + M)
    w = normal((N, K), 12, 0.05)
    b = normal((N,), 13)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("path", ["mfma", "valu"])
@pytest.mark.parametrize("M", [1, 3, 8])
@pytest.mark.parametrize("N,K", [(4104, 912), (264, 144)])
def test_w8a16_both_paths(pkg, dev, gemv_path, path, M, N, K):
    gemv_path(path)
    x = normal((M, K), 21 + M)
    q, s = int8_weights(N, K, 22)
    b = normal((N,), 23)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("path", ["mfma", "valu"])
def test_w8a16_onehot_exact_both_paths(pkg, dev, gemv_path, path):
    gemv_path(path)
    d = np.load(GOLDEN / "w8_onehot.npz")
    q, cols = torch.from_numpy(d["q"]), d["cols"]
    M = 5
    rows = np.resize(np.arange(len(cols)), M)
    x = torch.zeros((M, q.shape[1]), dtype=torch.float16)
    x[np.arange(M), cols[rows]] = 1
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), torch.ones(q.shape[0], dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.int32), d["y"][rows])


@pytest.mark.parametrize("M", [5, 64])
def test_w8a16_onehot_is_exact(pkg, dev, M):
    # scale 1 and one-hot activations: y must be the int8 weight column itself
    d = np.load(GOLDEN / "w8_onehot.npz")
    q, cols = torch.from_numpy(d["q"]), d["cols"]
    rows = np.resize(np.arange(len(cols)), M)
    x = torch.zeros((M, q.shape[1]), dtype=torch.float16)
    x[np.arange(M), cols[rows]] = 1
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), torch.ones(q.shape[0], dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.int32), d["y"][rows])


def test_w8a16_all_codes_exact(pkg, dev):
    # every int8 code in every position of a 16-byte load
    q = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).reshape(16, 16).repeat(1, 4)  # [16, 64]
    x = torch.zeros((16, 64), dtype=torch.float16)
    for m in range(16):
        x[m, m * 4] = 1  # picks column 4m
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), torch.ones(16, dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    exp = q.numpy().astype(np.int32)[:, [4 * m for m in range(16)]].T
    assert np.array_equal(y.cpu().numpy().astype(np.int32), exp)


def test_w8a16_bias_and_scale_linearity(pkg, dev):
    x = normal((16, 896), 8)
    q, s = int8_weights(512, 896, 9)
    b = normal((512,), 10)
    y1 = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    y2 = pkg.w8a16_linear(x.to(dev), q.to(dev), (2 * s).to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y1.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL
    assert ref.max_rel_err(np32(y2.cpu()), 2 * ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy())) <= TOL
