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


@pytest.mark.parametrize("M,N", [(128, 151936), (200, 151936), (256, 133144)])
def test_w8a16_many_tiles_with_bias(pkg, dev, M, N):
    # one row of output tiles over more tiles than a round of workgroups,
    # with a ragged last tile column and the bias epilogue
    K = 896
    x = normal((M, K), 500 + M)
    q, s = int8_weights(N, K, 501)
    b = normal((N,), 502)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    want = ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())
    assert ref.max_rel_err(np32(y.cpu()), want) <= TOL


@pytest.fixture
def gemv_path(knobs):
    """Force the decode kernel: "mfma" (16-row MFMA tiles, K split over
    waves), "valu" (row streaming) or "pair" (8-row tiles, whole-line
    loads, each row read as two MFMA rows, K <= 1024)."""

    def force(path):
        knobs(gemv_path=path)

    return force


@pytest.mark.parametrize("path", ["mfma", "valu", "pair"])
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


@pytest.mark.parametrize("path", ["mfma", "valu", "pair"])
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


@pytest.mark.parametrize("path", ["mfma", "valu", "pair"])
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


@pytest.fixture
def gemv_kgroups(knobs):
    """Force the number of workgroups that split K per row group (1 = unsplit)."""

    def force(kg):
        knobs(gemv_path="mfma", gemv_kg=kg)

    return force


@pytest.mark.parametrize("kg", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("N,K", [(896, 4864), (72, 4104), (8, 8200)])
def test_gemv_k_groups(pkg, dev, gemv_kgroups, kg, M, N, K):
    # K split over workgroups that combine fp32 partial tiles in the workspace;
    # ragged K groups (K not a multiple of kg steps) and a partial 16-row tile
    gemv_kgroups(kg)
    x = normal((M, K), 31 + M)
    w = normal((N, K), 32, 0.05)
    b = normal((N,), 33)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("kg", [2, 5, 8])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_w8a16_k_groups(pkg, dev, gemv_kgroups, kg, M):
    gemv_kgroups(kg)
    N, K = 904, 4864
    x = normal((M, K), 41 + M)
    q, s = int8_weights(N, K, 42)
    b = normal((N,), 43)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL


def test_w8a16_onehot_exact_k_groups(pkg, dev, gemv_kgroups):
    # one-hot rows land in one K group; the others add exact zeros
    gemv_kgroups(4)
    d = np.load(GOLDEN / "w8_onehot.npz")
    q, cols = torch.from_numpy(d["q"]), d["cols"]
    M = 5
    rows = np.resize(np.arange(len(cols)), M)
    x = torch.zeros((M, q.shape[1]), dtype=torch.float16)
    x[np.arange(M), cols[rows]] = 1
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), torch.ones(q.shape[0], dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.int32), d["y"][rows])


def test_gemv_long_k_splits_by_default(pkg, dev):
    """A long-K GEMV on 2560 rows (8192 -> 2560) splits K over workgroups by
    default; the result is deterministic (partials are added in K-group
    order) and one workspace serves calls of different shapes back to back."""
    lib = pkg.load_library()
    N, K = 2560, 8192
    assert lib.hxmi_gemv_workspace_bytes(1, N, K) > 0
    assert lib.hxmi_gemv_workspace_bytes(1, 4864, 896) == 0
    nbytes = max(lib.hxmi_gemv_workspace_bytes(m, N, K) for m in (1, 16))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)  # counters zero before first use
    w = normal((N, K), 51, 0.05).to(dev)
    outs = []
    for M in (1, 16, 1, 16, 1):
        x = normal((M, K), 52 + M).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        rc = lib.hxmi_gemv_f16(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K, K, K, N,
                               ws.data_ptr(), nbytes, None)
        assert rc == 0, lib.hxmi_last_error()
        outs.append(y.cpu())
        assert ref.max_rel_err(np32(outs[-1]), ref.linear(x.cpu().numpy(), w.cpu().numpy())) <= TOL
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[0], outs[4]) and torch.equal(outs[1], outs[3])


def test_gemv_k_groups_graph_replays(pkg, dev):
    """Captured split-K GEMV: the arrival counters reset themselves, so every
    replay (with eager calls on the same workspace between them) matches."""
    M, N, K = 1, 2560, 8192
    lib = pkg.load_library()
    nbytes = lib.hxmi_gemv_workspace_bytes(M, N, K)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)  # counters zero before first use
    x = normal((M, K), 61).to(dev)
    w = normal((N, K), 62, 0.05).to(dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()

    def call(stream):
        rc = lib.hxmi_gemv_f16(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K, K, K, N, ws.data_ptr(),
                               nbytes, stream)
        assert rc == 0, lib.hxmi_last_error()

    call(None)
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(s.cuda_stream)
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        call(None)  # eager call between replays, same workspace
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


@pytest.mark.parametrize("M", [1, 7, 16])
@pytest.mark.parametrize("N,K", [(2056, 1024), (40, 8), (300, 520), (33000, 896), (1004, 72), (151936, 896)])
def test_gemv_pair(pkg, dev, gemv_path, M, N, K):
    # x staged for the whole K: K up to 1024, ragged 128-byte windows and
    # 8-row tiles, more tiles than waves (each wave strides over several),
    # the lm_head shape
    gemv_path("pair")
    x = normal((M, K), 71 + M)
    w = normal((N, K), 72, 0.05)
    b = normal((N,), 73)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("M", [7, 16])
@pytest.mark.parametrize("wg", [8, 3])
def test_gemv_pair_many_tiles_per_wave(pkg, dev, gemv_path, knobs, M, wg):
    """With few workgroups every wave walks many 8-row tiles: at M > 4 the
    first 6 tiles' outputs are held back until the wave's last tile and the
    later ones are stored as they finish; both halves must land."""
    gemv_path("pair")
    knobs(gemv_pair_wg=wg)
    N, K = 8192 + 40, 896
    x = normal((M, K), 74 + M)
    w = normal((N, K), 75, 0.05)
    b = normal((N,), 76)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("M", [1, 16])
def test_gemv_pair_strided_output_keeps_padding(pkg, dev, gemv_path, M):
    """fp16 whole-line kernel writing into a wider row-major buffer: the
    result lands in the first N columns and the padding is untouched."""
    gemv_path("pair")
    N, K, ldy = 8192 + 24, 640, 8192 + 64
    x = normal((M, K), 77 + M)
    w = normal((N, K), 78, 0.05)
    buf = torch.full((M, ldy), -7.0, dtype=torch.float16, device=dev)
    pkg.gemv(x.to(dev), w.to(dev), out=buf[:, :N])
    torch.cuda.synchronize()
    got = buf.cpu()
    assert ref.max_rel_err(np32(got[:, :N]), ref.linear(x.numpy(), w.numpy())) <= TOL
    assert torch.all(got[:, N:] == -7.0)


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("N,K", [(2056, 1024), (24, 16), (33000, 896), (1000, 144)])
def test_w8a16_pair(pkg, dev, gemv_path, M, N, K):
    gemv_path("pair")
    x = normal((M, K), 81 + M)
    q, s = int8_weights(N, K, 82)
    b = normal((N,), 83)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("M", [9, 16])
@pytest.mark.parametrize("N,K", [(2056, 1024), (40, 8), (33000, 896)])
def test_gemv_valu_two_row_blocks(pkg, dev, gemv_path, M, N, K):
    # M > 8 on the row-streaming kernel: lanes write rows c and c + 8
    gemv_path("valu")
    x = normal((M, K), 91 + M)
    w = normal((N, K), 92, 0.05)
    y = pkg.gemv(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy())) <= TOL


def test_gemv_k_groups_workspace_counters_return_to_zero(pkg, dev, gemv_kgroups):
    """K groups meet on per-tile counters at the workspace's head: zero when a
    call starts, zero again when it ends, whatever the partial area holds."""
    gemv_kgroups(3)
    lib = pkg.load_library()
    M, N, K = 4, 896, 4864
    nbytes = lib.hxmi_gemv_workspace_bytes(M, N, K)
    cwords = 16384 // 8  # HXMI_WORKSPACE_COUNTER_BYTES of 64-bit counters
    assert nbytes > cwords * 8
    ws = torch.zeros(nbytes // 8, dtype=torch.int64, device=dev)
    ws[cwords:] = (torch.arange(nbytes // 8 - cwords, device=dev) % 5) | (1 << 8)
    x, w = normal((M, K), 70).to(dev), normal((N, K), 71, 0.05).to(dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    exp = ref.linear(x.cpu().numpy(), w.cpu().numpy())
    for _ in range(3):
        rc = lib.hxmi_gemv_f16(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K, K, K, N, ws.data_ptr(),
                               nbytes, None)
        assert rc == 0, lib.hxmi_last_error()
        torch.cuda.synchronize()
        assert int(ws[:cwords].abs().sum()) == 0
        assert ref.max_rel_err(np32(y.cpu()), exp) <= TOL


@pytest.mark.parametrize("ks", ["8", "16"])
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("N,K", [(896, 4864), (2048, 5632), (1004, 2056), (40, 8), (300, 1288)])
def test_gemv_pair_ksplit(pkg, dev, gemv_path, knobs, ks, M, N, K):
    # whole-line loads with K split over the workgroup's waves: down
    # projections, ragged windows and 8-row tiles, waves left without K
    gemv_path("ksplit")
    knobs(gemv_ks=int(ks))
    x = normal((M, K), 91 + M)
    w = normal((N, K), 92, 0.05)
    b = normal((N,), 93)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(x.numpy(), w.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("ks", ["8", "16"])
@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("N,K", [(896, 4864), (1000, 2064), (24, 16)])
def test_w8a16_pair_ksplit(pkg, dev, gemv_path, knobs, ks, M, N, K):
    gemv_path("ksplit")
    knobs(gemv_ks=int(ks))
    x = normal((M, K), 95 + M)
    q, s = int8_weights(N, K, 96)
    b = normal((N,), 97)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL


def test_w8a16_onehot_exact_pair_ksplit(pkg, dev, gemv_path):
    gemv_path("ksplit")
    d = np.load(GOLDEN / "w8_onehot.npz")
    q, cols = torch.from_numpy(d["q"]), d["cols"]
    M = 5
    rows = np.resize(np.arange(len(cols)), M)
    x = torch.zeros((M, q.shape[1]), dtype=torch.float16)
    x[np.arange(M), cols[rows]] = 1
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), torch.ones(q.shape[0], dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.int32), d["y"][rows])


@pytest.mark.parametrize("M", [1, 16])
def test_w8a16_pair_ragged_rows_strided_out(pkg, dev, gemv_path, M):
    # N % 8 == 4 (a half-empty last 8-row tile: its scale and bias loads run
    # past N and must read zero), output rows with a leading dimension > N
    gemv_path("pair")
    N, K = 1004, 896
    x = normal((M, K), 101 + M)
    q, s = int8_weights(N, K, 102)
    b = normal((N,), 103)
    big = torch.full((M, 1008), 7.0, dtype=torch.float16, device=dev)
    y = big[:, :N]
    pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev), out=y)
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL
    assert torch.all(big[:, N:].cpu() == 7.0)  # nothing written past N


# ---- bf16 -------------------------------------------------------------------------------------------


@pytest.mark.parametrize("K,N", QWEN)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_bf16_qwen_shapes(pkg, dev, M, K, N):
    """bf16 activations and weights on the same kernels and plans as fp16
    (bf16 MFMA / v_dot2_f32_bf16), fp32 accumulation, bf16 out."""
    x = normal((M, K), 300 + M, dtype=torch.bfloat16)
    w = normal((N, K), 400 + K % 7, 0.02, dtype=torch.bfloat16)
    y = pkg.gemv(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(np32(x), np32(w))) <= TOL


@pytest.mark.parametrize("path", ["mfma", "valu", "pair", "ksplit"])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_gemv_bf16_every_kernel(pkg, dev, knobs, path, M):
    """Each of the four GEMV kernels forced in turn, with a bias, on a shape
    every one of them takes (K <= 1024 for the whole-line kernel, ragged N)."""
    knobs(gemv_path=path)
    K, N = 1024 if path != "ksplit" else 2048, 1020
    x = normal((M, K), 11, dtype=torch.bfloat16)
    w = normal((N, K), 12, 0.03, dtype=torch.bfloat16)
    b = normal((N,), 13, dtype=torch.bfloat16)
    y = pkg.gemv(x.to(dev), w.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.linear(np32(x), np32(w), np32(b))) <= TOL


def test_gemv_bf16_exact_integers(pkg, dev):
    """Small integers are exact in bf16 and their sums exact in fp32: every
    output bf16-rounds the exact product."""
    g = torch.Generator().manual_seed(14)
    x = torch.randint(-3, 4, (4, 896), generator=g).to(torch.bfloat16)
    w = torch.randint(-3, 4, (2048, 896), generator=g).to(torch.bfloat16)
    y = pkg.gemv(x.to(dev), w.to(dev)).cpu()
    exact = (x.double() @ w.double().T).to(torch.bfloat16)
    assert torch.equal(y, exact)


@pytest.mark.parametrize("M", [64, 256])
@pytest.mark.parametrize("N,K", [(264, 144), (520, 912), (4104, 208), (896, 848)])
def test_w8a16_gemm_k_not_a_multiple_of_the_k_step(pkg, dev, M, N, K):
    """The int8-weight MFMA GEMM (M > 16) reads each 16-byte chunk of int8
    codes once per pair of 16-deep substeps; a K that ends inside a 64-deep
    step leaves chunks past K, which must read as zero, in the last step.
    (896x848 at M = 256 takes the short-K split path, slices of >= 256.)"""
    x = normal((M, K), 61 + M)
    q, s = int8_weights(N, K, 62)
    b = normal((N,), 63)
    y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev), bias=b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.w8a16_linear(x.numpy(), q.numpy(), s.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("tile", [None, 3, 4, 5, 6, 8, 12, 13])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_w8a16_gemm_integer_exact_every_tile(pkg, dev, tile, splits):
    """Small-integer activations, int8 codes and unit scales: every fp32 sum
    is exact, so each tile shape and K split must return the exactly rounded
    product (the codes' k order in the paired reads must match the
    activations' in every substep)."""
    g = torch.Generator().manual_seed(64)
    M, N, K = 96, 200, 784  # K % 64 = 16; K >= 512 so a K split applies
    x = torch.randint(-3, 4, (M, K), generator=g).half()
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.ones(N, dtype=torch.float16)
    with pkg.tuning(w8_tile=tile, splitk=splits):
        y = pkg.w8a16_linear(x.to(dev), q.to(dev), s.to(dev))
        torch.cuda.synchronize()
    exact = x.double() @ q.double().T
    assert np.array_equal(y.cpu().numpy(), exact.numpy().astype(np.float16))
