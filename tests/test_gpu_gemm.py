"""GPU parity of the MFMA GEMM (through the C ABI) against the oracle."""
import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import TOL, f16_round, normal, np32, uniform
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

TILES = list(range(16))  # every instantiated tile shape (TileId)
NT_ONLY = {14}  # 128x192 takes k-contiguous B only (a forced override of it in NN runs the picker's tile)


def skip_nn(tile, layout):
    if layout == "nn" and tile in NT_ONLY:
        pytest.skip("128x192 tile: k-contiguous B only")


def run_gemm(pkg, dev, a, b, layout, **kw):
    out = pkg.gemm(a.to(dev), b.to(dev), b_layout=layout, **kw)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("seed_a, seed_b", [(0, 1)])
def test_config1_gemm_1024_nn(pkg, dev, seed_a, seed_b):
    # single fp16 GEMM C = A.B, M=N=K=1024, U[-1,1], fp32 acc, fp16 out
    a = uniform((1024, 1024), seed_a)
    b = uniform((1024, 1024), seed_b)
    c = run_gemm(pkg, dev, a, b, "nn")
    assert ref.max_rel_err(np32(c), ref.matmul(a.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("tile", TILES)
def test_gemm_exact_integer_every_tile(pkg, dev, force_tile, layout, tile):
    skip_nn(tile, layout)
    d = np.load(GOLDEN / f"gemm_int_{layout}.npz")
    force_tile(tile)
    a = torch.from_numpy(d["a"]).half()
    b = torch.from_numpy(d["b"]).half()
    c = run_gemm(pkg, dev, a, b, layout)
    assert np.array_equal(c.numpy(), f16_round(d["c"])), f"tile {tile}"


@pytest.mark.parametrize("tile", TILES)
def test_gemm_bias_exact_every_tile(pkg, dev, force_tile, tile):
    d = np.load(GOLDEN / "gemm_int_epi.npz")
    force_tile(tile)
    a, b = torch.from_numpy(d["a"]).half(), torch.from_numpy(d["b"]).half()
    bias = torch.from_numpy(d["bias"]).half()
    c = run_gemm(pkg, dev, a, b, "nt", epilogue="bias", bias=bias.to(dev))
    assert np.array_equal(c.numpy(), f16_round(d["c"]))


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (33, 72, 40), (130, 264, 200), (300, 136, 520), (197, 64, 64),
                                   (64, 64, 0), (5, 24, 8)])
@pytest.mark.parametrize("tile", [None, 0, 3, 6, 7, 8, 9, 10, 11, 12, 13])
def test_gemm_ragged_shapes(pkg, dev, force_tile, layout, M, N, K, tile):
    force_tile(tile)
    a = uniform((M, K), 2)
    b = uniform((K, N) if layout == "nn" else (N, K), 3)
    c = run_gemm(pkg, dev, a, b, layout)
    assert ref.max_rel_err(np32(c), ref.matmul(a.numpy(), b.numpy(), layout)) <= TOL


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("M,N,K,lda", [(37, 45, 29, 29), (16, 16, 197, 197), (20, 33, 24, 31)])
def test_gemm_unaligned_elementwise_path(pkg, dev, layout, M, N, K, lda):
    a_full = uniform((M, lda), 4)
    a = a_full[:, :K]
    b = uniform((K, N) if layout == "nn" else (N, K), 5)
    c = pkg.gemm(a_full.to(dev)[:, :K], b.to(dev), b_layout=layout)
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(c.cpu()), ref.matmul(a.numpy(), b.numpy(), layout)) <= TOL


def _nan_padded(t, cols):
    """t as the leading columns of a wider buffer whose other columns are NaN:
    any read of them that reaches a result shows up as NaN."""
    full = torch.full((t.shape[0], cols), float("nan"), dtype=t.dtype)
    full[:, : t.shape[1]] = t
    return full


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("M,N,K", [(5, 24, 1), (33, 40, 3), (64, 72, 13), (130, 264, 197), (300, 136, 517),
                                   (1024, 1024, 999), (197, 197, 197), (7, 9, 11)])
def test_gemm_ragged_k_and_n_on_mfma(pkg, dev, layout, M, N, K):
    """K and N not multiples of 8 on the MFMA path: operands are views of
    NaN-padded buffers (leading dims rounded up to 8), so an element past K
    that reaches a sum, or a store past N, is caught."""
    k8, n8 = (K + 7) // 8 * 8, (N + 7) // 8 * 8
    a = uniform((M, K), 31)
    b = uniform((K, N) if layout == "nn" else (N, K), 32)
    ap = _nan_padded(a, k8).to(dev)
    bp = (_nan_padded(b, n8) if layout == "nn" else _nan_padded(b, k8)).to(dev)
    outp = torch.full((M, n8), 7.0, dtype=torch.float16, device=dev)
    pkg.gemm(ap[:, :K], bp[:, : b.shape[1]], b_layout=layout, out=outp[:, :N])
    torch.cuda.synchronize()
    c = outp.cpu()
    assert ref.max_rel_err(np32(c[:, :N]), ref.matmul(a.numpy(), b.numpy(), layout)) <= TOL
    assert (c[:, N:] == 7.0).all()  # padding columns untouched


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("K", [1, 5, 197])
def test_gemm_ragged_k_exact_integer(pkg, dev, layout, K):
    """Small integers give exact fp32 sums: the ragged-K path must return the
    exactly rounded products bit for bit."""
    g = torch.Generator().manual_seed(33)
    M, N = 130, 72
    a = torch.randint(-4, 5, (M, K), generator=g).half()
    b = torch.randint(-4, 5, (K, N) if layout == "nn" else (N, K), generator=g).half()
    k8 = (K + 7) // 8 * 8
    ap = _nan_padded(a, k8).to(dev)
    bp = b.to(dev) if layout == "nn" else _nan_padded(b, k8).to(dev)
    c = pkg.gemm(ap[:, :K], bp if layout == "nn" else bp[:, :K], b_layout=layout)
    torch.cuda.synchronize()
    exact = a.double() @ (b.double() if layout == "nn" else b.double().T)
    assert np.array_equal(c.cpu().numpy(), f16_round(exact.numpy()))


@pytest.mark.parametrize("epi", ["bias", "gelu_tanh", "bias_gelu_tanh", "silu_mul"])
def test_gemm_ragged_k_epilogues(pkg, dev, epi):
    M, N, K = 200, 96 if epi == "silu_mul" else 93, 301
    x = normal((M, K), 34)
    w = normal((N, K), 35, std=0.05)
    bias = normal((N,), 36, std=0.1)
    xp, wp = _nan_padded(x, 304).to(dev), _nan_padded(w, 304).to(dev)
    n_out = N // 2 if epi == "silu_mul" else N
    outp = torch.empty((M, 104), dtype=torch.float16, device=dev)
    kw = {"bias": bias.to(dev)} if "bias" in epi else {}
    pkg.gemm(xp[:, :K], wp[:, :K], b_layout="nt", epilogue=epi, out=outp[:, :n_out], **kw)
    torch.cuda.synchronize()
    exp = ref.gemm_epilogue(x.numpy(), w.numpy(), "nt", epi, bias.numpy() if "bias" in epi else None)
    assert ref.max_rel_err(np32(outp[:, :n_out].cpu()), exp) <= TOL


def test_gemm_ragged_bf16(pkg, dev):
    M, N, K = 150, 77, 123
    a = uniform((M, K), 37, dtype=torch.bfloat16)
    b = uniform((N, K), 38, dtype=torch.bfloat16)
    ap, bp = _nan_padded(a, 128).to(dev), _nan_padded(b, 128).to(dev)
    outp = torch.empty((M, 80), dtype=torch.bfloat16, device=dev)
    pkg.gemm(ap[:, :K], bp[:, :K], b_layout="nt", out=outp[:, :N])
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(outp[:, :N].cpu()), ref.matmul(np32(a), np32(b), "nt")) <= TOL


def test_composite_attention_runs_the_mfma_gemms(pkg, dev):
    """Head dim 80 takes the reference's three steps (Q.K^T, softmax, P.V)
    with S and P padded to 200 keys: both GEMMs on the MFMA path."""
    q, k, v = (normal((24, 197, 80), 39 + i) for i in range(3))
    o = pkg.attention(q.to(dev), k.to(dev), v.to(dev), 80**-0.5)
    torch.cuda.synchronize()
    exp = ref.sdpa(q.numpy(), k.numpy(), v.numpy(), 80**-0.5)
    assert ref.max_err_vs_scale(np32(o.cpu()), exp) <= TOL


@pytest.mark.parametrize("epi", ["bias", "gelu_tanh", "bias_gelu_tanh"])
@pytest.mark.parametrize("tile", [None, 0, 3, 6, 7, 8, 9, 10, 11, 12, 13])
def test_gemm_epilogues(pkg, dev, force_tile, epi, tile):
    force_tile(tile)
    M, N, K = 300, 264, 256
    a = normal((M, K), 6)
    w = normal((N, K), 7, 0.05)
    bias = normal((N,), 8, 0.5)
    c = run_gemm(pkg, dev, a, w, "nt", epilogue=epi, bias=bias.to(dev))
    exp = ref.gemm_epilogue(a.numpy(), w.numpy(), "nt", epi, bias.numpy())
    assert ref.max_rel_err(np32(c), exp) <= TOL


@pytest.mark.parametrize("epi", ["bias", "bias_gelu_tanh"])
@pytest.mark.parametrize("tile", [None, 3, 6, 8, 12])
def test_gemm_bias_n_not_a_multiple_of_8(pkg, dev, force_tile, epi, tile):
    """N % 8 != 0 with K % 8 == 0: the epilogue reads the bias from global
    memory element by element instead of the per-tile LDS copy (which takes
    whole 16-byte chunks); the padding columns of the output stay untouched."""
    force_tile(tile)
    M, N, K = 200, 93, 256
    a = normal((M, K), 40)
    w = normal((N, K), 41, 0.05)
    bias = normal((N,), 42, 0.5)
    outp = torch.full((M, 96), 7.0, dtype=torch.float16, device=dev)
    pkg.gemm(a.to(dev), w.to(dev), b_layout="nt", epilogue=epi, bias=bias.to(dev), out=outp[:, :N])
    torch.cuda.synchronize()
    c = outp.cpu()
    exp = ref.gemm_epilogue(a.numpy(), w.numpy(), "nt", epi, bias.numpy())
    assert ref.max_rel_err(np32(c[:, :N]), exp) <= TOL
    assert (c[:, N:] == 7.0).all()


@pytest.mark.parametrize("tile", [None, 0, 1, 2, 3, 4, 11, 12, 13, 14])
def test_gemm_silu_mul(pkg, dev, force_tile, tile):
    force_tile(tile)
    M, I, K = 200, 320, 256
    x = normal((M, K), 9)
    wg = normal((I, K), 10, 0.05)
    wu = normal((I, K), 11, 0.05)
    packed = pkg.pack_gate_up(wg.to(dev), wu.to(dev))
    h = pkg.linear(x.to(dev), packed, epilogue="silu_mul")
    torch.cuda.synchronize()
    exp = ref.silu_mul_linear(x.numpy(), wg.numpy(), wu.numpy())
    assert ref.max_rel_err(np32(h.cpu()), exp) <= TOL


@pytest.mark.parametrize("epi", [None, "bias_gelu_tanh", "silu_mul"])
def test_gemm_bf16_tile_128x192(pkg, dev, force_tile, epi):
    # the 8-wave 128x192 tile on bf16 operands, with a ragged last tile
    # column (N = 416: 32 of its 192 columns) and the epilogues it runs in
    # the ViT MLP and the LLaMA gate/up projection
    force_tile(14)
    M, N, K = 200, 416, 320
    a = normal((M, K), 45, dtype=torch.bfloat16)
    w = normal((N, K), 46, 0.05, dtype=torch.bfloat16)
    bias = normal((N,), 47, 0.5, dtype=torch.bfloat16) if epi == "bias_gelu_tanh" else None
    y = pkg.linear(a.to(dev), w.to(dev), None if bias is None else bias.to(dev),
                   epilogue="gelu_tanh" if epi == "bias_gelu_tanh" else epi)
    torch.cuda.synchronize()
    # (silu_mul: w holds packed gate/up rows, which the oracle unpacks itself)
    exp = ref.gemm_epilogue(np32(a), np32(w), "nt", epi, None if bias is None else np32(bias))
    assert tuple(y.shape) == (M, N // 2 if epi == "silu_mul" else N)
    assert ref.max_rel_err(np32(y.cpu()), exp) <= TOL


def test_gemm_tile_128x192_override_nn_runs_picked_tile(pkg, dev, force_tile):
    # 128x192 takes k-contiguous B only: forced on an NN GEMM, the picker's
    # tile runs instead and the integer product stays exact
    force_tile(14)
    d = np.load(GOLDEN / "gemm_int_nn.npz")
    c = run_gemm(pkg, dev, torch.from_numpy(d["a"]).half(), torch.from_numpy(d["b"]).half(), "nn")
    assert np.array_equal(c.numpy(), f16_round(d["c"]))


def test_gemm_alpha(pkg, dev):
    a, b = uniform((64, 128), 12), uniform((96, 128), 13)
    c = run_gemm(pkg, dev, a, b, "nt", alpha=0.125)
    assert ref.max_rel_err(np32(c), 0.125 * ref.matmul(a.numpy(), b.numpy(), "nt")) <= TOL


@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_gemm_bf16(pkg, dev, layout):
    a = uniform((256, 320), 14, dtype=torch.bfloat16)
    b = uniform((320, 192) if layout == "nn" else (192, 320), 15, dtype=torch.bfloat16)
    c = run_gemm(pkg, dev, a, b, layout)
    # bf16 output rounding is 2^-9 relative
    assert ref.max_rel_err(np32(c), ref.matmul(np32(a), np32(b), layout)) <= TOL


def test_gemm_strided_views(pkg, dev):
    base = uniform((128, 200), 16)
    a = base[:, 8:136]  # lda = 200, 16-byte aligned rows
    b = uniform((128, 96), 17)
    c = pkg.gemm(base.to(dev)[:, 8:136], b.to(dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(c.cpu()), ref.matmul(a.numpy(), b.numpy())) <= TOL


def test_gemm_output_view_untouched_outside(pkg, dev):
    a, b = uniform((40, 64), 18), uniform((64, 48), 19)
    out = torch.full((40, 64), 7.0, dtype=torch.float16, device=dev)
    pkg.gemm(a.to(dev), b.to(dev), out=out[:, :48])
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.all(o[:, 48:] == 7.0)
    assert ref.max_rel_err(np32(o[:, :48]), ref.matmul(a.numpy(), b.numpy())) <= TOL


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("tile", [None, 0, 11])
def test_gemm_4096_cube(pkg, dev, force_tile, layout, tile):
    force_tile(tile)
    a = uniform((4096, 4096), 20)
    b = uniform((4096, 4096), 21)
    c = run_gemm(pkg, dev, a, b, layout)
    assert ref.max_rel_err(np32(c), ref.matmul(a.numpy(), b.numpy(), layout)) <= TOL


@pytest.mark.parametrize("name,N,K", [("qkv", 2560, 2048), ("o", 2048, 2048), ("down", 2048, 5632)])
def test_tinyllama_projections(pkg, dev, name, N, K):
    x = normal((512, K), 22)
    w = normal((N, K), 23, 0.02)
    y = run_gemm(pkg, dev, x, w, "nt")
    assert ref.max_rel_err(np32(y), ref.linear(x.numpy(), w.numpy())) <= TOL


def test_bgemm_vit_attention_products(pkg, dev):
    q = normal((96, 197, 64), 24)
    k = normal((96, 197, 64), 25)
    v = normal((96, 197, 64), 26)
    s = pkg.bgemm(q.to(dev), k.to(dev), b_layout="nt", alpha=0.125)
    p = pkg.softmax(s)
    o = pkg.bgemm(p, v.to(dev), b_layout="nn")
    torch.cuda.synchronize()
    s_ref = 0.125 * ref.bmm(q.numpy(), k.numpy(), "nt")
    assert ref.max_rel_err(np32(s.cpu()), s_ref) <= TOL
    p_ref = ref.softmax(np32(s.cpu()))
    assert ref.max_rel_err(np32(p.cpu()), p_ref) <= TOL
    # the three-kernel pipeline keeps S and P in fp16 between kernels (as the
    # reference's bmm -> softmax -> bmm lowering does), so its output is
    # judged relative to the output scale
    o_ref = ref.sdpa(q.numpy(), k.numpy(), v.numpy(), 0.125)
    assert ref.max_err_vs_scale(np32(o.cpu()), o_ref) <= TOL
    o_ref_p16 = ref.bmm(np32(p.cpu()), v.numpy())  # same fp16 P: elementwise bound holds
    assert ref.max_rel_err(np32(o.cpu()), o_ref_p16) <= TOL


@pytest.fixture
def force_splits(knobs):
    return lambda s: knobs(splitk=s)


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("splits", [2, 3, 4, 8])
@pytest.mark.parametrize("K", [2048, 2056, 3000 - 3000 % 8])  # even, ragged last slice, odd slice count
def test_gemm_split_k(pkg, dev, force_splits, layout, splits, K):
    force_splits(splits)
    M, N = 200, 264
    a = uniform((M, K), 30)
    b = uniform((K, N) if layout == "nn" else (N, K), 31)
    c = run_gemm(pkg, dev, a, b, layout)
    assert ref.max_rel_err(np32(c), ref.matmul(a.numpy(), b.numpy(), layout)) <= TOL


@pytest.mark.parametrize("epi", ["bias", "gelu_tanh", "bias_gelu_tanh", "silu_mul"])
def test_gemm_split_k_epilogues(pkg, dev, force_splits, epi):
    force_splits(4)
    M, N, K = 130, 320, 4096
    a = normal((M, K), 32)
    w = normal((N, K), 33, 0.02)
    bias = normal((N,), 34, 0.5)
    c = run_gemm(pkg, dev, a, w, "nt", epilogue=epi, bias=bias.to(dev))
    exp = ref.gemm_epilogue(a.numpy(), w.numpy(), "nt", epi, bias.numpy())
    assert ref.max_rel_err(np32(c), exp) <= TOL


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_gemm_split_k_every_tile_exact(pkg, dev, force_tile, force_splits, tile, layout):
    # integer-valued operands: every partial tile and their fp32 sum are
    # exact, so the fixed-up output must equal the rounded exact product
    skip_nn(tile, layout)
    force_tile(tile)
    force_splits(3)
    M, N, K = 300, 264, 2112
    a = torch.randint(-2, 3, (M, K), generator=torch.Generator().manual_seed(40)).half()
    b = torch.randint(-2, 3, (K, N) if layout == "nn" else (N, K), generator=torch.Generator().manual_seed(41)).half()
    c = run_gemm(pkg, dev, a, b, layout)
    assert np.array_equal(c.numpy(), f16_round(ref.matmul(a.numpy(), b.numpy(), layout))), f"tile {tile}"


def test_gemm_split_k_bf16(pkg, dev, force_splits):
    force_splits(4)
    M, N, K = 256, 384, 4096
    a = normal((M, K), 42, dtype=torch.bfloat16)
    w = normal((N, K), 43, 0.02, dtype=torch.bfloat16)
    c = run_gemm(pkg, dev, a, w, "nt")
    assert ref.max_rel_err(np32(c), ref.linear(np32(a), np32(w))) <= TOL


def test_gemm_split_k_deterministic_graph_replays(pkg, dev, force_splits):
    """The last slice to arrive adds the partial tiles in slice order, so
    repeated calls are bit-identical; the arrival counters reset themselves,
    so graph replays with eager calls on the same workspace between them
    match too, and one workspace serves two shapes back to back."""
    force_splits(4)
    lib = pkg.load_library()
    shapes = [(512, 2048, 5632), (200, 640, 4096)]
    nbytes = max(lib.hxmi_gemm_workspace_bytes(M, N, K, 1, 0) for M, N, K in shapes)
    assert nbytes > 0
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)  # counters zero before first use
    ops = []
    for i, (M, N, K) in enumerate(shapes):
        x = normal((M, K), 44 + i).to(dev)
        w = normal((N, K), 46 + i, 0.02).to(dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ops.append((x, w, y, M, N, K))

    def call(op, stream):
        x, w, y, M, N, K = op
        rc = lib.hxmi_gemm_f16(x.data_ptr(), w.data_ptr(), y.data_ptr(), None, M, N, K, K, K, N, 1, 0, 1.0,
                               ws.data_ptr(), nbytes, stream)
        assert rc == 0, lib.hxmi_last_error()

    eager = []
    for op in ops:
        call(op, None)
        torch.cuda.synchronize()
        eager.append(op[2].clone())
        exp = ref.linear(op[0].cpu().numpy(), op[1].cpu().numpy())
        assert ref.max_rel_err(np32(op[2].cpu()), exp) <= TOL
    for op, e in zip(ops, eager):
        call(op, None)
        torch.cuda.synchronize()
        assert torch.equal(op[2], e)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(ops[0], s.cuda_stream)
    for _ in range(3):
        ops[0][2].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ops[0][2], eager[0])
        call(ops[1], None)  # another shape on the same workspace between replays
        torch.cuda.synchronize()
        assert torch.equal(ops[1][2], eager[1])


def test_gemm_split_k_workspace_counters_return_to_zero(pkg, dev, force_splits):
    """The workspace protocol: arrival counters zero when a call starts, zero
    again when it ends; whatever an earlier user left in the partial-tile
    area (here int64 words that look like tagged counts) does not matter."""
    force_splits(3)
    lib = pkg.load_library()
    M, N, K = 200, 640, 4096
    nbytes = lib.hxmi_gemm_workspace_bytes(M, N, K, 1, 0)
    cwords = 16384 // 8  # HXMI_WORKSPACE_COUNTER_BYTES of 64-bit counters
    assert nbytes > cwords * 8
    ws = torch.zeros(nbytes // 8, dtype=torch.int64, device=dev)
    ws[cwords:] = (torch.arange(nbytes // 8 - cwords, device=dev) % 7) | (1 << 8)
    x, w = normal((M, K), 60).to(dev), normal((N, K), 61, 0.02).to(dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    exp = ref.linear(x.cpu().numpy(), w.cpu().numpy())
    first = None
    for _ in range(3):
        rc = lib.hxmi_gemm_f16(x.data_ptr(), w.data_ptr(), y.data_ptr(), None, M, N, K, K, K, N, 1, 0, 1.0,
                               ws.data_ptr(), nbytes, None)
        assert rc == 0, lib.hxmi_last_error()
        torch.cuda.synchronize()
        assert int(ws[:cwords].abs().sum()) == 0
        assert ref.max_rel_err(np32(y.cpu()), exp) <= TOL
        first = y.clone() if first is None else first
        assert torch.equal(y, first)


def test_gemm_split_k_default_down_projection(pkg, dev):
    # TinyLlama down projection: the dispatcher splits K by itself
    assert pkg.load_library().hxmi_gemm_workspace_bytes(512, 2048, 5632, 1, 0) > 0
    x = normal((512, 5632), 35)
    w = normal((2048, 5632), 36, 0.02)
    y = run_gemm(pkg, dev, x, w, "nt")
    assert ref.max_rel_err(np32(y), ref.linear(x.numpy(), w.numpy())) <= TOL


@pytest.mark.parametrize("tile", TILES)
def test_gemm_f32_out_every_tile(pkg, dev, force_tile, tile):
    # fp32 output straight from the accumulators (HexKL's f16 x f16 -> f32
    # matmul, w [n_inner, n_col]: NN): integer operands, so every tile's
    # result is exact
    skip_nn(tile, "nn")
    force_tile(tile)
    g = torch.Generator().manual_seed(44)
    act = torch.randint(-3, 4, (300, 200), generator=g).half()
    w = torch.randint(-3, 4, (200, 264), generator=g).half()
    out = pkg.hexkl_matmul(act.to(dev), w.to(dev)).cpu()
    assert np.array_equal(out.numpy(), ref.matmul(act.numpy(), w.numpy()).astype(np.float32)), f"tile {tile}"


def test_hexkl_compat_matmul(pkg, dev):
    # hexkl_linalg_matmul/wrapper.cpp:30-67: 1024x64 . 64x512, N(0,0.5)
    # rounded to 4 decimals, |diff| <= 1e-2 against a CPU triple loop
    act = torch.round(normal((1024, 64), 27, 0.5, torch.float32) * 1e4) / 1e4
    w = torch.round(normal((64, 512), 28, 0.5, torch.float32) * 1e4) / 1e4
    act, w = act.half(), w.half()
    out = pkg.hexkl_matmul(act.to(dev), w.to(dev)).cpu()
    assert out.dtype == torch.float32
    assert np.max(np.abs(out.numpy() - ref.matmul(act.numpy(), w.numpy()))) <= 1e-2
