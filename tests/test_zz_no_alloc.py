"""The allocation-free GEMM entry point (hxmi_gemm_f16_noalloc): its split-K
partials live in the library's per-GPU scratch array.  Checked through the
C ABI against hxmi_gemm_f16 with a caller workspace (same kernels, same
split, so bit-identical) and against the oracle, on two calls in a row, the
second smaller, then once more at the first size."""
import pytest
import torch

from gpu_util import TOL, normal, np32
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

# (M, N, K) that split K by default: the TinyLlama down projection, a
# smaller 200 x 640 x 4096 projection
SHAPES = [(512, 2048, 5632), (200, 640, 4096), (512, 2048, 5632)]


def _operands(M, N, K, seed, dev):
    return normal((M, K), seed).to(dev), normal((N, K), seed + 1, 0.02).to(dev)


def test_noalloc_gemm_matches_workspace_gemm(pkg, dev):
    lib = pkg.load_library()
    for i, (M, N, K) in enumerate(SHAPES):
        print(f"[noalloc] call {i}: M={M} N={N} K={K}", flush=True)
        nbytes = lib.hxmi_gemm_workspace_bytes(M, N, K, 1, 0)
        assert 0 < nbytes <= 33554432  # splits, and fits the scratch
        x, w = _operands(M, N, K, 80 + i, dev)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        y_ws = torch.full((M, N), 7.0, dtype=torch.float16, device=dev)
        y_na = torch.full((M, N), -7.0, dtype=torch.float16, device=dev)
        rc = lib.hxmi_gemm_f16(x.data_ptr(), w.data_ptr(), y_ws.data_ptr(), None, M, N, K, K, K, N, 1, 0, 1.0,
                               ws.data_ptr(), nbytes, None)
        assert rc == 0, lib.hxmi_last_error()
        rc = lib.hxmi_gemm_f16_noalloc(x.data_ptr(), w.data_ptr(), y_na.data_ptr(), None, M, N, K, K, K, N, 1, 0,
                                       1.0, None)
        assert rc == 0, lib.hxmi_last_error()
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ws), f"call {i}"
        assert ref.max_rel_err(np32(y_na.cpu()), ref.linear(x.cpu().numpy(), w.cpu().numpy())) <= TOL


def test_noalloc_gemm_epilogue_on_current_stream(pkg, dev):
    """SiLU-mul epilogue, launched on a non-default stream."""
    lib = pkg.load_library()
    M, I, K = 256, 1024, 4096
    x = normal((M, K), 90).to(dev)
    wg, wu = normal((I, K), 91, 0.02).to(dev), normal((I, K), 92, 0.02).to(dev)
    wp = pkg.pack_gate_up(wg, wu)
    assert lib.hxmi_gemm_workspace_bytes(M, 2 * I, K, 1, 2) > 0
    s = torch.cuda.Stream()
    y = torch.empty((M, I), dtype=torch.float16, device=dev)
    with torch.cuda.stream(s):
        rc = lib.hxmi_gemm_f16_noalloc(x.data_ptr(), wp.data_ptr(), y.data_ptr(), None, M, 2 * I, K, K, K, I, 1, 2,
                                       1.0, s.cuda_stream)
    assert rc == 0, lib.hxmi_last_error()
    s.synchronize()
    exp = ref.silu_mul_linear(x.cpu().numpy(), wg.cpu().numpy(), wu.cpu().numpy())
    assert ref.max_rel_err(np32(y.cpu()), exp) <= TOL
