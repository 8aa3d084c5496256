"""GPU parity of the RMSNorm and softmax row kernels."""
import numpy as np
import pytest
import torch

from gpu_util import TOL, normal, np32, uniform
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [(512, 2048), (127, 513), (3, 8), (64, 4096), (5, 8200), (1, 520)])
def test_rmsnorm(pkg, dev, rows, cols):
    x = normal((rows, cols), 1)
    g = (1 + normal((cols,), 2, 0.02, torch.float32)).half()
    y = pkg.rms_norm(x.to(dev), g.to(dev), 1e-5)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert ref.max_rel_err(y.astype(np.float32), ref.rms_norm(x.numpy(), g.numpy(), 1e-5)) <= TOL
    # HF order (round the normalised value to fp16 before the weight): within
    # one fp16 ulp of the oracle's HF-order result
    hf = ref.rms_norm_hf(x.numpy(), g.numpy(), 1e-5).astype(np.float32)
    assert np.max(np.abs(y.astype(np.float32) - hf) / np.maximum(np.abs(hf), 1e-3)) <= 2 ** -9


def test_rmsnorm_reference_test_shape_uniform(pkg, dev):
    # test_rms_norm.py:19-20, 65-67: 127 x 513, rand inputs and weights
    x = uniform((127, 513), 3, 0, 1)
    g = uniform((513,), 4, 0, 1)
    y = pkg.rms_norm(x.to(dev), g.to(dev), 1e-5)
    torch.cuda.synchronize()
    assert np.max(np.abs(np32(y.cpu()) - ref.rms_norm(x.numpy(), g.numpy(), 1e-5))) <= 1e-2


def test_rmsnorm_constant_and_zero_rows(pkg, dev):
    x = torch.zeros((4, 256), dtype=torch.float16)
    x[1] = 3.0
    g = torch.ones(256, dtype=torch.float16)
    y = pkg.rms_norm(x.to(dev), g.to(dev), 1e-5).cpu().numpy().astype(np.float32)
    assert not np.any(y[0]) and not np.any(y[2:])
    assert np.allclose(y[1], 3.0 / np.sqrt(9.0 + 1e-5), rtol=2 ** -10)


def test_rmsnorm_bf16(pkg, dev):
    x = normal((64, 2048), 5, dtype=torch.bfloat16)
    g = (1 + normal((2048,), 6, 0.02, torch.float32)).to(torch.bfloat16)
    y = pkg.rms_norm(x.to(dev), g.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.rms_norm(np32(x), np32(g), 1e-6)) <= TOL


@pytest.mark.parametrize("rows,cols,scale", [(96 * 197, 197, 0.125), (128, 128, 1.0), (7, 3000, 0.5), (33, 1, 1.0),
                                             (5, 64, 2.0), (9, 1024, 1.0)])
def test_softmax(pkg, dev, rows, cols, scale):
    x = normal((rows, cols), 7)
    y = pkg.softmax(x.to(dev), scale)
    torch.cuda.synchronize()
    y = np32(y.cpu())
    assert ref.max_rel_err(y, ref.softmax(x.numpy(), scale)) <= TOL
    assert np.allclose(y.sum(-1), 1.0, atol=2e-3)


def test_softmax_reference_test_tolerance(pkg, dev):
    # test_softmax.py:19-21, 91-94: 128 x 128 rand, atol 1e-3 for fp16
    x = uniform((128, 128), 8, 0, 1)
    y = pkg.softmax(x.to(dev))
    torch.cuda.synchronize()
    assert np.max(np.abs(np32(y.cpu()) - ref.softmax(x.numpy()))) <= 1e-3


def test_softmax_shift_invariance_and_uniform(pkg, dev):
    x = normal((16, 197), 9)
    y1 = pkg.softmax(x.to(dev))
    y2 = pkg.softmax((x.float() + 3.0).half().to(dev))
    u = pkg.softmax(torch.zeros((4, 197), dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y2.cpu()), np32(y1.cpu())) <= TOL
    assert np.allclose(np32(u.cpu()), 1 / 197, rtol=2 ** -10)


def test_softmax_bf16(pkg, dev):
    x = normal((64, 197), 10, dtype=torch.bfloat16)
    y = pkg.softmax(x.to(dev), 0.125)
    torch.cuda.synchronize()
    assert ref.max_rel_err(np32(y.cpu()), ref.softmax(np32(x), 0.125)) <= TOL


def _softmax_widths():
    # every elements-per-lane count of both lane groupings (32 lanes a row up
    # to 512 columns, 64 up to 1024) at both ends, and the three-pass width
    w = set()
    for e in range(1, 17):
        w.update({32 * e - 31, 32 * e})
    for e in range(9, 17):
        w.update({64 * e - 63, 64 * e})
    return sorted(w | {1025})


def test_softmax_every_lane_count(pkg, dev):
    # odd row counts: the last wave's second row group is past the matrix
    for i, cols in enumerate(_softmax_widths()):
        rows = 3 + 2 * (i % 3)
        x = normal((rows, cols), 100 + i)
        y = np32(pkg.softmax(x.to(dev), 0.7).cpu())
        want = ref.softmax(x.numpy(), 0.7)
        assert ref.max_rel_err(y, want) <= TOL, cols
        assert np.allclose(y.sum(-1), 1.0, atol=2e-3), cols


@pytest.mark.parametrize("scale", [-0.3, 0.0, 0.125])
def test_softmax_scale_sign_and_masked_entries(pkg, dev, scale):
    # the row extremum is taken on the raw values: the smallest one for a
    # negative scale; -inf entries (masked scores) get weight 0
    x = normal((37, 197), 11)
    if scale != 0.0:  # (inf * 0 is NaN)
        x[::3, 5::7] = float("-inf") if scale > 0 else float("inf")
    y = np32(pkg.softmax(x.to(dev), scale).cpu())
    want = ref.softmax(x.numpy(), scale)
    assert ref.max_rel_err(y, want) <= TOL
    if scale != 0.0:
        assert not np.any(y[::3, 5::7])
    # a row with every entry masked is NaN, as in torch
    z = torch.full((3, 40), float("-inf"), dtype=torch.float16)
    z[1] = 0
    yz = np32(pkg.softmax(z.to(dev), 1.0).cpu())
    assert np.isnan(yz[0]).all() and np.isnan(yz[2]).all() and np.allclose(yz[1], 1 / 40, rtol=2 ** -10)


def test_softmax_strided_rows(pkg, dev):
    # leading dimensions past the row: padded score rows as attention keeps them
    base = normal((19, 256), 12)
    out = torch.full((19, 224), 5.0, dtype=torch.float16, device=dev)
    y = pkg.softmax(base.to(dev)[:, :197], 0.125, out=out[:, :197])
    got = np32(out.cpu())
    assert ref.max_rel_err(np32(y.cpu()), ref.softmax(base[:, :197].numpy(), 0.125)) <= TOL
    assert np.all(got[:, 197:] == 5.0)


@pytest.mark.parametrize("rows,cols", [(5, 197), (7, 1), (3, 255), (9, 64), (4, 129), (1, 3)])
def test_softmax_output_neighbours_untouched(pkg, dev, rows, cols):
    # odd row counts (the last wave's second row group is past the matrix)
    # and odd element counts: the output's neighbours in a larger buffer
    # stay untouched
    x = normal((rows, cols), 13)
    buf = torch.full((rows * cols + 8,), 7.0, dtype=torch.float16, device=dev)
    out = buf[:rows * cols].view(rows, cols)
    y = pkg.softmax(x.to(dev), 0.3, out=out)
    got = np32(buf.cpu())
    assert ref.max_rel_err(np32(y.cpu()), ref.softmax(x.numpy(), 0.3)) <= TOL
    assert np.all(got[rows * cols:] == 7.0)


def test_softmax_unaligned_and_strided_rows_every_width(pkg, dev):
    # rows starting 2 bytes past a 4-byte boundary, and padded rows, agree
    # with the oracle at every width <= 256
    for i, cols in enumerate([1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 197, 255, 256]):
        rows = 3 + (i % 4)
        flat = normal((rows * cols + 1,), 200 + i)
        x = flat.to(dev)[1:].view(rows, cols)
        y = pkg.softmax(x, 0.5)
        assert ref.max_rel_err(np32(y.cpu()), ref.softmax(flat[1:].view(rows, cols).numpy(), 0.5)) <= TOL, cols
        base = normal((rows, cols + 24), 300 + i)
        ys = pkg.softmax(base.to(dev)[:, :cols], 0.5)
        assert ref.max_rel_err(np32(ys.cpu()), ref.softmax(base[:, :cols].numpy(), 0.5)) <= TOL, cols
