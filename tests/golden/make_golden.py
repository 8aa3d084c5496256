"""Write the known-answer fixtures in this directory.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its tests compare with
PyTorch on unseeded inputs), so these fixtures are exact answers computed
here with Python integers, independently of numpy/torch arithmetic:

  gemm_int_{nn,nt}.npz   small-integer fp16 operands (|v| <= 8) whose fp32
                         sums are exact and representable in fp16: every
                         correct fp16-in / fp32-accumulate GEMM must
                         reproduce C bit-for-bit (the config-1 check of
                         test_matmul_benchmark.py:91-92, made exact).
  gemm_int_epi.npz       the same with bias (integer) for the bias epilogue.
  w8_onehot.npz          int8 weights, scale 1, one-hot activations: y must
                         equal a weight column exactly (dequant is exact).
  tile_model.npz         the VTCM tile sizes the reference's lit test pins
                         (qcom_hexagon_backend/test/Conversion/LinalgToLLVM/
                         vtcm_tiling_static.mlir:80-88).
"""
from __future__ import annotations

import pathlib
import random

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent


def int_matrix(rng: random.Random, rows: int, cols: int, lo: int = -8, hi: int = 8) -> list[list[int]]:
    return [[rng.randint(lo, hi) for _ in range(cols)] for _ in range(rows)]


def int_matmul(a: list[list[int]], b: list[list[int]], b_nt: bool) -> list[list[int]]:
    m, k = len(a), len(a[0])
    n = len(b) if b_nt else len(b[0])
    out = []
    for i in range(m):
        row = []
        for j in range(n):
            s = 0
            for t in range(k):
                s += a[i][t] * (b[j][t] if b_nt else b[t][j])
            row.append(s)
        out.append(row)
    return out


def main() -> None:
    rng = random.Random(20240601)
    # sizes straddle the 64-wide tile and the 8-element vector granularity
    m, n, k = 72, 80, 96
    a = int_matrix(rng, m, k)
    b_nn = int_matrix(rng, k, n)
    b_nt = int_matrix(rng, n, k)
    c_nn = int_matmul(a, b_nn, False)
    c_nt = int_matmul(a, b_nt, True)
    # |c| <= 96 * 64 = 6144: the fp32 sum is exact and a correct kernel's
    # fp16 output is that integer rounded once to fp16 (round-to-nearest-even)
    for c in (c_nn, c_nt):
        assert max(abs(v) for row in c for v in row) < 65504
    np.savez_compressed(HERE / "gemm_int_nn.npz", a=np.array(a, np.int32), b=np.array(b_nn, np.int32), c=np.array(c_nn, np.int64))
    np.savez_compressed(HERE / "gemm_int_nt.npz", a=np.array(a, np.int32), b=np.array(b_nt, np.int32), c=np.array(c_nt, np.int64))

    bias = [rng.randint(-16, 16) for _ in range(n)]
    c_b = [[c_nt[i][j] + bias[j] for j in range(n)] for i in range(m)]
    np.savez_compressed(HERE / "gemm_int_epi.npz", a=np.array(a, np.int32), b=np.array(b_nt, np.int32),
             bias=np.array(bias, np.int32), c=np.array(c_b, np.int64))

    nq, kq = 64, 128
    q = [[rng.randint(-127, 127) for _ in range(kq)] for _ in range(nq)]
    cols = [3, 0, 127, 64, 100]
    # y[m][n] = q[n][cols[m]] for one-hot x rows
    y = [[q[j][c] for j in range(nq)] for c in cols]
    np.savez_compressed(HERE / "w8_onehot.npz", q=np.array(q, np.int8), cols=np.array(cols, np.int32), y=np.array(y, np.int32))

    # lit: the generic over (d0=2048 parallel, d1=8192 reduction, d2=1024
    # parallel), f16 x f16 -> f32, is tiled to [64, 4096, 64]
    np.savez_compressed(HERE / "tile_model.npz", dims=np.array([2048, 8192, 1024]), tile=np.array([64, 4096, 64]))


if __name__ == "__main__":
    main()
