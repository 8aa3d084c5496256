"""Shared helpers for the GPU parity tests: seeded CPU generation (copied to
the GPU afterwards, so inputs are identical for kernel and oracle)."""
import numpy as np
import torch

TOL = 1e-2  # max relative error of fp16 outputs vs the fp32 oracle


def gen(seed):
    return torch.Generator().manual_seed(seed)


def uniform(shape, seed, lo=-1.0, hi=1.0, dtype=torch.float16):
    return (torch.rand(shape, generator=gen(seed)) * (hi - lo) + lo).to(dtype)


def normal(shape, seed, std=1.0, dtype=torch.float16):
    return (torch.randn(shape, generator=gen(seed)) * std).to(dtype)


def np32(t):
    return t.float().numpy()


def f16_round(x):
    """Round exact values once to fp16 (what a correct fp32-accumulate,
    fp16-store kernel returns for exactly representable sums)."""
    return np.asarray(x, dtype=np.float64).astype(np.float16)
