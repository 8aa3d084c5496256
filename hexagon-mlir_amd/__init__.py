"""hexagon_mlir_amd — MI355X-native replacement of Hexagon-MLIR's matmul / GEMV /
RMSNorm / softmax hot path.

Layers:
  * ``csrc/``      hand-written HIP kernels for gfx950 behind the C ABI of
                   ``include/hxmi.h`` (built into ``lib/libhxmi.so``);
  * ``hxmi``       ctypes binding and torch-tensor ops over that ABI;
  * ``backend``    the reference's Python surface (``HexagonOptions``,
                   ``TorchMLIRHexagonLauncher.run_torch_mlir``) on top of it.

The directory name carries a dash, so it is imported under the module name
``hexagon_mlir_amd`` (see ``load_package`` in the repository's
``__graft_entry__.py``).
"""
from . import hxmi, weights
from .hxmi import (
    HxmiError,
    HxmiNotBuiltError,
    attention,
    bgemm,
    fold_rms_weight,
    gemm,
    gemv,
    hexkl_matmul,
    linear,
    load_library,
    pack_gate_up,
    quantize_int8,
    rms_norm,
    rms_norm_linear,
    set_tuning,
    softmax,
    tuning,
    w8a16_linear,
)

__all__ = [
    "hxmi",
    "weights",
    "HxmiError",
    "HxmiNotBuiltError",
    "attention",
    "bgemm",
    "fold_rms_weight",
    "gemm",
    "gemv",
    "hexkl_matmul",
    "linear",
    "load_library",
    "pack_gate_up",
    "quantize_int8",
    "rms_norm",
    "rms_norm_linear",
    "set_tuning",
    "softmax",
    "tuning",
    "w8a16_linear",
]
