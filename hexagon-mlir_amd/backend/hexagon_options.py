"""Compile options, field-for-field the reference's HexagonOptions
(qcom_hexagon_backend/backend/hexagon_options.py:16-101), so callers that
build ``HexagonOptions(...).__dict__`` or edit that dict keep working.

What the fields mean on MI355X (fields not listed are accepted and recorded
but have no GPU meaning; they affected Hexagon code generation only):

  enableVTCMTiling, enableConvertToHexagonmem, enableHexagonmemCopyToDMA,
  enableDoubleBuffering
      The GPU kernels always stage operand tiles global->LDS with
      double-buffered direct-to-LDS loads; these flags are accepted and do not
      switch that off.
  enableHexKL
      Matrix multiplies always run on the MFMA units.
  fusion
      True: the launcher fuses bias / SiLU-mul / tanh-GELU into the producing
      GEMM, RMSNorm chains into one row kernel and attention into one
      kernel.  False: those elementwise ops run as separate kernels.
  tileSizes
      "" = heuristic GEMM tile; "BM,BN" (e.g. "256,256") forces that tile.
  iterations
      Timing loop count of the Test_Info report (as the generated main()).
  lowerConstantsInSeparateSharedObjects
      The planned module's constants (weights after RMSNorm folding and
      gate/up packing) are written to <func>.constants.safetensors in the
      run's artifact folder and read back from there before the run.
  enableLWP
      Per-op timing in the light-weight profiler's format: a kernel enqueued
      before and after every planned op stamps the GPU's wall clock into a
      record buffer, written to lwp.json ({"entries": [{"id", "cyc"}]},
      begin/end pairs per op id) in the run's artifact folder.
"""
import hashlib
import os
from dataclasses import dataclass
from typing import Tuple


@dataclass(frozen=True)
class HexagonOptions:
    allow_fp8e4nv: bool = False
    allowed_dot_input_precisions: Tuple[str] = ("ieee",)
    arch_triple: str = "hexagon"
    arch_features: str = f'+hvxv{os.getenv("HEXAGON_ARCH_VERSION")},+hvx-length128b'
    vectorize: int = 1
    vector_length: int = 32
    num_threads: int = 4
    data_layout: str = (
        "e-m:e-p:32:32:32-a:0-n16:32-i64:64:64-i32:32:32-i16:16:16-i1:8:8-f32:32:"
        "32-f64:64:64-v32:32:32-v64:64:64-v512:512:512-v1024:1024:1024-v2048:2048:2048"
    )
    num_warps: int = 1
    num_stages: int = 1
    num_ctas: int = 1
    shared: bool = False
    cluster_dims: tuple = (1, 1, 1)
    supported_fp8_dtypes: Tuple[str, ...] = ()
    sanitize_overflow: bool = True
    debug: bool = False
    name: str = "Hexagon"
    htp_kernel_gen: bool = False
    target_artifact: str = "o"
    iterations: int = 10

    fusion: bool = True
    fusionAllowRecompute: bool = False
    fusionDoMultiUse: bool = True

    enableBufferization: bool = True
    enableCollapseAddressSpace: bool = True
    enableConvTiling: bool = False
    enableDoubleBuffering: bool = False
    convTilingFactor: int = -1
    convTileHeightDim: bool = False
    convTileOCDim: bool = False
    enableConvertToHexagonmem: bool = True
    enableHexagonmemCopyToDMA: bool = False
    enableHexKL: bool = False
    enableMultiThreading: bool = False
    enableSCFThreading: bool = False
    enableSplitReduction: bool = False
    enableVectorization: bool = True
    enableVTCMTiling: bool = True
    enableHVXInlining: bool = False
    enableSeedLayoutConversions: bool = False

    tileSizes: str = ""

    lowerConstantsInSeparateSharedObjects: bool = False

    enableLWP: bool = False
    disableLWPLoop: bool = False
    LWPloopDepth: int = 1

    def __post_init__(self):
        valid_artifacts = {"o", "llir", "so"}
        if self.target_artifact not in valid_artifacts:
            raise ValueError(
                f"Invalid target_artifact '{self.target_artifact}'. "
                f"Must be one of: {', '.join(sorted(valid_artifacts))}"
            )

    def hash(self):
        key = "_".join([f"{name}-{val}" for name, val in self.__dict__.items()])
        return hashlib.md5(key.encode("utf-8")).hexdigest()


def options_from_dict(options: dict) -> HexagonOptions:
    """Validate an options dict the way the reference's pipeline reads one:
    unknown keys are an error (setLinalgToLLVMOptions looks every option up
    with .at(), MLLVMIRTranslation.cpp:54-99), missing keys take defaults."""
    known = HexagonOptions.__dataclass_fields__
    unknown = sorted(k for k in options if k not in known)
    if unknown:
        raise KeyError(f"unknown HexagonOptions field(s): {', '.join(unknown)}")
    return HexagonOptions(**options)
