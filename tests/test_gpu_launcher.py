"""GPU end-to-end through the reference-compatible launcher."""
import json
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

from gpu_util import TOL, normal, np32, uniform
from oracle import hot_path as ref
from test_backend import Block, QKVIn, block_inputs, fold_lwp

pytestmark = pytest.mark.gpu


class MatMul(nn.Module):
    """benchmark_models/micro_bench/test_matmul_benchmark.py:22-31."""

    def __init__(self, transpose_b=False):
        super().__init__()
        self.transpose_b = transpose_b

    def forward(self, a, b):
        if self.transpose_b:
            b = b.transpose(-2, -1)
        return torch.matmul(a, b)


@pytest.fixture(scope="module")
def backend(pkg):
    import hexagon_mlir_amd.backend as b

    return b


@pytest.mark.parametrize("transpose_b", [False, True])
def test_micro_bench_matmul_flow(backend, dev, tmp_path, capsys, transpose_b):
    a = uniform((1024, 1024), 0)
    b = uniform((1024, 1024), 1)
    model = MatMul(transpose_b)
    path = str(tmp_path / "mm.pt2")
    backend.write_program_to_file(backend.export_program(model, [a, b]), path)
    opts = backend.HexagonOptions(enableVTCMTiling=True, enableVectorization=True).__dict__
    launcher = backend.TorchMLIRHexagonLauncher()
    out = launcher.run_torch_mlir(path, [a, b], "mm", base_dir_for_artifacts=str(tmp_path), iterations=5,
                                  options=opts)
    assert [p for p, _ in launcher.last_plan.kernels] == ["matmul"]
    text = capsys.readouterr().out
    perf = float(re.search(r"Perf:\s*([0-9]+(?:\.[0-9]+)?)", text).group(1))
    assert perf > 0 and re.search(r"Units:\s*([a-zA-Z]+)", text).group(1) == "us"
    reference = model(a.float(), b.float())
    # the micro-bench's own check (test_matmul_benchmark.py:91-92)
    assert torch.allclose(out[0].float(), reference, rtol=1e-3, atol=1e-3)
    assert ref.max_rel_err(np32(out[0]), reference.numpy()) <= TOL


def test_block_through_launcher(backend, dev, tmp_path):
    torch.manual_seed(0)
    model = Block().half()
    inputs = block_inputs(2)
    path = str(tmp_path / "block.pt2")
    backend.write_program_to_file(backend.export_program(model, inputs), path)
    launcher = backend.TorchMLIRHexagonLauncher()
    opts = backend.HexagonOptions(enableLWP=True).__dict__
    outs = launcher.run_torch_mlir(path, inputs, "block", str(tmp_path), iterations=2, options=opts)
    pats = sorted(p for p, _ in launcher.last_plan.kernels)
    assert pats == ["attention", "attention", "linear", "linear_gelu", "rms_norm", "rms_silu_mul"]
    exp = model.float()(*[t.float() for t in inputs])
    for o, e in zip(outs, exp):
        assert o.device.type == "cpu" and o.dtype == torch.float16
        assert ref.max_err_vs_scale(np32(o), e.detach().numpy()) <= TOL
    folder = next(p for p in tmp_path.iterdir() if p.is_dir() and p.name.startswith("block-"))
    assert (folder / "lwp.json").exists() and (folder / "perf.txt").exists() and (folder / "block.plan.txt").exists()
    back = backend.read_output_tensor(folder / "_mlir_ciface_block_o0.raw")
    assert torch.equal(back, outs[0])
    # LWP: region 0 is the whole run, regions 1..n the planned ops, each
    # closed once, nested in region 0, with non-negative GPU time
    lwp = json.loads((folder / "lwp.json").read_text())
    summary = fold_lwp(lwp["entries"])
    n_ops = len(summary) - 1
    assert n_ops >= len(pats) and set(summary) == set(range(n_ops + 1))
    assert all(cnt == 1 for _, cnt, _ in summary.values())
    assert all(summary[i][2] == 0 for i in range(1, n_ops + 1)) and summary[0][2] is None
    assert all(tot >= 0 for tot, _, _ in summary.values())
    assert sum(summary[i][0] for i in range(1, n_ops + 1)) <= summary[0][0]
    assert lwp["cyc_hz"] > 0
    # the run takes between 1 us and 1 s of GPU time
    assert 1e-6 <= summary[0][0] / lwp["cyc_hz"] <= 1.0
    dump = (folder / "lwp_infodump.txt").read_text().strip().split("\n")
    ids = sorted(int(re.search(r"corresponds to ID (\d+)", line).group(1)) for line in dump)
    assert ids == list(range(n_ops + 1))


def test_tile_sizes_apply_to_their_run_only(backend, pkg, dev, tmp_path):
    """tileSizes forces the GEMM tile of the runs of that plan and nothing
    else: no environment variable, no thread override left behind."""
    import os

    a, b = uniform((256, 512), 20), uniform((512, 384), 21)
    path = str(tmp_path / "mm.pt2")
    model = MatMul()
    backend.write_program_to_file(backend.export_program(model, [a, b]), path)
    launcher = backend.TorchMLIRHexagonLauncher()
    opts = backend.HexagonOptions(tileSizes="64,64").__dict__
    out = launcher.run_torch_mlir(path, [a, b], "mm", str(tmp_path), options=opts)
    assert launcher.last_plan.gemm_tile is not None
    assert "HXMI_GEMM_TILE" not in os.environ
    assert pkg.set_tuning("gemm_tile", None) is None  # no override left on this thread
    plain = backend.TorchMLIRHexagonLauncher().run_torch_mlir(path, [a, b], "mm2", str(tmp_path))
    assert ref.max_rel_err(np32(out[0]), ref.matmul(a.numpy(), b.numpy())) <= TOL
    assert ref.max_rel_err(np32(plain[0]), ref.matmul(a.numpy(), b.numpy())) <= TOL


def test_fusion_off_gives_same_numbers(backend, dev, tmp_path):
    torch.manual_seed(0)
    model = Block().half()
    inputs = block_inputs(3)
    path = str(tmp_path / "b.pt2")
    backend.write_program_to_file(backend.export_program(model, inputs), path)
    on = backend.TorchMLIRHexagonLauncher().run_torch_mlir(path, inputs, "on", str(tmp_path),
                                                           options=backend.HexagonOptions(fusion=True).__dict__)
    off = backend.TorchMLIRHexagonLauncher().run_torch_mlir(path, inputs, "off", str(tmp_path),
                                                            options=backend.HexagonOptions(fusion=False).__dict__)
    for a, b in zip(on, off):
        assert ref.max_err_vs_scale(np32(a), np32(b)) <= TOL


def test_rmsnorm_folded_into_qkv_on_gpu(backend, dev, tmp_path):
    """Qwen2-style q/k/v with bias after an RMSNorm: three GEMMs, the first
    takes the row statistics, no RMSNorm kernel; compared with the fp32 model."""
    torch.manual_seed(0)
    model = QKVIn(256).half()
    x = torch.randn(77, 256, generator=torch.Generator().manual_seed(5)).half()
    path = str(tmp_path / "qkv.pt2")
    backend.write_program_to_file(backend.export_program(model, [x]), path)
    launcher = backend.TorchMLIRHexagonLauncher()
    outs = launcher.run_torch_mlir(path, [x], "qkv", str(tmp_path), iterations=2)
    assert sorted(p for p, _ in launcher.last_plan.kernels) == ["rms_linear"] * 3
    exp = model.float()(x.float())
    for o, e in zip(outs, exp):
        assert ref.max_err_vs_scale(np32(o), e.detach().numpy()) <= TOL


def test_constants_in_separate_artifact(backend, dev, tmp_path):
    """lowerConstantsInSeparateSharedObjects: the folded / packed weights go
    to <func>.constants.safetensors and the run reads them back from it; the
    outputs are bit-identical to a run without the option."""
    from safetensors import safe_open

    torch.manual_seed(0)
    model = QKVIn(256).half()
    x = torch.randn(33, 256, generator=torch.Generator().manual_seed(6)).half()
    path = str(tmp_path / "qkv.pt2")
    backend.write_program_to_file(backend.export_program(model, [x]), path)
    plain = backend.TorchMLIRHexagonLauncher().run_torch_mlir(path, [x], "plain", str(tmp_path))
    launcher = backend.TorchMLIRHexagonLauncher()
    opts = backend.HexagonOptions(lowerConstantsInSeparateSharedObjects=True).__dict__
    split = launcher.run_torch_mlir(path, [x], "split", str(tmp_path), options=opts)
    for a, b in zip(plain, split):
        assert torch.equal(a, b)
    folder = next(p for p in tmp_path.iterdir() if p.is_dir() and p.name.startswith("split-"))
    art = folder / "split.constants.safetensors"
    with safe_open(str(art), framework="pt") as f:
        keys = set(f.keys())
        assert f.metadata()["format"] == "hxmi-constants"
    names = {k for k, _ in launcher.last_plan.module.named_buffers()}
    names |= {k for k, _ in launcher.last_plan.module.named_parameters()}
    assert keys == names and any("rmsfold" in k for k in keys)
