"""GPU end-to-end through the reference-compatible launcher."""
import json
import re

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from gpu_util import TOL, normal, np32, uniform
from oracle import hot_path as ref
from test_backend import RMS, Block, QKVIn, block_inputs, fold_lwp

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


# ---- the launcher at the benchmark configs' sizes -------------------------------------------


class TinyLlamaBlock(nn.Module):
    """One LLaMA decoder layer at TinyLlama-1.1B's sizes (hidden 2048, 32
    query heads / 4 key-value heads of 64, intermediate 5632) as HF writes
    it: RMSNorm, q/k/v, causal grouped-query SDPA, o + residual, RMSNorm,
    SiLU(gate) * up, down + residual (RoPE left out: it is elementwise work
    outside the path)."""

    def __init__(self, h=2048, heads=32, kv_heads=4, inter=5632):
        super().__init__()
        self.heads, self.kv_heads, self.hd = heads, kv_heads, h // heads
        self.norm1, self.norm2 = RMS(h), RMS(h)
        self.q = nn.Linear(h, h, bias=False)
        self.k = nn.Linear(h, kv_heads * self.hd, bias=False)
        self.v = nn.Linear(h, kv_heads * self.hd, bias=False)
        self.o = nn.Linear(h, h, bias=False)
        self.gate = nn.Linear(h, inter, bias=False)
        self.up = nn.Linear(h, inter, bias=False)
        self.down = nn.Linear(inter, h, bias=False)
        for lin in (self.q, self.k, self.v, self.o, self.gate, self.up, self.down):
            nn.init.normal_(lin.weight, std=0.02)

    def forward(self, x):
        S = x.shape[0]
        hs = self.norm1(x)
        q = self.q(hs).view(S, self.heads, self.hd).transpose(0, 1)
        k = self.k(hs).view(S, self.kv_heads, self.hd).transpose(0, 1)
        v = self.v(hs).view(S, self.kv_heads, self.hd).transpose(0, 1)
        att = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        x = x + self.o(att.transpose(0, 1).reshape(S, -1))
        hs = self.norm2(x)
        return x + self.down(F.silu(self.gate(hs)) * self.up(hs))


def tinyllama_oracle(m, x):
    """The same layer from the oracle's functions in fp32, each projection's
    output rounded to fp16 as the fp16 forward stores it."""
    w = lambda lin: lin.weight.detach().numpy()  # noqa: E731
    r16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    S, hd = x.shape[0], m.hd
    xf = x.float().numpy()
    hs = ref.rms_norm_hf(xf, m.norm1.weight.detach().numpy(), m.norm1.eps)
    q, k, v = (r16(ref.linear(hs, w(lin))) for lin in (m.q, m.k, m.v))
    q = q.reshape(S, m.heads, hd).transpose(1, 0, 2)
    k = k.reshape(S, m.kv_heads, hd).transpose(1, 0, 2)
    v = v.reshape(S, m.kv_heads, hd).transpose(1, 0, 2)
    att = r16(ref.sdpa(q, k, v, 1.0 / np.sqrt(hd), causal=1, kv_group=m.heads // m.kv_heads))
    x1 = r16(xf + r16(ref.linear(att.transpose(1, 0, 2).reshape(S, -1), w(m.o))))
    hs2 = ref.rms_norm_hf(x1, m.norm2.weight.detach().numpy(), m.norm2.eps)
    a = r16(ref.silu_mul_linear(hs2, w(m.gate), w(m.up)))
    return x1 + r16(ref.linear(a, w(m.down)))


class ViTBlock(nn.Module):
    """ViT-B/16 attention + MLP at batch 8 (197 tokens, 12 heads of 64,
    MLP 768 -> 3072 -> 768 with tanh-GELU): q/k/v are given, as in the
    benchmark config; the MLP reads its own input."""

    def __init__(self, e=768, f=3072):
        super().__init__()
        self.fc1 = nn.Linear(e, f)
        self.fc2 = nn.Linear(f, e)
        for lin in (self.fc1, self.fc2):
            nn.init.normal_(lin.weight, std=0.02)
            nn.init.normal_(lin.bias, std=0.02)

    def forward(self, q, k, v, x):
        att = F.scaled_dot_product_attention(q, k, v)
        return att, self.fc2(F.gelu(self.fc1(x), approximate="tanh"))


def test_launcher_at_config_sizes(backend, dev, tmp_path, capsys):
    """A 512-token TinyLlama-shaped layer and the ViT-B/16 batch-8 block
    through run_torch_mlir: the plan uses the fused kernels (RMSNorm folded
    into the projections, SiLU-mul and GELU epilogues, fused attention) and
    the outputs match the oracle's composition of the same layer."""
    torch.manual_seed(0)
    tl = TinyLlamaBlock().half()
    x = torch.randn(512, 2048, generator=torch.Generator().manual_seed(7)).half()
    path = str(tmp_path / "tinyllama.pt2")
    backend.write_program_to_file(backend.export_program(tl, [x]), path)
    launcher = backend.TorchMLIRHexagonLauncher()
    out = launcher.run_torch_mlir(path, [x], "tinyllama", str(tmp_path), iterations=3)
    pats = sorted(p for p, _ in launcher.last_plan.kernels)
    print(f"[launcher] tinyllama plan {pats}", flush=True)
    assert pats == ["attention", "linear", "linear", "rms_linear", "rms_linear", "rms_linear", "rms_silu_mul"]
    want = tinyllama_oracle(tl.float(), x)
    err = ref.max_err_vs_scale(np32(out[0]), want)
    print(f"[launcher] tinyllama layer max err vs scale {err:.2e}, elementwise {ref.max_rel_err(np32(out[0]), want):.2e}",
          flush=True)
    assert err <= TOL

    vit = ViTBlock().half()
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(8, 12, 197, 64, generator=g).half() for _ in range(3))
    xv = torch.randn(8 * 197, 768, generator=g).half()
    path = str(tmp_path / "vit.pt2")
    backend.write_program_to_file(backend.export_program(vit, [q, k, v, xv]), path)
    launcher = backend.TorchMLIRHexagonLauncher()
    att, y = launcher.run_torch_mlir(path, [q, k, v, xv], "vit", str(tmp_path), iterations=3)
    pats = sorted(p for p, _ in launcher.last_plan.kernels)
    print(f"[launcher] vit plan {pats}", flush=True)
    assert pats == ["attention", "linear", "linear_gelu"]
    want_att = ref.sdpa(q.numpy(), k.numpy(), v.numpy(), 0.125)
    assert ref.max_err_vs_scale(np32(att), want_att) <= TOL
    vf = vit.float()
    h = ref.gemm_epilogue(xv.float().numpy(), vf.fc1.weight.detach().numpy(), "nt", "bias_gelu_tanh",
                          vf.fc1.bias.detach().numpy())
    h16 = h.astype(np.float16).astype(np.float32)  # fc1's output as the fp16 forward stores it
    want_y = ref.linear(h16, vf.fc2.weight.detach().numpy(), vf.fc2.bias.detach().numpy())
    err = ref.max_err_vs_scale(np32(y), want_y)
    print(f"[launcher] vit mlp max err vs scale {err:.2e}, elementwise {ref.max_rel_err(np32(y), want_y):.2e}",
          flush=True)
    assert err <= TOL
    text = capsys.readouterr().out
    perfs = [float(p) for p in re.findall(r"Perf:\s*([0-9]+(?:\.[0-9]+)?)", text)]
    assert len(perfs) == 2 and all(p > 0 for p in perfs)
    print(f"[launcher] Test_Info perf (us): tinyllama layer {perfs[0]}, vit block {perfs[1]}", flush=True)
