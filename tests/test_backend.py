"""CPU tests of the reference-compatible Python surface (backend/)."""
import os
import re
import struct
import types

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import hot_path as ref


@pytest.fixture(scope="module")
def backend(pkg):
    import hexagon_mlir_amd.backend as b

    return b


# ---- HexagonOptions ------------------------------------------------------------------


def test_options_defaults_and_validation(backend):
    o = backend.HexagonOptions()
    # hot-path flags keep the reference defaults (hexagon_options.py:48-70)
    assert o.enableVTCMTiling and o.fusion and o.enableVectorization and not o.enableHexKL
    assert o.iterations == 10 and o.tileSizes == "" and o.target_artifact == "o"
    with pytest.raises(ValueError, match="Invalid target_artifact"):
        backend.HexagonOptions(target_artifact="exe")
    assert backend.HexagonOptions().hash() == backend.HexagonOptions().hash()
    assert backend.HexagonOptions(fusion=False).hash() != o.hash()


def test_options_dict_round_trip(backend):
    d = backend.HexagonOptions(enableLWP=True).__dict__
    assert backend.options_from_dict(d).enableLWP
    d2 = dict(d)
    d2["enableVTCMTiling"] = False  # callers mutate the dict (run_tinyllama.py:185-198)
    assert not backend.options_from_dict(d2).enableVTCMTiling
    with pytest.raises(KeyError, match="notAnOption"):
        backend.options_from_dict({"notAnOption": 1})


# ---- raw tensor files ----------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.int8, torch.int32, torch.int64, torch.uint8])
def test_raw_output_round_trip(backend, tmp_path, dtype):
    t = (torch.arange(24) - 7).reshape(2, 3, 4).to(dtype)
    p = tmp_path / "o0.raw"
    backend.write_output_tensor(p, t)
    data = p.read_bytes()
    # tensor.h:232-257: int32 dtype id, int64 rank, int64 shape, data
    assert struct.unpack_from("<i", data, 0)[0] == backend.DTYPE_IDS[dtype]
    assert struct.unpack_from("<q", data, 4)[0] == 3
    assert struct.unpack_from("<3q", data, 12) == (2, 3, 4)
    assert len(data) == 12 + 24 + 24 * t.element_size()
    back = backend.read_output_tensor(p)
    assert back.dtype == dtype and torch.equal(back, t)


def test_raw_rank0_and_errors(backend, tmp_path):
    p = tmp_path / "s.raw"
    backend.write_output_tensor(p, torch.tensor(3.5))
    assert backend.read_output_tensor(p).item() == 3.5
    p.write_bytes(struct.pack("<iq", 2, 1) + struct.pack("<q", 4) + b"\0" * 8)  # 4 floats need 16 bytes
    with pytest.raises(ValueError, match="data bytes"):
        backend.read_output_tensor(p)
    assert backend.to_torch_type(1) == torch.float16 and backend.to_torch_type(4) == torch.int8
    with pytest.raises(KeyError):
        backend.to_torch_type(99)


def test_raw_input_is_bare_data(backend, tmp_path):
    t = torch.randn(5, 3).half()
    p = tmp_path / "t0.raw"
    backend.write_input_tensor(p, t)
    assert p.read_bytes() == t.numpy().tobytes()


# ---- report and artifact folder ----------------------------------------------------------


def test_test_info_parses_like_the_reference(backend):
    text = backend.format_test_info("_mlir_ciface_mm", 12.5)
    # benchmark_models/micro_bench/test_matmul_benchmark.py:84-88
    assert float(re.search(r"Perf:\s*([0-9]+(?:\.[0-9]+)?)", text).group(1)) == 12.5
    assert re.search(r"Units:\s*([a-zA-Z]+)", text).group(1) == "us"
    assert "Result:Pass" in text and text.startswith("Test_Info: {")


def test_timestamped_folder(backend, tmp_path, monkeypatch):
    p = backend.create_timestamped_folder("mm", str(tmp_path))
    assert os.path.isdir(p) and os.path.basename(p).startswith("mm-")
    monkeypatch.setenv("HEXAGON_MLIR_DUMP_DIR", str(tmp_path))
    assert os.path.dirname(backend.create_timestamped_folder("x")) == str(tmp_path)
    with pytest.raises(AssertionError):
        backend.create_timestamped_folder("x", str(tmp_path / "missing"))


# ---- graph planner --------------------------------------------------------------------------


class RMS(nn.Module):
    """HF LlamaRMSNorm forward."""

    def __init__(self, h):
        super().__init__()
        self.weight = nn.Parameter(1 + 0.02 * torch.randn(h))
        self.eps = 1e-5

    def forward(self, x):
        dt = x.dtype
        x = x.to(torch.float32)
        v = x.pow(2).mean(-1, keepdim=True)
        x = x * torch.rsqrt(v + self.eps)
        return self.weight * x.to(dt)


class Block(nn.Module):
    def __init__(self, h=64, inter=128):
        super().__init__()
        self.norm = RMS(h)
        self.gate = nn.Linear(h, inter, bias=False)
        self.up = nn.Linear(h, inter, bias=False)
        self.down = nn.Linear(inter, h, bias=False)
        self.fc1 = nn.Linear(h, 96)

    def forward(self, x, q, k, v):
        hs = self.norm(x)
        m = self.down(F.silu(self.gate(hs)) * self.up(hs))
        y = F.gelu(self.fc1(m), approximate="tanh")
        a = torch.softmax(q @ k.transpose(-1, -2) * 0.125, dim=-1) @ v
        b = F.scaled_dot_product_attention(q, k, v)
        return y, a, b, F.rms_norm(x, (x.shape[-1],), self.norm.weight, 1e-5)


def block_inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(4, 64, generator=g).half()
    q, k, v = (torch.randn(2, 3, 16, 8, generator=g).half() for _ in range(3))
    return [x, q, k, v]


class OraclePkg(types.SimpleNamespace):
    """Stands in for the kernels on CPU, computing each call with the oracle,
    so the planner's rewiring (which tensors go where) is checked numerically."""

    @staticmethod
    def rms_norm(x, w, eps):
        return torch.from_numpy(ref.rms_norm_hf(x.numpy(), w.detach().numpy(), eps))

    @staticmethod
    def linear(x, w, b=None, epilogue=None):
        lead, x2 = x.shape[:-1], x.reshape(-1, x.shape[-1]).numpy()
        wn, bn = w.detach().numpy(), None if b is None else b.detach().numpy()
        if epilogue == "silu_mul":
            y = ref.gemm_epilogue(x2, wn, "nt", "silu_mul")
        elif epilogue == "gelu_tanh":
            y = ref.gemm_epilogue(x2, wn, "nt", "gelu_tanh" if bn is None else "bias_gelu_tanh", bn)
        else:
            y = ref.linear(x2, wn, bn)
        return torch.from_numpy(y).half().reshape(*lead, y.shape[-1])

    @staticmethod
    def attention(q, k, v, scale, mask=None, causal=0):
        if mask is not None and mask.dtype == torch.bool:
            mask = torch.where(mask, 0.0, float("-inf"))
        m = None if mask is None else mask.float().numpy()
        out = ref.sdpa(q.numpy(), k.numpy(), v.numpy(), scale, mask=m, causal=causal,
                       kv_group=q.shape[-3] // k.shape[-3])
        return torch.from_numpy(out).half()

    @staticmethod
    def pack_gate_up(wg, wu):
        return torch.from_numpy(ref.pack_gate_up(wg.numpy(), wu.numpy()))

    @staticmethod
    def fold_rms_weight(w, g):
        return (w.float() * g.float()[None, :]).half()

    @staticmethod
    def rms_norm_linear(x, w, eps, epilogue=None, bias=None, rscale_out=None, rscale_in=None):
        xn = ref.rms_norm(x.numpy(), np.ones(x.shape[-1], np.float32), eps)
        if rscale_out is not None:
            xf = x.float().numpy()
            rscale_out.copy_(torch.from_numpy(1 / np.sqrt((xf * xf).mean(-1) + eps)))
        if rscale_in is not None:  # the scales a previous call published
            xn = x.float().numpy() * rscale_in.numpy()[:, None]
        if epilogue == "silu_mul":
            y = ref.gemm_epilogue(xn, w.numpy(), "nt", "silu_mul")
        else:
            y = ref.linear(xn, w.numpy(), None if bias is None else bias.numpy())
        return torch.from_numpy(y).half()


class QKVIn(nn.Module):
    """Qwen2-style attention input: RMSNorm, then q/k/v projections with bias
    (q and v consume the norm, k a second one without bias)."""

    def __init__(self, h=64):
        super().__init__()
        self.norm = RMS(h)
        self.norm2 = RMS(h)
        self.q = nn.Linear(h, 64)
        self.k = nn.Linear(h, 32, bias=False)
        self.v = nn.Linear(h, 32)

    def forward(self, x):
        hs = self.norm(x)
        return self.q(hs), self.v(hs), self.k(self.norm2(x))


@pytest.fixture
def oracle_kernels(monkeypatch):
    from hexagon_mlir_amd.backend import graph

    monkeypatch.setattr(graph, "_pkg", lambda: OraclePkg())


def test_planner_matches_hot_path_patterns(backend, oracle_kernels):
    torch.manual_seed(0)
    model = Block().half()
    ep = backend.export_program(model, block_inputs())
    plan = backend.plan_program(ep, torch.device("cpu"), fusion=True)
    pats = sorted(p for p, _ in plan.kernels)
    # the norm feeding only gate/up is folded into that GEMM; F.rms_norm of
    # the output stays a kernel
    assert pats == ["attention", "attention", "linear", "linear_gelu", "rms_norm", "rms_silu_mul"], pats
    # nothing of the hot path is left to torch
    left = " ".join(plan.torch_ops)
    for op in ("linear", "matmul", "softmax", "rsqrt", "silu", "gelu", "rms_norm", "scaled_dot"):
        assert op not in left, left


class MaskedAttn(nn.Module):
    """Decoder-style attention calls: a padding mask, a causal one over
    grouped K/V heads, and one the fused kernel cannot take (head dim 8),
    which runs the three steps with the masked softmax."""

    def forward(self, q, k, v, kg, vg, m, q8, k8, v8, m8):
        a = F.scaled_dot_product_attention(q, k, v, attn_mask=m)
        b = F.scaled_dot_product_attention(q, kg, vg, is_causal=True, enable_gqa=True)
        c = F.scaled_dot_product_attention(q8, k8, v8, attn_mask=m8)
        return a, b, c


def test_planner_routes_masked_causal_gqa_attention(backend, oracle_kernels):
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 4, 16, 64, generator=g).half() for _ in range(3))
    kg, vg = (torch.randn(1, 2, 16, 64, generator=g).half() for _ in range(2))
    m = torch.zeros(1, 1, 16, 16).half()
    m[..., 12:] = float("-inf")
    q8, k8, v8 = (torch.randn(1, 2, 16, 8, generator=g).half() for _ in range(3))
    m8 = torch.zeros(16, 16).half()
    args = [q, k, v, kg, vg, m, q8, k8, v8, m8]
    ep = backend.export_program(MaskedAttn(), args)
    plan = backend.plan_program(ep, torch.device("cpu"), fusion=True)
    assert sorted(p for p, _ in plan.kernels) == ["attention", "attention", "attention"]
    assert not any("scaled_dot" in t for t in plan.torch_ops)
    a, b, c = plan(*args)
    ex = lambda x: x.float().numpy()  # noqa: E731
    assert ref.max_err_vs_scale(ex(a), ref.sdpa(ex(q), ex(k), ex(v), mask=ex(m))) < 1e-2
    assert ref.max_err_vs_scale(ex(b), ref.sdpa(ex(q), ex(kg), ex(vg), causal=1, kv_group=2)) < 1e-2
    assert ref.max_err_vs_scale(ex(c), ref.sdpa(ex(q8), ex(k8), ex(v8), mask=ex(m8))) < 1e-2


def test_planner_without_fusion_keeps_elementwise_ops(backend, oracle_kernels):
    torch.manual_seed(0)
    plan = backend.plan_program(backend.export_program(Block().half(), block_inputs()), torch.device("cpu"),
                                fusion=False)
    pats = [p for p, _ in plan.kernels]
    assert "silu_mul" not in pats and "linear_gelu" not in pats and pats.count("linear") == 4
    assert any("silu" in t for t in plan.torch_ops) and any("gelu" in t for t in plan.torch_ops)


def test_planner_folds_rmsnorm_into_projections(backend, oracle_kernels):
    torch.manual_seed(0)
    model = QKVIn().half()
    x = torch.randn(6, 64, generator=torch.Generator().manual_seed(2)).half()
    plan = backend.plan_program(backend.export_program(model, [x]), torch.device("cpu"), fusion=True)
    assert sorted(p for p, _ in plan.kernels) == ["rms_linear"] * 3, plan.kernels
    assert not any("rsqrt" in t or "linear" in t for t in plan.torch_ops), plan.torch_ops
    got = plan.module(x)
    exp = model.float()(x.float())
    for g_, e in zip(got, exp):
        assert ref.max_err_vs_scale(g_.float().numpy(), e.detach().numpy()) < 1e-2


def test_planner_keeps_rmsnorm_with_other_users(backend, oracle_kernels):
    class Two(nn.Module):
        def __init__(self):
            super().__init__()
            self.norm = RMS(64)
            self.q = nn.Linear(64, 32, bias=False)

        def forward(self, x):
            hs = self.norm(x)
            return self.q(hs), hs * 2

    plan = backend.plan_program(backend.export_program(Two().half(), [torch.randn(4, 64).half()]),
                                torch.device("cpu"), fusion=True)
    assert sorted(p for p, _ in plan.kernels) == ["linear", "rms_norm"]


def test_planner_rewiring_is_numerically_right(backend, oracle_kernels):
    torch.manual_seed(0)
    model = Block().half()
    inputs = block_inputs(1)
    plan = backend.plan_program(backend.export_program(model, inputs), torch.device("cpu"), fusion=True)
    got = plan.module(*inputs)
    exp = model.float()(*[t.float() for t in inputs])
    for g, e in zip(got, exp):
        assert ref.max_err_vs_scale(g.float().numpy(), e.detach().numpy()) < 1e-2


def test_planner_leaves_fp32_to_torch(backend):
    torch.manual_seed(0)
    model = Block().float()
    plan = backend.plan_program(backend.export_program(model, [t.float() for t in block_inputs()]),
                                torch.device("cpu"))
    assert plan.kernels == []


def test_etm_is_not_available(backend, tmp_path):
    with pytest.raises(NotImplementedError):
        backend.TorchMLIRHexagonLauncher(torch.device("cpu")).run_torch_mlir(
            "missing.pt2", [], "f", str(tmp_path), enable_etm=True)


# ---- LWP region timing files --------------------------------------------------------


def fold_lwp(entries):
    """The pairing rule of the reference's region tooling
    (test/python/process_lwp.py:20-60), restated: a record whose id is on top
    of the stack of open regions closes it, any other record opens a region
    (an id may not reopen while open); returns {id: (total, count, parent)}."""
    stack, summary = [], {}
    for e in entries:
        rid, cyc = e["id"], e["cyc"]
        if stack and stack[-1][0] == rid:
            _, start, parent = stack.pop()
            tot, cnt, par = summary.get(rid, (0, 0, None))
            summary[rid] = (tot + cyc - start, cnt + 1, par if par is not None else parent)
        else:
            assert rid not in [s[0] for s in stack], f"region {rid} reopened while open"
            stack.append((rid, cyc, stack[-1][0] if stack else None))
    assert not stack, f"regions left open: {stack}"
    return summary


def test_lwp_files_follow_the_reference_layout(backend):
    from hexagon_mlir_amd.backend import lwp

    entries = [{"id": 0, "cyc": 100}, {"id": 1, "cyc": 110}, {"id": 1, "cyc": 150}, {"id": 2, "cyc": 150},
               {"id": 2, "cyc": 400}, {"id": 0, "cyc": 401}]
    text = lwp.lwp_json(entries, 100_000_000)
    d = json_loads(text)
    assert d["entries"] == entries and d["cyc_hz"] == 100_000_000
    # prof_utils.cc:37-60 writes one {"id", "cyc"} object per record, in order
    assert re.search(r'"entries": \[\n    \{\n      "id": 0,\n      "cyc": 100\n    \},', text)
    s = fold_lwp(d["entries"])
    assert s == {1: (40, 1, 0), 2: (250, 1, 0), 0: (301, 1, None)}
    dump = lwp.infodump_lines([(0, [0], ["func"]), (1, [3], ["linear_1: hx_linear"]), (2, [5, 6], ["a", "b"])])
    # the line format process_lwp.py:63-88 reads
    pat = re.compile(r"Location ([\d,\s]+) corresponds to ID (\d+)")
    parsed = {}
    for line in dump.strip().split("\n"):
        loc, ops = line.split(" | Collected ops:", 1)
        m = pat.search(loc)
        parsed[int(m.group(2))] = ([int(v) for v in m.group(1).split(",")], [o.strip() for o in ops.split(",")])
    assert parsed == {0: ([0], ["func"]), 1: ([3], ["linear_1: hx_linear"]), 2: ([5, 6], ["a", "b"])}


def test_lwp_pairing_rejects_interleaved_regions():
    with pytest.raises(AssertionError, match="reopened"):
        fold_lwp([{"id": 1, "cyc": 0}, {"id": 2, "cyc": 1}, {"id": 1, "cyc": 2}])


def json_loads(text):
    import json

    return json.loads(text)
