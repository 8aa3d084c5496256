"""GPU parity at the benchmark's full sizes, on the exact inputs, weights and
calls bench.py times (its own make_block / make_vit), against the oracle:

* the TinyLlama-1.1B prefill block, 512 tokens (RMSNorm statistics in the
  QKV GEMM, the row scales reused by the gate/up GEMM with its SiLU-mul
  epilogue over 2048 -> 11264, the O and down projections), stage by stage
  and end to end;
* the ViT-B/16 MLP at batch 8 (fc1 1576x768 -> 3072 + bias + tanh-GELU, fc2
  3072 -> 768 + bias) and its attention over 96 heads of 197 tokens.

Stage checks feed each kernel's own fp16 input to the oracle (elementwise
max relative error <= 1e-2); the end-to-end checks chain the oracle's own
fp16-rounded stages and compare relative to the output's scale, as the
other multi-kernel tests do."""
import numpy as np
import pytest
import torch

import bench
from gpu_util import TOL, np32
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

EPS = 1e-5


@pytest.fixture(scope="module")
def block(pkg, dev):
    step, gate_up, t, buf = bench.make_block(pkg, torch, dev)
    step()
    torch.cuda.synchronize()
    cpu = {k: np32(v.cpu()) for k, v in t.items() if isinstance(v, torch.Tensor)}
    out = {k: v.cpu() for k, v in buf.items()}
    return gate_up, t, buf, cpu, out


def _xn(cpu):
    """The RMSNorm of x without its weight (the weight is folded into the GEMM weights), fp32."""
    return ref.rms_norm(cpu["x"], np.ones(cpu["x"].shape[1], np.float32), EPS)


def _gate_up_exact(cpu):
    g, u = ref.unpack_gate_up_cols(cpu["wgu_f"].T, cpu["wgu_f"].shape[0])  # [K, I] each
    return ref.silu_mul_linear(_xn(cpu), g.T, u.T)


def test_tinyllama_gate_up_at_bench_shape(block):
    """The headline's dominant kernel exactly as bench.py launches it: M=512,
    N=11264 packed columns, K=2048, folded norm weight, rscale_in from the
    QKV call, SiLU-mul epilogue."""
    _, t, buf, cpu, out = block
    assert tuple(out["h"].shape) == (512, 5632)
    assert ref.max_rel_err(np32(out["h"]), _gate_up_exact(cpu)) <= TOL
    # the row scales the QKV GEMM published are the fp32 rsqrt(mean(x^2) + eps)
    rs = 1.0 / np.sqrt(np.mean(cpu["x"].astype(np.float64) ** 2, axis=1) + EPS)
    assert np.max(np.abs(out["rs"].numpy() - rs) / rs) <= 1e-5


def test_tinyllama_gate_up_repeat_is_identical(block):
    """Relaunching the gate/up GEMM alone (as the bench's roofline loop does)
    rewrites the same bits."""
    gate_up, _, buf, _, out = block
    for _ in range(3):
        gate_up()
    torch.cuda.synchronize()
    assert torch.equal(buf["h"].cpu(), out["h"])


def test_tinyllama_block_stages(block):
    _, t, buf, cpu, out = block
    assert ref.max_rel_err(np32(out["qkv"]), ref.linear(_xn(cpu), cpu["wqkv_f"])) <= TOL
    assert ref.max_rel_err(np32(out["o"]), ref.linear(cpu["xa"], cpu["wo"])) <= TOL
    # down projection (K = 5632 splits K into the workspace) on the kernel's own h
    assert ref.max_rel_err(np32(out["d"]), ref.linear(np32(out["h"]), cpu["wd"])) <= TOL


def test_tinyllama_block_end_to_end_vs_hf_order(block):
    """The block against the unfused HF order: RMSNorm rounded to fp16 before
    the weight and each projection, h rounded to fp16 before the down
    projection."""
    _, t, buf, cpu, out = block
    xn = ref.rms_norm_hf(cpu["x"], cpu["gn"], EPS).astype(np.float16).astype(np.float32)
    qkv = ref.linear(xn, cpu["wqkv"])
    h = ref.silu_mul_linear(xn, cpu["wg"], cpu["wu"]).astype(np.float16).astype(np.float32)
    d = ref.linear(h, cpu["wd"])
    for got, exp in ((out["qkv"], qkv), (out["h"], h), (out["d"], d)):
        o = np32(got)
        assert ref.max_err_vs_scale(o, exp) <= TOL
        assert np.sqrt(np.mean((o - exp) ** 2)) <= 3e-3 * np.sqrt(np.mean(exp**2))


@pytest.fixture(scope="module")
def vit(pkg, dev):
    step, attention, t, buf = bench.make_vit(pkg, torch, dev)
    step()
    torch.cuda.synchronize()
    cpu = {k: np32(v.cpu()) for k, v in t.items()}
    out = {k: v.cpu() for k, v in buf.items()}
    return cpu, out


def test_vit_fc1_bias_gelu_full_size(vit):
    cpu, out = vit
    assert tuple(out["h"].shape) == (1576, 3072)
    exp = ref.gemm_epilogue(cpu["x"], cpu["w1"], "nt", "bias_gelu_tanh", cpu["b1"])
    assert ref.max_rel_err(np32(out["h"]), exp) <= TOL


def test_vit_fc2_bias_full_size(vit):
    cpu, out = vit
    assert tuple(out["y"].shape) == (1576, 768)
    exp = ref.gemm_epilogue(np32(out["h"]), cpu["w2"], "nt", "bias", cpu["b2"])
    assert ref.max_rel_err(np32(out["y"]), exp) <= TOL


def test_vit_mlp_end_to_end(vit):
    cpu, out = vit
    h = ref.gemm_epilogue(cpu["x"], cpu["w1"], "nt", "bias_gelu_tanh", cpu["b1"])
    y = ref.gemm_epilogue(h.astype(np.float16).astype(np.float32), cpu["w2"], "nt", "bias", cpu["b2"])
    o = np32(out["y"])
    assert ref.max_err_vs_scale(o, y) <= TOL
    assert np.sqrt(np.mean((o - y) ** 2)) <= 3e-3 * np.sqrt(np.mean(y**2))


def test_vit_attention_full_batch(vit):
    """96 (batch x head) slices of 197 tokens, head dim 64, scale 1/8."""
    cpu, out = vit
    exp = ref.sdpa(cpu["q"], cpu["k"], cpu["v"], 0.125)
    o = np32(out["attn"])
    assert ref.max_err_vs_scale(o, exp) <= TOL
    assert np.sqrt(np.mean((o - exp) ** 2)) <= 2e-3 * np.sqrt(np.mean(exp**2))


def test_bench_self_checks_pass(block, vit, pkg, dev):
    """bench.py's own torch-fp32 check of one step accepts these outputs (it
    exits non-zero before timing anything otherwise)."""
    _, t, buf, _, _ = block
    assert max(bench.check_block(torch, t, buf).values()) <= TOL
    step, _, tv, bv = bench.make_vit(pkg, torch, dev)
    step()
    torch.cuda.synchronize()
    assert max(bench.check_vit(torch, tv, bv).values()) <= TOL
