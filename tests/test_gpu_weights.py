"""GPU parity of the weight formats: the int8 quantiser kernel
(hxmi_quantize_int8_rows_f16) bit-exact against the oracle, and decoder
layers packed by the loader (fused QKV with bias, interleaved gate/up, folded
RMSNorm, int8 codes) run through the kernels against the oracle applied to
the checkpoint's own unpacked tensors."""
import numpy as np
import pytest
import torch

from ckpt_util import CFG_QWEN25_05B, CFG_TINYLLAMA, hf_state_dict
from gpu_util import TOL, normal, np32
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu


def _quant_check(pkg, dev, w):
    q, s = pkg.quantize_int8(w.to(dev))
    q_ref, s_ref = ref.quantize_int8_rows(w.numpy())
    assert np.array_equal(s.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    return q, s


@pytest.mark.parametrize("N,K", [(896, 4864), (4864, 896), (1152, 896), (5, 8), (3, 520)])
def test_quantizer_bit_exact(pkg, dev, N, K):
    print(f"quantize_int8 N={N} K={K}", flush=True)
    _quant_check(pkg, dev, normal((N, K), N + K, 0.02))


def test_quantizer_edge_rows(pkg, dev):
    K = 64
    rows = np.zeros((8, K), np.float32)
    rows[1, 3] = 1e-6                                       # subnormal scale
    rows[2, :9] = np.array([127, 0.5, 1.5, 2.5, -2.5, 3.5, 100.5, -126.5, 126.5]) * 2.0 ** -6  # ties
    rows[3] = np.linspace(-0.05, 0.05, K)                    # max at both ends
    rows[4, 10] = -60000.0                                   # near the fp16 range limit
    rows[5, :] = 0.0123                                      # constant row
    rows[6, 7] = np.float16(1.0) + np.float16(2.0 ** -10)    # a scale that rounds down and is bumped
    rows[7] = -np.abs(np.random.default_rng(0).standard_normal(K)) * 0.02  # all negative
    w = torch.from_numpy(rows.astype(np.float16))
    q, s = _quant_check(pkg, dev, w)
    assert s[0].item() == 1 and not q[0].any()


def test_quantizer_strided_view(pkg, dev):
    big = normal((300, 1024), 7, 0.02)
    view = big[:, :512]  # ldw 1024
    q, s = pkg.quantize_int8(big.to(dev)[:, :512])
    q_ref, s_ref = ref.quantize_int8_rows(view.numpy())
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_quantized_linear_error_bound(pkg, dev):
    """w8a16 on the quantiser's codes stays within sum_k |x_k| * s_n / 2 of
    the fp16 weights' product (the per-element bound |w - q s| <= s / 2)."""
    w = normal((4864, 896), 11, 0.02)
    x = normal((16, 896), 12)
    q, s = pkg.quantize_int8(w.to(dev))
    y8 = pkg.w8a16_linear(x.to(dev), q, s).cpu()
    exact = ref.w8a16_linear(x.numpy(), q.cpu().numpy(), s.cpu().numpy())
    assert ref.max_rel_err(np32(y8), exact) <= TOL
    y16 = ref.linear(x.numpy(), w.numpy())
    bound = np.abs(np32(x)).sum(axis=1)[:, None] * np32(s.cpu())[None, :] / 2
    assert np.all(np.abs(exact - y16) <= bound * (1 + 1e-4) + 1e-6)


def _layer_inputs(c, M, seed):
    x = normal((M, c["hidden_size"]), seed)
    h = normal((M, c["num_attention_heads"] * (c["hidden_size"] // c["num_attention_heads"])), seed + 1)
    return x, h


@pytest.mark.parametrize("cfg,bias,M", [(CFG_QWEN25_05B, True, 16), (CFG_TINYLLAMA, False, 64)])
def test_packed_fp16_layer_through_kernels(pkg, dev, cfg, bias, M):
    W = pkg.weights
    print(f"packed fp16 layer {cfg['model_type']} M={M}", flush=True)
    sd = hf_state_dict(cfg, vocab=1024, qkv_bias=bias)
    c = W.DecoderConfig.from_hf(cfg)
    m = W.pack_model(sd, c, dev)
    L = m.layers[0]
    p = "model.layers.0."
    x, attn = _layer_inputs(cfg, M, 21)
    xd = x.to(dev)
    # QKV: RMSNorm folded, q/k/v concatenated, bias added after the norm
    qkv = pkg.rms_norm_linear(xd, L.qkv.weight, c.eps, bias=L.qkv.bias).cpu()
    xn = ref.rms_norm_hf(x.numpy(), sd[p + "input_layernorm.weight"].numpy(), c.eps)
    exp = np.concatenate([ref.linear(xn, sd[p + f"self_attn.{n}_proj.weight"].numpy(),
                                     sd[p + f"self_attn.{n}_proj.bias"].numpy() if bias else None)
                          for n in "qkv"], axis=1)
    assert ref.max_err_vs_scale(np32(qkv), exp) <= TOL
    # O projection
    o = pkg.linear(attn.to(dev), L.o.weight).cpu()
    assert ref.max_rel_err(np32(o), ref.linear(attn.numpy(), sd[p + "self_attn.o_proj.weight"].numpy())) <= TOL
    # gate/up with the post-attention norm folded and the SiLU-mul epilogue, then down
    h = pkg.rms_norm_linear(xd, L.gate_up.weight, c.eps, epilogue="silu_mul")
    xn2 = ref.rms_norm_hf(x.numpy(), sd[p + "post_attention_layernorm.weight"].numpy(), c.eps)
    h_exp = ref.silu_mul_linear(xn2, sd[p + "mlp.gate_proj.weight"].numpy(), sd[p + "mlp.up_proj.weight"].numpy())
    assert ref.max_err_vs_scale(np32(h.cpu()), h_exp) <= TOL
    d = pkg.linear(h, L.down.weight).cpu()
    assert ref.max_rel_err(np32(d), ref.linear(np32(h.cpu()), sd[p + "mlp.down_proj.weight"].numpy())) <= TOL
    # lm_head (tied to the embeddings for Qwen2)
    head = sd["model.embed_tokens.weight" if c.tie_word_embeddings else "lm_head.weight"]
    y = pkg.gemv(xd, m.lm_head.weight).cpu() if M <= 16 else pkg.linear(xd, m.lm_head.weight).cpu()
    assert ref.max_rel_err(np32(y), ref.linear(x.numpy(), head.numpy())) <= TOL


def test_packed_int8_layer_through_kernels(pkg, dev):
    W = pkg.weights
    cfg = CFG_QWEN25_05B
    sd = hf_state_dict(cfg, vocab=1024, qkv_bias=True)
    c = W.DecoderConfig.from_hf(cfg)
    m = W.pack_model(sd, c, dev, fold_norm=False, int8=True)
    L = m.layers[0]
    p = "model.layers.0."
    # the codes are the oracle quantiser's, on the packed fp16 layouts
    qkv16 = np.concatenate([sd[p + f"self_attn.{n}_proj.weight"].numpy() for n in "qkv"])
    gu16 = ref.pack_gate_up(sd[p + "mlp.gate_proj.weight"].numpy(), sd[p + "mlp.up_proj.weight"].numpy())
    for lin, w16 in ((L.qkv, qkv16), (L.gate_up, gu16), (L.down, sd[p + "mlp.down_proj.weight"].numpy()),
                     (m.lm_head, sd["model.embed_tokens.weight"].numpy())):
        q_ref, s_ref = ref.quantize_int8_rows(w16)
        assert lin.is_int8
        assert np.array_equal(lin.weight.cpu().numpy(), q_ref) and np.array_equal(lin.scale.cpu().numpy(), s_ref)
    # decode step pieces: RMSNorm kernel, then the int8 GEMV with the q/k/v bias
    for M in (1, 16):
        x = normal((M, c.hidden), 30 + M)
        xn = pkg.rms_norm(x.to(dev), L.input_norm, c.eps)
        assert ref.max_err_vs_scale(np32(xn.cpu()), ref.rms_norm_hf(x.numpy(), L.input_norm.cpu().numpy(),
                                                                    c.eps)) <= TOL
        y = pkg.w8a16_linear(xn, L.qkv.weight, L.qkv.scale, L.qkv.bias).cpu()
        exp = ref.w8a16_linear(np32(xn.cpu()), L.qkv.weight.cpu().numpy(), L.qkv.scale.cpu().numpy(),
                               L.qkv.bias.cpu().numpy())
        assert ref.max_rel_err(np32(y), exp) <= TOL


def test_packed_file_loads_to_gpu_and_runs_identically(pkg, dev, tmp_path):
    W = pkg.weights
    cfg = CFG_QWEN25_05B
    sd = hf_state_dict(cfg, vocab=1024, qkv_bias=True)
    c = W.DecoderConfig.from_hf(cfg)
    m = W.pack_model(sd, c, dev)
    f = tmp_path / "qwen_layer0.safetensors"
    W.save_packed(f, m)
    back = W.load_packed(f, dev)
    assert back.folded_norm and back.layers[0].qkv.weight.device.type == "cuda"
    x = normal((16, c.hidden), 40).to(dev)
    a = pkg.rms_norm_linear(x, m.layers[0].qkv.weight, c.eps, bias=m.layers[0].qkv.bias)
    b = pkg.rms_norm_linear(x, back.layers[0].qkv.weight, c.eps, bias=back.layers[0].qkv.bias)
    assert torch.equal(a, b)
    mi = W.pack_model(sd, c, dev, fold_norm=False, int8=True)
    W.save_packed(tmp_path / "i8.safetensors", mi)
    bi = W.load_packed(tmp_path / "i8.safetensors", dev)
    assert bi.int8 and torch.equal(bi.layers[0].down.weight, mi.layers[0].down.weight)
    assert torch.equal(bi.layers[0].down.scale, mi.layers[0].down.scale)
