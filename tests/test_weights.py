"""CPU checks of the int8 quantiser's oracle and of the weight loader's
layouts, files and errors.  The GPU side (the quantiser kernel bit-exact
against the oracle, packed layers through the kernels) is
tests/test_gpu_weights.py."""
import json

import numpy as np
import pytest
import torch

from ckpt_util import CFG_LLAMA, CFG_QWEN, hf_state_dict
from oracle import hot_path as ref

# ---- oracle quantiser pins ----------------------------------------------------------


def _all_positive_fp16() -> np.ndarray:
    bits = np.arange(1, 0x7C00, dtype=np.uint16)  # every positive finite fp16
    return bits.view(np.float16)


def test_quantizer_known_answer_integer_grid():
    """w = c * 2^-7 with integer c and max |c| = 127: the scale is exactly
    2^-7 and the codes are c themselves."""
    rng = np.random.default_rng(0)
    c = rng.integers(-127, 128, size=(16, 64))
    c[:, 5] = np.where(rng.integers(0, 2, 16) == 1, 127, -127)
    w = (c * 2.0 ** -7).astype(np.float16)
    q, s = ref.quantize_int8_rows(w)
    assert np.all(s == np.float16(2.0 ** -7))
    assert np.array_equal(q.astype(np.int64), c)


def test_quantizer_ties_round_half_to_even():
    s0 = 2.0 ** -6
    halves = np.array([0.5, 1.5, 2.5, -2.5, 3.5, 100.5, -126.5, 126.5])
    row = np.concatenate([[127.0], halves]) * s0
    q, s = ref.quantize_int8_rows(row.astype(np.float16)[None, :])
    assert s[0] == np.float16(s0)
    assert [int(v) for v in q[0, 1:]] == [round(h) for h in halves]  # Python rounds half to even


def test_quantizer_scale_is_smallest_covering_fp16():
    """Brute force over every positive fp16: s is the smallest v with
    127 * v >= max|w| (and no code clips)."""
    cand = _all_positive_fp16().astype(np.float64)
    rng = np.random.default_rng(1)
    amax = np.concatenate([
        (rng.standard_normal(400) * 0.05),
        rng.uniform(1e-7, 1e-4, 100),  # scales in the fp16 subnormal range
        rng.uniform(1, 60000, 100),
        _all_positive_fp16()[rng.integers(0, 0x7B00, 200)].astype(np.float64),
    ])
    amax = np.abs(amax).astype(np.float16)
    amax = amax[amax > 0]
    w = np.zeros((amax.size, 8), np.float16)
    w[:, 3] = amax
    w[::2, 3] *= np.float16(-1)
    q, s = ref.quantize_int8_rows(w)
    for i, a in enumerate(amax.astype(np.float64)):
        want = cand[np.searchsorted(127.0 * cand, a)]  # first v with 127 v >= a
        assert float(s[i]) == want, (a, float(s[i]), want)
    assert np.all(np.abs(q[:, 3].astype(np.int64)) <= 127)


def test_quantizer_zero_row_and_error_bound():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float16)
    w[7] = 0
    q, s = ref.quantize_int8_rows(w)
    assert s[7] == 1 and not q[7].any()
    err = np.abs(w.astype(np.float64) - q.astype(np.float64) * s.astype(np.float64)[:, None])
    assert np.all(err <= s.astype(np.float64)[:, None] * (0.5 + 1e-6))
    nz = np.arange(64) != 7
    assert np.all(np.abs(q[nz]).max(axis=1) == 127)


def test_quantizer_sign_symmetry_and_power_of_two_equivariance():
    """quantize(-w) = (-q, s) and quantize(w * 2^j) = (q, s * 2^j) exactly
    while every scale stays a normal fp16."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((32, 128)) * 0.03).astype(np.float16)
    q, s = ref.quantize_int8_rows(w)
    qn, sn = ref.quantize_int8_rows(-w)
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    for j in (-3, 1, 5):
        qj, sj = ref.quantize_int8_rows((w.astype(np.float32) * 2.0 ** j).astype(np.float16))
        assert np.array_equal(qj, q)
        assert np.array_equal(sj, (s.astype(np.float32) * 2.0 ** j).astype(np.float16))


# ---- loader layouts (CPU: no kernels involved with fold_norm=False, int8=False) -----

def test_config_from_hf_defaults(pkg):
    W = pkg.weights
    c = W.DecoderConfig.from_hf({"hidden_size": 896, "intermediate_size": 4864, "num_hidden_layers": 24,
                                 "num_attention_heads": 14, "num_key_value_heads": 2, "rms_norm_eps": 1e-6,
                                 "tie_word_embeddings": True, "model_type": "qwen2"})
    assert (c.head_dim, c.qkv_rows, c.eps, c.tie_word_embeddings) == (64, 1152, 1e-6, True)
    c = W.DecoderConfig.from_hf({"hidden_size": 2048, "intermediate_size": 5632, "num_hidden_layers": 22,
                                 "num_attention_heads": 32})
    assert (c.kv_heads, c.head_dim, c.eps, c.tie_word_embeddings) == (32, 64, 1e-5, False)


@pytest.mark.parametrize("cfg,bias", [(CFG_LLAMA, False), (CFG_QWEN, True)])
def test_pack_layout_on_cpu(pkg, cfg, bias):
    W = pkg.weights
    sd = hf_state_dict(cfg, qkv_bias=bias)
    c = W.DecoderConfig.from_hf(cfg)
    m = W.pack_model(sd, c, torch.device("cpu"), fold_norm=False)
    assert len(m.layers) == 2 and not m.int8 and not m.folded_norm
    for i, layer in enumerate(m.layers):
        p = f"model.layers.{i}.self_attn."
        exp = torch.cat([sd[p + "q_proj.weight"], sd[p + "k_proj.weight"], sd[p + "v_proj.weight"]])
        assert torch.equal(layer.qkv.weight, exp) and layer.qkv.shape == (c.qkv_rows, c.hidden)
        if bias:
            assert torch.equal(layer.qkv.bias, torch.cat([sd[p + f"{n}_proj.bias"] for n in "qkv"]))
        else:
            assert layer.qkv.bias is None
        mp = f"model.layers.{i}.mlp."
        gu = ref.pack_gate_up(sd[mp + "gate_proj.weight"].numpy(), sd[mp + "up_proj.weight"].numpy())
        assert np.array_equal(layer.gate_up.weight.numpy(), gu)
        assert torch.equal(layer.down.weight, sd[mp + "down_proj.weight"])
        assert torch.equal(layer.input_norm, sd[f"model.layers.{i}.input_layernorm.weight"])
    head = sd["model.embed_tokens.weight"] if cfg["tie_word_embeddings"] else sd["lm_head.weight"]
    assert torch.equal(m.lm_head.weight, head)


def test_packed_file_round_trip(pkg, tmp_path):
    W = pkg.weights
    sd = hf_state_dict(CFG_QWEN, qkv_bias=True)
    c = W.DecoderConfig.from_hf(CFG_QWEN)
    m = W.pack_model(sd, c, torch.device("cpu"), fold_norm=False, layers=[1])
    f = tmp_path / "packed.safetensors"
    W.save_packed(f, m)
    back = W.load_packed(f, torch.device("cpu"))
    assert back.config == c and back.extra["layer_index"] == [1] and not back.folded_norm
    for n in ("qkv", "o", "gate_up", "down"):
        a, b = getattr(m.layers[0], n), getattr(back.layers[0], n)
        assert torch.equal(a.weight, b.weight)
        assert (a.bias is None) == (b.bias is None) and (a.bias is None or torch.equal(a.bias, b.bias))
    assert torch.equal(back.norm, m.norm) and torch.equal(back.lm_head.weight, m.lm_head.weight)


def test_read_checkpoint_directory_and_shards(pkg, tmp_path):
    from safetensors.torch import save_file

    W = pkg.weights
    sd = hf_state_dict(CFG_LLAMA)
    keys = sorted(sd)
    half = len(keys) // 2
    shards = {"model-00001-of-00002.safetensors": keys[:half], "model-00002-of-00002.safetensors": keys[half:]}
    for name, ks in shards.items():
        save_file({k: sd[k] for k in ks}, str(tmp_path / name))
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {k: n for n, ks in shards.items() for k in ks}}))
    (tmp_path / "config.json").write_text(json.dumps(CFG_LLAMA))
    got, cfg = W.read_checkpoint(tmp_path)
    assert cfg == W.DecoderConfig.from_hf(CFG_LLAMA)
    assert set(got) == set(sd) and all(torch.equal(got[k], sd[k]) for k in sd)
    inferred = W.infer_config(got, heads=4, kv_heads=2)
    assert inferred == cfg


def test_loader_errors(pkg, tmp_path):
    W = pkg.weights
    c = W.DecoderConfig.from_hf(CFG_QWEN)
    sd = hf_state_dict(CFG_QWEN, qkv_bias=True)
    del sd["model.layers.0.self_attn.k_proj.bias"]
    with pytest.raises(ValueError, match="biases"):
        W.pack_decoder_layer(sd, 0, c, torch.device("cpu"), fold_norm=False)
    del sd["model.layers.1.mlp.up_proj.weight"]
    with pytest.raises(KeyError, match="up_proj"):
        W.pack_decoder_layer(sd, 1, c, torch.device("cpu"), fold_norm=False)
    bad = W.DecoderConfig(**{**c.__dict__, "heads": 8})
    with pytest.raises(ValueError, match="do not match"):
        W.pack_decoder_layer(hf_state_dict(CFG_QWEN), 0, bad, torch.device("cpu"), fold_norm=False)
    with pytest.raises(ValueError, match="fold_norm"):
        W.pack_decoder_layer(hf_state_dict(CFG_QWEN), 0, c, torch.device("cpu"), fold_norm=True, int8=True)
    # folding and quantising run on the GPU kernels: no CPU path
    with pytest.raises(pkg.HxmiError, match="GPU"):
        W.pack_decoder_layer(hf_state_dict(CFG_QWEN), 0, c, torch.device("cpu"))
    with pytest.raises(pkg.HxmiError, match="GPU"):
        pkg.quantize_int8(torch.zeros(8, 8, dtype=torch.float16))
    from safetensors.torch import save_file

    other = tmp_path / "other.safetensors"
    save_file({"x": torch.zeros(2)}, str(other), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="hxmi-packed"):
        W.load_packed(other, torch.device("cpu"))


def test_read_single_file_and_version_check(pkg, tmp_path):
    from safetensors.torch import save_file

    W = pkg.weights
    sd = hf_state_dict(CFG_QWEN)
    f = tmp_path / "model.safetensors"
    save_file(sd, str(f))
    got, cfg = W.read_checkpoint(f)
    assert cfg is None and set(got) == set(sd)
    inferred = W.infer_config(got, heads=4, kv_heads=1, eps=1e-6)
    assert inferred.tie_word_embeddings and inferred.head_dim == 32 and inferred.layers == 2
    m = W.pack_model(got, inferred, torch.device("cpu"), fold_norm=False)
    out = tmp_path / "p.safetensors"
    W.save_packed(out, m)
    # a file written by a later format version is refused, not misread
    from safetensors import safe_open

    with safe_open(str(out), framework="pt") as fh:
        meta = dict(fh.metadata())
        tensors = {k: fh.get_tensor(k) for k in fh.keys()}
    meta["version"] = "2"
    save_file(tensors, str(tmp_path / "v2.safetensors"), metadata=meta)
    with pytest.raises(ValueError, match="version 2"):
        W.load_packed(tmp_path / "v2.safetensors", torch.device("cpu"))


def test_int8_packing_needs_the_gpu(pkg):
    W = pkg.weights
    c = W.DecoderConfig.from_hf(CFG_LLAMA)
    with pytest.raises(pkg.HxmiError, match="GPU"):
        W.pack_model(hf_state_dict(CFG_LLAMA), c, torch.device("cpu"), fold_norm=False, int8=True)
