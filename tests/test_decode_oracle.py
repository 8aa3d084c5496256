"""Pin oracle.decode_step, the oracle the persistent decode step is compared with.

The step is the HF Qwen2 forward of one token at position 0
(benchmark_models/run_qwen2.5-0.5b.py:171-173,224-233).  transformers'
Qwen2ForCausalLM, built from a small random config on the CPU (nothing is
downloaded), is the library routine it reduces to; the oracle must agree
with it in fp32 and, with fp16 rounding on, with its fp16 forward.  Closed
forms cover what a random model could hide: with zero o/down projections the
residual stream is the embedding itself, and the attention output of every
query head is v of its own key/value head.
"""
import numpy as np
import pytest
import torch

from oracle import hot_path as ref

transformers = pytest.importorskip("transformers")


def hf_model(layers=2, hidden=64, inter=96, heads=4, kv_heads=2, vocab=50, seed=0, bias_scale=0.5):
    cfg = transformers.Qwen2Config(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                                   num_attention_heads=heads, num_key_value_heads=kv_heads, vocab_size=vocab,
                                   rms_norm_eps=1e-6, max_position_embeddings=32, tie_word_embeddings=False)
    torch.manual_seed(seed)
    m = transformers.Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():
        # non-trivial norm weights and biases, weights large enough that every term matters
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * (0.2 if p.dim() == 2 else bias_scale))
        for layer in m.model.layers:
            layer.input_layernorm.weight.add_(1.0)
            layer.post_attention_layernorm.weight.add_(1.0)
        m.model.norm.weight.add_(1.0)
    return m


def stacked(m):
    """The model's weights in the step's layout (numpy fp32)."""
    ls = m.model.layers
    t = lambda x: x.detach().float().numpy()
    cat = lambda *xs: np.concatenate([t(x) for x in xs], axis=0)
    return dict(
        w_qkv=np.stack([cat(l.self_attn.q_proj.weight, l.self_attn.k_proj.weight, l.self_attn.v_proj.weight)
                        for l in ls]),
        b_qkv=np.stack([cat(l.self_attn.q_proj.bias, l.self_attn.k_proj.bias, l.self_attn.v_proj.bias) for l in ls]),
        w_o=np.stack([t(l.self_attn.o_proj.weight) for l in ls]),
        w_gu=np.stack([cat(l.mlp.gate_proj.weight, l.mlp.up_proj.weight) for l in ls]),
        w_down=np.stack([t(l.mlp.down_proj.weight) for l in ls]),
        g_attn=np.stack([t(l.input_layernorm.weight) for l in ls]),
        g_mlp=np.stack([t(l.post_attention_layernorm.weight) for l in ls]),
        g_final=t(m.model.norm.weight),
        w_lm=t(m.lm_head.weight),
    )


def run_hf(m, token):
    with torch.no_grad():
        out = m.model(input_ids=torch.tensor([[token]]), position_ids=torch.tensor([[0]]), use_cache=False)
        h = out.last_hidden_state[0, 0]
        return h.float().numpy(), m.lm_head(h).float().numpy()


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (4, 4), (4, 1)])
def test_decode_step_matches_hf_qwen2_fp32(heads, kv_heads):
    m = hf_model(heads=heads, kv_heads=kv_heads, seed=heads + kv_heads)
    w = stacked(m)
    tok = 11
    x = m.model.embed_tokens.weight[tok].detach().numpy()
    out = ref.decode_step(x, heads=heads, kv_heads=kv_heads, eps=1e-6, fp16=False, **w)
    h_hf, logits_hf = run_hf(m, tok)
    assert np.abs(out["h"] - h_hf).max() < 1e-4 * max(1.0, np.abs(h_hf).max())
    assert np.abs(out["logits"] - logits_hf).max() < 1e-4 * max(1.0, np.abs(logits_hf).max())


def test_decode_step_fp16_rounding_matches_hf_fp16_forward():
    m = hf_model(layers=3, seed=5)
    w32 = stacked(m)
    mh = m.half()
    try:
        h_hf, logits_hf = run_hf(mh, 3)
    except RuntimeError as e:  # a CPU build without fp16 kernels
        pytest.skip(f"torch CPU fp16 forward unavailable: {e}")
    w16 = {k: v.astype(np.float16) for k, v in w32.items()}
    x = mh.model.embed_tokens.weight[3].detach().numpy()
    out16 = ref.decode_step(x, heads=4, kv_heads=2, eps=1e-6, fp16=True, **w16)
    out32 = ref.decode_step(x, heads=4, kv_heads=2, eps=1e-6, fp16=False, **w16)
    scale = np.abs(h_hf).max()
    err16 = np.abs(out16["h"] - h_hf).max() / scale
    err32 = np.abs(out32["h"] - h_hf).max() / scale
    # the fp16-rounding oracle tracks HF's fp16 forward to fp16 noise, closer than the fp32 forward does
    assert err16 < 4e-3
    assert err16 <= err32
    assert np.abs(out16["logits"] - logits_hf).max() / np.abs(logits_hf).max() < 1e-2


def test_decode_step_zero_projections_keep_the_embedding():
    r = np.random.default_rng(2)
    L, H, I, heads, kvh = 3, 32, 48, 4, 2
    kv = H // heads * kvh
    x = r.standard_normal(H).astype(np.float32)
    g = r.uniform(0.5, 1.5, (L, H)).astype(np.float32)
    gf = r.uniform(0.5, 1.5, H).astype(np.float32)
    w = dict(w_qkv=r.standard_normal((L, H + 2 * kv, H)).astype(np.float32), b_qkv=None,
             w_o=np.zeros((L, H, H), np.float32), w_gu=r.standard_normal((L, 2 * I, H)).astype(np.float32),
             w_down=np.zeros((L, H, I), np.float32), g_attn=g, g_mlp=g, g_final=gf)
    out = ref.decode_step(x, heads=heads, kv_heads=kvh, eps=1e-6, fp16=False, **w)
    assert np.array_equal(out["x"], x)
    want = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * gf
    assert np.abs(out["h"] - want).max() < 1e-5


def test_decode_step_attention_routes_each_head_to_its_kv_head():
    # o projection = identity, v bias = a distinct constant per kv head, all
    # q/k/v weights zero: x1 = x + att, att[head i] = bias of kv head i // grp
    L, H, I, heads, kvh = 1, 32, 16, 4, 2
    hd, kv, grp = H // heads, H // heads * kvh, heads // kvh
    x = np.zeros(H, np.float32)
    x[0] = 1.0  # keeps RMSNorm finite
    b = np.zeros((L, H + 2 * kv), np.float32)
    for j in range(kvh):
        b[0, H + kv + j * hd:H + kv + (j + 1) * hd] = 10.0 * (j + 1) + np.arange(hd)
    w = dict(w_qkv=np.zeros((L, H + 2 * kv, H), np.float32), b_qkv=b, w_o=np.eye(H, dtype=np.float32)[None],
             w_gu=np.zeros((L, 2 * I, H), np.float32), w_down=np.zeros((L, H, I), np.float32),
             g_attn=np.ones((L, H), np.float32), g_mlp=np.ones((L, H), np.float32),
             g_final=np.ones(H, np.float32))
    out = ref.decode_step(x, heads=heads, kv_heads=kvh, eps=1e-6, fp16=False, **w)
    att = out["x"] - x
    for i in range(heads):
        np.testing.assert_array_equal(att[i * hd:(i + 1) * hd], 10.0 * (i // grp + 1) + np.arange(hd))
