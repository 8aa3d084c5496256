"""Random decoder checkpoints with Hugging Face LLaMA / Qwen2 tensor names,
for the weight-loader tests (CPU and GPU)."""
import torch

CFG_LLAMA = dict(hidden_size=128, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, rms_norm_eps=1e-5, model_type="llama", tie_word_embeddings=False)
CFG_QWEN = dict(hidden_size=128, intermediate_size=160, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=1, rms_norm_eps=1e-6, model_type="qwen2", tie_word_embeddings=True)


def hf_state_dict(cfg: dict, vocab: int = 256, seed: int = 0, qkv_bias: bool = False) -> dict:
    """A random checkpoint with Hugging Face LLaMA / Qwen2 tensor names."""
    g = torch.Generator().manual_seed(seed)
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    nh, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = H // nh

    def w(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).half()

    sd = {"model.embed_tokens.weight": w(vocab, H), "model.norm.weight": (1 + w(H)).half()}
    if not cfg["tie_word_embeddings"]:
        sd["lm_head.weight"] = w(vocab, H)
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = (1 + w(H)).half()
        sd[p + "post_attention_layernorm.weight"] = (1 + w(H)).half()
        sd[p + "self_attn.q_proj.weight"] = w(nh * D, H)
        sd[p + "self_attn.k_proj.weight"] = w(nkv * D, H)
        sd[p + "self_attn.v_proj.weight"] = w(nkv * D, H)
        sd[p + "self_attn.o_proj.weight"] = w(H, nh * D)
        if qkv_bias:
            sd[p + "self_attn.q_proj.bias"] = w(nh * D)
            sd[p + "self_attn.k_proj.bias"] = w(nkv * D)
            sd[p + "self_attn.v_proj.bias"] = w(nkv * D)
        sd[p + "mlp.gate_proj.weight"] = w(I, H)
        sd[p + "mlp.up_proj.weight"] = w(I, H)
        sd[p + "mlp.down_proj.weight"] = w(H, I)
    return sd

# one layer of each model the decoder configs are shaped on
CFG_QWEN25_05B = dict(hidden_size=896, intermediate_size=4864, num_hidden_layers=1, num_attention_heads=14,
                      num_key_value_heads=2, rms_norm_eps=1e-6, model_type="qwen2", tie_word_embeddings=True)
CFG_TINYLLAMA = dict(hidden_size=2048, intermediate_size=5632, num_hidden_layers=1, num_attention_heads=32,
                     num_key_value_heads=4, rms_norm_eps=1e-5, model_type="llama", tie_word_embeddings=False)
