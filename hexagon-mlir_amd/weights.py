"""Weight formats the kernels read, and a loader that turns LLaMA / Qwen2
decoder checkpoints (Hugging Face tensor names, safetensors files) into them.

The reference compiles a whole model through torch-mlir with its weights as
constants of the compiled module (benchmark_models/run_tinyllama.py:70-88);
``lowerConstantsInSeparateSharedObjects`` moves those constants into artifacts
of their own (triton_qcom_hexagon_backend_api.cc:196-214).  Here the kernels
are compiled once and weights are data: prepared once at load time into the
layouts below, kept in HBM, and optionally written to a packed safetensors
file that a later process loads straight to the GPU without repacking.

Layouts (row-major; ``nn.Linear``'s ``[out_features, in_features]`` is
already the NT operand, so no transposed copy is made):

  fp16 projection   ``W [N, K]`` fp16.
  fused QKV         q, k and v rows concatenated, ``[Hq*D + 2*Hkv*D, K]``;
                    the q/k/v biases (Qwen2) concatenated the same way.
  packed gate/up    ``[2I, K]`` in 16-row blocks alternating gate and up, the
                    order the SiLU-mul epilogue pairs its output columns in.
  folded RMSNorm    ``fp16(W * g[None, :])`` for the projections that read
                    the normalised rows (QKV from ``input_layernorm``, gate/up
                    from ``post_attention_layernorm``); ``rms_norm_linear``
                    applies ``rsqrt(mean(x^2) + eps)`` per row.
  int8 weight-only  codes ``q [N, K]`` int8 in [-127, 127] with per-row fp16
                    scales ``s [N]``, ``W ~= q * s[:, None]``
                    (``quantize_int8``), the layout ``w8a16_linear`` reads.
                    The reference's int8 tile shape {8, 8, 32}
                    (include/hexagon/Common/Common.h:24) orders bytes for HVX
                    registers; MFMA fragments load straight from rows, so the
                    codes stay row-major.  The norm weights stay separate
                    (the int8 path runs ``rms_norm`` before its GEMV).

Weight preparation runs on the GPU kernels (``fold_rms_weight``,
``quantize_int8``); the concatenations and the gate/up interleave are copies.
"""
from __future__ import annotations

import json
import os
from dataclasses import asdict, dataclass, field
from typing import Mapping, Optional

import torch

from . import hxmi

FORMAT = "hxmi-packed"
VERSION = 1


@dataclass
class DecoderConfig:
    """The checkpoint facts the packed layouts depend on (Hugging Face
    ``config.json`` names in the comments)."""
    hidden: int                    # hidden_size
    intermediate: int              # intermediate_size
    layers: int                    # num_hidden_layers
    heads: int                     # num_attention_heads
    kv_heads: int                  # num_key_value_heads
    head_dim: int                  # head_dim (hidden / heads when absent)
    eps: float = 1e-5              # rms_norm_eps
    tie_word_embeddings: bool = False
    model_type: str = "llama"

    @classmethod
    def from_hf(cls, cfg: Mapping) -> "DecoderConfig":
        heads = int(cfg["num_attention_heads"])
        return cls(
            hidden=int(cfg["hidden_size"]),
            intermediate=int(cfg["intermediate_size"]),
            layers=int(cfg["num_hidden_layers"]),
            heads=heads,
            kv_heads=int(cfg.get("num_key_value_heads") or heads),
            head_dim=int(cfg.get("head_dim") or int(cfg["hidden_size"]) // heads),
            eps=float(cfg.get("rms_norm_eps", 1e-5)),
            tie_word_embeddings=bool(cfg.get("tie_word_embeddings", False)),
            model_type=str(cfg.get("model_type", "llama")),
        )

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


@dataclass
class Linear:
    """One projection in the layout its kernel reads: fp16 ``weight [N, K]``
    (``scale`` None), or int8 codes ``weight`` with fp16 ``scale [N]``."""
    weight: torch.Tensor
    scale: Optional[torch.Tensor] = None
    bias: Optional[torch.Tensor] = None

    @property
    def is_int8(self) -> bool:
        return self.scale is not None

    @property
    def shape(self) -> tuple[int, int]:
        return tuple(self.weight.shape)


@dataclass
class PackedLayer:
    qkv: Linear
    o: Linear
    gate_up: Linear
    down: Linear
    input_norm: torch.Tensor
    post_norm: torch.Tensor


@dataclass
class PackedModel:
    config: DecoderConfig
    layers: list[PackedLayer]
    norm: Optional[torch.Tensor] = None
    lm_head: Optional[Linear] = None
    folded_norm: bool = True
    int8: bool = False
    extra: dict = field(default_factory=dict)


# ---- reading Hugging Face checkpoints -----------------------------------------------

def read_checkpoint(path: str | os.PathLike) -> tuple[dict[str, torch.Tensor], Optional[DecoderConfig]]:
    """Tensors of a safetensors checkpoint (one file, or a directory with
    ``model.safetensors`` or a sharded ``model.safetensors.index.json``) on
    the CPU, and its ``config.json`` when the directory has one.  Only
    safetensors is read: nothing in the files is executed."""
    from safetensors.torch import load_file

    path = os.fspath(path)
    cfg = None
    if os.path.isdir(path):
        cj = os.path.join(path, "config.json")
        if os.path.exists(cj):
            with open(cj) as f:
                cfg = DecoderConfig.from_hf(json.load(f))
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                shards = sorted(set(json.load(f)["weight_map"].values()))
            files = [os.path.join(path, s) for s in shards]
        else:
            files = [os.path.join(path, "model.safetensors")]
    else:
        files = [path]
    sd: dict[str, torch.Tensor] = {}
    for fn in files:
        sd.update(load_file(fn, device="cpu"))
    return sd, cfg


def infer_config(sd: Mapping[str, torch.Tensor], heads: int, kv_heads: Optional[int] = None,
                 eps: float = 1e-5) -> DecoderConfig:
    """A DecoderConfig from tensor shapes, for checkpoints without a
    config.json (head counts cannot be read from the shapes)."""
    kv_heads = kv_heads or heads
    q = sd["model.layers.0.self_attn.q_proj.weight"]
    layers = 1 + max(int(k.split(".")[2]) for k in sd if k.startswith("model.layers."))
    return DecoderConfig(hidden=q.shape[1], intermediate=sd["model.layers.0.mlp.gate_proj.weight"].shape[0],
                         layers=layers, heads=heads, kv_heads=kv_heads, head_dim=q.shape[0] // heads, eps=eps,
                         tie_word_embeddings="lm_head.weight" not in sd)


# ---- packing -------------------------------------------------------------------------

def _half(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.float16).contiguous()


def _linear(w: torch.Tensor, bias: Optional[torch.Tensor], int8: bool) -> Linear:
    if int8:
        q, s = hxmi.quantize_int8(w)
        return Linear(q, s, bias)
    return Linear(w, None, bias)


def pack_decoder_layer(sd: Mapping[str, torch.Tensor], index: int, config: DecoderConfig,
                       device: torch.device, fold_norm: bool = True, int8: bool = False) -> PackedLayer:
    """Layer ``index`` of a LLaMA / Qwen2 checkpoint (``model.layers.<i>.*``)
    in the kernels' layouts.  ``fold_norm`` folds the two RMSNorm weights into
    QKV and gate/up (fp16 only); ``int8`` quantises every projection."""
    if fold_norm and int8:
        raise ValueError("the int8 path keeps the norms separate: fold_norm must be False with int8")
    p = f"model.layers.{index}."

    def get(name: str) -> torch.Tensor:
        key = p + name
        if key not in sd:
            raise KeyError(f"checkpoint has no tensor {key!r}")
        return _half(sd[key], device)

    c = config
    wq, wk, wv = get("self_attn.q_proj.weight"), get("self_attn.k_proj.weight"), get("self_attn.v_proj.weight")
    if wq.shape != (c.heads * c.head_dim, c.hidden) or wk.shape != (c.kv_heads * c.head_dim, c.hidden) \
            or wv.shape != wk.shape:
        raise ValueError(f"layer {index}: q/k/v shapes {tuple(wq.shape)}, {tuple(wk.shape)}, {tuple(wv.shape)} "
                         f"do not match the config")
    has_bias = [(p + f"self_attn.{n}_proj.bias") in sd for n in "qkv"]
    if any(has_bias) and not all(has_bias):
        raise ValueError(f"layer {index}: q/k/v biases must be all present or all absent")
    bqkv = torch.cat([get(f"self_attn.{n}_proj.bias") for n in "qkv"]) if all(has_bias) else None
    g1, g2 = get("input_layernorm.weight"), get("post_attention_layernorm.weight")
    qkv = torch.cat([wq, wk, wv], dim=0)
    gate_up = hxmi.pack_gate_up(get("mlp.gate_proj.weight"), get("mlp.up_proj.weight"))
    if fold_norm:
        qkv = hxmi.fold_rms_weight(qkv, g1)
        gate_up = hxmi.fold_rms_weight(gate_up, g2)
    return PackedLayer(
        qkv=_linear(qkv, bqkv, int8),
        o=_linear(get("self_attn.o_proj.weight"), None, int8),
        gate_up=_linear(gate_up, None, int8),
        down=_linear(get("mlp.down_proj.weight"), None, int8),
        input_norm=g1,
        post_norm=g2,
    )


def pack_model(sd: Mapping[str, torch.Tensor], config: DecoderConfig, device: torch.device,
               fold_norm: bool = True, int8: bool = False, layers: Optional[list[int]] = None,
               lm_head: bool = True) -> PackedModel:
    """Every decoder layer (or the listed ones), the final norm and the
    lm_head (the embedding matrix when the checkpoint ties them)."""
    idx = list(range(config.layers)) if layers is None else list(layers)
    packed = [pack_decoder_layer(sd, i, config, device, fold_norm, int8) for i in idx]
    norm = _half(sd["model.norm.weight"], device) if "model.norm.weight" in sd else None
    head = None
    if lm_head:
        key = "model.embed_tokens.weight" if config.tie_word_embeddings else "lm_head.weight"
        if key not in sd:
            raise KeyError(f"checkpoint has no tensor {key!r} for the lm_head")
        head = _linear(_half(sd[key], device), None, int8)
    return PackedModel(config, packed, norm, head, folded_norm=fold_norm, int8=int8,
                       extra={"layer_index": idx})


# ---- the packed file -----------------------------------------------------------------

def _flatten(model: PackedModel) -> dict[str, torch.Tensor]:
    out: dict[str, torch.Tensor] = {}

    def put_linear(name: str, lin: Optional[Linear]) -> None:
        if lin is None:
            return
        out[name + ".weight"] = lin.weight
        if lin.scale is not None:
            out[name + ".scale"] = lin.scale
        if lin.bias is not None:
            out[name + ".bias"] = lin.bias

    for i, layer in enumerate(model.layers):
        for n in ("qkv", "o", "gate_up", "down"):
            put_linear(f"layers.{i}.{n}", getattr(layer, n))
        out[f"layers.{i}.input_norm"] = layer.input_norm
        out[f"layers.{i}.post_norm"] = layer.post_norm
    if model.norm is not None:
        out["norm"] = model.norm
    put_linear("lm_head", model.lm_head)
    return {k: v.detach().to("cpu").contiguous() for k, v in out.items()}


def save_packed(path: str | os.PathLike, model: PackedModel) -> None:
    """Write the packed tensors and their layout description to one
    safetensors file."""
    from safetensors.torch import save_file

    meta = {
        "format": FORMAT,
        "version": str(VERSION),
        "config": json.dumps(asdict(model.config)),
        "folded_norm": "1" if model.folded_norm else "0",
        "int8": "1" if model.int8 else "0",
        "gate_up": "interleaved-16-rows",
        "layer_index": json.dumps(model.extra.get("layer_index", list(range(len(model.layers))))),
    }
    save_file(_flatten(model), os.fspath(path), metadata=meta)


def load_packed(path: str | os.PathLike, device: torch.device) -> PackedModel:
    """Read a file written by save_packed straight to ``device``."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    path = os.fspath(path)
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path} is not a {FORMAT} file")
    if int(meta.get("version", "0")) != VERSION:
        raise ValueError(f"{path}: packed format version {meta.get('version')} (this library reads {VERSION})")
    t = load_file(path, device=str(device))
    cfg = DecoderConfig(**json.loads(meta["config"]))
    idx = json.loads(meta["layer_index"])

    def lin(name: str) -> Optional[Linear]:
        if name + ".weight" not in t:
            return None
        return Linear(t[name + ".weight"], t.get(name + ".scale"), t.get(name + ".bias"))

    layers = [PackedLayer(qkv=lin(f"layers.{i}.qkv"), o=lin(f"layers.{i}.o"), gate_up=lin(f"layers.{i}.gate_up"),
                          down=lin(f"layers.{i}.down"), input_norm=t[f"layers.{i}.input_norm"],
                          post_norm=t[f"layers.{i}.post_norm"]) for i in range(len(idx))]
    return PackedModel(cfg, layers, t.get("norm"), lin("lm_head"), folded_norm=meta["folded_norm"] == "1",
                       int8=meta["int8"] == "1", extra={"layer_index": idx})
