"""Reads a transformers ``Qwen2ForCausalLM`` with PEFT LoRA on q/v and bitsandbytes NF4 base
layers into ``rus_amd.model.QLoRAQwen2`` (what ``Qwen2FusedEngine`` consumes).

Attribute paths follow the reference's extraction (solution/hostload.py:65-96 ``_extract_bnb_nf4``
and solution/ops.py:629-652): ``layer.self_attn.q_proj.base_layer.weight`` holds the packed uint8
codes and a ``quant_state`` with ``absmax`` (uint8), ``offset``, ``shape``, ``blocksize`` and
``state2`` (``absmax`` float32, ``code`` float32[256], ``blocksize``); LoRA lives in
``lora_A["default"]`` / ``lora_B["default"]`` with ``scaling["default"]`` and
``lora_dropout["default"].p``. Objects are duck-typed, so neither library needs to be importable.
"""

from __future__ import annotations

import torch

from .model import LayerWeights, QLoRAQwen2, Qwen2Config
from .quant import NF4Weight


def nf4_from_linear(mod) -> NF4Weight:
    base = getattr(mod, "base_layer", mod)
    w = base.weight
    qs = w.quant_state
    packed = getattr(w, "_cpu_packed", None)
    if packed is None:
        packed = w.data.detach().reshape(-1)
    absmax = getattr(w, "_cpu_absmax", None)
    if absmax is None:
        absmax = qs.absmax.detach().reshape(-1)
    absmax2 = getattr(w, "_cpu_absmax2", None)
    if absmax2 is None:
        absmax2 = qs.state2.absmax.detach().reshape(-1).float()
    code2 = getattr(w, "_cpu_code2", None)
    if code2 is None:
        code2 = qs.state2.code.detach().reshape(-1).float()
    off = qs.offset
    offset = float(off.item()) if isinstance(off, torch.Tensor) else float(off or 0.0)
    return NF4Weight(packed.to(torch.uint8), absmax.to(torch.uint8), code2, absmax2, offset,
                     (int(qs.shape[0]), int(qs.shape[1])), int(qs.blocksize),
                     int(qs.state2.blocksize))


def _bias(mod, dim: int) -> torch.Tensor:
    b = getattr(getattr(mod, "base_layer", mod), "bias", None)
    return torch.zeros(dim, dtype=torch.float16) if b is None else b.detach().to(torch.float16)


def model_from_causal_lm(causal_lm) -> QLoRAQwen2:
    c = causal_lm.config
    q0 = causal_lm.model.layers[0].self_attn.q_proj
    r = int(q0.lora_A["default"].weight.shape[0])
    scale = float(q0.scaling["default"])
    cfg = Qwen2Config(
        hidden_size=int(c.hidden_size), intermediate_size=int(c.intermediate_size),
        num_hidden_layers=len(causal_lm.model.layers),
        num_attention_heads=int(c.num_attention_heads),
        num_key_value_heads=int(c.num_key_value_heads), vocab_size=int(c.vocab_size),
        rms_norm_eps=float(getattr(c, "rms_norm_eps", 1e-6)),
        rope_theta=float(getattr(c, "rope_theta", 1e6)), lora_r=r, lora_alpha=scale * r,
        lora_dropout=float(getattr(q0.lora_dropout["default"], "p", 0.0)))
    layers = []
    meta = []
    for layer in causal_lm.model.layers:
        at, mlp = layer.self_attn, layer.mlp
        layers.append(LayerWeights(
            q=nf4_from_linear(at.q_proj), k=nf4_from_linear(at.k_proj),
            v=nf4_from_linear(at.v_proj), o=nf4_from_linear(at.o_proj),
            gate=nf4_from_linear(mlp.gate_proj), up=nf4_from_linear(mlp.up_proj),
            down=nf4_from_linear(mlp.down_proj),
            q_bias=_bias(at.q_proj, cfg.num_attention_heads * cfg.head_dim),
            k_bias=_bias(at.k_proj, cfg.num_key_value_heads * cfg.head_dim),
            v_bias=_bias(at.v_proj, cfg.num_key_value_heads * cfg.head_dim),
            ln1=layer.input_layernorm.weight.detach(), ln2=layer.post_attention_layernorm.weight.detach(),
            q_A=at.q_proj.lora_A["default"].weight, q_B=at.q_proj.lora_B["default"].weight,
            v_A=at.v_proj.lora_A["default"].weight, v_B=at.v_proj.lora_B["default"].weight))
        meta.append({"scale_q": float(at.q_proj.scaling["default"]),
                     "scale_v": float(at.v_proj.scaling["default"]),
                     "p_q": float(getattr(at.q_proj.lora_dropout["default"], "p", 0.0)),
                     "p_v": float(getattr(at.v_proj.lora_dropout["default"], "p", 0.0))})
    embed = causal_lm.model.embed_tokens.weight.detach().to(torch.float16)
    return QLoRAQwen2(cfg, layers, embed, causal_lm.model.norm.weight.detach(),
                      {"layer_lora_meta": meta})
