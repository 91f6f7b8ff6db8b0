"""Test helper: the attribute layout of a transformers Qwen2ForCausalLM with PEFT LoRA on q_proj /
v_proj over bitsandbytes 4-bit layers, built from a ``rus_amd.model.QLoRAQwen2`` with plain
namespaces (neither PEFT nor bitsandbytes is installed). The paths follow what the reference reads
(solution/hostload.py:65-96, solution/ops.py:629-652, 1041-1061)."""

from __future__ import annotations

from types import SimpleNamespace

import torch


def duck_causal_lm(m, dropout_p: float = 0.05, training: bool = True):
    cfg = m.config

    def lin(w, bias=None, lora=None):
        qs = SimpleNamespace(absmax=w.absmax, offset=torch.tensor(w.offset), shape=w.shape,
                             blocksize=w.blocksize,
                             state2=SimpleNamespace(absmax=w.absmax2, code=w.code2,
                                                    blocksize=w.super_blocksize))
        weight = SimpleNamespace(data=w.packed.view(-1, 1), quant_state=qs)
        mod = SimpleNamespace(base_layer=SimpleNamespace(weight=weight, bias=bias))
        if lora is not None:
            A, B = lora
            mod.lora_A = {"default": SimpleNamespace(weight=A)}
            mod.lora_B = {"default": SimpleNamespace(weight=B)}
            mod.scaling = {"default": cfg.lora_scaling}
            mod.lora_dropout = {"default": SimpleNamespace(p=dropout_p)}
        return mod

    layers = []
    for L in m.layers:
        attn = SimpleNamespace(q_proj=lin(L.q, L.q_bias, (L.q_A, L.q_B)),
                               k_proj=lin(L.k, L.k_bias),
                               v_proj=lin(L.v, L.v_bias, (L.v_A, L.v_B)), o_proj=lin(L.o))
        mlp = SimpleNamespace(gate_proj=lin(L.gate), up_proj=lin(L.up), down_proj=lin(L.down))
        layers.append(SimpleNamespace(self_attn=attn, mlp=mlp,
                                      input_layernorm=SimpleNamespace(weight=L.ln1),
                                      post_attention_layernorm=SimpleNamespace(weight=L.ln2)))
    hf_cfg = SimpleNamespace(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                             num_attention_heads=cfg.num_attention_heads,
                             num_key_value_heads=cfg.num_key_value_heads,
                             vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
                             rope_theta=cfg.rope_theta)
    return SimpleNamespace(config=hf_cfg, training=training, model=SimpleNamespace(
        layers=layers, embed_tokens=SimpleNamespace(weight=m.embed),
        norm=SimpleNamespace(weight=m.final_norm)))
