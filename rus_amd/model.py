"""A random-init QLoRA Qwen2 in the layout the fused engine consumes (no checkpoint, no network).

The reference builds its engine from a transformers ``Qwen2ForCausalLM`` whose linear layers are
bitsandbytes ``Linear4bit`` wrapped by PEFT LoRA (solution/ops.py:606-656, hostload.py:65-96).
Neither bitsandbytes nor PEFT is part of this build, so this module provides the same pieces as
plain tensors:

* per layer, seven NF4 double-quantised projections (q, k, v, o, gate, up, down; blocksize 64,
  absmax super-blocks of 256), q/k/v biases, two RMSNorm weights (fp32, as after
  ``prepare_model_for_kbit_training``) and LoRA A/B for q_proj and v_proj (fp32 trainable);
* a tied fp16 embedding / lm_head and the final norm.

Weights are drawn N(0, 0.02) (transformers' default ``initializer_range``); LoRA A and B are both
N(0, 0.02) as in the BASELINE configuration (PEFT would start B at zero).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .quant import NF4Weight, quantize_nf4


@dataclass
class Qwen2Config:
    hidden_size: int = 1536
    intermediate_size: int = 8960
    num_hidden_layers: int = 28
    num_attention_heads: int = 12
    num_key_value_heads: int = 2
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 2048
    lora_r: int = 16
    lora_alpha: float = 32.0
    lora_dropout: float = 0.05

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def lora_scaling(self) -> float:
        return self.lora_alpha / self.lora_r


def qwen2_1p5b() -> Qwen2Config:
    """Qwen2.5-1.5B-Instruct shapes."""
    return Qwen2Config()


@dataclass
class LayerWeights:
    q: NF4Weight
    k: NF4Weight
    v: NF4Weight
    o: NF4Weight
    gate: NF4Weight
    up: NF4Weight
    down: NF4Weight
    q_bias: torch.Tensor
    k_bias: torch.Tensor
    v_bias: torch.Tensor
    ln1: torch.Tensor
    ln2: torch.Tensor
    q_A: torch.nn.Parameter
    q_B: torch.nn.Parameter
    v_A: torch.nn.Parameter
    v_B: torch.nn.Parameter


@dataclass
class QLoRAQwen2:
    config: Qwen2Config
    layers: list[LayerWeights]
    embed: torch.Tensor  # fp16 [V, D], tied lm_head
    final_norm: torch.Tensor  # fp32 [D]
    meta: dict = field(default_factory=dict)

    def lora_parameters(self) -> list[torch.nn.Parameter]:
        """[q_A, q_B, v_A, v_B] per layer, in layer order (the order FusedQwen2StackFn expects)."""
        out = []
        for L in self.layers:
            out += [L.q_A, L.q_B, L.v_A, L.v_B]
        return out


def build_random_qlora_qwen2(cfg: Qwen2Config, device="cpu", seed: int = 0,
                             std: float = 0.02, norm_jitter: float = 0.05) -> QLoRAQwen2:
    """Random-init model; base weights are quantised on ``device`` and returned there."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    D, I, H, KV, hd = (cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads,
                       cfg.num_key_value_heads, cfg.head_dim)
    dev = torch.device(device)

    def w(rows, cols):
        return (torch.randn(rows, cols, generator=g) * std).to(device=dev, dtype=torch.float16)

    def vec(n, base=0.0, scale=std, dtype=torch.float16):
        return (base + torch.randn(n, generator=g) * scale).to(device=dev, dtype=dtype)

    layers = []
    for _ in range(cfg.num_hidden_layers):
        layers.append(LayerWeights(
            q=quantize_nf4(w(H * hd, D)), k=quantize_nf4(w(KV * hd, D)),
            v=quantize_nf4(w(KV * hd, D)), o=quantize_nf4(w(D, H * hd)),
            gate=quantize_nf4(w(I, D)), up=quantize_nf4(w(I, D)), down=quantize_nf4(w(D, I)),
            q_bias=vec(H * hd), k_bias=vec(KV * hd), v_bias=vec(KV * hd),
            ln1=vec(D, 1.0, norm_jitter, torch.float32), ln2=vec(D, 1.0, norm_jitter, torch.float32),
            q_A=torch.nn.Parameter(vec(cfg.lora_r * D, 0.0, std, torch.float32).view(cfg.lora_r, D)),
            q_B=torch.nn.Parameter(vec(H * hd * cfg.lora_r, 0.0, std, torch.float32).view(H * hd, cfg.lora_r)),
            v_A=torch.nn.Parameter(vec(cfg.lora_r * D, 0.0, std, torch.float32).view(cfg.lora_r, D)),
            v_B=torch.nn.Parameter(vec(KV * hd * cfg.lora_r, 0.0, std, torch.float32).view(KV * hd, cfg.lora_r)),
        ))
    embed = w(cfg.vocab_size, D)
    final = vec(D, 1.0, norm_jitter, torch.float32)
    return QLoRAQwen2(cfg, layers, embed, final, {"seed": seed, "std": std})


def lengths_lognormal(n_rows: int, median: float = 140.0, mean: float = 220.0, lo: int = 16,
                      hi: int = 512, seed: int = 0) -> list[int]:
    """Row lengths ~ lognormal(median, mean) clipped to [lo, hi] (BASELINE configs 3 and 5):
    mu = ln(median), sigma = sqrt(2 ln(mean / median))."""
    g = torch.Generator().manual_seed(seed)
    mu, sigma = math.log(median), math.sqrt(2 * math.log(mean / median))
    x = torch.exp(mu + sigma * torch.randn(n_rows, generator=g))
    return [int(v) for v in x.round().clamp(lo, hi).tolist()]
