"""CPU fp32 restatement of the packed QLoRA Qwen2 training step (TEST INFRASTRUCTURE ONLY).

What the reference's fused stack + chunked lm_head compute (solution/ops.py:736-1009 forward and
manual backward, ops.py:174-339, packing ops.py:1103-1127), written as a plain eager fp32
composition whose LoRA gradients come from torch autograd:

    h = embed[ids]
    per layer: x = RMSNorm(h); q = x Wq^T + bq + s_q (x A_q^T) B_q^T; k = x Wk^T + bk;
               v = x Wv^T + bv + s_v (x A_v^T) B_v^T; q, k <- NeoX RoPE(pos);
               h += causal GQA attention per packed row . Wo^T;
               x2 = RMSNorm(h); h += (silu(x2 Wg^T) * (x2 Wu^T)) Wd^T
    loss = sum CE(RMSNorm(h) E^T, shifted labels) / denom

with base weights dequantised by ``oracle.ops.nf4_dequant``. With ``dropout_seed`` the q- and
v-branch LoRA inputs are x * mask / (1 - p) with the counter-based masks of
``oracle.ops.dropout_keep_mask`` (streams 2*layer and 2*layer + 1, p = config.lora_dropout). Pinned against transformers' Qwen2ForCausalLM (eager attention) with the LoRA deltas
merged into the projection weights (tests/test_oracle_stack.py).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import ops as ref


def dequant_fp32(w) -> torch.Tensor:
    """fp16 dequantised NF4 weight (oracle), as float32."""
    out = ref.nf4_dequant(w.packed.cpu().numpy(), w.absmax.cpu().numpy(), w.code2.cpu().numpy(),
                          w.absmax2.cpu().numpy(), w.offset, w.shape, blocksize=w.blocksize,
                          super_blocksize=w.super_blocksize)
    return torch.from_numpy(out).float()


def dequant_model(model) -> list[dict]:
    out = []
    for L in model.layers:
        out.append({n: dequant_fp32(getattr(L, n)) for n in ("q", "k", "v", "o", "gate", "up", "down")})
    return out


def lora_leaves(model) -> list[torch.Tensor]:
    """CPU float32 copies of [q_A, q_B, v_A, v_B] per layer with requires_grad."""
    return [p.detach().float().cpu().clone().requires_grad_(True) for p in model.lora_parameters()]


def _rms(x, w, eps):
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def _rope(x, c, s):
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * c[:, None, :] + rot * s[:, None, :]


def _attention(q, k, v, row_lengths):
    n, hq, d = q.shape
    groups = hq // k.shape[1]
    out = torch.empty(n, hq, d)
    cur = 0
    for L in row_lengths:
        if L <= 0:
            continue
        qs, ks, vs = q[cur:cur + L], k[cur:cur + L], v[cur:cur + L]
        ks = ks.repeat_interleave(groups, dim=1)
        vs = vs.repeat_interleave(groups, dim=1)
        sc = torch.einsum("ihd,jhd->hij", qs, ks) / math.sqrt(d)
        mask = torch.ones(L, L, dtype=torch.bool).tril()
        sc = sc.masked_fill(~mask, float("-inf"))
        out[cur:cur + L] = torch.einsum("hij,jhd->ihd", torch.softmax(sc, dim=-1), vs)
        cur += L
    return out.reshape(n, hq * d)


def _dropped(x, seed, stream, p):
    if seed is None or p <= 0:
        return x
    keep = torch.from_numpy(ref.dropout_keep_mask(seed, stream, x.shape[0], x.shape[1], p))
    scale = torch.tensor(1.0) / (1.0 - torch.tensor(p, dtype=torch.float32))
    return torch.where(keep, x * scale, torch.zeros((), dtype=x.dtype))


def stack_forward(model, deq, lora, ids, pos, row_lengths, rope_dtype=torch.float16,
                  dropout_seed=None):
    """Final-norm hidden states [N, D] (fp32) of the packed batch."""
    cfg = model.config
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    cos, sin = ref.rope_tables(max(int(pos.max()) + 1, 1), hd, cfg.rope_theta, rope_dtype)
    c, s = cos[pos].float(), sin[pos].float()
    eps = cfg.rms_norm_eps
    h = model.embed.cpu().float()[ids]
    n = h.shape[0]
    for li, L in enumerate(model.layers):
        W = deq[li]
        qA, qB, vA, vB = lora[4 * li: 4 * li + 4]
        x = _rms(h, L.ln1.cpu().float(), eps)
        xq = _dropped(x, dropout_seed, 2 * li, cfg.lora_dropout)
        xv = _dropped(x, dropout_seed, 2 * li + 1, cfg.lora_dropout)
        q = x @ W["q"].t() + L.q_bias.cpu().float() + cfg.lora_scaling * ((xq @ qA.t()) @ qB.t())
        k = x @ W["k"].t() + L.k_bias.cpu().float()
        v = x @ W["v"].t() + L.v_bias.cpu().float() + cfg.lora_scaling * ((xv @ vA.t()) @ vB.t())
        q = _rope(q.view(n, hq, hd), c, s)
        k = _rope(k.view(n, hkv, hd), c, s)
        h = h + _attention(q, k, v.view(n, hkv, hd), row_lengths) @ W["o"].t()
        x2 = _rms(h, L.ln2.cpu().float(), eps)
        h = h + (F.silu(x2 @ W["gate"].t()) * (x2 @ W["up"].t())) @ W["down"].t()
    return _rms(h, model.final_norm.cpu().float(), eps)


def step_loss(model, deq, lora, ids, pos, shift_labels, row_lengths, num_items_in_batch=None,
              rope_dtype=torch.float16, dropout_seed=None):
    """Mean cross-entropy over labels != -100 (or sum / num_items_in_batch)."""
    final = stack_forward(model, deq, lora, ids, pos, row_lengths, rope_dtype, dropout_seed)
    logits = final @ model.embed.cpu().float().t()
    nll = F.cross_entropy(logits, shift_labels, ignore_index=-100, reduction="sum")
    denom = float(num_items_in_batch) if num_items_in_batch is not None else float((shift_labels != -100).sum())
    return nll / max(denom, 1.0), final
