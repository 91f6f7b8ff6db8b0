"""Unfused eager training step of the same QLoRA Qwen2 (comparison baseline, not the hot path).

This is what the reference's stack replaces: the transformers + PEFT + bitsandbytes forward under
torch autograd, which stores every activation and materialises the fp16 [N, V] logits and their
fp32 copy (README.md:10-11 of the reference). It uses the same NF4 weights, dequantised per use
like bitsandbytes' ``MatMul4Bit`` (forward and again in backward, only the input saved), fp16
activations, fp32 norm weights and LoRA on q/v with dropout. The dropout masks are the fused
stack's counter-based ones for a given seed (drawn by the dropout kernel on a tensor of ones and
applied with plain torch ops under autograd), so both paths drop the same elements.

Used by bench.py for the peak-memory / throughput comparison and by the GPU tests as a second,
independent GPU reference (the 28-layer step's loss and LoRA gradients).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import kernels as K


def _run_packed_sdpa(q_rot, k_rot, v_out, row_lengths, num_heads, num_kv_heads, head_dim):
    """Causal GQA attention per packed row with K/V expanded per group, as the reference's
    stack does it (solution/ops.py:669-696): torch SDPA, differentiable."""
    n_tokens = q_rot.shape[0]
    out = torch.empty((n_tokens, num_heads * head_dim), dtype=q_rot.dtype, device=q_rot.device)
    groups = num_heads // num_kv_heads
    cur = 0
    for L in row_lengths:
        if L <= 0:
            continue
        nxt = cur + L
        q = q_rot[cur:nxt].transpose(0, 1).unsqueeze(0)
        k = k_rot[cur:nxt].transpose(0, 1).unsqueeze(0)
        v = v_out[cur:nxt].transpose(0, 1).unsqueeze(0)
        if groups > 1:
            k = k.unsqueeze(2).expand(1, num_kv_heads, groups, L, head_dim).reshape(1, num_heads, L, head_dim)
            v = v.unsqueeze(2).expand(1, num_kv_heads, groups, L, head_dim).reshape(1, num_heads, L, head_dim)
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        out[cur:nxt] = o.squeeze(0).transpose(0, 1).reshape(L, num_heads * head_dim)
        cur = nxt
    return out


class _NF4Linear(torch.autograd.Function):
    """y = x W^T (+ b) with W dequantised in forward and re-dequantised in backward."""

    @staticmethod
    def forward(ctx, x, deq, bias):
        w = deq()
        ctx.deq = deq
        ctx.save_for_backward(x)
        return F.linear(x, w, bias)

    @staticmethod
    def backward(ctx, dy):
        w = ctx.deq()
        return dy @ w, None, None


def _deq_fn(ws, layer, seg):
    def f():
        # A private copy: the eager path holds several dequantised weights at once.
        return ws.dequant(layer, seg).clone()
    return f


def _rms(h, w, eps):
    hf = h.float()
    x = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps)).to(h.dtype)
    return (x.float() * w.float()).to(h.dtype)


def _rope(x, cos, sin):
    half = x.shape[-1] // 2
    xf = x.float()
    rot = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
    return (xf * cos[:, None, :].float() + rot * sin[:, None, :].float()).to(x.dtype)


def _dropped(x, seed, layer, meta):
    """(x_q, x_v) with the masks of streams 2*layer, 2*layer + 1, differentiable in x."""
    ones = torch.ones(x.shape, dtype=torch.float32, device=x.device)
    mq, mv = K.lora_dropout_fwd(ones, seed, 2 * layer, 2 * layer + 1, meta["p_q"], meta["p_v"])
    return (x.float() * mq).to(x.dtype), (x.float() * mv).to(x.dtype)


def eager_step_loss(engine, h_packed, pos_ids, shift_labels, row_lengths, training=True,
                    num_items_in_batch=None, seed=None):
    """Loss of the packed batch through plain torch autograd (gradients reach the LoRA params).
    ``seed``: the dropout seed tensor to use (default: the engine's last forward's)."""
    if seed is None:
        seed = engine.last_dropout_seed
    ws = engine.weight_stream
    cos, sin = engine.cos_table[pos_ids], engine.sin_table[pos_ids]
    hq, hkv, hd, eps = engine.num_heads, engine.num_kv_heads, engine.head_dim, engine.rms_eps
    h = h_packed
    n = h.shape[0]
    for l in range(engine.num_layers):
        ws.prefetch(l)
        ws.wait_slot(l)
        meta = engine.layer_lora_meta[l]
        qA, qB, vA, vB = (p.to(h.dtype) for p in engine.lora_params[4 * l: 4 * l + 4])
        x = _rms(h, engine.ln1_weights[l], eps)
        qkv = _NF4Linear.apply(x, _deq_fn(ws, l, "qkv"), engine.layer_biases[l])
        q, k, v = qkv.split([hq * hd, hkv * hd, hkv * hd], dim=-1)
        if training and (meta["p_q"] > 0 or meta["p_v"] > 0):
            xq, xv = _dropped(x, seed, l, meta)
        else:
            xq = xv = x
        q = q + meta["scale_q"] * F.linear(F.linear(xq, qA), qB)
        v = v + meta["scale_v"] * F.linear(F.linear(xv, vA), vB)
        q = _rope(q.reshape(n, hq, hd), cos, sin)
        k = _rope(k.reshape(n, hkv, hd), cos, sin)
        attn = _run_packed_sdpa(q, k, v.reshape(n, hkv, hd), row_lengths, hq, hkv, hd)
        h = h + _NF4Linear.apply(attn, _deq_fn(ws, l, "o"), None)
        x2 = _rms(h, engine.ln2_weights[l], eps)
        gu = _NF4Linear.apply(x2, _deq_fn(ws, l, "gu"), None)
        g, u = gu.chunk(2, dim=-1)
        h = h + _NF4Linear.apply(F.silu(g) * u, _deq_fn(ws, l, "down"), None)
        ws.release_slot(l)
    final = _rms(h, engine.final_norm_weight, eps)
    w = engine.host_head.gpu_weight
    logits = F.linear(final, w)  # fp16 [N, V], as transformers' lm_head
    nll = F.cross_entropy(logits.float(), shift_labels, ignore_index=-100, reduction="sum")
    if num_items_in_batch is None:
        denom = (shift_labels != -100).sum().clamp(min=1).float()
    else:
        denom = torch.tensor(max(float(num_items_in_batch), 1.0), device=h.device)
    return nll / denom


__all__ = ["eager_step_loss"]
