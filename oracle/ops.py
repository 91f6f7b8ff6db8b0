"""CPU restatement of the reference's per-operator arithmetic (test infrastructure only).

Every function cites the reference lines it follows. Floating-point work is eager torch on the CPU
in fp32 with the reference's casts: each product and sum is its own rounded op (no FMA), which is
also what the gfx950 kernels do, so the only differences left are reduction orders.
"""

from __future__ import annotations

import math

import numpy as np
import torch

# NF4 levels in code order, as in solution/kernels.py:76-83 (the QLoRA NF4 table, README.md:53).
NF4_LEVELS = np.array(
    [
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
    ],
    dtype=np.float32,
)

PRESCALE_GRAD = 65536.0  # solution/ops.py:171


def _up(x: torch.Tensor) -> torch.Tensor:
    """fp32 compute type (float64 inputs stay float64, for the float64 invariant checks)."""
    return x if x.dtype == torch.float64 else x.float()


# ---------------------------------------------------------------------------------------------
# NF4 double-quant dequant — solution/kernels.py:27-118 and launcher kernels.py:572-619
# ---------------------------------------------------------------------------------------------


def nf4_dequant(
    packed: np.ndarray,
    absmax: np.ndarray,
    code2: np.ndarray,
    absmax2: np.ndarray,
    offset,
    out_shape: tuple[int, int],
    split_bytes: tuple[int, int] | None = None,
    blocksize: int = 64,
    super_blocksize: int = 256,
    absmax2_bases: tuple[int, int] | None = None,
) -> np.ndarray:
    """fp16 weights from packed NF4 codes.

    byte b holds elements 2b (high nibble, kernels.py:66-68) and 2b+1 (low nibble); segment s of
    byte b is (b >= split1) + (b >= split2) (kernels.py:59-63); scale = fp32(fp32(code2[absmax[blk]]
    * absmax2[sup]) + off_s) with two roundings (kernels.py:64 without contraction, as
    bitsandbytes' dequantize_blockwise followed by ``absmax += offset``); value =
    fp16_rne(fp32(NF4[nib] * scale)) (kernels.py:90, 115). sup is the super-block index relative
    to the segment's first block plus the segment's absmax2 base; with the default bases this is
    the reference's global ``block // super_blocksize`` (kernels.py:53-57) whenever each segment
    holds a multiple of super_blocksize blocks.

    Pinned by: hand-computed known answers, a float64 brute force, segment-vs-separate equality
    and the quantise->dequantise error bound (tests/test_oracle.py).
    """
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.asarray(absmax, dtype=np.uint8).reshape(-1)
    code2 = np.asarray(code2, dtype=np.float32).reshape(-1)
    absmax2 = np.asarray(absmax2, dtype=np.float32).reshape(-1)
    n = int(out_shape[0]) * int(out_shape[1])
    nb = n // 2
    hb = blocksize // 2
    if isinstance(offset, (tuple, list)):
        offs = np.array([offset[0], offset[1], offset[2]], dtype=np.float32)
    else:
        offs = np.full(3, offset, dtype=np.float32)
    s1, s2 = (nb, nb) if split_bytes is None else (int(split_bytes[0]), int(split_bytes[1]))
    if absmax2_bases is None:
        n0 = -(-(s1 // hb) // super_blocksize) if s1 > 0 else 0
        n1 = -(-((s2 - s1) // hb) // super_blocksize) if s2 > s1 else 0
        absmax2_bases = (n0, n0 + n1)
    bases = np.array([0, absmax2_bases[0], absmax2_bases[1]], dtype=np.int64)
    first_blk = np.array([0, s1 // hb, s2 // hb], dtype=np.int64)

    b = np.arange(nb, dtype=np.int64)
    seg = (b >= s1).astype(np.int64) + (b >= s2).astype(np.int64)
    blk = b // hb
    sup = bases[seg] + (blk - first_blk[seg]) // super_blocksize
    scale = code2[absmax[blk]] * absmax2[sup]  # float32 * float32 -> float32
    scale = (scale + offs[seg]).astype(np.float32)
    byte = packed[:nb]
    out = np.empty(n, dtype=np.float32)
    out[0::2] = NF4_LEVELS[byte >> 4] * scale
    out[1::2] = NF4_LEVELS[byte & 15] * scale
    return out.astype(np.float16).reshape(out_shape)


def nf4_gemm(x: torch.Tensor, w16: np.ndarray, trans: bool = False,
             bias: torch.Tensor | None = None) -> torch.Tensor:
    """The product the fused NF4 GEMM computes, on the dequantised fp16 weight w16 [rows, cols]
    (``nf4_dequant``): trans=False -> fp16(x @ w16^T + bias) (F.linear, solution/ops.py:771, 810,
    710-724), trans=True -> fp16(x @ w16) (torch.mm, solution/ops.py:934, 939, 949, 993). The sum
    is taken in float64 (the exact value that an fp32-accumulating GEMM approximates) and rounded
    once to fp16. Pinned by numpy's float64 matmul (a library routine) on exactly representable
    inputs and by the dequant pins above."""
    xd = np.asarray(x.float().numpy(), dtype=np.float64)
    wd = np.asarray(w16, dtype=np.float64)
    y = xd @ (wd if trans else wd.T)
    if bias is not None:
        y = y + np.asarray(bias.float().numpy(), dtype=np.float64)[None, :]
    return torch.from_numpy(y.astype(np.float16))  # one rounding, float64 -> fp16


# ---------------------------------------------------------------------------------------------
# Residual + RMSNorm — solution/kernels.py:125-199, wrapper ops.py:30-54
# ---------------------------------------------------------------------------------------------


def rms_norm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, residual: torch.Tensor | None = None):
    """(y, h, rstd): h = T(x + res) (kernels.py:149), rstd = 1/sqrt(mean(h^2) + eps) in fp32
    (kernels.py:154-156), y = T(fp32(T(h*rstd)) * fp32(w)) (kernels.py:161-162; Qwen2RMSNorm's
    cast order). Pinned against transformers' Qwen2RMSNorm."""
    dt = x.dtype
    h = (_up(x) + _up(residual)).to(dt) if residual is not None else x
    hf = _up(h)
    var = (hf * hf).sum(-1, keepdim=True) / hf.shape[-1]
    rstd = 1.0 / torch.sqrt(var + eps)
    y = ((hf * rstd).to(dt).to(hf.dtype) * _up(w)).to(dt)
    return y, h, rstd.squeeze(-1)


def rms_norm_bwd(dy: torch.Tensor, h: torch.Tensor, w: torch.Tensor, rstd: torch.Tensor,
                 dresidual: torch.Tensor | None = None) -> torch.Tensor:
    """dx = T((w*dy - xhat*mean(xhat*w*dy)) * rstd + dres), xhat = h*rstd (kernels.py:190-197).
    Pinned against torch autograd of the forward formula in float64."""
    xh = _up(h) * _up(rstd).unsqueeze(-1)
    g = _up(w) * _up(dy)
    c = (xh * g).sum(-1, keepdim=True) / h.shape[-1]
    dx = (g - xh * c) * _up(rstd).unsqueeze(-1)
    if dresidual is not None:
        dx = dx + _up(dresidual)
    return dx.to(h.dtype)


# ---------------------------------------------------------------------------------------------
# LoRA delta + NeoX RoPE — solution/kernels.py:206-348, wrapper ops.py:88-164
# ---------------------------------------------------------------------------------------------


def rope_tables(max_pos: int, head_dim: int, theta: float, dtype=torch.float16):
    """cos/sin [max_pos, head_dim] as Qwen2RotaryEmbedding builds them (default rope type): inv
    = 1/theta^(2i/d) in fp32, freqs = pos*inv, emb = [freqs, freqs], cast to ``dtype``
    (the engine takes its cache from the model's rotary module, ops.py:655-666). Pinned against
    transformers' Qwen2RotaryEmbedding."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    pos = torch.arange(max_pos, dtype=torch.float32)
    freqs = pos[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _rot(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    lo, hi = x[..., :half], x[..., half:]
    out_lo = lo * c[..., :half] - hi * s[..., :half]
    out_hi = hi * c[..., half:] + lo * s[..., half:]
    return torch.cat([out_lo, out_hi], dim=-1)


def _rot_t(dy: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    half = dy.shape[-1] // 2
    lo, hi = dy[..., :half], dy[..., half:]
    dx_lo = lo * c[..., :half] + hi * s[..., half:]
    dx_hi = hi * c[..., half:] - lo * s[..., :half]
    return torch.cat([dx_lo, dx_hi], dim=-1)


def qkv_rope_fwd(qkv, cos, sin, pos_ids, q_lora=None, v_lora=None, scale_q=2.0, scale_v=2.0,
                 h_q=12, h_kv=2, head_dim=128):
    """(q, k, v) [n, h, d]: q = T(R(p)(q + s_q*ql)), k = T(R(p)k), v = T(v + s_v*vl), fp32 math,
    out_lo = a*cos_lo - b*sin_lo, out_hi = b*cos_hi + a*sin_hi (kernels.py:242-283). Pinned against
    transformers' apply_rotary_pos_emb and the reference test formula (test_kernels.py:111-124)."""
    dt = qkv.dtype
    n = qkv.shape[0]
    qd, kd = h_q * head_dim, h_kv * head_dim
    q = _up(qkv[:, :qd])
    k = _up(qkv[:, qd:qd + kd])
    v = _up(qkv[:, qd + kd:qd + 2 * kd])
    if q_lora is not None and v_lora is not None:
        q = q + _up(q_lora) * scale_q
        v = v + _up(v_lora) * scale_v
    c = _up(cos[pos_ids]).unsqueeze(1)
    s = _up(sin[pos_ids]).unsqueeze(1)
    qo = _rot(q.view(n, h_q, head_dim), c, s).to(dt)
    ko = _rot(k.view(n, h_kv, head_dim), c, s).to(dt)
    return qo, ko, v.view(n, h_kv, head_dim).to(dt)


def qkv_rope_bwd(dq, dk, dv, cos, sin, pos_ids, h_q=12, h_kv=2, head_dim=128,
                 scale_q: float | None = None, scale_v: float | None = None):
    """dqkv [n, (h_q+2h_kv)*d] = [R^T dQ | R^T dK | dV] (kernels.py:315-348); with scales also
    (dq_lora, dv_lora) = T(fp32(dQ_T)*s) from the rounded values (ops.py:144-147). Pinned by
    R^T R = I and against autograd of the forward."""
    dt = dq.dtype
    n = dq.shape[0]
    c = _up(cos[pos_ids]).unsqueeze(1)
    s = _up(sin[pos_ids]).unsqueeze(1)
    gq = _rot_t(_up(dq).view(n, h_q, head_dim), c, s).to(dt).view(n, -1)
    gk = _rot_t(_up(dk).view(n, h_kv, head_dim), c, s).to(dt).view(n, -1)
    gv = dv.reshape(n, -1).to(dt)
    dqkv = torch.cat([gq, gk, gv], dim=1)
    if scale_q is None:
        return dqkv
    return dqkv, (_up(gq) * scale_q).to(dt), (_up(gv) * scale_v).to(dt)


# ---------------------------------------------------------------------------------------------
# SwiGLU — solution/kernels.py:355-446, wrapper ops.py:57-85
# ---------------------------------------------------------------------------------------------


def swiglu_fwd(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """T(g*sigmoid(g)*u), sigmoid = 1/(1+exp(-g)) in fp32 (kernels.py:388-391). Pinned against
    F.silu."""
    gf = _up(g)
    sg = 1.0 / (1.0 + torch.exp(-gf))
    return ((gf * sg) * _up(u)).to(g.dtype)


def swiglu_bwd(dout: torch.Tensor, g: torch.Tensor, u: torch.Tensor):
    """(dg, du): du = T(dout*silu), dg = T((dout*u)*(s + silu*(1-s))) (kernels.py:435-439).
    Pinned against autograd of F.silu(g)*u."""
    gf, uf, df = _up(g), _up(u), _up(dout)
    sg = 1.0 / (1.0 + torch.exp(-gf))
    silu = gf * sg
    du = df * silu
    dg = (df * uf) * (sg + silu * (1.0 - sg))
    return dg.to(g.dtype), du.to(g.dtype)


# ---------------------------------------------------------------------------------------------
# LoRA-input dropout — solution/ops.py:775-777 (forward), 882-886 (recompute), 986-992 (backward)
# The reference replays torch's generator state; the build draws each mask from a counter-based
# Philox4x64-10 stream instead (same masks in forward, recompute and backward by construction).
# ---------------------------------------------------------------------------------------------

_PHILOX_M = (0xD2E7470EE14C6C93, 0xCA5A826395121157)
_PHILOX_W = (0x9E3779B97F4A7C15, 0xBB67AE8584CAA73B)
_LO32 = np.uint64(0xFFFFFFFF)


def _mulhilo64(a: int, b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(hi, lo) 64-bit halves of the 128-bit products a * b (uint64 arrays, 32-bit limbs)."""
    a_lo, a_hi = np.uint64(a & 0xFFFFFFFF), np.uint64(a >> 32)
    b_lo, b_hi = b & _LO32, b >> np.uint64(32)
    ll, lh, hl, hh = a_lo * b_lo, a_lo * b_hi, a_hi * b_lo, a_hi * b_hi
    mid = (ll >> np.uint64(32)) + (lh & _LO32) + (hl & _LO32)
    lo = (ll & _LO32) | ((mid & _LO32) << np.uint64(32))
    hi = hh + (lh >> np.uint64(32)) + (hl >> np.uint64(32)) + (mid >> np.uint64(32))
    return hi, lo


def philox4x64_10(counters: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x64 with 10 rounds (Salmon et al., SC'11) over uint64 counters [n, 4] -> [n, 4]."""
    c = [counters[:, i].astype(np.uint64).copy() for i in range(4)]
    k0, k1 = int(key[0]) & (2**64 - 1), int(key[1]) & (2**64 - 1)
    with np.errstate(over="ignore"):
        for _ in range(10):
            hi0, lo0 = _mulhilo64(_PHILOX_M[0], c[0])
            hi1, lo1 = _mulhilo64(_PHILOX_M[1], c[2])
            c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
            k0, k1 = (k0 + _PHILOX_W[0]) % 2**64, (k1 + _PHILOX_W[1]) % 2**64
    return np.stack(c, axis=1)


def dropout_keep_mask(seed: int, stream: int, n_rows: int, n_cols: int, p: float) -> np.ndarray:
    """bool [n_rows, n_cols]: element e = row * n_cols + col is kept when 32-bit word e % 8 of
    Philox4x64-10((e // 8, 0, 0, 0), (seed, stream)) (words w0.lo, w0.hi, ..., w3.hi) is
    >= round(p * 2^32)."""
    n = n_rows * n_cols
    nb = (n + 7) // 8
    ctr = np.zeros((nb, 4), dtype=np.uint64)
    ctr[:, 0] = np.arange(nb, dtype=np.uint64)
    w = philox4x64_10(ctr, (seed, stream))
    words = np.empty((nb, 8), dtype=np.uint64)
    words[:, 0::2] = w & _LO32
    words[:, 1::2] = w >> np.uint64(32)
    thresh = min(int(float(np.float32(p)) * 4294967296.0 + 0.5), 0xFFFFFFFF)
    return (words.reshape(-1)[:n] >= np.uint64(thresh)).reshape(n_rows, n_cols)


def dropout_keep_bits(seed: int, stream: int, n_rows: int, n_cols: int, p: float) -> np.ndarray:
    """The mask of ``dropout_keep_mask`` packed as int32 [n_rows, ceil(n_cols / 32)]: bit i of
    word w of a row is element 32 w + i of that row (0 past its end), the layout the fused LoRA
    kernels read (one launch per step forms every layer's masks in it)."""
    keep = dropout_keep_mask(seed, stream, n_rows, n_cols, p)
    words = (n_cols + 31) // 32
    padded = np.zeros((n_rows, words * 32), dtype=np.uint64)
    padded[:, :n_cols] = keep
    packed = (padded.reshape(n_rows, words, 32) << np.arange(32, dtype=np.uint64)).sum(-1)
    return packed.astype(np.uint32).view(np.int32)


def _drop(x: torch.Tensor, keep: np.ndarray, p: float) -> torch.Tensor:
    scale = torch.tensor(1.0, dtype=torch.float32) / (1.0 - torch.tensor(p, dtype=torch.float32))
    y = torch.where(torch.from_numpy(keep), x.float() * scale, torch.zeros((), dtype=torch.float32))
    return y.to(x.dtype)


def lora_dropout_fwd(x: torch.Tensor, seed: int, stream_a: int, stream_b: int, p_a: float,
                     p_b: float):
    """(dropout_a(x), dropout_b(x)) with x [rows, cols]: T(x * fp32(1 / (1 - p))) where kept."""
    r, c = x.shape
    return (_drop(x, dropout_keep_mask(seed, stream_a, r, c, p_a), p_a),
            _drop(x, dropout_keep_mask(seed, stream_b, r, c, p_b), p_b))


def lora_dropout_bwd_add(acc: torch.Tensor, ga: torch.Tensor, gb: torch.Tensor, seed: int,
                         stream_a: int, stream_b: int, p_a: float, p_b: float) -> torch.Tensor:
    """T(T(acc + dropout_a(ga)) + dropout_b(gb)): ops.py:988-992 with the forward's masks."""
    r, c = acc.shape
    ta = _drop(ga, dropout_keep_mask(seed, stream_a, r, c, p_a), p_a)
    tb = _drop(gb, dropout_keep_mask(seed, stream_b, r, c, p_b), p_b)
    return (acc.float() + ta.float()).to(acc.dtype).float().add(tb.float()).to(acc.dtype)


# ---------------------------------------------------------------------------------------------
# Rank-r LoRA branches — solution/ops.py:775-778 (forward), 975-992 (backward). Each product is
# an fp16 tensor computed with fp32 accumulation, as torch's fp16 F.linear / torch.mm.
# ---------------------------------------------------------------------------------------------


def _mm16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return (a.float() @ b.float()).half()


def lora_down_fwd(x, a_q, a_v, seed=None, stream_q=0, stream_v=1, p_q=0.0, p_v=0.0):
    """(mid_q, mid_v, x_q, x_v): x_q = drop_q(x), mid_q = fp16(x_q A_q^T) (ops.py:775-778)."""
    if seed is None:
        x_q = x_v = x
    else:
        x_q, x_v = lora_dropout_fwd(x, seed, stream_q, stream_v, p_q, p_v)
    return _mm16(x_q, a_q.t()), _mm16(x_v, a_v.t()), x_q, x_v


def lora_up(mid, b):
    """fp16(mid B^T): the LoRA delta the RoPE kernel adds (ops.py:776, 778)."""
    return _mm16(mid, b.t())


def lora_bwd_x(dq, dv, a_q, a_v, b_q, b_v, dx, seed=None, stream_q=0, stream_v=1, p_q=0.0,
               p_v=0.0):
    """(d_mid_q, d_mid_v, dx_new): d_mid = fp16(dq B), dx_branch = fp16(d_mid A), then the masked
    adds of ops.py:986-992."""
    dmq, dmv = _mm16(dq, b_q), _mm16(dv, b_v)
    dxq, dxv = _mm16(dmq, a_q), _mm16(dmv, a_v)
    if seed is None:
        out = (dx.float() + dxq.float()).half().float().add(dxv.float()).half()
    else:
        out = lora_dropout_bwd_add(dx, dxq, dxv, seed, stream_q, stream_v, p_q, p_v)
    return dmq, dmv, out


def lora_bwd_w(x_q, x_v, dq, dv, mid_q, mid_v, d_mid_q, d_mid_v):
    """(g_a_q, g_b_q, g_a_v, g_b_v) = (d_mid_q^T x_q, dq^T mid_q, ...) in fp16 (ops.py:975-981)."""
    return (_mm16(d_mid_q.t(), x_q), _mm16(dq.t(), mid_q), _mm16(d_mid_v.t(), x_v),
            _mm16(dv.t(), mid_v))


# ---------------------------------------------------------------------------------------------
# Chunked lm_head cross-entropy — solution/kernels.py:453-565, ops.py:174-349
# ---------------------------------------------------------------------------------------------


def lm_head_logits(h16: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """z16 = fp16(H·W^T) with fp32 accumulation (the fp16 torch.mm of ops.py:231), as fp32."""
    return (h16.float() @ w16.float().t()).to(torch.float16).float()


def lm_head_ce(h16: torch.Tensor, w16: torch.Tensor, labels: torch.Tensor,
               num_items_in_batch: float | None = None, v_chunk: int = 8192,
               need_grad: bool = True, grad_loss: float = 1.0) -> dict:
    """Per-token statistics and the hidden-state gradient of the vocab-chunked lm_head CE.

    Over fp16-rounded logits z: m = max z, s = sum e^{z-m}, w = sum e^{z-m} z; lse = m + ln s,
    entropy = lse - w/s, nll = lse - z[y] (0 for y = -100), argmax = first index of max
    (kernels.py:480-565); loss = sum(nll)/denom with denom = num_items_in_batch or #valid, >= 1
    (ops.py:268-277). Gradient: G = fp16((e^{z-lse} - 1[v=y]) * 2^16/denom), 0 on masked rows
    (kernels.py:517-531); dH = fp16((sum_v G W) * grad_loss/2^16) with the sum accumulated in fp32
    (the reference accumulates in fp16 across chunks, ops.py:283, 320, 337-338).
    Pinned against F.cross_entropy / logsumexp / softmax entropy / argmax and autograd on the
    full logits.
    """
    n, d = h16.shape
    V = w16.shape[0]
    labels = labels.reshape(-1).long()
    hf = h16.float()
    m = torch.full((n,), -float("inf"))
    s = torch.zeros(n)
    wsum = torch.zeros(n)
    best = torch.full((n,), -float("inf"))
    best_idx = torch.zeros(n, dtype=torch.long)
    target = torch.zeros(n)
    for start in range(0, V, v_chunk):
        end = min(start + v_chunk, V)
        z = (hf @ w16[start:end].float().t()).to(torch.float16).float()
        cmax, carg = z.max(dim=1)
        upd = cmax > best
        best_idx = torch.where(upd, carg + start, best_idx)
        best = torch.where(upd, cmax, best)
        m_new = torch.maximum(m, cmax)
        alpha = torch.exp(m - m_new)
        e = torch.exp(z - m_new[:, None])
        s = s * alpha + e.sum(1)
        wsum = wsum * alpha + (e * z).sum(1)
        m = m_new
        inr = (labels >= start) & (labels < end)
        if inr.any():
            idx = torch.nonzero(inr).squeeze(1)
            target[idx] = z[idx, labels[idx] - start]
    lse = m + torch.log(s)
    entropy = lse - wsum / s
    valid = labels != -100
    nll = torch.where(valid, lse - target, torch.zeros_like(lse))
    denom = float(num_items_in_batch) if num_items_in_batch is not None else float(valid.sum())
    denom = max(denom, 1.0)
    out = {"loss": nll.sum() / denom, "nll": nll, "lse": lse, "entropy": entropy,
           "argmax": best_idx, "denom": denom}
    if need_grad:
        scale = torch.where(valid, torch.full((n,), PRESCALE_GRAD / denom), torch.zeros(n))
        dh = torch.zeros(n, d)
        for start in range(0, V, v_chunk):
            end = min(start + v_chunk, V)
            wf = w16[start:end].float()
            z = (hf @ wf.t()).to(torch.float16).float()
            p = torch.exp(z - lse[:, None])
            onehot = torch.zeros_like(p)
            inr = (labels >= start) & (labels < end)
            if inr.any():
                idx = torch.nonzero(inr).squeeze(1)
                onehot[idx, labels[idx] - start] = 1.0
            g16 = ((p - onehot) * scale[:, None]).to(torch.float16).float()
            dh += g16 @ wf
        out["dh"] = (dh * (grad_loss / PRESCALE_GRAD)).to(torch.float16)
    return out


def softmax_stats_reference(z: torch.Tensor, labels: torch.Tensor) -> dict:
    """Library-routine statistics of full fp32 logits (the pin for ``lm_head_ce``)."""
    labels = labels.reshape(-1).long()
    lse = torch.logsumexp(z, dim=-1)
    p = torch.softmax(z, dim=-1)
    ent = lse - (p * z).sum(-1)
    nll = torch.nn.functional.cross_entropy(z, labels.clamp(min=0), reduction="none")
    nll = torch.where(labels != -100, nll, torch.zeros_like(nll))
    return {"lse": lse, "entropy": ent, "nll": nll, "argmax": z.argmax(-1)}


# ---------------------------------------------------------------------------------------------
# Varlen causal GQA attention — solution/ops.py:669-696 (_run_packed_sdpa) and its autograd
# backward (ops.py:903-928)
# ---------------------------------------------------------------------------------------------


def _rows(cu) -> list[tuple[int, int]]:
    cu = [int(c) for c in cu]
    return [(cu[i], cu[i + 1]) for i in range(len(cu) - 1) if cu[i + 1] > cu[i]]


def attention_varlen_fwd(q, k, v, cu, scale=None):
    """(out [n, h_q, d], lse [h_q, n]) in float64: per row [cu[i], cu[i+1]), causal softmax of
    scale * q k^T (k/v head g = h // (h_q / h_kv), as the expand+reshape of ops.py:690-692) times
    v; lse is the natural-log sum-exp of the scaled scores."""
    n, hq, d = q.shape
    grp = hq // k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    q, k, v = q.double(), k.double(), v.double()
    out = torch.zeros(n, hq, d, dtype=torch.float64)
    lse = torch.zeros(hq, n, dtype=torch.float64)
    for a, e in _rows(cu):
        ks = k[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)  # [h_q, L, d]
        vs = v[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)
        s = scale * (q[a:e].transpose(0, 1) @ ks.transpose(1, 2))  # [h_q, L, L]
        causal = torch.ones(e - a, e - a, dtype=torch.bool).tril()
        s = s.masked_fill(~causal, float("-inf"))
        m = s.amax(-1, keepdim=True)
        p = torch.exp(s - m)
        den = p.sum(-1, keepdim=True)
        out[a:e] = ((p / den) @ vs).transpose(0, 1)
        lse[:, a:e] = (m + torch.log(den)).squeeze(-1)
    return out, lse


def attention_varlen_bwd(dout, q, k, v, cu, scale=None):
    """(dq, dk, dv) in float64 by the softmax adjoint per row and head: P = softmax(S),
    dV = P^T dO, dP = dO V^T, dS = P o (dP - rowsum(dO o O)), dQ = scale dS K, dK = scale dS^T Q;
    dk / dv sum the query heads sharing a KV head (the adjoint of the expand of ops.py:690-692)."""
    n, hq, d = q.shape
    hkv = k.shape[1]
    grp = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    q, k, v, dout = q.double(), k.double(), v.double(), dout.double()
    dq = torch.zeros(n, hq, d, dtype=torch.float64)
    dk = torch.zeros(n, hkv, d, dtype=torch.float64)
    dv = torch.zeros(n, hkv, d, dtype=torch.float64)
    for a, e in _rows(cu):
        L = e - a
        qh = q[a:e].transpose(0, 1)
        ks = k[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)
        vs = v[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)
        do = dout[a:e].transpose(0, 1)
        s = scale * (qh @ ks.transpose(1, 2))
        s = s.masked_fill(~torch.ones(L, L, dtype=torch.bool).tril(), float("-inf"))
        p = torch.softmax(s, dim=-1)
        o = p @ vs
        dvs = p.transpose(1, 2) @ do
        dp = do @ vs.transpose(1, 2)
        ds = p * (dp - (do * o).sum(-1, keepdim=True))
        dq[a:e] = (scale * (ds @ ks)).transpose(0, 1)
        dks = scale * (ds.transpose(1, 2) @ qh)
        dk[a:e] = dks.reshape(hkv, grp, L, d).sum(1).transpose(0, 1)
        dv[a:e] = dvs.reshape(hkv, grp, L, d).sum(1).transpose(0, 1)
    return dq, dk, dv


def fp16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 numbers at |x| (subnormal spacing below 2^-14)."""
    a = x.abs().float().clamp(min=2.0**-14)
    e = torch.floor(torch.log2(a))
    return torch.pow(2.0, e - 10)


__all__ = [name for name in dir() if not name.startswith("_") and name not in ("math", "np", "torch")]
