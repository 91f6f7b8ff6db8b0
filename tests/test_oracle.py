"""Pins the CPU oracle (oracle/ops.py) before it is trusted as the checker of the gfx950 kernels.

Each oracle function is checked against something that does not restate its formula: literal
known answers, a float64 element-by-element brute force, library routines (transformers'
Qwen2RMSNorm / Qwen2RotaryEmbedding / apply_rotary_pos_emb, F.silu, F.cross_entropy, torch
autograd), or invariants that a plausible mistake (swapped nibbles, FMA-contracted scale, wrong
super-block index, wrong sign in the rotation, transposed adjoint, dropped term) would break.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as ref
from rus_amd import quant

# ---------------------------------------------------------------------------------------------
# NF4 dequant
# ---------------------------------------------------------------------------------------------


def _code2_linear() -> np.ndarray:
    return ((np.arange(256, dtype=np.float32) - 128.0) / 128.0).astype(np.float32)


def test_nf4_known_answers_nibble_order():
    # scale = code2[192] * absmax2[0] + off = 0.5 * 2.0 + 0.5 = 1.5 (exact); values by hand.
    packed = np.array([0x0F, 0xF0, 0x87, 0x3C, 0xE1, 0x00, 0x00, 0x00], dtype=np.uint8)
    out = ref.nf4_dequant(packed, np.array([192], np.uint8), _code2_linear(),
                          np.array([2.0], np.float32), 0.5, (1, 16), blocksize=64)
    bits = out.reshape(-1).view(np.uint16)[:10]
    expect = [0xBE00, 0x3E00,  # 0x0F -> (-1.0, +1.0) * 1.5: high nibble is the EVEN element
              0x3E00, 0xBE00,  # 0xF0
              0x2FA4, 0x0000,  # 0x87 -> (0.0796*1.5, 0)
              0xB8BD, 0x394A,  # 0x3C
              0x3C56, 0xBC2D]  # 0xE1
    assert [int(b) for b in bits] == expect


def test_nf4_scale_has_two_roundings_not_fma():
    # code2 value c, absmax2 a and offset o chosen so that fp32(fp32(c*a)+o) differs from the
    # fused fma(c, a, o) by enough to change the fp16 output of level 1.0 (code 15).
    c = np.array([3209721674], np.uint32).view(np.float32)[0]
    a = np.array([994703209], np.uint32).view(np.float32)[0]
    o = float(np.array([993388834], np.uint32).view(np.float32)[0])
    code2 = np.zeros(256, np.float32)
    code2[7] = c
    packed = np.full(32, 0xF7, np.uint8)  # (1.0, 0.0) pairs
    out = ref.nf4_dequant(packed, np.array([7], np.uint8), code2, np.array([a], np.float32), o,
                          (1, 64))
    assert int(out.reshape(-1).view(np.uint16)[0]) == 3164  # fused FMA would give 3165
    assert int(out.reshape(-1).view(np.uint16)[1]) == 0


def _brute_force(packed, absmax, code2, absmax2, offs, splits, bases, n, blocksize, sbs):
    """Element-by-element float64 evaluation with explicit fp32 rounding steps."""
    hb = blocksize // 2
    out = np.empty(n, np.float16)
    starts = [0, splits[0], splits[1]]
    for e in range(n):
        b = e // 2
        seg = int(b >= splits[0]) + int(b >= splits[1])
        nib = (int(packed[b]) >> 4) if e % 2 == 0 else (int(packed[b]) & 15)
        blk = b // hb
        sup = bases[seg] + (blk - starts[seg] // hb) // sbs
        prod = np.float32(float(code2[absmax[blk]]) * float(absmax2[sup]))
        scale = np.float32(float(prod) + float(np.float32(offs[seg])))
        val = np.float32(float(ref.NF4_LEVELS[nib]) * float(scale))
        out[e] = np.float16(val)
    return out


def test_nf4_matches_float64_brute_force_three_segments():
    rng = np.random.default_rng(5)
    blocksize, sbs = 64, 4  # small super-block so that bases matter
    seg_blocks = [5, 3, 6]  # not multiples of sbs: exercises per-segment super-block bases
    n = sum(seg_blocks) * blocksize
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    absmax = rng.integers(0, 256, n // blocksize, dtype=np.uint8)
    code2 = np.sort(rng.uniform(-1, 1, 256)).astype(np.float32)
    n2 = [-(-b // sbs) for b in seg_blocks]
    absmax2 = rng.uniform(0.01, 0.1, sum(n2)).astype(np.float32)
    offs = (0.013, 0.021, 0.034)
    hb = blocksize // 2
    splits = (seg_blocks[0] * hb, (seg_blocks[0] + seg_blocks[1]) * hb)
    bases = (0, n2[0], n2[0] + n2[1])
    got = ref.nf4_dequant(packed, absmax, code2, absmax2, offs, (1, n), split_bytes=splits,
                          blocksize=blocksize, super_blocksize=sbs)
    want = _brute_force(packed, absmax, code2, absmax2, offs, splits, bases, n, blocksize, sbs)
    assert np.array_equal(got.reshape(-1).view(np.uint16), want.view(np.uint16))


def test_nf4_fused_segments_equal_separate_dequants():
    torch.manual_seed(0)
    parts = [quant.quantize_nf4((torch.randn(r, 128) * 0.02).half()) for r in (96, 32, 32)]
    fused, splits, offs, bases = quant.concat_segments(parts)
    got = ref.nf4_dequant(fused.packed.numpy(), fused.absmax.numpy(), fused.code2.numpy(),
                          fused.absmax2.numpy(), offs, fused.shape, split_bytes=splits,
                          absmax2_bases=bases)
    sep = np.concatenate([ref.nf4_dequant(p.packed.numpy(), p.absmax.numpy(), p.code2.numpy(),
                                          p.absmax2.numpy(), p.offset, p.shape) for p in parts])
    assert np.array_equal(got.view(np.uint16), sep.view(np.uint16))


def test_nf4_roundtrip_error_bound():
    # Quantise -> dequantise: every element lies within half the widest NF4 gap of its block's
    # (double-quantised) absmax, plus the absmax quantisation error.
    torch.manual_seed(1)
    w = (torch.randn(256, 192) * 0.02).half()
    q = quant.quantize_nf4(w)
    deq = ref.nf4_dequant(q.packed.numpy(), q.absmax.numpy(), q.code2.numpy(), q.absmax2.numpy(),
                          q.offset, q.shape).astype(np.float32).reshape(-1, 64)
    wf = w.float().numpy().reshape(-1, 64)
    true_absmax = np.abs(wf).max(axis=1, keepdims=True)
    max_gap = float(np.max(np.diff(ref.NF4_LEVELS)))
    err = np.abs(deq - wf)
    # absmax after double quant differs from the true absmax by at most one 8-bit code step of
    # its super block (relative 1/127 of absmax2 ~ a few % of absmax here).
    assert np.all(err <= true_absmax * (max_gap / 2 + 0.06) + 1e-4)
    assert np.abs(deq - wf).mean() < 0.1 * np.abs(wf).mean() + 1e-4


def test_nf4_all_zero_block_and_tail():
    packed = np.full(40, 0x77, np.uint8)  # code 7 = 0.0 everywhere
    out = ref.nf4_dequant(packed, np.array([200, 3], np.uint8), _code2_linear(),
                          np.array([1.0], np.float32), 0.25, (1, 80))
    assert np.all(out == 0)


# ---------------------------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------------------------


def _hf_rmsnorm(hidden: int, w: torch.Tensor, eps: float):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    m = Qwen2RMSNorm(hidden, eps=eps)
    with torch.no_grad():
        m.weight.copy_(w.float())
    if w.dtype == torch.float16:
        m = m.half()
    return m


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("wdtype", [torch.float16, torch.float32])
def test_rmsnorm_matches_transformers(dtype, wdtype):
    torch.manual_seed(0)
    x = torch.randn(64, 1536).to(dtype)
    res = torch.randn(64, 1536).to(dtype)
    w = (1 + 0.05 * torch.randn(1536)).to(wdtype)
    y, h, rstd = ref.rms_norm_fwd(x, w, 1e-6, residual=res)
    assert torch.equal(h, (x + res) if dtype == torch.float16 else (x + res))
    hf = _hf_rmsnorm(1536, w, 1e-6)
    want = hf(h).to(dtype).float()
    diff = (y.float() - want).abs()
    if dtype == torch.float16:
        assert torch.all(diff <= ref.fp16_ulp(want))  # at most one ulp (mean vs sum/n, rsqrt)
        assert (diff == 0).float().mean() > 0.99
    else:
        assert torch.allclose(y.float(), want, rtol=1e-6, atol=1e-6)


def test_rmsnorm_bwd_matches_float64_autograd():
    torch.manual_seed(1)
    h = torch.randn(32, 1536).half()
    w = (1 + 0.05 * torch.randn(1536)).half()
    dy = torch.randn(32, 1536).half()
    dres = torch.randn(32, 1536).half()
    _, _, rstd = ref.rms_norm_fwd(h, w, 1e-6)
    got = ref.rms_norm_bwd(dy, h, w, rstd, dresidual=dres).float()
    hd = h.double().requires_grad_(True)
    yd = w.double() * hd * torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-6)
    yd.backward(dy.double())
    want = (hd.grad + dres.double()).float()
    assert torch.allclose(got, want, rtol=2e-3, atol=2e-3)


def test_rmsnorm_bwd_orthogonal_to_input_when_unit_weight():
    # RMSNorm is scale invariant: with w = 1 and no residual, dx . h = 0 for every row.
    torch.manual_seed(2)
    h = torch.randn(16, 512, dtype=torch.float32)
    w = torch.ones(512)
    _, _, rstd = ref.rms_norm_fwd(h, w, 0.0)
    dx = ref.rms_norm_bwd(torch.randn(16, 512), h, w, rstd)
    dots = (dx * h).sum(-1) / (dx.norm(dim=-1) * h.norm(dim=-1))
    assert dots.abs().max() < 1e-5


# ---------------------------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------------------------


def test_rope_tables_match_qwen2_rotary_embedding():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                      rope_theta=1e6, max_position_embeddings=2048)
    rot = Qwen2RotaryEmbedding(cfg)
    pos = torch.arange(2048).unsqueeze(0)
    c_hf, s_hf = rot(torch.empty(1, 2048, 128, dtype=torch.float16), pos)
    c, s = ref.rope_tables(2048, 128, 1e6, torch.float16)
    assert torch.equal(c, c_hf[0]) and torch.equal(s, s_hf[0])


def test_rope_fwd_matches_transformers_apply_rotary_pos_emb():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    torch.manual_seed(3)
    n, hq, hkv, d = 37, 12, 2, 128
    qkv = torch.randn(n, (hq + 2 * hkv) * d)
    ql, vl = torch.randn(n, hq * d), torch.randn(n, hkv * d)
    cos, sin = torch.randn(64, d), torch.randn(64, d)  # arbitrary tables: lo/hi halves differ
    pos = torch.randint(0, 64, (n,))
    q, k, v = ref.qkv_rope_fwd(qkv, cos, sin, pos, ql, vl, 2.0, 2.0, hq, hkv, d)
    q_in = (qkv[:, :hq * d] + ql * 2.0).view(n, hq, d).transpose(0, 1).unsqueeze(0)
    k_in = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d).transpose(0, 1).unsqueeze(0)
    qh, kh = apply_rotary_pos_emb(q_in, k_in, cos[pos].unsqueeze(0), sin[pos].unsqueeze(0))
    assert torch.allclose(q, qh[0].transpose(0, 1), rtol=1e-6, atol=1e-5)
    assert torch.allclose(k, kh[0].transpose(0, 1), rtol=1e-6, atol=1e-5)
    assert torch.allclose(v.reshape(n, -1), qkv[:, (hq + hkv) * d:] + vl * 2.0)


def test_rope_bwd_is_adjoint_and_inverse():
    torch.manual_seed(4)
    n, hq, hkv, d = 21, 4, 2, 32
    c64, s64 = ref.rope_tables(128, d, 1e4, torch.float64)
    pos = torch.randint(0, 128, (n,))
    x = torch.randn(n, (hq + 2 * hkv) * d, dtype=torch.float64)
    y = torch.randn(n, hq, d, dtype=torch.float64)
    q, k, v = ref.qkv_rope_fwd(x, c64, s64, pos, h_q=hq, h_kv=hkv, head_dim=d)
    # <R x, y> == <x, R^T y> (adjoint) on the Q heads.
    g = ref.qkv_rope_bwd(y, torch.zeros(n, hkv, d, dtype=torch.float64),
                         torch.zeros(n, hkv, d, dtype=torch.float64), c64, s64, pos, hq, hkv, d)
    assert torch.allclose((q * y).sum(), (x[:, :hq * d] * g[:, :hq * d]).sum(), rtol=1e-12)
    # R^T R = I for exact (float64) cos/sin; rotation preserves each head's norm; dV copies.
    back = ref.qkv_rope_bwd(q, k, v, c64, s64, pos, hq, hkv, d)
    assert torch.allclose(back, x, atol=1e-12)
    assert torch.allclose(q.norm(dim=-1), x[:, :hq * d].view(n, hq, d).norm(dim=-1))
    # position 0 is the identity.
    q0, _, _ = ref.qkv_rope_fwd(x, c64, s64, torch.zeros(n, dtype=torch.long), h_q=hq, h_kv=hkv,
                                head_dim=d)
    assert torch.allclose(q0.reshape(n, -1), x[:, :hq * d])


def test_rope_lora_grads_scale_rounded_values():
    torch.manual_seed(6)
    n = 9
    c, s = ref.rope_tables(16, 128, 1e6, torch.float16)
    pos = torch.randint(0, 16, (n,))
    dq, dk, dv = (torch.randn(n, 12, 128).half(), torch.randn(n, 2, 128).half(),
                  torch.randn(n, 2, 128).half())
    dqkv, dql, dvl = ref.qkv_rope_bwd(dq, dk, dv, c, s, pos, scale_q=2.0, scale_v=0.5)
    assert torch.equal(dql, (dqkv[:, :1536].float() * 2.0).half())
    assert torch.equal(dvl, (dqkv[:, 1792:].float() * 0.5).half())


# ---------------------------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------------------------


def test_swiglu_matches_silu_and_autograd():
    torch.manual_seed(7)
    g = torch.randn(33, 1001, dtype=torch.float64) * 3
    u = torch.randn(33, 1001, dtype=torch.float64)
    assert torch.allclose(ref.swiglu_fwd(g, u), F.silu(g) * u, rtol=1e-12, atol=1e-12)
    gr, ur = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    dout = torch.randn_like(g)
    (F.silu(gr) * ur).backward(dout)
    dg, du = ref.swiglu_bwd(dout, g, u)
    assert torch.allclose(dg, gr.grad, rtol=1e-10, atol=1e-12)
    assert torch.allclose(du, ur.grad, rtol=1e-10, atol=1e-12)


def test_swiglu_fp16_within_one_ulp_of_float64():
    torch.manual_seed(8)
    g = torch.randn(64, 512).half()
    u = torch.randn(64, 512).half()
    want = (F.silu(g.double()) * u.double()).half().float()
    got = ref.swiglu_fwd(g, u).float()
    assert torch.all((got - want).abs() <= ref.fp16_ulp(want))


# ---------------------------------------------------------------------------------------------
# LoRA-input dropout (Philox4x64-10 counter-based masks)
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("key", [(0, 0), (1, 2), (2**64 - 1, 12345), (20251201, 55)])
@pytest.mark.parametrize("block", [1, 7, 2**40 + 3])
def test_philox_matches_numpy_bit_generator(key, block):
    # numpy.random.Philox is Philox4x64-10; it increments its 256-bit counter before each block.
    raw = np.random.Philox(key=np.array(key, dtype=np.uint64),
                           counter=np.array([block - 1, 0, 0, 0], dtype=np.uint64)).random_raw(4 * 3)
    ctr = np.zeros((3, 4), dtype=np.uint64)
    ctr[:, 0] = np.arange(block, block + 3, dtype=np.uint64)
    got = ref.philox4x64_10(ctr, key)
    assert np.array_equal(got.reshape(-1), raw.astype(np.uint64))


def test_philox_counter_wraps_like_numpy():
    raw = np.random.Philox(key=[3, 4], counter=[2**64 - 1] * 4).random_raw(4)
    got = ref.philox4x64_10(np.zeros((1, 4), dtype=np.uint64), (3, 4))
    assert np.array_equal(got.reshape(-1), raw.astype(np.uint64))


def test_dropout_mask_rate_and_independence():
    n_rows, n_cols, p = 625, 1600, 0.05  # 1e6 elements
    m = ref.dropout_keep_mask(7, 0, n_rows, n_cols, p)
    frac = 1.0 - m.mean()
    assert abs(frac - p) < 5 * math.sqrt(p * (1 - p) / m.size)
    m2 = ref.dropout_keep_mask(7, 1, n_rows, n_cols, p)
    m3 = ref.dropout_keep_mask(8, 0, n_rows, n_cols, p)
    both = ((~m) & (~m2)).mean()  # independent streams: P(both dropped) = p^2
    assert abs(both - p * p) < 5 * math.sqrt(p * p * (1 - p * p) / m.size)
    assert (m != m3).any()
    assert ref.dropout_keep_mask(7, 0, n_rows, n_cols, 0.0).all()
    # the mask of an element depends on its row-major index only, not on the row count
    assert np.array_equal(ref.dropout_keep_mask(7, 0, 10, n_cols, p), m[:10])


def test_dropout_keep_bits_layout():
    # The packed layout against an independent unpacking (numpy's little-endian bit order) and
    # known answers: p = 0 keeps every element and pads the last word's tail with zeros.
    keep = ref.dropout_keep_mask(3, 5, 7, 72, 0.3)
    bits = ref.dropout_keep_bits(3, 5, 7, 72, 0.3)
    assert bits.shape == (7, 3) and bits.dtype == np.int32
    unpacked = np.unpackbits(bits.view(np.uint8).reshape(7, 12), axis=1, bitorder="little")
    assert np.array_equal(unpacked[:, :72].astype(bool), keep)
    assert not unpacked[:, 72:].any()
    full = ref.dropout_keep_bits(3, 5, 2, 40, 0.0).view(np.uint32)
    assert (full[:, 0] == 0xFFFFFFFF).all() and (full[:, 1] == 0xFF).all()


def test_dropout_fwd_values_and_bwd_rounding_order():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 96, generator=g).half()
    a, b = ref.lora_dropout_fwd(x, 11, 4, 5, 0.05, 0.1)
    ka = ref.dropout_keep_mask(11, 4, 37, 96, 0.05)
    kt = torch.from_numpy(ka)
    scale = torch.tensor(1.0) / (1.0 - torch.tensor(0.05))
    assert torch.equal(a[~kt], torch.zeros_like(a[~kt]))
    assert torch.equal(a[kt], (x[kt].float() * scale).half())
    assert not torch.equal(a, b)
    a0, _ = ref.lora_dropout_fwd(x, 11, 4, 5, 0.0, 0.0)
    assert torch.equal(a0, x)
    # backward: the reference's sequence of fp16 tensor ops (mask*scale, then two in-place adds)
    acc = torch.randn(37, 96, generator=g).half()
    ga = torch.randn(37, 96, generator=g).half()
    gb = torch.randn(37, 96, generator=g).half()
    da, _ = ref.lora_dropout_fwd(ga, 11, 4, 5, 0.05, 0.1)
    _, db = ref.lora_dropout_fwd(gb, 11, 4, 5, 0.05, 0.1)
    want = acc.clone().add_(da).add_(db)
    assert torch.equal(ref.lora_dropout_bwd_add(acc, ga, gb, 11, 4, 5, 0.05, 0.1), want)


# ---------------------------------------------------------------------------------------------
# Rank-r LoRA branches
# ---------------------------------------------------------------------------------------------


def test_lora_branch_grads_match_float64_autograd():
    # q_lora = s * ((drop(x) A^T) B^T): the closed-form d_mid / dx / gA / gB of the oracle against
    # float64 autograd of the same function (same masks), within the fp16 roundings.
    g = torch.Generator().manual_seed(12)
    n, d, dq_dim, dv_dim, r = 37, 64, 48, 16, 8
    x = torch.randn(n, d, generator=g).half()
    aq, av = ((torch.randn(r, d, generator=g) * 0.1).half() for _ in range(2))
    bq = (torch.randn(dq_dim, r, generator=g) * 0.1).half()
    bv = (torch.randn(dv_dim, r, generator=g) * 0.1).half()
    dq = torch.randn(n, dq_dim, generator=g).half()
    dv = torch.randn(n, dv_dim, generator=g).half()
    dx0 = torch.randn(n, d, generator=g).half()
    seed, pq, pv = 77, 0.1, 0.2
    mid_q, mid_v, xq, xv = ref.lora_down_fwd(x, aq, av, seed, 4, 5, pq, pv)
    dmq, dmv, dx = ref.lora_bwd_x(dq, dv, aq, av, bq, bv, dx0, seed, 4, 5, pq, pv)
    gaq, gbq, gav, gbv = ref.lora_bwd_w(xq, xv, dq, dv, mid_q, mid_v, dmq, dmv)

    kq = torch.from_numpy(ref.dropout_keep_mask(seed, 4, n, d, pq)).double() / (1 - pq)
    kv = torch.from_numpy(ref.dropout_keep_mask(seed, 5, n, d, pv)).double() / (1 - pv)
    X = x.double().requires_grad_(True)
    A_q, A_v, B_q, B_v = (t.double().requires_grad_(True) for t in (aq, av, bq, bv))
    ql = ((X * kq) @ A_q.t()) @ B_q.t()
    vl = ((X * kv) @ A_v.t()) @ B_v.t()
    ((ql * dq.double()).sum() + (vl * dv.double()).sum()).backward()

    def close(a, b, tol):
        return float((a.double() - b).abs().max()) <= tol * float(b.abs().max())

    assert close(mid_q, (X * kq).detach() @ A_q.detach().t(), 2e-3)
    assert close(dx.double() - dx0.double(), X.grad, 5e-3)
    assert close(gaq, A_q.grad, 5e-3) and close(gav, A_v.grad, 5e-3)
    assert close(gbq, B_q.grad, 5e-3) and close(gbv, B_v.grad, 5e-3)
    assert close(dmq, dq.double() @ B_q.detach(), 2e-3)


# ---------------------------------------------------------------------------------------------
# Chunked lm_head cross-entropy
# ---------------------------------------------------------------------------------------------


def _ce_case(seed=9, n=48, d=64, V=1031, masked=8):
    torch.manual_seed(seed)
    h = torch.randn(n, d).half()
    w = (torch.randn(V, d) * 0.2).half()
    labels = torch.randint(0, V, (n,))
    labels[:masked] = -100
    labels[-1] = V - 1  # label in the last, partial chunk
    return h, w, labels


def test_ce_matches_library_routines_on_full_logits():
    h, w, labels = _ce_case()
    out = ref.lm_head_ce(h, w, labels, v_chunk=256)  # 1031 = 4 full chunks + 7
    z = ref.lm_head_logits(h, w)
    lib = ref.softmax_stats_reference(z, labels)
    assert torch.allclose(out["lse"], lib["lse"], atol=1e-5)
    assert torch.allclose(out["entropy"], lib["entropy"], atol=1e-5)
    assert torch.allclose(out["nll"], lib["nll"], atol=1e-5)
    assert torch.equal(out["argmax"], lib["argmax"])  # first index of the max, as torch.argmax
    loss_lib = F.cross_entropy(z, labels, ignore_index=-100)
    assert torch.allclose(out["loss"], loss_lib, atol=1e-6)
    assert torch.all(out["entropy"] >= -1e-6) and torch.all(out["entropy"] <= math.log(1031) + 1e-5)


def test_ce_grad_matches_autograd():
    h, w, labels = _ce_case(seed=10)
    out = ref.lm_head_ce(h, w, labels, v_chunk=300)
    hr = h.float().requires_grad_(True)
    z = hr @ w.float().t()
    F.cross_entropy(z, labels, ignore_index=-100).backward()
    assert torch.allclose(out["dh"].float(), hr.grad, rtol=1e-2, atol=1e-4)
    # rows with label -100 get no gradient
    assert torch.all(out["dh"][:8] == 0)


def test_ce_all_masked_and_num_items():
    h, w, labels = _ce_case(seed=11)
    allm = torch.full_like(labels, -100)
    out = ref.lm_head_ce(h, w, allm, v_chunk=512)
    assert float(out["loss"]) == 0.0 and out["denom"] == 1.0 and torch.all(out["dh"] == 0)
    out2 = ref.lm_head_ce(h, w, labels, num_items_in_batch=100, v_chunk=512, need_grad=False)
    assert torch.allclose(out2["loss"], out2["nll"].sum() / 100)


def test_ce_tie_takes_first_index():
    h = torch.ones(2, 8).half()
    w = torch.zeros(20, 8).half()
    w[3] = 1
    w[17] = 1  # equal logits at 3 and 17 (17 is in a later chunk)
    out = ref.lm_head_ce(h, w, torch.tensor([3, -100]), v_chunk=8, need_grad=False)
    assert out["argmax"].tolist() == [3, 3]


# ---------------------------------------------------------------------------------------------
# Varlen causal GQA attention
# ---------------------------------------------------------------------------------------------


def _attn_inputs(lens, hq=4, hkv=2, d=16, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    n = sum(lens)
    q = torch.randn(n, hq, d, generator=g, dtype=dtype)
    k = torch.randn(n, hkv, d, generator=g, dtype=dtype)
    v = torch.randn(n, hkv, d, generator=g, dtype=dtype)
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    return q, k, v, cu


def test_attention_matches_sdpa_per_row():
    # The reference's own routine: torch SDPA per row with K/V expanded to the query heads.
    q, k, v, cu = _attn_inputs([5, 1, 12, 7], hq=6, hkv=2, d=32, dtype=torch.float32)
    out, _ = ref.attention_varlen_fwd(q, k, v, cu)
    for a, e in zip(cu[:-1], cu[1:]):
        L = e - a
        kb = k[a:e].transpose(0, 1).unsqueeze(1).expand(2, 3, L, 32).reshape(6, L, 32)
        vb = v[a:e].transpose(0, 1).unsqueeze(1).expand(2, 3, L, 32).reshape(6, L, 32)
        sd = F.scaled_dot_product_attention(q[a:e].transpose(0, 1)[None], kb[None], vb[None],
                                            is_causal=True)[0].transpose(0, 1)
        torch.testing.assert_close(out[a:e].float(), sd, rtol=1e-5, atol=1e-6)


def test_attention_closed_forms():
    # q = 0: every allowed key scores 0, so out is the causal running mean of v and
    # lse = log(#keys); a row of length 1 returns its own v.
    q, k, v, cu = _attn_inputs([9, 1, 4])
    out, lse = ref.attention_varlen_fwd(torch.zeros_like(q), k, v, cu)
    for a, e in zip(cu[:-1], cu[1:]):
        for t in range(a, e):
            mean = v[a:t + 1].mean(0).repeat_interleave(2, dim=0)
            torch.testing.assert_close(out[t], mean, rtol=1e-12, atol=1e-12)
            torch.testing.assert_close(lse[:, t], torch.full((4,), math.log(t - a + 1),
                                                             dtype=torch.float64))
    out1, _ = ref.attention_varlen_fwd(q, k, v, cu)
    torch.testing.assert_close(out1[9], v[9].repeat_interleave(2, dim=0))
    # lse = log sum_j exp(scale q.k_j) over j <= t, brute force for one element.
    _, lse = ref.attention_varlen_fwd(q, k, v, cu)
    t, h = 12, 3
    s = [math.exp((q[t, h] @ k[j, h // 2]).item() / 4.0) for j in range(10, t + 1)]
    assert abs(lse[h, t].item() - math.log(sum(s))) < 1e-12


def test_attention_bwd_matches_float64_autograd():
    q, k, v, cu = _attn_inputs([7, 3, 11], hq=6, hkv=2, d=8, seed=3)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    out, _ = ref.attention_varlen_fwd(q, k, v, cu)
    dout = torch.randn_like(out)
    gq, gk, gv = torch.autograd.grad(out, (q, k, v), dout)
    dq, dk, dv = ref.attention_varlen_bwd(dout, q.detach(), k.detach(), v.detach(), cu)
    for a, b in ((dq, gq), (dk, gk), (dv, gv)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)
