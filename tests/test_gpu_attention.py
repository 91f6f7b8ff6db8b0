"""GPU tests of the varlen causal GQA attention kernels against the CPU oracle
(oracle.ops.attention_varlen_fwd / _bwd, float64 on the same fp16 inputs).

Tolerances follow the kernels' two roundings: P (forward) and dS (backward) are rounded to fp16
for their MFMA products, relative error at most 2^-11 each, and the stored O that the backward's
D = rowsum(dO o O) reads is fp16. Each element's bound is that error carried through the
absolute values of the other operand (computed here in float64 from the same inputs), doubled,
plus one fp16 ulp of the output. lse is fp32: 1e-5 absolute.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ops as ref
from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS16 = 2.0**-11


def _inputs(lens, hq, hkv, seed, qk_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    n = sum(lens)
    q = (torch.randn(n, hq, 128, generator=g) * qk_scale).half()
    k = (torch.randn(n, hkv, 128, generator=g) * qk_scale).half()
    v = torch.randn(n, hkv, 128, generator=g).half()
    dout = torch.randn(n, hq, 128, generator=g).half()
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    return q, k, v, dout, cu


def _dev(*ts):
    return [t.to(DEV) for t in ts]


def _bounds(q, k, v, dout, cu):
    """float64 per-element error bounds (before doubling) for out, dq, dk, dv."""
    n, hq, d = q.shape
    hkv = k.shape[1]
    grp = hq // hkv
    sc = 1.0 / math.sqrt(d)
    q, k, v, dout = q.double(), k.double(), v.double(), dout.double()
    bo = torch.zeros(n, hq, d, dtype=torch.float64)
    bq = torch.zeros_like(bo)
    bk = torch.zeros(n, hkv, d, dtype=torch.float64)
    bv = torch.zeros_like(bk)
    for a, e in zip(cu[:-1], cu[1:]):
        L = e - a
        if L == 0:
            continue
        qh = q[a:e].transpose(0, 1)
        ks = k[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)
        vs = v[a:e].repeat_interleave(grp, dim=1).transpose(0, 1)
        do = dout[a:e].transpose(0, 1)
        s = sc * (qh @ ks.transpose(1, 2))
        s = s.masked_fill(~torch.ones(L, L, dtype=torch.bool).tril(), float("-inf"))
        p = torch.softmax(s, -1)
        o = p @ vs
        ds = p * (do @ vs.transpose(1, 2) - (do * o).sum(-1, keepdim=True))
        # |dS| rounding + P * sum|dO||O| (fp16 O in D)
        eds = EPS16 * ds.abs() + p * EPS16 * (do.abs() * o.abs()).sum(-1, keepdim=True)
        bo[a:e] = (EPS16 * (p @ vs.abs())).transpose(0, 1)
        bq[a:e] = (sc * (eds @ ks.abs())).transpose(0, 1)
        bk[a:e] = (sc * (eds.transpose(1, 2) @ qh.abs())).reshape(hkv, grp, L, d).sum(1).transpose(0, 1)
        bv[a:e] = (EPS16 * (p.transpose(1, 2) @ do.abs())).reshape(hkv, grp, L, d).sum(1).transpose(0, 1)
    return bo, bq, bk, bv


def _check(name, got, want, bound):
    g = got.double().cpu()
    tol = 2.0 * bound + ref.fp16_ulp(want.float()).double() + 1e-6
    err = (g - want).abs()
    bad = err > tol
    assert not bool(bad.any()), (
        f"{name}: {int(bad.sum())} elements out of tolerance, worst excess "
        f"{float((err - tol).max()):.3e} (max err {float(err.max()):.3e})")


def _run(lens, hq, hkv, seed, qk_scale=1.0, check_bwd=True):
    q, k, v, dout, cu = _inputs(lens, hq, hkv, seed, qk_scale)
    out_ref, lse_ref = ref.attention_varlen_fwd(q, k, v, cu)
    bo, bq, bk, bv = _bounds(q, k, v, dout, cu)
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    out, lse = K.attn_varlen_fwd(qd, kd, vd, cud, lens=lens)
    torch.cuda.synchronize()
    _check("out", out, out_ref, bo)
    torch.testing.assert_close(lse.double().cpu(), lse_ref, rtol=1e-6, atol=1e-5)
    if not check_bwd:
        return
    dq_ref, dk_ref, dv_ref = ref.attention_varlen_bwd(dout, q, k, v, cu)
    dq, dk, dv = K.attn_varlen_bwd(dd, qd, kd, vd, out, lse, cud, lens=lens)
    torch.cuda.synchronize()
    _check("dq", dq, dq_ref, bq)
    _check("dk", dk, dk_ref, bk)
    _check("dv", dv, dv_ref, bv)


@pytest.mark.parametrize("lens,hq,hkv", [
    ([1, 17, 32, 33, 64, 100], 12, 2),  # edges of the 32-token blocks, rows at ragged offsets
    ([40, 7], 4, 4),                     # no GQA
    ([70, 1, 1, 5], 8, 1),               # MQA, single-token rows
])
def test_attention_matches_oracle(lens, hq, hkv):
    _run(lens, hq, hkv, seed=sum(lens) + hq)


def test_attention_longest_row():
    _run([512], 12, 2, seed=7)


def test_attention_bench_shaped_batch():
    # 4 rows with lognormal lengths (median 140, mean 220, clipped to [16, 512]) + a padding row
    # of the kind a captured-graph bucket appends.
    rng = np.random.default_rng(11)
    lens = [int(x) for x in np.clip(rng.lognormal(math.log(140), 0.92, 4), 16, 512)]
    lens.append(256 - sum(lens) % 256)
    _run(lens, 12, 2, seed=3)


def test_attention_peaked_scores():
    # Large logits: the running max moves across key blocks (online-softmax rescaling).
    _run([96, 45], 12, 2, seed=5, qk_scale=3.0)


def test_attention_rising_scores():
    # Scores that grow along the row by more than 2^8 per key block: the running maximum
    # (and its lazily updated reference point) moves on every block.
    lens = [200, 70]
    q, k, v, dout, cu = _inputs(lens, 12, 2, seed=8)
    ramp = torch.cat([torch.linspace(0.0, 1.0, L) for L in lens])
    k = (k.float() * 0.1 + 4.0 * ramp[:, None, None]).half()
    q = (q.float() * 0.1 + 1.0).half()
    out_ref, lse_ref = ref.attention_varlen_fwd(q, k, v, cu)
    bo, bq, bk, bv = _bounds(q, k, v, dout, cu)
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    out, lse = K.attn_varlen_fwd(qd, kd, vd, cud)
    dq, dk, dv = K.attn_varlen_bwd(dd, qd, kd, vd, out, lse, cud)
    torch.cuda.synchronize()
    _check("out", out, out_ref, bo)
    torch.testing.assert_close(lse.double().cpu(), lse_ref, rtol=1e-6, atol=1e-4)
    dq_ref, dk_ref, dv_ref = ref.attention_varlen_bwd(dout, q, k, v, cu)
    _check("dq", dq, dq_ref, bq)
    _check("dk", dk, dk_ref, bk)
    _check("dv", dv, dv_ref, bv)


def test_attention_deterministic_and_extra_blocks():
    lens = [33, 90]
    q, k, v, dout, cu = _inputs(lens, 12, 2, seed=1)
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    o1, l1 = K.attn_varlen_fwd(qd, kd, vd, cud)
    o2, l2 = K.attn_varlen_fwd(qd, kd, vd, cud, max_blocks=K.attn_max_blocks(123, 2) + 40)
    g1 = K.attn_varlen_bwd(dd, qd, kd, vd, o1, l1, cud)
    g2 = K.attn_varlen_bwd(dd, qd, kd, vd, o2, l2, cud, max_blocks=64)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_attention_matches_torch_flash_on_device():
    # Same call as the engine's previous path (aten flash attention, varlen, causal).
    lens = [50, 130, 16]
    q, k, v, dout, cu = _inputs(lens, 12, 2, seed=9)
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    out, _ = K.attn_varlen_fwd(qd, kd, vd, cud)
    o_t = torch.ops.aten._flash_attention_forward(qd, kd, vd, cud, cud, max(lens), max(lens), 0.0,
                                                  True, False)[0]
    torch.cuda.synchronize()
    assert (out.float() - o_t.float()).abs().max().item() < 4e-3


@pytest.mark.parametrize("lens,hq,hkv", [([33, 90, 1, 200], 12, 2), ([40, 7], 4, 4), ([70, 5], 8, 1)])
def test_attention_partials_equal_group_sum(lens, hq, hkv):
    # The partial-output backward: dq is the group-summing backward's bit for bit, and each KV
    # head's per-query-head partials summed in head order and rounded once are its dk / dv.
    q, k, v, dout, cu = _inputs(lens, hq, hkv, seed=sum(lens))
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    out, lse = K.attn_varlen_fwd(qd, kd, vd, cud)
    dq, dk, dv = K.attn_varlen_bwd(dd, qd, kd, vd, out, lse, cud)
    dq_p, dk_p, dv_p = K.attn_varlen_bwd_parts(dd, qd, kd, vd, out, lse, cud)
    torch.cuda.synchronize()
    assert torch.equal(dq_p, dq)
    grp = hq // hkv
    for part, full in ((dk_p, dk), (dv_p, dv)):
        acc = part.view(hkv, grp, -1, 128)[:, 0].clone()
        for j in range(1, grp):
            acc += part.view(hkv, grp, -1, 128)[:, j]
        assert torch.equal(acc.half().permute(1, 0, 2).contiguous(), full)


def test_rope_mid_over_attention_partials_equals_group_sum_path():
    # Attention partials -> RoPE backward that sums them equals attention group sum -> RoPE
    # backward, for all five outputs, bit for bit (bench-shaped heads, rank 16).
    lens = [100, 37, 250]
    hq, hkv, hd, r = 12, 2, 128, 16
    q, k, v, dout, cu = _inputs(lens, hq, hkv, seed=21)
    qd, kd, vd, dd = _dev(q, k, v, dout)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    n = sum(lens)
    g = torch.Generator().manual_seed(5)
    ang = torch.rand(600, hd, generator=g) * 6.3
    cos, sin = ang.cos().half().to(DEV), ang.sin().half().to(DEV)
    pos = torch.randint(0, 600, (n,), generator=g).to(DEV)
    bqt = (torch.randn(r, hq * hd, generator=g) * 0.05).half().to(DEV)
    bvt = (torch.randn(r, hkv * hd, generator=g) * 0.05).half().to(DEV)
    out, lse = K.attn_varlen_fwd(qd, kd, vd, cud)
    dq, dk, dv = K.attn_varlen_bwd(dd, qd, kd, vd, out, lse, cud)
    want = K.qkv_rope_bwd_lora_mid(dq, dk, dv, cos, sin, pos, 2.0, 0.5, bqt, bvt,
                                   h_q=hq, h_kv=hkv, head_dim=hd)
    dq_p, dk_p, dv_p = K.attn_varlen_bwd_parts(dd, qd, kd, vd, out, lse, cud)
    got = K.qkv_rope_bwd_lora_mid_parts(dq_p, dk_p, dv_p, cos, sin, pos, 2.0, 0.5, bqt, bvt,
                                        h_q=hq, h_kv=hkv, head_dim=hd)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
