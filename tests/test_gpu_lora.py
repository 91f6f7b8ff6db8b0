"""GPU tests of the fused rank-r LoRA kernels against the CPU oracle (oracle.ops.lora_*).

Every output is an fp16 value that the reference rounds once from an fp32 sum; the kernels sum
in a different order, so each element may differ by one fp16 ulp (at the larger of the two
magnitudes; plus 1e-6 for sums that cancel to near zero). Dropout masks, copies of dropped rows and the untouched elements are
bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as ref
from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, want, ulps=1.0, a=None, b=None):
    """One fp16 ulp at the larger of the two magnitudes (a sum landing on a power of two rounds
    into the wider binade), plus, for a product a @ b, the fp32 accumulation error of either
    summation order: 2 sqrt(K) 2^-24 (|a| @ |b|), which matters only where the sum cancels."""
    g, w = got.float().cpu(), want.float()
    tol = ulps * ref.fp16_ulp(torch.maximum(g.abs(), w.abs())) + 1e-6
    if a is not None:
        k = a.shape[1]
        tol = tol + 2.0 * k ** 0.5 * 2.0**-24 * (a.float().abs() @ b.float().abs())
    ok = (g - w).abs() <= tol
    return bool(ok.all()), float(((g - w).abs() - tol).max())


def _inputs(n, d, dq_dim, dv_dim, r, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g).half()
    aq, av = ((torch.randn(r, d, generator=g) * 0.05).half() for _ in range(2))
    bq = (torch.randn(dq_dim, r, generator=g) * 0.05).half()
    bv = (torch.randn(dv_dim, r, generator=g) * 0.05).half()
    return g, x, aq, av, bq, bv


def _bits(seed_v, stream0, n, d, p_even, p_odd):
    """Device keep bits of two streams and their oracle values (bit-exact)."""
    seed = torch.tensor([seed_v], dtype=torch.int64, device=DEV)
    bits = K.dropout_keep_bits(seed, stream0, 2, n, d, p_even, p_odd)
    torch.cuda.synchronize()
    for s, p in ((0, p_even), (1, p_odd)):
        want = ref.dropout_keep_bits(seed_v, stream0 + s, n, d, p)
        assert np.array_equal(bits[s].cpu().numpy(), want)
    return bits[0], bits[1]


@pytest.mark.parametrize("n,d,streams", [(1, 1536, 2), (37, 40, 3), (300, 1536, 56)])
def test_dropout_keep_bits_match_oracle(n, d, streams):
    seed_v = 77 + n
    seed = torch.tensor([seed_v], dtype=torch.int64, device=DEV)
    bits = K.dropout_keep_bits(seed, 4, streams, n, d, 0.05, 0.3)
    torch.cuda.synchronize()
    for s in (0, 1, streams - 1):
        want = ref.dropout_keep_bits(seed_v, 4 + s, n, d, 0.05 if s % 2 == 0 else 0.3)
        assert np.array_equal(bits[s].cpu().numpy(), want), s


@pytest.mark.parametrize("r", [4, 8, 16, 32])
@pytest.mark.parametrize("drop", [False, True])
@pytest.mark.parametrize("n", [1, 37, 300])
def test_lora_down_and_rope_mid(r, drop, n):
    h_q, h_kv, hd = 12, 2, 128
    d = 1536
    g, x, aq, av, bq, bv = _inputs(n, d, h_q * hd, h_kv * hd, r, seed=r * 100 + n)
    seed_v = 4242
    args = (seed_v, 6, 7, 0.05, 0.1) if drop else (None,)
    mq, mv, xq, xv = ref.lora_down_fwd(x, aq, av, *args)
    bits = _bits(seed_v, 6, n, d, 0.05, 0.1) if drop else (None, None)
    out = K.lora_down_fwd(x.to(DEV), aq.to(DEV), av.to(DEV), *bits, 0.05, 0.1)
    torch.cuda.synchronize()
    for got, want, xx, aa in zip(out[:2], (mq, mv), (xq, xv), (aq, av)):
        ok, err = _close(got, want, a=xx, b=aa.t())
        assert ok, err
    # RoPE with the deltas formed from (mid, B), against the oracle given the same mid values
    qkv = torch.randn(n, (h_q + 2 * h_kv) * hd, generator=g).half()
    cos, sin = ref.rope_tables(512, hd, 1e6)
    pos = torch.randint(0, 512, (n,), generator=g)
    mid_q, mid_v = out[0].cpu(), out[1].cpu()
    want = ref.qkv_rope_fwd(qkv, cos, sin, pos, ref.lora_up(mid_q, bq), ref.lora_up(mid_v, bv),
                            2.0, 2.0, h_q, h_kv, hd)
    got = K.qkv_rope_fwd_mid(qkv.to(DEV), out[0], out[1], bq.to(DEV), bv.to(DEV), cos.to(DEV),
                             sin.to(DEV), pos.to(DEV), 2.0, 2.0, h_q, h_kv, hd)
    torch.cuda.synchronize()
    # Each delta element may differ by one fp16 ulp of its value (fp32 sums in another order);
    # the output then moves by at most scale * (ulp(d_lo) |cos| + ulp(d_hi) |sin|) before its own
    # rounding (one output ulp). K has no delta: one ulp.
    half = hd // 2
    c, sn = cos[pos].float().unsqueeze(1), sin[pos].float().unsqueeze(1)
    for gt, wt, delta, heads, rot in ((got[0], want[0], ref.lora_up(mid_q, bq), h_q, True),
                                      (got[1], want[1], None, h_kv, True),
                                      (got[2], want[2], ref.lora_up(mid_v, bv), h_kv, False)):
        wt = wt.reshape(gt.shape).float()
        tol = ref.fp16_ulp(wt)
        if delta is not None:
            u = ref.fp16_ulp(delta.float()).view(n, heads, hd)
            if rot:
                u_sw = torch.cat([u[..., half:], u[..., :half]], dim=-1)
                tol = tol + 2.0 * (u * c.abs() + u_sw * sn.abs())
            else:
                tol = tol + 2.0 * u
        err = (gt.float().cpu() - wt).abs()
        assert bool((err <= tol + 1e-6).all()), float((err - tol).max())


@pytest.mark.parametrize("r", [4, 8, 16, 32])
@pytest.mark.parametrize("drop", [False, True])
@pytest.mark.parametrize("n", [5, 300])
def test_lora_bwd_x_and_w(r, drop, n):
    d, dq_dim, dv_dim = 1536, 1536, 256
    g, x, aq, av, bq, bv = _inputs(n, d, dq_dim, dv_dim, r, seed=7 + r + n)
    dq = torch.randn(n, dq_dim, generator=g).half()
    dv = torch.randn(n, dv_dim, generator=g).half()
    dx = torch.randn(n, d, generator=g).half()
    seed_v = 99
    dargs = (seed_v, 2, 3, 0.05, 0.05) if drop else (None,)
    bits = _bits(seed_v, 2, n, d, 0.05, 0.05) if drop else (None, None)
    dmq, dmv, dx_want = ref.lora_bwd_x(dq, dv, aq, av, bq, bv, dx, *dargs)
    dxd = dx.to(DEV)
    ts = [t.t().contiguous().to(DEV) for t in (aq, av, bq, bv)]
    got_mq, got_mv = K.lora_bwd_x(dq.to(DEV), dv.to(DEV), *ts, dxd, *bits, 0.05, 0.05)
    torch.cuda.synchronize()
    for got, want, dd, bb in ((got_mq, dmq, dq, bq), (got_mv, dmv, dv, bv)):
        ok, err = _close(got, want, a=dd, b=bb)
        assert ok, err
    # dx: with the kernel's own d_mid (the oracle fed the same values), two chained roundings
    dxq = ref._mm16(got_mq.cpu(), aq)
    dxv = ref._mm16(got_mv.cpu(), av)
    if drop:
        dx_ref = ref.lora_dropout_bwd_add(dx, dxq, dxv, seed_v, 2, 3, 0.05, 0.05)
    else:
        dx_ref = (dx.float() + dxq.float()).half().float().add(dxv.float()).half()
    # each branch product may differ by one ulp of itself; scaled by the dropout factor and
    # rounded again (one ulp of the scaled term), then each of the two chained roundings (the
    # intermediate dx + term_q, then the result) adds one ulp of its value
    sc = 1.0 / 0.95 if drop else 1.0
    inter = (dx.float() + dxq.float() * sc).half().float()
    tol = (ref.fp16_ulp(dx_ref.float()) + ref.fp16_ulp(inter) +
           sc * (ref.fp16_ulp(dxq.float()) + ref.fp16_ulp(dxv.float())) +
           ref.fp16_ulp(sc * dxq.float()) + ref.fp16_ulp(sc * dxv.float()))
    err = (dxd.float().cpu() - dx_ref.float()).abs()
    assert bool((err <= tol + 1e-6).all()), float((err - tol).max())

    # weight gradients from the kernel's d_mid and a forward's mid; the dropped rows are formed
    # in the kernel from x and the keep bits
    mq, mv, xq, xv = ref.lora_down_fwd(x, aq, av, *((seed_v, 2, 3, 0.05, 0.05) if drop else (None,)))
    want = ref.lora_bwd_w(xq, xv, dq, dv, mq, mv, got_mq.cpu(), got_mv.cpu())
    outs = [torch.full(w.shape, 7.0, dtype=torch.float16, device=DEV) for w in want]
    K.lora_bwd_w(x.to(DEV), dq.to(DEV), dv.to(DEV), mq.to(DEV), mv.to(DEV), got_mq, got_mv, *outs,
                 *bits, 0.05, 0.05)
    torch.cuda.synchronize()
    operands = ((got_mq.cpu().t(), xq), (dq.t(), mq), (got_mv.cpu().t(), xv), (dv.t(), mv))
    for got, w, (aa, bb) in zip(outs, want, operands):
        ok, err = _close(got, w, a=aa, b=bb)
        assert ok, err


@pytest.mark.parametrize("r", [16, 32])
def test_lora_split_reductions_see_each_calls_partials(r):
    """The rank-r reductions are split over blocks whose partial sums meet in a workspace (and
    counters) that consecutive calls reuse: back-to-back calls with new inputs must each match
    the products of their own inputs, and a repeated input reproduces its outputs bit for bit
    (fixed summation order), whatever ran in between."""
    n, d, dq_dim, dv_dim = 707, 1536, 1536, 256
    sets = []
    for s in range(3):
        g, x, aq, av, bq, bv = _inputs(n, d, dq_dim, dv_dim, r, seed=500 + s)
        dq = torch.randn(n, dq_dim, generator=g).half()
        dv = torch.randn(n, dv_dim, generator=g).half()
        sets.append((x, aq, av, bq, bv, dq, dv))
    first = {}
    for rep in range(2):
        for i, (x, aq, av, bq, bv, dq, dv) in enumerate(sets):
            xd, dqd, dvd = x.to(DEV), dq.to(DEV), dv.to(DEV)
            ts = [t.t().contiguous().to(DEV) for t in (aq, av, bq, bv)]
            mq, mv = K.lora_down_fwd(xd, aq.to(DEV), av.to(DEV))
            dmq, dmv = K.lora_bwd_x(dqd, dvd, *ts, torch.zeros_like(xd))
            gs = [torch.empty(shp, dtype=torch.float16, device=DEV)
                  for shp in ((r, d), (dq_dim, r), (r, d), (dv_dim, r))]
            K.lora_bwd_w(xd, dqd, dvd, mq, mv, dmq, dmv, *gs)
            outs = [t.cpu() for t in (mq, mv, dmq, dmv, *gs)]
            if rep == 1:
                assert all(torch.equal(a, b) for a, b in zip(outs, first[i])), i
                continue
            first[i] = outs
            checks = ((outs[0], x, aq.t()), (outs[1], x, av.t()), (outs[2], dq, bq),
                      (outs[3], dv, bv), (outs[4], outs[2].t(), x), (outs[5], dq.t(), outs[0]),
                      (outs[6], outs[3].t(), x), (outs[7], dv.t(), outs[1]))
            for k, (got, a, b) in enumerate(checks):
                want = (a.float() @ b.float()).half()
                ok, err = _close(got, want, a=a, b=b)
                assert ok, (i, k, err)


def test_lora_kernels_reject_bad_rank_and_layout():
    x = torch.randn(8, 64, device=DEV).half()
    a = torch.randn(6, 64, device=DEV).half()
    with pytest.raises(ValueError, match="rank"):
        K.lora_down_fwd(x, a, a)
    a4 = torch.randn(4, 64, device=DEV).half()
    bad = torch.zeros(8, 3, dtype=torch.int32, device=DEV)  # 64 columns need 2 words per row
    with pytest.raises(ValueError, match="bits_q"):
        K.lora_down_fwd(x, a4, a4, bad, None, 0.1, 0.0)


@pytest.mark.parametrize("n", [1, 3, 300, 707])
def test_rope_bwd_mid_matches_rope_bwd_and_oracle_products(n):
    # The RoPE backward with the rank-16 products: its packed and scaled outputs equal the plain
    # kernel's bit for bit; d_mid = fp16(dq_lora B) within one ulp (different fp32 sum order).
    hq, hkv, hd, r = 12, 2, 128, 16
    g = torch.Generator().manual_seed(300 + n)
    dq = torch.randn(n, hq, hd, generator=g).half()
    dk = torch.randn(n, hkv, hd, generator=g).half()
    dv = torch.randn(n, hkv, hd, generator=g).half()
    n_pos = 600
    ang = torch.rand(n_pos, hd, generator=g) * 6.3
    cos, sin = ang.cos().half(), ang.sin().half()
    pos = torch.randint(0, n_pos, (n,), generator=g)
    bq = (torch.randn(hq * hd, r, generator=g) * 0.05).half()
    bv = (torch.randn(hkv * hd, r, generator=g) * 0.05).half()
    args = tuple(t.to(DEV) for t in (dq, dk, dv, cos, sin, pos)) + (2.0, 0.5)
    assert K.rope_bwd_mid_supported(hq, hkv, hd, r)
    got = K.qkv_rope_bwd_lora_mid(*args, bq.t().contiguous().to(DEV), bv.t().contiguous().to(DEV),
                                  h_q=hq, h_kv=hkv, head_dim=hd)
    want = K.qkv_rope_bwd_lora(*args, h_q=hq, h_kv=hkv, head_dim=hd)
    torch.cuda.synchronize()
    for a, b in zip(got[:3], want):
        assert torch.equal(a, b)
    for gm, x, b in ((got[3], want[1].cpu(), bq), (got[4], want[2].cpu(), bv)):
        ok, err = _close(gm, ref._mm16(x, b), a=x, b=b)
        assert ok, err


@pytest.mark.parametrize("r", [8, 16])
@pytest.mark.parametrize("drop", [False, True])
@pytest.mark.parametrize("n", [1, 37, 707])
def test_lora_bwd_xw_equals_bwd_x_then_bwd_w(r, drop, n):
    # The expansion beside the weight gradients in one launch runs the same per-wave and
    # per-block code as the two separate launches: dx and all four gradients are bit-identical.
    d, dq_dim, dv_dim = 1536, 1536, 256
    g, x, aq, av, bq, bv = _inputs(n, d, dq_dim, dv_dim, r, seed=900 + r + n)
    dq = torch.randn(n, dq_dim, generator=g).half()
    dv = torch.randn(n, dv_dim, generator=g).half()
    dx = torch.randn(n, d, generator=g).half().to(DEV)
    mq = (torch.randn(n, r, generator=g) * 0.5).half().to(DEV)
    mv = (torch.randn(n, r, generator=g) * 0.5).half().to(DEV)
    bits = _bits(77, 6, n, d, 0.05, 0.1) if drop else (None, None)
    ts = [t.t().contiguous().to(DEV) for t in (aq, av, bq, bv)]
    xd, dqd, dvd = x.to(DEV), dq.to(DEV), dv.to(DEV)
    dx_a = dx.clone()
    dmq, dmv = K.lora_bwd_x(dqd, dvd, *ts, dx_a, *bits, 0.05, 0.1)
    shapes = ((r, d), (dq_dim, r), (r, d), (dv_dim, r))
    outs_a = [torch.full(sh, 7.0, dtype=torch.float16, device=DEV) for sh in shapes]
    outs_b = [torch.full(sh, 7.0, dtype=torch.float16, device=DEV) for sh in shapes]
    K.lora_bwd_w(xd, dqd, dvd, mq, mv, dmq, dmv, *outs_a, *bits, 0.05, 0.1)
    dx_b = dx.clone()
    K.lora_bwd_w(xd, dqd, dvd, mq, mv, dmq, dmv, *outs_b, *bits, 0.05, 0.1,
                 expand=(ts[0], ts[1], dx_b))
    torch.cuda.synchronize()
    assert torch.equal(dx_a, dx_b)
    for a, b in zip(outs_a, outs_b):
        assert torch.equal(a, b)


# ---------------------------------------------------------------------------------------------
# LoRA-down by blocks of four token rows (rus_lora_down_rows) and the same product carried by the
# per-layer dequant launch beside the input norm (rus_nf4_dequant_multi_norm with `down`).

@pytest.mark.parametrize("r", [4, 8, 16])
@pytest.mark.parametrize("drop", [False, True])
@pytest.mark.parametrize("n,d", [(1, 1536), (37, 1536), (301, 1536), (6, 64), (9, 2048)])
def test_lora_down_rows_matches_oracle(r, drop, n, d):
    _, x, aq, av, _, _ = _inputs(n, d, 8, 8, r, seed=7 * r + n + d)
    seed_v = 515
    args = (seed_v, 2, 3, 0.05, 0.1) if drop else (None,)
    mq, mv, xq, xv = ref.lora_down_fwd(x, aq, av, *args)
    bits = _bits(seed_v, 2, n, d, 0.05, 0.1) if drop else (None, None)
    out = K.lora_down_rows(x.to(DEV), aq.to(DEV), av.to(DEV), *bits, 0.05, 0.1)
    torch.cuda.synchronize()
    for got, want, xx, aa in zip(out, (mq, mv), (xq, xv), (aq, av)):
        ok, err = _close(got, want, a=xx, b=aa.t())
        assert ok, err
    # the split-K kernel of rus_lora_down_fwd gives the same values within one ulp each way
    old = K.lora_down_fwd(x.to(DEV), aq.to(DEV), av.to(DEV), *bits, 0.05, 0.1)
    for got, o, xx, aa in zip(out, old, (xq, xv), (aq, av)):
        ok, err = _close(got, o.cpu(), ulps=2.0, a=xx, b=aa.t())
        assert ok, err


@pytest.mark.parametrize("drop", [False, True])
@pytest.mark.parametrize("n", [3, 300])
def test_dequant_launch_carries_norm_and_lora_down_bitwise(drop, n):
    """The input norm and its LoRA-down carried by a layer's dequant launch give the bits of the
    standalone norm followed by rus_lora_down_rows, and the weights of the plain dequant."""
    from rus_amd import model as M
    from rus_amd.hostload import WeightStream

    cfg = M.Qwen2Config(num_hidden_layers=1, hidden_size=1536, intermediate_size=256,
                        num_attention_heads=12, num_key_value_heads=2, vocab_size=64)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=3)
    ws = WeightStream(model.layers, DEV, resident=True)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, 1536, generator=g).half().to(DEV)
    res = torch.randn(n, 1536, generator=g).half().to(DEV)
    lnw = (torch.rand(1536, generator=g) + 0.5).to(DEV)
    aq, av = ((torch.randn(16, 1536, generator=g) * 0.05).half().to(DEV) for _ in range(2))
    bits = _bits(99, 0, n, 1536, 0.05, 0.1) if drop else (None, None)
    want_w = [w.clone() for w in ws.dequant_layer(0).values()]
    y0, h0, r0 = K.rms_norm_fwd(x, lnw, 1e-6, residual=res)
    m0 = K.lora_down_rows(y0, aq, av, *bits, 0.05, 0.1)
    torch.cuda.synchronize()
    y1, h1, r1, pend = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
    m1 = pend.carry_lora_down(aq, av, *bits, 0.05, 0.1)
    got_w = ws.dequant_layer(0, norm=pend)
    assert pend.done
    torch.cuda.synchronize()
    for a, b in zip((y1, h1, r1, *m1), (y0, h0, r0, *m0)):
        assert torch.equal(a, b)
    for a, b in zip(got_w.values(), want_w):
        assert torch.equal(a, b)
    # a norm that runs on its own runs its carried LoRA-down too
    y2, _, _, pend2 = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
    m2 = pend2.carry_lora_down(aq, av, *bits, 0.05, 0.1)
    pend2.run()
    torch.cuda.synchronize()
    assert torch.equal(y2, y0) and all(torch.equal(a, b) for a, b in zip(m2, m0))


@pytest.mark.parametrize("d,r,n", [(2048, 8, 301), (512, 4, 5), (1024, 16, 257)])
def test_carried_lora_down_widths_ranks_and_ragged_tokens(d, r, n):
    """The carried LoRA-down's LDS stage at other widths (2048 fills it exactly), ranks 4 / 8 and
    token counts that leave a partial last block of four: the bits of the norm followed by
    rus_lora_down_rows, with dropout, and the mids against the oracle's fp16 product."""
    from rus_amd import model as M
    from rus_amd.hostload import WeightStream

    cfg = M.Qwen2Config(num_hidden_layers=1, hidden_size=d, intermediate_size=256,
                        num_attention_heads=d // 128, num_key_value_heads=2, vocab_size=64)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=5)
    ws = WeightStream(model.layers, DEV, resident=True)
    g = torch.Generator().manual_seed(n + d)
    x = torch.randn(n, d, generator=g).half().to(DEV)
    res = torch.randn(n, d, generator=g).half().to(DEV)
    lnw = (torch.rand(d, generator=g) + 0.5).to(DEV)
    aq, av = ((torch.randn(r, d, generator=g) * 0.05).half().to(DEV) for _ in range(2))
    bits = _bits(7, 0, n, d, 0.05, 0.1)
    y0, _, _ = K.rms_norm_fwd(x, lnw, 1e-6, residual=res)
    m0 = K.lora_down_rows(y0, aq, av, *bits, 0.05, 0.1)
    _, _, _, pend = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
    m1 = pend.carry_lora_down(aq, av, *bits, 0.05, 0.1)
    ws.dequant_layer(0, norm=pend)
    assert pend.done
    torch.cuda.synchronize()
    for a, b in zip(m1, m0):
        assert torch.equal(a, b)
    # against the oracle: fp16(drop(y) A^T) from the same keep bits, within 2 fp16 ulps
    yc = y0.cpu()
    for (mid, a_fac, b_bits, p) in ((m1[0], aq, bits[0], 0.05), (m1[1], av, bits[1], 0.1)):
        keep = torch.from_numpy(np.unpackbits(
            b_bits.cpu().numpy().view(np.uint8), axis=1, bitorder="little")[:, :d].astype(bool))
        xd = torch.where(keep, (yc.float() * (1.0 / (1.0 - p))).half(), torch.zeros((), dtype=torch.float16))
        ok, err = _close(mid.cpu(), (xd.float() @ a_fac.cpu().float().t()).half(), ulps=2.0,
                         a=xd, b=a_fac.cpu().t())
        assert ok, err


@pytest.mark.parametrize("n_layers,shapes", [(3, [(16, 1536), (1536, 16), (16, 1536), (256, 16)]),
                                             (2, [(3, 5), (7, 2)]), (1, [(1, 1)])])
def test_lora_cast_t_matches_torch_cast_and_transposes(n_layers, shapes):
    # rus_lora_cast_t: fp16 of the flat fp32 factors (torch's round-to-nearest-even cast,
    # bitwise) and every layer's segments transposed into [n_layers, cols, rows] regions.
    n = n_layers * sum(r * c for r, c in shapes)
    flat = torch.randn(n, device=DEV) * 3.0
    flat[::97] = 65520.0  # rounds to inf in fp16, as torch's cast does
    out = torch.empty(n, dtype=torch.float16, device=DEV)
    out_t = torch.empty_like(out)
    K.lora_cast_t(flat, n_layers, shapes, out, out_t)
    only = torch.empty_like(out)
    K.lora_cast_t(flat, n_layers, shapes, only)
    torch.cuda.synchronize()
    want = flat.half()
    assert torch.equal(out, want) and torch.equal(only, want)
    per = sum(r * c for r, c in shapes)
    off = 0
    for r, c in shapes:
        seg = want.view(n_layers, per)[:, off: off + r * c].reshape(n_layers, r, c)
        region = out_t[n_layers * off: n_layers * (off + r * c)].view(n_layers, c, r)
        assert torch.equal(region, seg.transpose(1, 2)), (r, c)
        off += r * c


def test_engine_lora_fp16_t_is_the_cast_launch_copy():
    # The engine's step casts: lora_fp16_t returns the copies written beside lora_fp16's
    # (no further launch), equal to the transposes of the fp16 factors.
    from rus_amd import model as M
    from rus_amd.ops import Qwen2FusedEngine

    cfg = M.Qwen2Config(hidden_size=512, intermediate_size=256, num_hidden_layers=2,
                        num_attention_heads=4, num_key_value_heads=2, vocab_size=1000, lora_r=16)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=1)
    eng = Qwen2FusedEngine(model, DEV, resident_weights=True)
    lora16 = eng.lora_fp16()
    t = eng.lora_fp16_t(lora16)
    for p, a, b in zip(eng.lora_params, lora16, t):
        assert torch.equal(a, p.detach().half()) and torch.equal(b, a.t())
    # factors from elsewhere (views of another flat fp16 buffer): the transposes are formed
    again = eng.lora_views(torch.cat([x.reshape(-1) for x in lora16]))
    for a, b in zip(again, eng.lora_fp16_t(again)):
        assert torch.equal(b, a.t())
