"""GPU tests of the fused NF4 W4A16 products (rus_nf4_gemm) against the CPU oracle.

The kernel decodes the NF4 weight exactly as rus_nf4_dequant does and sums in fp32 on MFMA; the
oracle sums the same fp16 operands in float64 and rounds once. Each output may therefore differ
by one fp16 ulp (at the larger magnitude) plus the fp32 accumulation error of a K-term sum,
2 sqrt(K) 2^-24 (|x| @ |W|), which matters only where the sum cancels.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as ref
from rus_amd import kernels as K
from rus_amd import quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weight(rows_per_seg, cols, seed, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    parts = [quant.quantize_nf4((torch.randn(r, cols, generator=g) * scale).half())
             for r in rows_per_seg]
    fused, splits, offs, bases = quant.concat_segments(parts)
    w16 = ref.nf4_dequant(fused.packed.numpy(), fused.absmax.numpy(), fused.code2.numpy(),
                          fused.absmax2.numpy(), offs, fused.shape, split_bytes=splits,
                          absmax2_bases=bases)
    op = K.NF4Operand(fused.packed.to(DEV), fused.absmax.to(DEV), fused.absmax2.to(DEV),
                      fused.code2.to(DEV), offs, fused.shape, split_bytes=splits,
                      absmax2_bases=bases)
    return op, w16


def _tol(got, want, x, w16, trans):
    g, w = got.float().cpu(), want.float()
    wa = torch.from_numpy(np.abs(w16.astype(np.float32)))
    mag = x.float().abs() @ (wa if trans else wa.t())
    k = x.shape[1]
    tol = ref.fp16_ulp(torch.maximum(g.abs(), w.abs())) + 2.0 * k ** 0.5 * 2.0**-24 * mag + 1e-6
    return g, w, tol


def _check(got, want, x, w16, trans):
    g, w, tol = _tol(got, want, x, w16, trans)
    err = (g - w).abs()
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("m", [1, 37, 300])
@pytest.mark.parametrize("split", [0, 1, 2, 3])
def test_nf4_gemm_segments_match_oracle(trans, m, split):
    # Three row segments (own offsets and absmax2 bases), two 64-column tiles, several steps.
    op, w16 = _weight((64, 128, 64), 320, seed=11 + m)
    n_in = 256 if trans else 320
    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, n_in, generator=g).half()
    bias = None if trans else (torch.randn(256, generator=g) * 0.1).half()
    sp = K.nf4_gemm_plan(m, 256, 320, trans, split)[0] if split else 0  # nearest valid split
    got = K.nf4_gemm(x.to(DEV), op, trans=trans, bias=None if bias is None else bias.to(DEV),
                     split=sp)
    torch.cuda.synchronize()
    _check(got, ref.nf4_gemm(x, w16, trans, bias), x, w16, trans)


@pytest.mark.parametrize("trans", [False, True])
def test_nf4_gemm_strided_rows_and_out(trans):
    op, w16 = _weight((128,), 192, seed=3)
    n_in, n_out = (128, 192) if trans else (192, 128)
    g = torch.Generator().manual_seed(4)
    xb = torch.randn(70, n_in + 24, generator=g).half()
    x = xb[:, :n_in]  # row stride n_in + 24
    out = torch.full((70, n_out + 12), 7.0, dtype=torch.float16, device=DEV)
    got = K.nf4_gemm(xb.to(DEV)[:, :n_in], op, trans=trans, out=out[:, :n_out])
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    _check(got, ref.nf4_gemm(x, w16, trans), x, w16, trans)
    assert torch.all(out[:, n_out:] == 7.0)  # nothing written past the view


# The layer products of the bench workload (Qwen2.5-1.5B shapes, ~707 packed tokens):
# [q|k|v], o, [gate|up], down weights, forward (x W^T) and input-gradient (dy W) products.
LAYER = {"qkv": ((1536, 256, 256), 1536), "o": ((1536,), 1536), "gu": ((8960, 8960), 1536),
         "down": ((1536,), 8960)}


@pytest.mark.parametrize("seg", list(LAYER))
def test_nf4_gemm_layer_shapes_match_dequant_then_gemm(seg):
    rows_per_seg, cols = LAYER[seg]
    op, w16 = _weight(rows_per_seg, cols, seed=len(seg))
    rows = sum(rows_per_seg)
    wd = torch.from_numpy(w16).to(DEV).float()
    g = torch.Generator().manual_seed(7)
    m = 707
    for trans in (False, True):
        n_in = rows if trans else cols
        x = torch.randn(m, n_in, generator=g).half()
        xd = x.to(DEV)
        got = K.nf4_gemm(xd, op, trans=trans)
        again = K.nf4_gemm(xd, op, trans=trans)
        want = ((xd.float() @ (wd if trans else wd.t()))).half()  # fp32 GEMM, one rounding
        torch.cuda.synchronize()
        assert torch.equal(got, again)  # fixed summation order
        g_, w_, tol = _tol(got, want.cpu(), x, w16, trans)
        err = (g_ - w_).abs()
        assert bool((err <= 2 * tol).all()), (trans, float((err - 2 * tol).max()))


def test_nf4_gemm_split_partials_fresh_each_call():
    """Split products meet in a workspace and counters that consecutive calls reuse: each call
    must match its own inputs, and a repeated input reproduces its output bit for bit."""
    op, w16 = _weight((1536,), 8960, seed=21)
    m = 707
    assert K.nf4_gemm_plan(m, 1536, 8960, False)[0] > 1
    g = torch.Generator().manual_seed(22)
    xs = [torch.randn(m, 8960, generator=g).half() for _ in range(3)]
    first = []
    for rep in range(2):
        for i, x in enumerate(xs):
            got = K.nf4_gemm(x.to(DEV), op).cpu()
            if rep:
                assert torch.equal(got, first[i]), i
            else:
                first.append(got)
                _check(got, ref.nf4_gemm(x, w16), x, w16, False)
