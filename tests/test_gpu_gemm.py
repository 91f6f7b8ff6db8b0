"""GPU parity of the split-K projection product rus_gemm_parts (the MLP input gradient
d_norm2 = torch.mm(d_gu, W_gu), solution/ops.py:939) against an fp32 product of the same fp16
operands on the CPU.

Every partial is checked on its own K range (a wrong split boundary or a dropped stage shows up
in one part even when the sum hides it). Tolerance: the kernel and the CPU both accumulate fp16
products in fp32, in different orders, so each output is within 1e-4 relative plus 2e-5 * sqrt(K)
absolute (|a|, |b| <= 1: the products' fp32 rounding error grows like sqrt(K)); a misplaced
element is off by O(1).
"""

from __future__ import annotations

import math

import pytest
import torch

from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(m, n, k, b_kn, seed, pad_a=0, pad_b=0):
    g = torch.Generator().manual_seed(seed)
    a = (torch.rand(m, k + pad_a, generator=g) * 2 - 1).half()
    rows, cols = (k, n) if b_kn else (n, k)
    b = (torch.rand(rows, cols + pad_b, generator=g) * 2 - 1).half()
    return a, b


def _check(a, b, b_kn, n_split, k):
    m = a.shape[0]
    parts = K.gemm_parts(a.to(DEV), b.to(DEV), b_kn, n_split)
    torch.cuda.synchronize()
    sp = K.gemm_parts_count(k, n_split)
    assert parts.shape[0] == sp
    per = -(-k // n_split)
    per = -(-per // 64) * 64  # the pieces are round_up(ceil(k / n_split), 64) columns
    bf = b.float() if b_kn else b.float().t()
    af = a.float()
    got = parts.cpu()
    for s in range(sp):
        lo, hi = s * per, min(k, (s + 1) * per)
        want = af[:, lo:hi] @ bf[lo:hi]
        tol = 1e-4 * want.abs() + 2e-5 * math.sqrt(hi - lo) + 1e-6
        err = (got[s] - want).abs()
        assert torch.all(err <= tol), (s, err.max().item())


@pytest.mark.parametrize("b_kn", [True, False])
@pytest.mark.parametrize("m,n,k,n_split", [
    (876, 1536, 17920, 10),   # the gu input gradient of the bench batch
    (707, 1536, 17920, 14),
    (300, 200, 1536, 3),      # ragged M and N edges
    (1, 8, 64, 1),            # smallest shape
    (257, 264, 192, 2),
    (64, 1536, 8960, 7),
])
def test_gemm_parts_matches_fp32_product(m, n, k, n_split, b_kn):
    a, b = _operands(m, n, k, b_kn, seed=m + n + k)
    _check(a, b, b_kn, n_split, k)


@pytest.mark.parametrize("b_kn", [True, False])
def test_gemm_parts_strided_operands(b_kn):
    m, n, k = 130, 264, 320
    a, b = _operands(m, n, k, b_kn, seed=5, pad_a=24, pad_b=40)
    a_d, b_d = a.to(DEV), b.to(DEV)
    a_v = a_d[:, :k]
    b_v = b_d[:, :n] if b_kn else b_d[:, :k]
    parts = K.gemm_parts(a_v, b_v, b_kn, 3)
    want = a[:, :k].float() @ (b[:, :n].float() if b_kn else b[:, :k].float().t())
    got = parts.sum(0).cpu()
    assert torch.all((got - want).abs() <= 1e-4 * want.abs() + 2e-5 * math.sqrt(k) * 2)


def test_gemm_parts_feeds_norm_backward():
    """The partials summed by the norm backward equal the norm backward of their sum (the path the
    engine takes for d_norm2, ops.py:939-943)."""
    m, n, k = 300, 1536, 17920
    a, b = _operands(m, n, k, True, seed=11)
    a_d, b_d = a.to(DEV), b.to(DEV)
    parts = K.gemm_parts(a_d, b_d, True, 8)
    g = torch.Generator().manual_seed(3)
    h = torch.randn(m, n, generator=g).half().to(DEV)
    w = (torch.rand(n, generator=g) + 0.5).half().to(DEV)
    rstd = (torch.rand(m, generator=g) + 0.5).float().to(DEV)
    dx_parts = K.rms_norm_bwd_parts(parts, h, w, rstd)
    dx_sum = K.rms_norm_bwd(K.sum_splits(parts), h, w, rstd)
    torch.cuda.synchronize()
    assert torch.equal(dx_parts, dx_sum)


def test_gemm_parts_rejects_bad_shapes():
    a = torch.zeros(4, 96, dtype=torch.float16, device=DEV)  # K = 96 is not a multiple of 64
    b = torch.zeros(96, 8, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        K.gemm_parts(a, b, True, 1)
    a = torch.zeros(4, 64, dtype=torch.float16, device=DEV)
    b = torch.zeros(64, 12, dtype=torch.float16, device=DEV)  # N = 12 is not a multiple of 8
    with pytest.raises(RuntimeError, match="not a multiple of 8"):
        K.gemm_parts(a, b, True, 1)
    with pytest.raises(ValueError, match="inner dimensions"):
        K.gemm_parts(a, torch.zeros(32, 8, dtype=torch.float16, device=DEV), True, 1)
