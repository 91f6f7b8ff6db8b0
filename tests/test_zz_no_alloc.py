"""GPU test of rus_lora_down_fwd_noalloc, the allocation-free variant of rus_lora_down_fwd: called
through the C ABI, its outputs equal the workspace entry point's bit for bit (same kernels, same
summation order) on two calls in a row, the second with fewer tokens, with and without dropout
keep bits; shapes beyond its static scratch are rejected before any launch."""

from __future__ import annotations

import pytest
import torch

from rus_amd import _lib
from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc(x, a_q, a_v, bits, p):
    n, d = x.shape
    r = a_q.shape[0]
    mid_q = torch.empty((n, r), dtype=torch.float16, device=DEV)
    mid_v = torch.empty((n, r), dtype=torch.float16, device=DEV)
    bq = bits[0].data_ptr() if bits is not None else None
    bv = bits[1].data_ptr() if bits is not None else None
    _lib.call("rus_lora_down_fwd_noalloc", x.data_ptr(), n, d, x.stride(0), a_q.data_ptr(),
              a_v.data_ptr(), r, mid_q.data_ptr(), mid_v.data_ptr(), bq, bv, float(p), float(p),
              torch.cuda.current_stream().cuda_stream)
    return mid_q, mid_v


@pytest.mark.parametrize("r", [16, 32])
def test_noalloc_lora_down_equals_workspace_entry_point(r):
    g = torch.Generator().manual_seed(r)
    d = 1536
    a_q = (torch.randn(r, d, generator=g) * 0.02).half().to(DEV)
    a_v = (torch.randn(r, d, generator=g) * 0.02).half().to(DEV)
    seed = torch.tensor([1234], dtype=torch.int64, device=DEV)
    for n, dropout in ((1000, True), (300, True), (777, False), (45, False)):
        x = torch.randn(n, d, generator=g).half().to(DEV)
        bits = None
        p = 0.0
        if dropout:
            p = 0.05
            bits = K.dropout_keep_bits(seed, 0, 2, n, d, p, p)
        want = K.lora_down_fwd(x, a_q, a_v, *(bits if bits is not None else (None, None)), p, p)
        got = _noalloc(x, a_q, a_v, bits, p)
        torch.cuda.synchronize()
        assert torch.equal(got[0].cpu(), want[0].cpu()) and torch.equal(got[1].cpu(), want[1].cpu()), (n, dropout)


def test_noalloc_lora_down_rejects_beyond_static_scratch():
    d, r, n = 1536, 16, 10944
    # buffers of the full size, so that a regression of the host-side check would show as a
    # missing error rather than as accesses past small allocations
    x = torch.zeros((n, d), dtype=torch.float16, device=DEV)
    a = torch.zeros((r, d), dtype=torch.float16, device=DEV)
    mid_q = torch.zeros((n, r), dtype=torch.float16, device=DEV)
    mid_v = torch.zeros((n, r), dtype=torch.float16, device=DEV)
    # 10,944 tokens need 342 tiles of 32: one more than the static scratch holds (checked on the
    # host from the sizes alone, before anything is launched)
    with pytest.raises(RuntimeError, match="static scratch"):
        _lib.call("rus_lora_down_fwd_noalloc", x.data_ptr(), n, d, d, a.data_ptr(),
                  a.data_ptr(), r, mid_q.data_ptr(), mid_v.data_ptr(), None, None, 0.0, 0.0,
                  torch.cuda.current_stream().cuda_stream)
