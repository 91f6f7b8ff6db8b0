"""GPU parity of the AdamW kernel (rus_amd.optim.FlatAdamW, rus_adamw_step) against
torch.optim.AdamW (single-tensor path, fp32) on the same parameters and gradients.

The update is elementwise, so it is checked over several steps on sizes with and without a
partial last 16-byte pack, with and without weight decay. Tolerance: the two compute the same
fp32 update in different operation orders (torch's single-tensor path scales p by (1 - lr wd)
and forms m with lerp; this library rounds every product and sum of the formula as written), a
few fp32 ulps per step: parameters within rtol 2e-6 plus 5e-6 lr absolute (the update is at most
a few lr per step), exp_avg within rtol 2e-6 / atol 1e-6, exp_avg_sq within rtol 2e-6 / atol
1e-9, after six steps; the first step of a zero-moment start is checked in float64 against its
closed form p (1 - lr wd) - lr g / (|g| + eps).
"""

from __future__ import annotations

import pytest
import torch

from rus_amd import kernels as K
from rus_amd.optim import FlatAdamW

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("n", [1, 7, 4096, 2_179_072 + 3])
@pytest.mark.parametrize("lr,wd", [(2e-4, 0.01), (1e-3, 0.0), (5e-2, 0.1)])
def test_flat_adamw_matches_torch_adamw(n, lr, wd):
    g = torch.Generator(device=DEV).manual_seed(n + int(lr * 1e6))
    p0 = torch.randn(n, device=DEV, generator=g) * 0.05
    a = torch.nn.Parameter(p0.clone())
    b = torch.nn.Parameter(p0.clone())
    ours = FlatAdamW([a], lr=lr, weight_decay=wd)
    ref = torch.optim.AdamW([b], lr=lr, weight_decay=wd, foreach=False, fused=False)
    for step in range(6):
        grad = torch.randn(n, device=DEV, generator=g) * (10.0 ** (step % 3 - 2))
        a.grad = grad.clone()
        b.grad = grad.clone()
        ours.step()
        ref.step()
        torch.cuda.synchronize()
        assert torch.allclose(a, b, rtol=2e-6, atol=5e-6 * lr), step
    st_a, st_b = ours.state[a], ref.state[b]
    assert st_a["step"] == 6 and int(st_b["step"]) == 6
    for k, atol in (("exp_avg", 1e-6), ("exp_avg_sq", 1e-9)):
        assert torch.allclose(st_a[k], st_b[k], rtol=2e-6, atol=atol), k


def test_first_step_closed_form_and_skipped_grads():
    # From zero moments, step 1 gives m = (1-b1) g, v = (1-b2) g^2, so the update is
    # lr * g / (|g| + eps) after the decay p -> p (1 - lr wd): checked in float64.
    n = 1000
    g = torch.Generator(device=DEV).manual_seed(3)
    p0 = torch.randn(n, device=DEV, generator=g)
    grad = torch.randn(n, device=DEV, generator=g)
    a = torch.nn.Parameter(p0.clone())
    idle = torch.nn.Parameter(torch.ones(8, device=DEV))  # no gradient: left untouched
    opt = FlatAdamW([a, idle], lr=1e-2, weight_decay=0.1, eps=1e-8)
    a.grad = grad.clone()
    opt.step()
    torch.cuda.synchronize()
    p64, g64 = p0.double(), grad.double()
    want = p64 * (1 - 1e-2 * 0.1) - 1e-2 * g64 / (g64.abs() + 1e-8)
    assert torch.allclose(a.double(), want, rtol=1e-6, atol=1e-7)
    assert torch.equal(idle.detach(), torch.ones(8, device=DEV)) and not opt.state[idle]


def test_adamw_step_validates():
    p = torch.zeros(16, device=DEV)
    with pytest.raises(ValueError, match="float32"):
        K.adamw_step(p, torch.zeros(16, device=DEV, dtype=torch.float16), p.clone(), p.clone(),
                     1e-3, 0.9, 0.999, 1e-8, 0.0, 1)
    with pytest.raises(ValueError, match="step"):
        K.adamw_step(p, p.clone(), p.clone(), p.clone(), 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    with pytest.raises(ValueError, match="contiguous float32"):
        FlatAdamW([torch.nn.Parameter(torch.zeros(4, 4, device=DEV).t())])
