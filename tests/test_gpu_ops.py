"""GPU tests of the autograd surface (rus_amd.ops), mirroring solution/test_kernels.py:51-226:
each op's forward and its autograd backward against the reference test's eager formula evaluated
on the CPU (fp32 math on the same fp16/fp32 inputs), with the reference test's tolerances
(2e-3 for fp16, 1e-4 for fp32, test_kernels.py:14; lm_head loss 2e-3, dH 5e-3, argmax exact)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import ops as ref
from rus_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.float32: 1e-4}


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("has_residual", [False, True])
@pytest.mark.parametrize("shape", [(4, 128, 1536), (273, 1536)])
def test_rms_norm_autograd(dtype, has_residual, shape):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(shape, generator=g).to(dtype)
    w = torch.randn(shape[-1], generator=g).to(dtype)
    res = torch.randn(shape, generator=g).to(dtype) if has_residual else None
    gy = torch.randn(shape, generator=g).to(dtype)
    # reference formula (test_kernels.py:64-69), autograd on the CPU in fp32
    xr = x.detach().float().clone().requires_grad_(True)
    rr = res.detach().float().clone().requires_grad_(True) if has_residual else None
    h = (xr + rr).to(dtype).float() if has_residual else xr
    y_ref = w.float() * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype).float()
    y_ref.backward(gy.float())

    xd = x.to(DEV).requires_grad_(True)
    rd = res.to(DEV).requires_grad_(True) if has_residual else None
    if has_residual:
        y, hs = ops.rms_norm(xd, w.to(DEV), 1e-6, residual=rd)
        assert torch.equal(hs.cpu(), (x.float() + res.float()).to(dtype))
    else:
        y = ops.rms_norm(xd, w.to(DEV), 1e-6)
    y.backward(gy.to(DEV))
    tol = TOL[dtype]
    assert torch.allclose(y.float().cpu(), y_ref.detach(), rtol=tol, atol=tol)
    assert torch.allclose(xd.grad.float().cpu(), xr.grad, rtol=tol, atol=tol)
    if has_residual:
        assert torch.equal(rd.grad, xd.grad)  # the residual receives the same gradient


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n_tokens", [64, 311])
def test_qkv_lora_rope_autograd(dtype, n_tokens):
    g = torch.Generator().manual_seed(1)
    hq, hkv, hd = 12, 2, 128
    qd, kd = hq * hd, hkv * hd
    qkv = torch.randn(n_tokens, qd + 2 * kd, generator=g).to(dtype)
    ql = torch.randn(n_tokens, qd, generator=g).to(dtype)
    vl = torch.randn(n_tokens, kd, generator=g).to(dtype)
    cos = torch.randn(512, hd, generator=g).to(dtype)
    sin = torch.randn(512, hd, generator=g).to(dtype)
    pos = torch.randint(0, 512, (n_tokens,), generator=g)
    dq, dk, dv = (torch.randn(n_tokens, h, hd, generator=g).to(dtype) for h in (hq, hkv, hkv))

    # reference formula (test_kernels.py:111-131) with CPU autograd in fp32
    a = qkv.float().clone().requires_grad_(True)
    b = ql.float().clone().requires_grad_(True)
    c = vl.float().clone().requires_grad_(True)

    def rot_half(t):
        return torch.cat((-t[..., hd // 2:], t[..., : hd // 2]), dim=-1)

    q_ref = (a[:, :qd] + b * 2.0).view(n_tokens, hq, hd)
    k_ref = a[:, qd:qd + kd].view(n_tokens, hkv, hd)
    v_ref = (a[:, qd + kd:] + c * 2.0).view(n_tokens, hkv, hd)
    cp, sp = cos[pos].float().unsqueeze(1), sin[pos].float().unsqueeze(1)
    qr = (q_ref * cp + rot_half(q_ref) * sp).to(dtype)
    kr = (k_ref * cp + rot_half(k_ref) * sp).to(dtype)
    vr = v_ref.to(dtype)
    ((qr.float() * dq.float()).sum() + (kr.float() * dk.float()).sum()
     + (vr.float() * dv.float()).sum()).backward()

    A = qkv.to(DEV).requires_grad_(True)
    Bq = ql.to(DEV).requires_grad_(True)
    Cv = vl.to(DEV).requires_grad_(True)
    qo, ko, vo = ops.qkv_lora_rope(A, cos.to(DEV), sin.to(DEV), pos.to(DEV), q_lora=Bq, v_lora=Cv)
    ((qo.float() * dq.to(DEV).float()).sum() + (ko.float() * dk.to(DEV).float()).sum()
     + (vo.float() * dv.to(DEV).float()).sum()).backward()
    tol = TOL[dtype]
    for got, want in ((qo, qr), (ko, kr), (vo, vr), (A.grad, a.grad), (Bq.grad, b.grad), (Cv.grad, c.grad)):
        assert torch.allclose(got.float().cpu(), want.float().detach(), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("shape", [(4, 64, 8960), (3, 77, 1001)])
def test_mlp_glu_autograd(dtype, fused, shape):
    g = torch.Generator().manual_seed(2)
    gate = torch.randn(shape, generator=g).to(dtype)
    up = torch.randn(shape, generator=g).to(dtype)
    grad = torch.randn(shape, generator=g).to(dtype)
    gr, ur = gate.float().clone().requires_grad_(True), up.float().clone().requires_grad_(True)
    ref_out = F.silu(gr) * ur
    ref_out.backward(grad.float())
    if fused:
        gu = torch.cat([gate, up], dim=-1).to(DEV).requires_grad_(True)
        out = ops.mlp_glu(gu, None)
        out.backward(grad.to(DEV))
        dg, du = gu.grad[..., : shape[-1]], gu.grad[..., shape[-1]:]
    else:
        gd, ud = gate.to(DEV).requires_grad_(True), up.to(DEV).requires_grad_(True)
        out = ops.mlp_glu(gd, ud)
        out.backward(grad.to(DEV))
        dg, du = gd.grad, ud.grad
    tol = TOL[dtype]
    assert torch.allclose(out.float().cpu(), ref_out.detach(), rtol=tol, atol=tol)
    assert torch.allclose(dg.float().cpu(), gr.grad, rtol=tol, atol=tol)
    assert torch.allclose(du.float().cpu(), ur.grad, rtol=tol, atol=tol)


def test_chunked_lm_head_autograd():
    # test_kernels.py:189-226 (without the ChunkedLogitsProxy part, out of scope)
    g = torch.Generator().manual_seed(3)
    B, S, D, V = 2, 32, 256, 4099
    hidden = torch.randn(B, S, D, generator=g).half()
    weight = (torch.randn(V, D, generator=g) * 0.02).half()
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[:, :8] = -100
    shift = torch.full((B, S), -100, dtype=torch.long)
    shift[:, :-1] = labels[:, 1:]
    hr = hidden.float().clone().requires_grad_(True)
    logits = hr @ weight.float().t()
    loss_ref = F.cross_entropy(logits[:, :-1].reshape(-1, V), labels[:, 1:].reshape(-1), ignore_index=-100)
    loss_ref.backward()
    lf = logits.detach()
    ent_ref = torch.logsumexp(lf, -1) - (F.softmax(lf, -1) * lf).sum(-1)

    hd = hidden.to(DEV).requires_grad_(True)
    loss, nll, ent, amax = ops.chunked_lm_head(hd, shift.to(DEV), weight.to(DEV), v_chunk=1024)
    loss.backward()
    assert torch.allclose(loss.float().cpu(), loss_ref.detach(), rtol=2e-3, atol=2e-3)
    assert torch.allclose(hd.grad.float().cpu(), hr.grad, rtol=5e-3, atol=5e-3)
    assert torch.allclose(ent.view(B, S).cpu(), ent_ref, rtol=2e-3, atol=2e-3)
    z16 = ref.lm_head_logits(hidden.view(-1, D), weight)
    top2 = z16.topk(2, dim=-1).values
    near_tie = (top2[:, 0] - top2[:, 1]) <= ref.fp16_ulp(top2[:, 0])
    assert torch.all((amax.cpu() == z16.argmax(-1)) | near_tie)
    # backward scales by the incoming gradient on the device (no host read of grad_loss)
    hd.grad = None
    loss2, *_ = ops.chunked_lm_head(hd, shift.to(DEV), weight.to(DEV))
    (3.0 * loss2).backward()
    assert torch.allclose(hd.grad.float().cpu(), 3.0 * hr.grad, rtol=5e-3, atol=5e-3)
