"""GPU parity of the gfx950 bandwidth kernels against the CPU oracle (oracle/ops.py).

Case matrix follows the reference's kernel tests (solution/test_kernels.py:21-182) plus the
BASELINE shapes: NF4 dequant bit-exact in fp16 (single, fused 2/3-segment, unaligned super-blocks,
odd tails); RMSNorm / RoPE / SwiGLU within one fp16 ulp (tolerance written per test) and, where the
kernel uses the same correctly-rounded ops as the oracle, bit-exact.
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


def _ulp_ok(got: torch.Tensor, want: torch.Tensor, ulps: float = 1.0) -> torch.Tensor:
    """|got - want| <= ulps fp16 ulp(want), elementwise (float32 view of fp16 values)."""
    return (got.float() - want.float()).abs() <= ulps * ref.fp16_ulp(want.float())


# ---------------------------------------------------------------------------------------------
# NF4 dequant: bit-exact
# ---------------------------------------------------------------------------------------------


def _dequant_gpu(q: quant.NF4Weight, offs=None, splits=None, bases=None):
    return K.dequant_nf4_tensor(q.packed.to(DEV), q.absmax.to(DEV), q.code2.to(DEV),
                                q.absmax2.to(DEV), q.offset if offs is None else offs, q.shape,
                                split_bytes=splits, blocksize=q.blocksize,
                                super_blocksize=q.super_blocksize, absmax2_bases=bases)


def _dequant_ref(q: quant.NF4Weight, offs=None, splits=None, bases=None):
    return ref.nf4_dequant(q.packed.numpy(), q.absmax.numpy(), q.code2.numpy(), q.absmax2.numpy(),
                           q.offset if offs is None else offs, q.shape, split_bytes=splits,
                           blocksize=q.blocksize, super_blocksize=q.super_blocksize,
                           absmax2_bases=bases)


def _bits_equal(gpu: torch.Tensor, cpu: np.ndarray) -> bool:
    g = gpu.cpu().numpy().view(np.uint16)
    return np.array_equal(g, cpu.view(np.uint16))


@pytest.mark.parametrize("shape", [(1536, 1536), (2048, 1536), (8960, 1536), (3, 70), (1, 10), (5, 64)])
def test_nf4_dequant_bit_exact(shape):
    g = torch.Generator().manual_seed(42)
    w = (torch.randn(shape, generator=g) * 0.02).half()
    q = quant.quantize_nf4(w)
    out = _dequant_gpu(q)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and tuple(out.shape) == shape
    assert _bits_equal(out, _dequant_ref(q))


def test_nf4_dequant_fused_qkv_and_gu_bit_exact():
    g = torch.Generator().manual_seed(0)
    mk = lambda r, c: quant.quantize_nf4((torch.randn(r, c, generator=g) * 0.02).half())
    for parts in ([mk(1536, 1536), mk(256, 1536), mk(256, 1536)], [mk(8960, 1536), mk(8960, 1536)]):
        fused, splits, offs, bases = quant.concat_segments(parts)
        out = _dequant_gpu(fused, offs, splits, bases)
        torch.cuda.synchronize()
        assert _bits_equal(out, _dequant_ref(fused, offs, splits, bases))
        sep = np.concatenate([_dequant_ref(p) for p in parts])
        assert _bits_equal(out, sep)


def test_nf4_dequant_unaligned_super_blocks_and_out_buf():
    # Segment block counts (96*... ) that are not multiples of 256: per-segment absmax2 bases.
    g = torch.Generator().manual_seed(3)
    parts = [quant.quantize_nf4((torch.randn(r, 128, generator=g) * 0.02).half()) for r in (200, 72, 136)]
    fused, splits, offs, bases = quant.concat_segments(parts)
    ws = torch.full((fused.shape[0] * fused.shape[1] + 100,), 7.0, dtype=torch.float16, device=DEV)
    out = K.dequant_nf4_tensor(fused.packed.to(DEV), fused.absmax.to(DEV), fused.code2.to(DEV),
                               fused.absmax2.to(DEV), offs, fused.shape, out_buf=ws,
                               split_bytes=splits, absmax2_bases=bases)
    torch.cuda.synchronize()
    assert out.data_ptr() == ws.data_ptr()
    assert _bits_equal(out, np.concatenate([_dequant_ref(p) for p in parts]))
    assert torch.all(ws[fused.shape[0] * fused.shape[1]:] == 7.0)  # nothing written past the view


def test_nf4_dequant_segments_one_launch_bit_exact():
    # One launch over a layer's four segments ([q|k|v], o, [gate|up], down shapes at reduced width,
    # plus ragged ones), each into its own guarded buffer; must equal the per-segment oracle.
    g = torch.Generator().manual_seed(5)
    mk = lambda r, c: quant.quantize_nf4((torch.randn(r, c, generator=g) * 0.02).half())
    layer = [[mk(384, 256), mk(64, 256), mk(64, 256)], [mk(384, 384)], [mk(1000, 256), mk(1000, 256)],
             [mk(256, 1000)]]
    ragged = [[mk(3, 70)], [mk(200, 128), mk(72, 128), mk(136, 128)], [mk(1, 10)]]
    for segs in (layer, ragged):
        jobs, refs, bufs = [], [], []
        for parts in segs:
            fused, splits, offs, bases = quant.concat_segments(parts)
            n = fused.shape[0] * fused.shape[1]
            buf = torch.full((n + 64,), 7.0, dtype=torch.float16, device=DEV)
            bufs.append((buf, n))
            jobs.append({"packed": fused.packed.to(DEV), "absmax": fused.absmax.to(DEV),
                         "absmax2": fused.absmax2.to(DEV), "offset": offs, "out_shape": fused.shape,
                         "out_buf": buf, "split_bytes": splits, "absmax2_bases": bases})
            refs.append(np.concatenate([_dequant_ref(p) for p in parts]))
        outs = K.dequant_nf4_segments(jobs, segs[0][0].code2.to(DEV))
        torch.cuda.synchronize()
        for out, want, (buf, n) in zip(outs, refs, bufs):
            assert out.data_ptr() == buf.data_ptr()
            assert _bits_equal(out, want)
            assert torch.all(buf[n:] == 7.0)


@pytest.mark.parametrize("kind", ["fwd", "fwd_res", "bwd", "bwd_dres"])
@pytest.mark.parametrize("wdtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(707, 1536), (5, 896), (130, 2048), (33, 512)])
def test_dequant_with_riding_norm_equals_separate_launches(kind, wdtype, shape):
    # A deferred RMSNorm carried by the dequant launch writes exactly what its own launch writes,
    # and the weights are unchanged (bit-exact; the rows and the decode run the same code).
    g = torch.Generator().manual_seed(shape[0] + len(kind))
    n, d = shape
    q = quant.quantize_nf4((torch.randn(384, 256, generator=g) * 0.02).half())
    job = lambda buf: {"packed": q.packed.to(DEV), "absmax": q.absmax.to(DEV),
                       "absmax2": q.absmax2.to(DEV), "offset": q.offset, "out_shape": q.shape,
                       "out_buf": buf}
    x = torch.randn(shape, generator=g).half().to(DEV)
    other = torch.randn(shape, generator=g).half().to(DEV)
    w = (1 + 0.05 * torch.randn(d, generator=g)).to(wdtype).to(DEV)
    code2 = q.code2.to(DEV)
    if kind.startswith("fwd"):
        res = other if kind == "fwd_res" else None
        want = K.rms_norm_fwd(x, w, 1e-6, residual=res)
        *got, pend = K.rms_norm_fwd(x, w, 1e-6, residual=res, defer=True)
    else:
        _, h, rstd = K.rms_norm_fwd(other, w, 1e-6)
        dres = torch.randn(shape, generator=g).half().to(DEV) if kind == "bwd_dres" else None
        want = [K.rms_norm_bwd(x, h, w, rstd, dresidual=dres)]
        dx, pend = K.rms_norm_bwd(x, h, w, rstd, dresidual=dres, defer=True)
        got = [dx]
    assert pend.side is not None and not pend.done
    w_buf = torch.empty(q.shape[0] * q.shape[1], dtype=torch.float16, device=DEV)
    (w_out,) = K.dequant_nf4_segments([job(w_buf)], code2, norm=pend)
    assert pend.done
    pend.run()  # already enqueued: no second launch
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    assert _bits_equal(w_out, _dequant_ref(q))


def test_nf4_dequant_rejects_short_absmax():
    q = quant.quantize_nf4(torch.randn(64, 64).half())
    with pytest.raises(RuntimeError, match="absmax"):
        K.dequant_nf4_tensor(q.packed.to(DEV), q.absmax[:-1].to(DEV), q.code2.to(DEV),
                             q.absmax2.to(DEV), q.offset, q.shape)


# ---------------------------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("wdtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("has_residual", [False, True])
@pytest.mark.parametrize("shape", [(4, 128, 1536), (273, 1536), (880, 1536), (7, 1001), (5000, 896),
                                   (3, 8960)])
def test_rmsnorm_fwd_bwd(dtype, wdtype, has_residual, shape):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(shape, generator=g).to(dtype)
    res = torch.randn(shape, generator=g).to(dtype) if has_residual else None
    w = (1 + 0.05 * torch.randn(shape[-1], generator=g)).to(wdtype)
    dy = torch.randn(shape, generator=g).to(dtype)
    dres = torch.randn(shape, generator=g).to(dtype) if has_residual else None

    y, h, rstd = K.rms_norm_fwd(x.to(DEV), w.to(DEV), 1e-6, residual=None if res is None else res.to(DEV))
    dx = K.rms_norm_bwd(dy.to(DEV), h, w.to(DEV), rstd, dresidual=None if dres is None else dres.to(DEV))
    torch.cuda.synchronize()
    y_r, h_r, rstd_r = ref.rms_norm_fwd(x, w, 1e-6, residual=res)
    dx_r = ref.rms_norm_bwd(dy, h_r, w, rstd_r, dresidual=dres)

    assert torch.equal(h.cpu(), h_r)  # T(x + res): one correctly rounded add, exact
    assert torch.allclose(rstd.cpu(), rstd_r.reshape(-1), rtol=2e-6, atol=0)  # fp32 sum order only
    if dtype == torch.float16:
        # y = T(T(h*rstd) * w) rounds to fp16 twice; rstd may differ in its last fp32 bit (sum
        # order), so allow one fp16 ulp at each rounding: ulp(y) + ulp(T(h*rstd)) * |w|.
        n_r = (h_r.float() * rstd_r.unsqueeze(-1)).half().float()
        tol_y = ref.fp16_ulp(y_r) + ref.fp16_ulp(n_r) * w.float().abs()
        assert torch.all((y.cpu().float() - y_r.float()).abs() <= tol_y)
        assert (y.cpu() == y_r).float().mean() > 0.99  # and nearly all bit-exact
        # dx = T((g - xhat*c)*rstd + dres): one fp16 ulp plus an fp32 budget for the reduction
        # order of c under cancellation (1e-5 relative to the terms being cancelled).
        xh = h_r.float() * rstd_r.unsqueeze(-1)
        gw = w.float() * dy.float()
        c = (xh * gw).sum(-1, keepdim=True) / shape[-1]
        tol_dx = ref.fp16_ulp(dx_r) + 1e-5 * rstd_r.unsqueeze(-1) * (gw.abs() + (xh * c).abs())
        assert torch.all((dx.cpu().float() - dx_r.float()).abs() <= tol_dx)
        assert (dx.cpu() == dx_r).float().mean() > 0.98
    else:
        assert torch.allclose(y.cpu(), y_r, rtol=1e-5, atol=1e-6)
        assert torch.allclose(dx.cpu(), dx_r, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("wdtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n_parts", [1, 3, 4, 8, 11, 35])
@pytest.mark.parametrize("has_residual", [False, True])
@pytest.mark.parametrize("shape", [(707, 1536), (5, 896)])
def test_rmsnorm_bwd_over_split_partials_equals_reduce_then_bwd(wdtype, n_parts, has_residual,
                                                                shape):
    # dy = fp16(sum of fp32 partials in part order) formed inside the norm backward must equal,
    # bit for bit, the separate reduce kernel followed by rms_norm_bwd.
    g = torch.Generator().manual_seed(n_parts)
    n, d = shape
    x = torch.randn(shape, generator=g).half().to(DEV)
    w = (1 + 0.05 * torch.randn(d, generator=g)).to(wdtype).to(DEV)
    parts = (torch.randn((n_parts, n, d), generator=g) * 3).to(DEV)
    dres = torch.randn(shape, generator=g).half().to(DEV) if has_residual else None
    _, h, rstd = K.rms_norm_fwd(x, w, 1e-6)
    want = K.rms_norm_bwd(K.sum_splits(parts), h, w, rstd, dresidual=dres)
    got = K.rms_norm_bwd_parts(parts, h, w, rstd, dresidual=dres)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------------------------
# LoRA + RoPE
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n_tokens", [64, 311, 761])
@pytest.mark.parametrize("tables", ["random", "qwen"])
def test_rope_fwd_bwd_bit_exact(dtype, n_tokens, tables):
    hq, hkv, d = 12, 2, 128
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(n_tokens, (hq + 2 * hkv) * d, generator=g).to(dtype)
    ql = torch.randn(n_tokens, hq * d, generator=g).to(dtype)
    vl = torch.randn(n_tokens, hkv * d, generator=g).to(dtype)
    if tables == "random":  # the reference test's tables: cos/sin halves differ
        cos = torch.randn(512, d, generator=g).to(dtype)
        sin = torch.randn(512, d, generator=g).to(dtype)
    else:
        cos, sin = ref.rope_tables(2048, d, 1e6, dtype)
    pos = torch.randint(0, cos.shape[0], (n_tokens,), generator=g)
    dq = torch.randn(n_tokens, hq, d, generator=g).to(dtype)
    dk = torch.randn(n_tokens, hkv, d, generator=g).to(dtype)
    dv = torch.randn(n_tokens, hkv, d, generator=g).to(dtype)

    args = (cos.to(DEV), sin.to(DEV), pos.to(DEV))
    q, k, v = K.qkv_rope_fwd(qkv.to(DEV), *args, q_lora=ql.to(DEV), v_lora=vl.to(DEV),
                             scale_q=2.0, scale_v=2.0)
    q0, k0, v0 = K.qkv_rope_fwd(qkv.to(DEV), *args)
    dqkv = K.qkv_rope_bwd(dq.to(DEV), dk.to(DEV), dv.to(DEV), *args)
    dqkv2, dql, dvl = K.qkv_rope_bwd_lora(dq.to(DEV), dk.to(DEV), dv.to(DEV), *args, 2.0, 0.5)
    torch.cuda.synchronize()

    q_r, k_r, v_r = ref.qkv_rope_fwd(qkv, cos, sin, pos, ql, vl, 2.0, 2.0)
    q0_r, k0_r, v0_r = ref.qkv_rope_fwd(qkv, cos, sin, pos)
    dqkv_r, dql_r, dvl_r = ref.qkv_rope_bwd(dq, dk, dv, cos, sin, pos, scale_q=2.0, scale_v=0.5)
    # Same separately-rounded fp32 products and sums on both sides: bit-exact.
    for got, want in ((q, q_r), (k, k_r), (v, v_r), (q0, q0_r), (k0, k0_r), (v0, v0_r),
                      (dqkv, dqkv_r), (dqkv2, dqkv_r), (dql, dql_r), (dvl, dvl_r)):
        assert torch.equal(got.cpu(), want)


def test_rope_out_of_range_position_is_clamped_and_flagged():
    from rus_amd import _lib

    n, d = 8, 128
    qkv = torch.randn(n, 16 * d, device=DEV).half()
    cos, sin = ref.rope_tables(16, d, 1e6, torch.float16)
    cos, sin = cos.to(DEV), sin.to(DEV)
    pos = torch.tensor([0, 1, 2, 3, 4, 5, 6, 99], device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    q = torch.empty(n, 12, d, device=DEV, dtype=torch.float16)
    k = torch.empty(n, 2, d, device=DEV, dtype=torch.float16)
    v = torch.empty(n, 2, d, device=DEV, dtype=torch.float16)
    _lib.call("rus_qkv_lora_rope_fwd", qkv.data_ptr(), None, None, cos.data_ptr(), sin.data_ptr(),
              pos.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), n, qkv.stride(0), 0, 0,
              cos.stride(0), cos.shape[0], 2.0, 2.0, 12, 2, d, flag.data_ptr(), 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    q_r, _, _ = ref.qkv_rope_fwd(qkv.cpu(), cos.cpu(), sin.cpu(), torch.tensor([0, 1, 2, 3, 4, 5, 6, 15]))
    assert torch.equal(q.cpu(), q_r)


# ---------------------------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("shape", [(4, 64, 8960), (3, 77, 1001), (880, 8960)])
def test_swiglu_fwd_bwd(dtype, fused, shape):
    g = torch.Generator().manual_seed(2)
    gate = torch.randn(shape, generator=g).to(dtype)
    up = torch.randn(shape, generator=g).to(dtype)
    dout = torch.randn(shape, generator=g).to(dtype)
    out_r = ref.swiglu_fwd(gate, up)
    dg_r, du_r = ref.swiglu_bwd(dout, gate, up)
    if fused:
        gu = torch.cat([gate, up], dim=-1).to(DEV)
        out = K.mlp_glu_fwd(gu)
        dgu = torch.empty_like(gu)
        K.mlp_glu_bwd(dout.to(DEV), gu, None, dgu_out=dgu)
        K.mlp_glu_bwd(dout.to(DEV), gu)  # in place over gu
        torch.cuda.synchronize()
        n = shape[-1]
        dg, du = dgu[..., :n].cpu(), dgu[..., n:].cpu()
        assert torch.equal(gu.cpu(), dgu.cpu())  # in place == out of place
    else:
        out = K.mlp_glu_fwd(gate.to(DEV), up.to(DEV))
        dg, du = K.mlp_glu_bwd(dout.to(DEV), gate.to(DEV), up.to(DEV))
        torch.cuda.synchronize()
        dg, du = dg.cpu(), du.cpu()
    out = out.cpu()
    if dtype == torch.float16:
        # hardware exp2/rcp (~1 fp32 ulp) against the oracle's exp and divide: 1 fp16 ulp.
        assert torch.all(_ulp_ok(out, out_r))
        assert torch.all(_ulp_ok(dg, dg_r))
        assert torch.all(_ulp_ok(du, du_r))
    else:
        assert torch.allclose(out, out_r, rtol=1e-5, atol=1e-6)
        assert torch.allclose(dg, dg_r, rtol=1e-5, atol=1e-6)
        assert torch.allclose(du, du_r, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# LoRA-input dropout: bit-exact against the oracle's Philox masks
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("shape,strided", [((311, 1536), False), ((77, 1001), False), ((64, 256), True)])
def test_lora_dropout_fwd_bwd_bit_exact(dtype, shape, strided):
    g = torch.Generator().manual_seed(9)
    n, c = shape
    seed_v, sa, sb, pa, pb = 123456789, 6, 7, 0.05, 0.1
    x = torch.randn(n, c, generator=g).to(dtype)
    acc, ga, gb = (torch.randn(n, c, generator=g).to(dtype) for _ in range(3))
    seed = torch.tensor([seed_v], dtype=torch.int64, device=DEV)
    xd = x.to(DEV)
    if strided:  # rows of a wider buffer (the vector path needs 8-aligned strides)
        xd = torch.zeros(n, c + 64, dtype=dtype, device=DEV)[:, :c]
        xd.copy_(x.to(DEV))
    a, b = K.lora_dropout_fwd(xd, seed, sa, sb, pa, pb)
    wa, wb = ref.lora_dropout_fwd(x, seed_v, sa, sb, pa, pb)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), wa) and torch.equal(b.cpu(), wb)
    accd = acc.to(DEV)
    K.lora_dropout_bwd_add(accd, ga.to(DEV), gb.to(DEV), seed, sa, sb, pa, pb)
    torch.cuda.synchronize()
    assert torch.equal(accd.cpu(), ref.lora_dropout_bwd_add(acc, ga, gb, seed_v, sa, sb, pa, pb))
    # the kernel reads the seed from device memory on every launch
    seed.fill_(seed_v + 1)
    a2, _ = K.lora_dropout_fwd(xd, seed, sa, sb, pa, pb)
    torch.cuda.synchronize()
    assert torch.equal(a2.cpu(), ref.lora_dropout_fwd(x, seed_v + 1, sa, sb, pa, pb)[0])


@pytest.mark.parametrize("blocksize", [16, 32, 64])
@pytest.mark.parametrize("offset_bytes", [0, 4])
@pytest.mark.parametrize("shape", [(3, 1002), (2, 4098)])
def test_nf4_dequant_table_and_direct_paths_bit_exact(blocksize, offset_bytes, shape):
    # blocksize >= 32 takes the path with an LDS table of NF4 x scale per absmax block,
    # blocksize 16 the direct one; packed views 4 bytes into their allocation. 3 x 1002
    # elements leave a ragged tail past the last 4-byte unit; 2 x 4098 (4098 packed bytes) put
    # that tail just past the first 4 KiB block, in an absmax block of its own.
    g = torch.Generator().manual_seed(blocksize + offset_bytes)
    w = (torch.randn(*shape, generator=g) * 0.02).half()
    q = quant.quantize_nf4(w, blocksize=blocksize)
    packed = torch.zeros(q.packed.numel() + offset_bytes, dtype=torch.uint8, device=DEV)
    packed[offset_bytes:].copy_(q.packed.reshape(-1).to(DEV))
    out = K.dequant_nf4_tensor(packed[offset_bytes:], q.absmax.to(DEV), q.code2.to(DEV),
                               q.absmax2.to(DEV), q.offset, q.shape, blocksize=q.blocksize,
                               super_blocksize=q.super_blocksize)
    torch.cuda.synchronize()
    assert _bits_equal(out, _dequant_ref(q))


def test_gather_rows_from_host_and_transpose():
    # Embedding rows read over the bus by a kernel (ids on the device; no host synchronisation):
    # exact copies, zero rows and the error flag for ids out of range.
    g = torch.Generator().manual_seed(11)
    w = torch.randn(1000, 264, generator=g).half().pin_memory()
    ids = torch.randint(0, 1000, (77,), generator=g)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = K.gather_rows_from_host(w, ids.to("cuda"), err_flag=flag)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), w[ids]) and int(flag.item()) == 0
    bad = ids.clone()
    bad[5], bad[9] = -1, 1000
    out = K.gather_rows_from_host(w, bad.to("cuda"), err_flag=flag)
    torch.cuda.synchronize()
    want = w[ids].clone()
    want[5] = 0
    want[9] = 0
    assert torch.equal(out.cpu(), want) and int(flag.item()) == 1
    # W^T on the device: exact transpose, zero padding columns
    for n, d in ((1000, 264), (64, 128), (4099, 256)):
        src = torch.randn(n, d, generator=g).half().cuda()
        dst = torch.full((d, n + 70), 3.0, dtype=torch.float16, device="cuda")
        K.transpose_rows(src, dst)
        torch.cuda.synchronize()
        assert torch.equal(dst[:, :n].cpu(), src.cpu().t())
        assert torch.all(dst[:, n:].cpu() == 0)
