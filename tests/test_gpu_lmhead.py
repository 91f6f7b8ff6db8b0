"""GPU parity of the vocab-tiled lm_head cross-entropy (fp16 MFMA) against the CPU oracle.

Cases follow solution/test_kernels.py:189-226 (B=2, S=32, D=256, V=4099, chunk 1024, masked
prompt labels) plus the BASELINE config 2 shape (N=2048, D=1536, V=151936, 10% labels -100),
whose per-token results, hidden gradient and loss are checked against the oracle for every
token.

Tolerances (written per assertion): loss / entropy / lse within 1e-3 absolute; nll within 1e-3
plus one fp16 ulp of the target logit (the fp32 accumulation order of an MFMA differs from the
CPU GEMM, so the fp16 rounding of a logit can land one ulp apart); argmax equal except where the
oracle's top two fp16 logits are within one ulp; hidden gradient within rtol 1e-2.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ops as ref
from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_against_oracle(h, w, labels, out, rows=None, denom=None, check_dh=True):
    nll, lse, ent, amax, dn, dh_pre = out[:6]
    rows = torch.arange(h.shape[0]) if rows is None else rows
    o = ref.lm_head_ce(h[rows], w, labels[rows], num_items_in_batch=denom, v_chunk=16384,
                       need_grad=check_dh)
    lse_g, ent_g, nll_g = lse.cpu()[rows], ent.cpu()[rows], nll.cpu()[rows]
    assert torch.all((lse_g - o["lse"]).abs() <= 1e-3)
    assert torch.all((ent_g - o["entropy"]).abs() <= 1e-3)
    lab = labels[rows]
    tgt_ulp = torch.zeros_like(o["nll"])
    valid = lab != -100
    if valid.any():
        z_t = (h[rows][valid].float() * w[lab[valid]].float()).sum(-1).half().float()
        tgt_ulp[valid] = ref.fp16_ulp(z_t)
    assert torch.all((nll_g - o["nll"]).abs() <= 1e-3 + tgt_ulp)
    # argmax: exact unless the oracle's top-2 fp16 logits are within one ulp of each other.
    z = ref.lm_head_logits(h[rows], w)
    top2 = z.topk(2, dim=-1).values
    near_tie = (top2[:, 0] - top2[:, 1]) <= ref.fp16_ulp(top2[:, 0])
    am = amax.cpu()[rows]
    assert torch.all((am == o["argmax"]) | near_tie)
    assert torch.all(z.gather(1, am[:, None]).squeeze(1) >= top2[:, 0] - ref.fp16_ulp(top2[:, 0]))
    if check_dh:
        dh = K.lm_head_dh_reduce(dh_pre.unsqueeze(0), 1.0 / 65536.0, torch.float16).cpu()[rows]
        want = o["dh"].float()
        scale = want.abs().max().item() + 1e-12
        assert torch.allclose(dh.float(), want, rtol=1e-2, atol=1e-2 * scale)
    return o


@pytest.mark.parametrize("v_chunk", [None, 1024])
def test_lmhead_reference_case(v_chunk):
    # solution/test_kernels.py:192-220: B=2, S=32, D=256, V=4099, chunk 1024, 8 masked labels/row.
    g = torch.Generator().manual_seed(3)
    B, S, D, V = 2, 32, 256, 4099
    hidden = torch.randn(B, S, D, generator=g).half()
    weight = (torch.randn(V, D, generator=g) * 0.02).half()
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[:, :8] = -100
    shift = torch.full((B, S), -100, dtype=torch.long)
    shift[:, :-1] = labels[:, 1:]
    h2, lab = hidden.view(-1, D), shift.view(-1)
    out = K.lm_head_ce(h2.to(DEV), weight.to(DEV), lab.to(DEV), v_chunk=v_chunk)
    torch.cuda.synchronize()
    o = _check_against_oracle(h2, weight, lab, out)
    loss = out[0].sum().cpu() / out[4].cpu()
    assert abs(float(loss) - float(o["loss"])) <= 1e-3
    assert abs(float(out[6].cpu()) - float(loss)) <= 1e-6 * abs(float(loss))  # device loss kernel
    # Full-logit library reference, as the reference test does (test_kernels.py:203-217).
    z = h2.float() @ weight.float().t()
    loss_lib = torch.nn.functional.cross_entropy(z, lab, ignore_index=-100)
    assert abs(float(loss) - float(loss_lib)) <= 2e-3


@pytest.mark.parametrize("v_chunk", [None, 8192])
def test_lmhead_unpadded_vocab_chunked(v_chunk):
    g = torch.Generator().manual_seed(4)
    N, D, V = 777, 1536, 32901  # V not a multiple of 64: padded K in the gradient GEMM
    h = torch.randn(N, D, generator=g).half()
    w = (torch.randn(V, D, generator=g) * 0.02).half()
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < 0.1] = -100
    lab[-1] = V - 1
    out = K.lm_head_ce(h.to(DEV), w.to(DEV), lab.to(DEV), v_chunk=v_chunk)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, 64), torch.tensor([N - 1])])
    denom = float(out[4].item())
    _check_against_oracle(h, w, lab, out, rows=rows, denom=denom)


def test_lmhead_baseline_config2_all_tokens():
    # H [2048,1536] ~ N(0,1), W [151936,1536] ~ N(0,0.02), 10% labels -100:
    # every token's statistics and hidden-gradient row against the oracle, and the loss.
    g = torch.Generator().manual_seed(0)
    N, D, V = 2048, 1536, 151936
    h = torch.randn(N, D, generator=g).half()
    w = (torch.randn(V, D, generator=g) * 0.02).half()
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < 0.1] = -100
    out = K.lm_head_ce(h.to(DEV), w.to(DEV), lab.to(DEV))
    torch.cuda.synchronize()
    denom = float(out[4].item())
    assert denom == float((lab != -100).sum())
    o = _check_against_oracle(h, w, lab, out, denom=denom)
    assert abs(float(out[6].cpu()) - float(o["loss"])) <= 1e-3
    nll = out[0].cpu()
    assert torch.all(nll[lab == -100] == 0)
    # size-independent invariants over every token: 0 <= H <= ln V, lse >= max logit.
    ent = out[2].cpu()
    assert torch.all(ent >= -1e-4) and torch.all(ent <= torch.log(torch.tensor(float(V))) + 1e-4)


def test_lmhead_token_block_size_leaves_the_statistics_unchanged():
    # 1100 tokens in five 256-token blocks and in two (768 + 332, the default for a small
    # vocabulary, which allows any block size but never one block for all tokens):
    # each token's logits, statistics and argmax are formed from its own row alone, so they are
    # bit-identical; the hidden gradient's split-K sum order follows the block's split count, so
    # it agrees within rtol 1e-3 and both match the oracle on a sample of tokens.
    g = torch.Generator().manual_seed(11)
    N, D, V = 1100, 256, 5000
    h = torch.randn(N, D, generator=g).half()
    w = (torch.randn(V, D, generator=g) * 0.05).half()
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < 0.1] = -100
    assert K.lm_head_token_blocks(N, K.lm_head_block_tokens(V)) == [(0, 768), (768, N)]
    two = K.lm_head_ce(h.to(DEV), w.to(DEV), lab.to(DEV))
    five = K.lm_head_ce(h.to(DEV), w.to(DEV), lab.to(DEV), block_tokens=256)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 3, 4, 6):
        assert torch.equal(two[i].cpu(), five[i].cpu()), i
    assert torch.allclose(two[5].cpu(), five[5].cpu(), rtol=1e-3, atol=1e-3 * two[5].abs().max().item())
    rows = torch.cat([torch.arange(0, 20), torch.arange(760, 780), torch.arange(1080, 1100)])
    _check_against_oracle(h, w, lab, two, rows=rows, denom=float(two[4].item()))
    _check_against_oracle(h, w, lab, five, rows=rows, denom=float(five[4].item()))


def test_lmhead_all_masked_and_ties():
    N, D, V = 8, 64, 700
    h = torch.ones(N, D).half()
    w = torch.zeros(V, D).half()
    w[3] = 0.01
    w[600] = 0.01  # tie between index 3 and 600 (different 256-row partials)
    lab = torch.full((N,), -100, dtype=torch.long)
    nll, lse, ent, amax, denom, dh_pre, loss = K.lm_head_ce(h.to(DEV), w.to(DEV), lab.to(DEV))
    torch.cuda.synchronize()
    assert float(denom.item()) == 1.0 and float(loss.item()) == 0.0
    assert torch.all(nll.cpu() == 0)
    assert torch.all(amax.cpu() == 3)
    assert torch.all(dh_pre.cpu() == 0)


def test_lmhead_num_items_in_batch_scales_gradient():
    g = torch.Generator().manual_seed(5)
    N, D, V = 100, 128, 1000
    h = torch.randn(N, D, generator=g).half().to(DEV)
    w = (torch.randn(V, D, generator=g) * 0.05).half().to(DEV)
    lab = torch.randint(0, V, (N,), generator=g).to(DEV)
    a = K.lm_head_ce(h, w, lab)
    b = K.lm_head_ce(h, w, lab, num_items_in_batch=2 * N)
    torch.cuda.synchronize()
    assert float(a[4].item()) == N and float(b[4].item()) == 2 * N
    assert torch.allclose(a[5].cpu() * 0.5, b[5].cpu(), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("n,d,v,start", [(37, 128, 1031, 0), (300, 256, 4099, 0), (64, 64, 700, 256)])
def test_kept_logits_gradient_equals_recomputed_gradient(n, d, v, start):
    # Single-pass head: the statistics pass keeps its fp16 logits in the gradient buffer and the
    # elementwise pass turns them into the gradient; both must give the bits of the recompute
    # GEMM's epilogue. Ragged vocabulary (v % 64 != 0), masked labels, labels outside the range.
    g = torch.Generator().manual_seed(n + v)
    h = torch.randn(n, d, generator=g).half()
    w = (torch.randn(start + v, d, generator=g) * 0.05).half()
    lab = torch.randint(0, start + v, (n,), generator=g)
    lab[torch.rand(n, generator=g) < 0.2] = -100
    hd, wd, ld = h.to(DEV), w[start:].to(DEV), lab.to(DEV)
    kp = (v + 63) // 64 * 64
    parts = K.LMHeadPartials(start // 256 + K.lm_head_num_parts(v), n, DEV)
    parts.m.fill_(-float("inf"))
    parts.s.zero_()
    parts.w.zero_()
    parts.idx.fill_(0)
    tgt_a = torch.zeros(n, dtype=torch.float32, device=DEV)
    tgt_b = torch.zeros(n, dtype=torch.float32, device=DEV)
    z = torch.full((n, kp + 64), 7.0, dtype=torch.float16, device=DEV)  # stride > kp
    K.lm_head_ce_fwd_chunk(hd, wd, ld, start, parts, tgt_a, logits_out=z[:, :kp])
    m_keep = parts.m.clone()
    K.lm_head_ce_fwd_chunk(hd, wd, ld, start, parts, tgt_b)
    torch.cuda.synchronize()
    assert torch.equal(m_keep, parts.m) and torch.equal(tgt_a, tgt_b)
    zc = z.cpu()
    assert torch.all(zc[:, v:kp] == 0) and torch.all(zc[:, kp:] == 7.0)
    # the kept logits are fp16(H.W^T) of an fp32 accumulation: the two fp32 sums differ by at
    # most d * 2^-24 * sum|h_i w_i| (summation order), then each rounds to fp16 (an ulp apart at
    # most, taken at the larger binade)
    want = (h.float() @ w[start:].float().T).half().float()
    acc_err = d * 2.0 ** -24 * (h.abs().float() @ w[start:].abs().float().T)
    assert torch.all((zc[:, :v].float() - want).abs() <= 2 * ref.fp16_ulp(want) + acc_err)
    lse = torch.randn(n, generator=g).abs().to(DEV) + zc[:, :v].float().amax(1).to(DEV)
    denom = torch.tensor([float((lab != -100).sum())], dtype=torch.float32, device=DEV)
    g_ref = torch.empty((n, kp), dtype=torch.float16, device=DEV)
    K.lm_head_ce_grad_logits(hd, wd, ld, lse, denom, start, g_ref)
    K.lm_head_ce_grad_from_logits(z[:, :kp], ld, lse, denom, v, start)
    torch.cuda.synchronize()
    assert torch.equal(z[:, :kp].cpu(), g_ref.cpu())
    assert torch.all(z[:, kp:].cpu() == 7.0)


@pytest.mark.parametrize("n,d,v,chunk", [(300, 256, 5000, 1024), (700, 1536, 20000, 8192)])
def test_single_pass_head_chunking_and_streaming(n, d, v, chunk):
    # The single-pass head over different vocabulary chunkings: statistics bit-identical (the
    # per-256-row partials do not depend on the chunking), hidden gradient within rtol 1e-2 of the
    # oracle. A HostHead streamed from pinned host memory with the same chunk gives the resident
    # head's bits, including the gradient; back-to-back calls without the gradient (which leave a
    # streamed slot's last reader to the next call's prefetch) and with it, on fresh inputs.
    from rus_amd import ops
    from rus_amd.hostload import HostHead

    g = torch.Generator().manual_seed(n + v)
    w = (torch.randn(v, d, generator=g) * 0.03).half()
    lab = torch.randint(0, v, (n,), generator=g)
    lab[torch.rand(n, generator=g) < 0.1] = -100
    lab[0] = v - 1  # a label in the last (partial) chunk
    labd = lab.to(DEV)
    streamed = HostHead(w, DEV, v_chunk=chunk, resident=False)
    resident = HostHead(w, DEV, v_chunk=chunk, resident=True)
    for step, need_grad in enumerate((False, False, True, True, False)):
        h = torch.randn(n, d, generator=g).half()
        outs = []
        for head in (streamed, resident):
            hd = h.to(DEV).requires_grad_(need_grad)
            with torch.set_grad_enabled(need_grad):
                loss, nll, ent, amax = ops.chunked_lm_head(hd, labd, head, v_chunk=chunk)
            if need_grad:
                loss.backward()
            torch.cuda.synchronize()
            outs.append((loss.detach().cpu(), nll.cpu(), ent.cpu(), amax.cpu(),
                         hd.grad.cpu() if need_grad else None))
        for a, b in zip(outs[0][:4], outs[1][:4]):
            assert torch.equal(a, b), step
        if need_grad:
            assert torch.equal(outs[0][4], outs[1][4]), step
    # the last gradient against the oracle; other chunkings agree on the statistics bitwise
    out = K.lm_head_ce(h.to(DEV), w.to(DEV), labd, v_chunk=chunk)
    auto = K.lm_head_ce(h.to(DEV), w.to(DEV), labd)
    torch.cuda.synchronize()
    # the token-blocked default forms the statistics per row (another fp32 summation order):
    # same argmax, lse / nll / entropy / loss within a few fp32 ulps of the chunked pass
    assert torch.equal(out[3].cpu(), auto[3].cpu())
    for i in (0, 1, 2, 6):
        assert torch.allclose(out[i].cpu(), auto[i].cpu(), rtol=1e-6, atol=2e-5), i
    rows = torch.arange(0, min(n, 40))
    _check_against_oracle(h, w, lab, out, rows=rows, denom=float(out[4].item()))
    _check_against_oracle(h, w, lab, auto, rows=rows, denom=float(auto[4].item()))


def test_chunk_choice_bounds_the_logit_buffer():
    # The default chunk keeps the per-chunk fp16 logits within the 128 MiB budget at any token
    # count and, from a few hundred tokens up, below the whole vocabulary (the [N, V] logits are
    # never held); a small vocabulary fits one chunk.
    assert K.LM_CHUNK_BUDGET == 128 << 20
    for n in (1, 707, 2048, 8192, 65536):
        c = K.lm_head_chunk_cols(n, 151936)
        assert c % 256 == 0 and c >= 256
        assert n * c * 2 <= max(K.LM_CHUNK_BUDGET, n * 256 * 2)
        if n >= 512:
            assert c < 151936
    assert K.lm_head_chunk_cols(64, 4099) >= 4099


@pytest.mark.parametrize("n,d,v", [(37, 128, 1031), (256, 1536, 20000), (5, 64, 700)])
def test_row_kernel_statistics_and_gradient(n, d, v):
    # Logits GEMM + per-row kernel: statistics against the oracle (1e-3; argmax exact unless an
    # oracle near-tie); the in-place gradient equals, bit for bit, the recompute GEMM's epilogue
    # given the same lse (same formula on the same fp16 logits), zeros past the vocabulary.
    g = torch.Generator().manual_seed(n * 7 + v)
    h = torch.randn(n, d, generator=g).half()
    w = (torch.randn(v, d, generator=g) * 0.05).half()
    lab = torch.randint(0, v, (n,), generator=g)
    lab[torch.rand(n, generator=g) < 0.2] = -100
    lab[0] = v - 1
    hd, wd, ld = h.to(DEV), w.to(DEV), lab.to(DEV)
    kp = (v + 63) // 64 * 64
    z = torch.full((n, kp + 64), 7.0, dtype=torch.float16, device=DEV)
    K.lm_head_ce_logits(hd, wd, z[:, :kp])
    lse = torch.empty(n, device=DEV)
    nll, ent = torch.empty_like(lse), torch.empty_like(lse)
    amax = torch.empty(n, dtype=torch.int64, device=DEV)
    zc = z.clone()
    K.lm_head_ce_rows(zc[:, :kp], v, ld, None, lse, nll, ent, amax)  # statistics only
    torch.cuda.synchronize()
    assert torch.equal(zc.cpu(), z.cpu())
    assert torch.all(z[:, v:kp].cpu() == 0) and torch.all(z[:, kp:].cpu() == 7.0)
    denom = torch.tensor([float(max((lab != -100).sum(), 1))], device=DEV)
    lse2, nll2, ent2 = torch.empty_like(lse), torch.empty_like(lse), torch.empty_like(lse)
    amax2 = torch.empty_like(amax)
    K.lm_head_ce_rows(z[:, :kp], v, ld, denom, lse2, nll2, ent2, amax2)
    g_ref = torch.empty((n, kp), dtype=torch.float16, device=DEV)
    K.lm_head_ce_grad_logits(hd, wd, ld, lse2, denom, 0, g_ref)
    torch.cuda.synchronize()
    assert torch.equal(lse.cpu(), lse2.cpu()) and torch.equal(amax.cpu(), amax2.cpu())
    assert torch.equal(z[:, :kp].cpu(), g_ref.cpu())
    assert torch.all(z[:, kp:].cpu() == 7.0)
    o = ref.lm_head_ce(h, w, lab, v_chunk=4096, need_grad=False)
    assert torch.all((lse.cpu() - o["lse"]).abs() <= 1e-3)
    assert torch.all((ent.cpu() - o["entropy"]).abs() <= 1e-3)
    zo = ref.lm_head_logits(h, w)
    tgt_ulp = torch.zeros(n)
    valid = lab != -100
    tgt_ulp[valid] = ref.fp16_ulp(zo[valid, lab[valid]])
    assert torch.all((nll.cpu() - o["nll"]).abs() <= 1e-3 + tgt_ulp)
    top2 = zo.topk(2, dim=-1).values
    near_tie = (top2[:, 0] - top2[:, 1]) <= ref.fp16_ulp(top2[:, 0])
    assert torch.all((amax.cpu() == o["argmax"]) | near_tie)
