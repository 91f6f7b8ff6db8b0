"""GPU tests of the fused packed Qwen2 stack (FusedQwen2StackFn + chunked lm_head).

* Against the CPU oracle (oracle/stack.py, pinned to transformers' Qwen2ForCausalLM) on a small
  model with dropout off: loss within 2e-3 relative, every LoRA gradient tensor within 1e-2 in
  relative Frobenius norm (||g - g_ref|| <= 1e-2 ||g_ref||; fp16 activations against fp32).
* Streamed (pinned host, two slots) and HBM-resident weights give bit-identical results, and so
  do the host-streamed lm_head / embedding and the host-offloaded layer inputs.
* With dropout on, the fused stack (forward masks re-drawn in the backward recompute) matches a
  plain autograd eager step using the same counter-based masks (rus_amd.eager_reference) and the
  CPU oracle given the oracle's own Philox masks: same tolerances.
"""

from __future__ import annotations

import pytest
import torch

from oracle import stack as ostack
from rus_amd import model as M
from rus_amd import ops
from rus_amd.eager_reference import eager_step_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


def small_config(layers=2, dropout=0.0):
    return M.Qwen2Config(hidden_size=512, intermediate_size=256, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, vocab_size=1000,
                         lora_r=4, lora_alpha=8.0, lora_dropout=dropout)


def _batch(cfg, lengths, seed=0):
    g = torch.Generator().manual_seed(seed)
    S = max(lengths)
    B = len(lengths)
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=g)
    mask = torch.zeros(B, S, dtype=torch.long)
    for b, L in enumerate(lengths):
        mask[b, :L] = 1
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    labels[0, :5] = -100
    return ids, mask, labels


def _fused_step(engine, pb, training=True):
    for p in engine.lora_params:
        p.grad = None
    h = engine.host_head.embed(pb.input_ids.to(DEV))
    final = ops.FusedQwen2StackFn.apply(h, pb.pos_ids.to(DEV), pb.row_lengths, engine, training,
                                        *engine.lora_params)
    loss, nll, ent, amax = ops.chunked_lm_head(final, pb.shift_labels.to(DEV), engine.host_head)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), [p.grad.detach().cpu().clone() for p in engine.lora_params]


def _rel(a, b):
    return float((a.float() - b.float()).norm() / (b.float().norm() + 1e-30))


@pytest.mark.parametrize("resident,head,offload", [(False, True, False), (True, True, False),
                                                 (False, False, True), (True, False, False)])
def test_fused_stack_matches_cpu_oracle(resident, head, offload):
    # head=False: the lm_head / embedding streamed from pinned host memory (HostHead); offload:
    # layer inputs kept in pinned host memory for the backward recompute (InputStream).
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=1, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=resident, resident_head=head,
                                  offload_inputs=offload, v_chunk=256)
    ids, mask, labels = _batch(cfg, [37, 64, 21])
    pb = ops.pack_varlen(ids, mask, labels)
    loss, grads = _fused_step(engine, pb, training=False)

    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                                   pb.row_lengths)
    loss_ref.backward()
    assert abs(float(loss) - float(loss_ref)) <= 2e-3 * abs(float(loss_ref))
    for gi, (g_f, leaf) in enumerate(zip(grads, lora)):
        assert _rel(g_f, leaf.grad) <= 1e-2, (gi, _rel(g_f, leaf.grad))


@pytest.mark.parametrize("resident,recompute", [(False, True), (True, False)])
def test_fused_nf4_gemm_stack_matches_cpu_oracle(resident, recompute):
    # Every base-weight product through the dequant-in-GEMM kernel (no fp16 weight copies).
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=1, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=resident, gemm="fused",
                                  recompute=recompute)
    ids, mask, labels = _batch(cfg, [37, 64, 21])
    pb = ops.pack_varlen(ids, mask, labels)
    loss, grads = _fused_step(engine, pb, training=False)
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                                   pb.row_lengths)
    loss_ref.backward()
    assert abs(float(loss) - float(loss_ref)) <= 2e-3 * abs(float(loss_ref))
    for gi, (g_f, leaf) in enumerate(zip(grads, lora)):
        assert _rel(g_f, leaf.grad) <= 1e-2, (gi, _rel(g_f, leaf.grad))
    # and twice in a row bit for bit (fixed-order sums, counters left at zero)
    loss2, grads2 = _fused_step(engine, pb, training=False)
    assert torch.equal(loss, loss2) and all(torch.equal(a, b) for a, b in zip(grads, grads2))


def test_streamed_and_resident_weights_agree_bitwise():
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=2, std=0.05)
    ids, mask, labels = _batch(cfg, [30, 50], seed=1)
    pb = ops.pack_varlen(ids, mask, labels)
    out = []
    for resident, unit, ov in ((False, "layer", False), (False, "model", False),
                               (True, "layer", False), (False, "model", True),
                               (True, "layer", True)):
        engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=resident, stream_unit=unit,
                                      overlap=ov)
        out.append(_fused_step(engine, pb, training=False))
        out.append(_fused_step(engine, pb, training=False))  # second step: the other buffer
    for o in out[1:]:
        assert torch.equal(out[0][0], o[0])
        for a, b in zip(out[0][1], o[1]):
            assert torch.equal(a, b)


def test_dropout_masks_match_eager_autograd_and_oracle():
    cfg = small_config(dropout=0.05)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=3, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
    ids, mask, labels = _batch(cfg, [40, 33, 60], seed=2)
    pb = ops.pack_varlen(ids, mask, labels)
    loss_f, grads_f = _fused_step(engine, pb, training=True)
    seed = engine.last_dropout_seed

    for p in engine.lora_params:
        p.grad = None
    h = engine.host_head.embed(pb.input_ids.to(DEV))
    loss_e = eager_step_loss(engine, h, pb.pos_ids.to(DEV), pb.shift_labels.to(DEV),
                             pb.row_lengths, training=True, seed=seed)
    loss_e.backward()
    torch.cuda.synchronize()
    assert abs(float(loss_f) - float(loss_e)) <= 2e-3 * abs(float(loss_e))
    for gi, (g_f, p) in enumerate(zip(grads_f, engine.lora_params)):
        assert _rel(g_f, p.grad.cpu()) <= 1e-2, (gi, _rel(g_f, p.grad.cpu()))
    # the CPU oracle with its own Philox masks for the same seed
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                                   pb.row_lengths, dropout_seed=int(seed.item()))
    loss_ref.backward()
    assert abs(float(loss_f) - float(loss_ref)) <= 2e-3 * abs(float(loss_ref))
    for gi, (g_f, leaf) in enumerate(zip(grads_f, lora)):
        assert _rel(g_f, leaf.grad) <= 1e-2, (gi, _rel(g_f, leaf.grad))
    # and the masks were really applied: without dropout the gradients differ
    for p in engine.lora_params:
        p.grad = None
    _, grads_nodrop = _fused_step(engine, pb, training=False)
    assert _rel(grads_nodrop[0], grads_f[0]) > 1e-2
    # each training forward draws a new seed
    _fused_step(engine, pb, training=True)
    assert int(engine.last_dropout_seed.item()) == int(seed.item()) + 1


def test_fused_causal_lm_forward_scatter():
    cfg = small_config(layers=1)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=4, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
    ids, mask, labels = _batch(cfg, [12, 20], seed=3)
    loss, nll, ent, amax = ops.fused_causal_lm_forward(engine, ids.to(DEV), mask.to(DEV),
                                                       labels.to(DEV), training=False)
    loss.backward()
    assert nll.shape == ids.shape and ent.shape == ids.shape and amax.shape == ids.shape
    assert torch.all(nll[0, 12:].cpu() == 0)  # padding
    assert all(p.grad is not None for p in engine.lora_params)


def test_fused_lora_kernels_match_library_gemm_path():
    # The fused LoRA kernels against the same stack with torch GEMMs for the rank-r products
    # (same dropout masks): loss within 1e-3 relative, LoRA gradients within 5e-3.
    cfg = small_config(dropout=0.05)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=6, std=0.05)
    ids, mask, labels = _batch(cfg, [45, 20, 61], seed=4)
    pb = ops.pack_varlen(ids, mask, labels)
    out = []
    for fused in (True, False):
        engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True, lora_kernels=fused,
                                      dropout_seed=555)
        assert engine.fused_lora == fused
        out.append(_fused_step(engine, pb, training=True))
    assert abs(float(out[0][0]) - float(out[1][0])) <= 1e-3 * abs(float(out[1][0]))
    for gi, (a, b) in enumerate(zip(out[0][1], out[1][1])):
        assert _rel(a, b) <= 5e-3, (gi, _rel(a, b))


@pytest.mark.parametrize("dropout,lora_kernels", [(0.0, True), (0.1, True), (0.1, False)])
def test_saved_activations_match_recompute_bitwise(dropout, lora_kernels):
    # recompute on / off, each without and with the second stream (dequant ahead, LoRA-down
    # beside the q/k/v GEMM): the same bits
    cfg = small_config(dropout=dropout)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=4, std=0.05)
    ids, mask, labels = _batch(cfg, [45, 70, 12], seed=3)
    pb = ops.pack_varlen(ids, mask, labels)
    out = []
    for recompute, ov in ((True, False), (False, False), (True, True), (False, True)):
        engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True, dropout_seed=123,
                                      lora_kernels=lora_kernels, recompute=recompute, overlap=ov)
        out.append(_fused_step(engine, pb, training=True))
    for o in out[1:]:
        assert torch.equal(out[0][0], o[0])
        for a, b in zip(out[0][1], o[1]):
            assert torch.equal(a, b)


def test_engine_has_one_attention_path():
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=4, std=0.05)
    for other in ("varlen_aten", "sdpa_rows"):
        with pytest.raises(ValueError, match="only attention path"):
            ops.Qwen2FusedEngine(model, DEV, attention=other)


@pytest.mark.parametrize("recompute", [True, False])
def test_host_streams_agree_bitwise_with_hbm_residency(recompute):
    # Streamed head (embedding rows gathered on the device from pinned host memory, vocabulary
    # chunks through the two-slot ring) and inputs offloaded to the host: the same bits as the
    # HBM-resident head and inputs, given the same vocabulary chunk; two steps in a row.
    cfg = small_config(dropout=0.1)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=7, std=0.05)
    ids, mask, labels = _batch(cfg, [33, 58, 27], seed=5)
    pb = ops.pack_varlen(ids, mask, labels)
    out = []
    for head, offload in ((True, False), (False, True), (False, False), (True, True)):
        engine = ops.Qwen2FusedEngine(model, DEV, resident_head=head, offload_inputs=offload,
                                      v_chunk=256, dropout_seed=77, recompute=recompute)
        for _ in range(2):
            for p in engine.lora_params:
                p.grad = None
            h = engine.host_head.embed(pb.input_ids.to(DEV))
            final = ops.FusedQwen2StackFn.apply(h, pb.pos_ids.to(DEV), pb.row_lengths, engine,
                                                True, *engine.lora_params)
            loss, nll, ent, amax = ops.chunked_lm_head(final, pb.shift_labels.to(DEV),
                                                       engine.host_head, v_chunk=256)
            loss.backward()
            torch.cuda.synchronize()
            out.append((loss.detach().cpu(), nll.cpu(), ent.cpu(), amax.cpu(),
                        [p.grad.detach().cpu().clone() for p in engine.lora_params]))
    for i in range(0, len(out), 2):  # the engines' second steps draw the same masks
        for a, b in zip(out[0][:4], out[i][:4]):
            assert torch.equal(a, b), i
        for a, b in zip(out[0][4], out[i][4]):
            assert torch.equal(a, b), i
        assert torch.equal(out[1][0], out[i + 1][0])
    if not engine.host_head.resident:
        assert int(engine.host_head.embed_error.item()) == 0


def test_patched_qwen2_forward_returns_loss_and_logits_proxy():
    # transformers' Qwen2ForCausalLM.forward, patched, on the attribute layout of a PEFT +
    # bitsandbytes model: the fused engine's loss and a ChunkedLogitsProxy whose statistics are
    # the fused head's (padding positions: nll 0, the batch-mean entropy).
    pytest.importorskip("transformers")
    from duck_hf import duck_causal_lm
    from transformers.models.qwen2 import modeling_qwen2

    import torch.nn.functional as F

    cfg = small_config(layers=1)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=8, std=0.05)
    duck = duck_causal_lm(model, dropout_p=0.0, training=False)
    ids, mask, labels = _batch(cfg, [17, 29], seed=6)
    ids, mask, labels = ids.to(DEV), mask.to(DEV), labels.to(DEV)
    unpatched = modeling_qwen2.Qwen2ForCausalLM.forward
    try:
        assert ops.install_runtime_patches()["transformers_qwen2"]
        out = modeling_qwen2.Qwen2ForCausalLM.forward(duck, input_ids=ids, attention_mask=mask,
                                                      labels=labels)
    finally:
        modeling_qwen2.Qwen2ForCausalLM.forward = unpatched
    engine = duck.__dict__["_rus_fused_engine"]
    loss_f, nll, ent, amax = ops.fused_causal_lm_forward(engine, ids, mask, labels,
                                                         training=False)
    torch.cuda.synchronize()
    assert torch.equal(out.loss.detach().cpu(), loss_f.detach().cpu())
    proxy = out.logits
    assert isinstance(proxy, ops.ChunkedLogitsProxy) and proxy.shape == (2, 29, cfg.vocab_size)
    assert torch.equal(proxy.argmax(-1).cpu(), amax.cpu())
    assert torch.all(proxy.per_token_nll[0, 17:].cpu() == 0)
    mean_ent = ent[mask.bool()].mean()
    assert torch.allclose(ent[0, 17:], mean_ent.expand(12))
    # the trainer's shifted loss from the proxy equals the fused loss
    V = cfg.vocab_size
    ce = F.cross_entropy(proxy[:, :-1].reshape(-1, V), labels[:, 1:].reshape(-1),
                         ignore_index=-100)
    assert torch.allclose(ce.cpu(), out.loss.detach().float().cpu(), rtol=1e-5, atol=1e-6)
    out.loss.backward()
    assert all(p.grad is not None for p in engine.lora_params)
    # the patched forward against the CPU oracle (fp32, pinned to transformers' Qwen2) on the same
    # batch: loss within 2e-3 relative, every real token's entropy within 1e-3 absolute, its nll
    # within 1e-2, its argmax equal wherever the oracle's top two logits differ by more than 1e-2
    # (measured: loss 2e-5 relative, entropy 3.5e-4, nll 3.3e-3, every argmax equal)
    pb = ops.pack_varlen(ids.cpu(), mask.cpu(), labels.cpu())
    with torch.no_grad():
        loss_ref, final = ostack.step_loss(model, ostack.dequant_model(model),
                                           ostack.lora_leaves(model), pb.input_ids, pb.pos_ids,
                                           pb.shift_labels, pb.row_lengths)
        logits = final @ model.embed.cpu().float().t()
        logp = torch.log_softmax(logits, -1)
        ent_ref = -(logp.exp() * logp).sum(-1)
        nll_ref = F.cross_entropy(logits, pb.shift_labels, ignore_index=-100, reduction="none")
        top2 = logits.topk(2, -1).values
    assert abs(float(out.loss.detach()) - float(loss_ref)) <= 2e-3 * abs(float(loss_ref))
    real = mask.bool().cpu()  # row-major real positions: the packed token order
    assert float((proxy.per_token_entropy.cpu()[real].float() - ent_ref).abs().max()) <= 1e-3
    assert float((proxy.per_token_nll.cpu()[real].float() - nll_ref).abs().max()) <= 1e-2
    clear = (top2[:, 0] - top2[:, 1]) > 1e-2
    assert torch.equal(proxy.argmax(-1).cpu()[real][clear], logits.argmax(-1)[clear])


def test_lm_head_layouts_agree_through_the_engine():
    # The engine's default head (one pass over vocabulary chunks) and the token-blocked head
    # (lm_v_chunk = 0) on the same step: the same statistics up to fp32 summation order.
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=3, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
    ids, mask, labels = _batch(cfg, [37, 64, 21], seed=4)
    ids, mask, labels = ids.to(DEV), mask.to(DEV), labels.to(DEV)
    out = {}
    for layout in (None, 0, 256):
        engine.lm_v_chunk = layout
        for p in engine.lora_params:
            p.grad = None
        loss, nll, ent, amax = ops.fused_causal_lm_forward(engine, ids, mask, labels,
                                                           training=False)
        loss.backward()
        torch.cuda.synchronize()
        out[layout] = (float(loss.detach()), nll.detach().cpu(), ent.detach().cpu(),
                       amax.cpu(), [p.grad.detach().cpu().clone() for p in engine.lora_params])
    base = out[None]
    for layout in (0, 256):
        loss, nll, ent, amax, grads = out[layout]
        assert abs(loss - base[0]) <= 1e-5 * abs(base[0]), (layout, loss, base[0])
        assert float((nll - base[1]).abs().max()) <= 1e-4
        assert float((ent - base[2]).abs().max()) <= 1e-4
        assert torch.equal(amax, base[3])
        for gi, (a, b) in enumerate(zip(grads, base[4])):
            assert _rel(a, b) <= 1e-3, (layout, gi, _rel(a, b))
