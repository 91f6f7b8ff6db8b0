"""GPU tests of the captured-graph training step (rus_amd.graph.GraphedTrainStep).

* One replay equals the CPU oracle (dropout off: loss within 2e-3 relative, every LoRA gradient
  within 1e-2 relative Frobenius norm) and the eager autograd path of the same engine.
* With dropout on, replay k uses seed base + k: matches the oracle with that seed's Philox masks.
* Replays are repeatable: several replays, with eager work and synchronisations in between and
  another bucket's graph replayed between them, give bitwise-identical loss and gradients.
* Streamed weights (per-layer slots with the copies captured in the graph, or whole-model
  buffers copied outside it) and resident weights agree bitwise.
* The captured graphs contain no memset nodes.
* ``time_replays()`` brackets each replay with one event pair, and only while it is on.
"""

from __future__ import annotations

import pytest
import torch

from oracle import stack as ostack
from rus_amd import model as M
from rus_amd import ops
from rus_amd.graph import GraphedTrainStep

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
    return ids.to(DEV), mask.to(DEV), labels.to(DEV)


def _rel(a, b):
    return float((a.float() - b.float()).norm() / (b.float().norm() + 1e-30))


def _grads(engine):
    return [p.grad.detach().cpu().clone() for p in engine.lora_params]


def _oracle(model, batch, seed=None):
    pb = ops.pack_varlen(*(t.cpu() for t in batch))
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                               pb.row_lengths, dropout_seed=seed)
    loss.backward()
    return float(loss), [leaf.grad for leaf in lora]


def test_graph_step_matches_oracle_and_eager():
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=1, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
    batch = _batch(cfg, [37, 64, 21])
    gs = GraphedTrainStep(engine, bucket=64, training=False)
    loss_g = float(gs.step(*batch))
    torch.cuda.synchronize()
    grads_g = _grads(engine)

    loss_o, grads_o = _oracle(model, batch)
    assert abs(loss_g - loss_o) <= 2e-3 * abs(loss_o)
    for gi, (a, b) in enumerate(zip(grads_g, grads_o)):
        assert _rel(a, b) <= 1e-2, (gi, _rel(a, b))

    for p in engine.lora_params:
        p.grad = None
    loss_e, *_ = ops.fused_causal_lm_forward(engine, *batch, training=False)
    loss_e.backward()
    torch.cuda.synchronize()
    assert abs(loss_g - float(loss_e)) <= 1e-3 * abs(float(loss_e))
    for gi, (a, p) in enumerate(zip(grads_g, engine.lora_params)):
        assert _rel(a, p.grad.cpu()) <= 5e-3, (gi, _rel(a, p.grad.cpu()))


def test_graph_fused_nf4_gemm_replays_repeat_and_match_eager():
    # The dequant-in-GEMM products inside a captured step: workspace from the graph pool,
    # arrival counters left at zero by every replay; replays separated by eager work.
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=1, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                  gemm="fused", recompute=False)
    batch = _batch(cfg, [37, 64, 21])
    for p in engine.lora_params:
        p.grad = None
    loss_e, *_ = ops.fused_causal_lm_forward(engine, *batch, training=False)
    loss_e.backward()
    torch.cuda.synchronize()
    grads_e = [p.grad.detach().cpu().clone() for p in engine.lora_params]
    gs = GraphedTrainStep(engine, bucket=64, training=False)
    first = None
    for rep in range(3):
        loss_g = float(gs.step(*batch))
        torch.cuda.synchronize()
        grads_g = [g.clone() for g in _grads(engine)]
        if first is None:
            first = (loss_g, grads_g)
            assert abs(loss_g - float(loss_e)) <= 1e-3 * abs(float(loss_e))
            for gi, (a, b) in enumerate(zip(grads_g, grads_e)):
                assert _rel(a, b) <= 5e-3, (gi, _rel(a, b))
        else:
            assert loss_g == first[0]
            assert all(torch.equal(a, b) for a, b in zip(grads_g, first[1]))
        x = torch.randn(300, 512, device=DEV).half()  # eager work between replays
        (x @ x.t()).sum().item()


def test_graph_dropout_seed_advances_per_replay():
    cfg = small_config(dropout=0.05)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=3, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True, dropout_seed=1000)
    batch = _batch(cfg, [40, 33, 60], seed=2)
    gs = GraphedTrainStep(engine, bucket=64, training=True)
    losses = []
    for k in range(2):
        losses.append(float(gs.step(*batch)))
        torch.cuda.synchronize()
        grads = _grads(engine)
        assert int(engine.dropout_seed.item()) == 1001 + k
        loss_o, grads_o = _oracle(model, batch, seed=1001 + k)
        assert abs(losses[-1] - loss_o) <= 2e-3 * abs(loss_o)
        for gi, (a, b) in enumerate(zip(grads, grads_o)):
            assert _rel(a, b) <= 1e-2, (k, gi, _rel(a, b))
    assert losses[0] != losses[1]  # different masks


@pytest.mark.parametrize("unit", ["resident", "layer", "model"])
def test_graph_replays_repeatable_across_buckets(unit):
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=5, std=0.05)
    resident = unit == "resident"
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=resident,
                                  stream_unit="layer" if resident else unit)
    a = _batch(cfg, [30, 50], seed=1)
    b = _batch(cfg, [90, 70, 12], seed=2)
    gs = GraphedTrainStep(engine, bucket=64, training=False, census=True)
    ref_loss = float(gs.step(*a))
    torch.cuda.synchronize()
    ref_grads = _grads(engine)
    gs.time_replays()  # an event pair around each replay (after its copy wait)
    for it in range(3):
        x = torch.randn(256, 256, device=DEV)  # unrelated eager work between replays
        (x @ x).sum().item()
        float(gs.step(*b))
        torch.cuda.synchronize()
        loss = float(gs.step(*a))
        torch.cuda.synchronize()
        assert loss == ref_loss, it
        for g0, g1 in zip(ref_grads, _grads(engine)):
            assert torch.equal(g0, g1), it
    ms = gs.replay_ms()
    assert len(ms) == 6 and all(0 < t < 1e4 for t in ms), ms
    gs.time_replays(False)
    gs.step(*a)
    assert gs.replay_ms() == []
    assert len(gs.graphs) == 2
    for cap in gs.graphs.values():
        # one graph per whole-model weight buffer
        assert len(cap.node_counts) == engine.weight_stream.n_buffers
        assert engine.weight_stream.n_buffers == (2 if unit == "model" else 1)
        for c in cap.node_counts.values():
            print("graph nodes", unit, c)
            assert c["memset"] == 0 and c["kernel"] > 50
            if unit == "layer":
                # each layer's packed image is one H2D copy into its slot, at least once
                assert c["memcpy"] >= cfg.num_hidden_layers
    # resident and streamed weights give the same bits
    if not resident:
        eng_r = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
        gr = GraphedTrainStep(eng_r, bucket=64, training=False)
        assert float(gr.step(*a)) == ref_loss
        torch.cuda.synchronize()
        for g0, g1 in zip(ref_grads, _grads(eng_r)):
            assert torch.equal(g0, g1)


def test_graph_saved_activations_match_recompute_bitwise():
    # The captured step with activations kept from the forward (and with the second stream:
    # dequant ahead, LoRA-down beside the q/k/v GEMM; or with one dequant per step, the backward
    # reading the forward's fp16 weights) gives the recompute's bits, dropout included, on two
    # buckets and repeated replays.
    cfg = small_config(dropout=0.1)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=6, std=0.05)
    a = _batch(cfg, [30, 50], seed=1)
    b = _batch(cfg, [90, 70, 12], seed=2)
    res = []
    for recompute, ov, once in ((True, False, False), (False, False, False), (False, True, False),
                                (False, False, True), (True, False, True)):
        engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                      dropout_seed=77, recompute=recompute, overlap=ov,
                                      dequant_once=once)
        gs = GraphedTrainStep(engine, bucket=64, training=True)
        out = []
        for batch in (a, b, a):
            out.append(float(gs.step(*batch)))
            torch.cuda.synchronize()
            out.append(_grads(engine))
        res.append(out)
    for other in res[1:]:
        for x, y in zip(res[0], other):
            if isinstance(x, float):
                assert x == y
            else:
                for g0, g1 in zip(x, y):
                    assert torch.equal(g0, g1)
    # one dequant per step needs the packed weights on the device for the whole step and the
    # dequant on the step's own stream
    with pytest.raises(ValueError, match="dequant"):
        ops.Qwen2FusedEngine(model, DEV, stream_unit="layer", dequant_once=True)
    with pytest.raises(ValueError, match="dequant_once"):
        ops.Qwen2FusedEngine(model, DEV, stream_unit="model", overlap=True, dequant_once=True)


@pytest.mark.parametrize("resident", [True, False])
def test_host_packed_batches_match_device_packed_bitwise(resident):
    # Host (CPU) batches are packed on the host into a pinned image that the graph's first kernel
    # copies; the replays must give the device-packed steps' loss and gradients bit for bit, also
    # when the two images alternate and another bucket runs in between (whole-model streaming
    # pairs each image with a weight buffer; resident weights alternate the images per step).
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=9, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=resident,
                                  stream_unit="layer" if resident else "model")
    gs_dev = GraphedTrainStep(engine, bucket=64, training=False)
    gs_host = GraphedTrainStep(engine, bucket=64, training=False)
    a = _batch(cfg, [37, 64, 21], seed=3)
    b = _batch(cfg, [100, 9], seed=4)
    want = {}
    for name, bt in (("a", a), ("b", b)):
        want[name] = (float(gs_dev.step(*bt)), _grads(engine))
    host = {"a": [t.cpu().pin_memory() for t in a], "b": [t.cpu().pin_memory() for t in b]}
    for name in ("a", "b", "a", "a", "b", "b", "a"):
        loss = float(gs_host.step(*host[name]))
        torch.cuda.synchronize()
        assert loss == want[name][0], name
        for x, y in zip(_grads(engine), want[name][1]):
            assert torch.equal(x, y), name
    assert gs_host.host_inputs and not gs_dev.host_inputs


def test_flat_lora_parameter_adamw_equals_per_factor_adamw():
    # The flat Parameter holds every factor (the LoRA parameters are its views) and receives the
    # step's flat gradient; AdamW over it gives the per-factor AdamW's values (elementwise).
    cfg = small_config()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=11, std=0.05)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True)
    gs = GraphedTrainStep(engine, bucket=64, training=False)
    flat = engine.flat_lora_parameter()
    batch = _batch(cfg, [50, 30], seed=5)
    start = [p.detach().clone() for p in engine.lora_params]
    gs.step(*batch)
    assert flat.grad is not None and flat.grad.data_ptr() == gs.grad32.data_ptr()
    torch.optim.AdamW(engine.lora_params, lr=1e-2, foreach=False).step()
    torch.cuda.synchronize()
    per_factor = [p.detach().clone() for p in engine.lora_params]
    with torch.no_grad():
        for p, s in zip(engine.lora_params, start):
            p.copy_(s)
    torch.optim.AdamW([flat], lr=1e-2, foreach=False).step()
    torch.cuda.synchronize()
    for p, want in zip(engine.lora_params, per_factor):
        assert torch.equal(p.detach(), want)
