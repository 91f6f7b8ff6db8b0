"""GPU tests of the BASELINE config 5 step at its real widths (the workload bench.py times).

* A 4-layer model with every Qwen2.5-1.5B width (hidden 1536, intermediate 8960, 12 / 2 heads,
  head_dim 128, vocab 151936, LoRA r=16 alpha=32 on q and v) through ``GraphedTrainStep`` with the
  bench's engine settings (whole-model streaming from pinned host memory, activations kept,
  native varlen attention, fused LoRA kernels, dequant + library GEMM, single-pass lm_head)
  against the fp32 CPU oracle (oracle/stack.py, pinned to transformers' Qwen2ForCausalLM):
  loss within 2e-3 relative, every LoRA gradient within 1e-2 relative Frobenius norm.
* The 28-layer model on a 4-row lognormal batch, by properties that hold at any size:
  activations kept vs recomputed give the same bits; replays are repeatable; whole-model,
  per-layer and resident weights, and one dequant per step instead of one per pass, give the
  same bits; the loss is finite and near ln V at random
  init; one step's loss is within 1e-3 (relative) of the plain autograd eager step
  (rus_amd.eager_reference) on the same weights and masks.
* The 28-layer model against the fp32 CPU oracle, on a short batch with dropout off and with
  the engine exactly as bench.py runs it (one dequant per step, buckets of 64, dropout on with
  the oracle's own Philox masks) on a 4-row lognormal batch of 695 tokens: loss within 2e-3
  relative; LoRA gradients within 1e-2 relative Frobenius norm of the oracle, except the listed
  tensors whose plain fp16 autograd step is itself further away (STRICT_SHORT / STRICT_BENCH):
  those within 1.25x that step's distance.
* The benchmarked loop for 16 steps (captured step + FlatAdamW) against the plain fp16 autograd
  step + torch.optim.AdamW: per-step losses within 2e-3 relative (the reference's acceptance is
  1% on the first step and 3% on the mean curve), parameter moves within 0.1 relative.

The reference's own acceptance for the full step is first-step loss within 1% of the base run
(harness/check_rules.py:29-30); the bounds here are tighter.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import stack as ostack
from rus_amd import model as M
from rus_amd import ops
from rus_amd.eager_reference import eager_step_loss
from rus_amd.graph import GraphedTrainStep

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    return float((a.float() - b.float()).norm() / (b.float().norm() + 1e-30))


def _batch(vocab, lengths, seed):
    g = torch.Generator().manual_seed(seed)
    S, B = max(lengths), len(lengths)
    ids = torch.randint(0, vocab, (B, S), generator=g)
    mask = torch.zeros(B, S, dtype=torch.long)
    for b, L in enumerate(lengths):
        mask[b, :L] = 1
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    return ids, mask, labels


def _graph_grads(engine):
    return [p.grad.detach().cpu().clone() for p in engine.lora_params]


def test_four_full_width_layers_graph_step_matches_oracle():
    cfg = M.Qwen2Config(num_hidden_layers=4, lora_dropout=0.0)
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=21)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                  recompute=False)
    assert engine.fused_lora and engine.attention == "varlen"
    ids, mask, labels = _batch(cfg.vocab_size, [61, 43], seed=5)
    gs = GraphedTrainStep(engine, training=True)
    loss = float(gs.step(ids, mask, labels))
    torch.cuda.synchronize()
    grads = _graph_grads(engine)

    pb = ops.pack_varlen(ids, mask, labels)
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                                   pb.row_lengths)
    loss_ref.backward()
    assert math.isfinite(loss)
    assert abs(loss - float(loss_ref)) <= 2e-3 * abs(float(loss_ref)), (loss, float(loss_ref))
    for gi, (g_f, leaf) in enumerate(zip(grads, lora)):
        assert _rel(g_f, leaf.grad) <= 1e-2, (gi, _rel(g_f, leaf.grad))


@pytest.fixture(scope="module")
def full_model():
    cfg = M.qwen2_1p5b()
    model = M.build_random_qlora_qwen2(cfg, DEV, seed=0)
    lengths = M.lengths_lognormal(4, seed=3)
    return cfg, model, _batch(cfg.vocab_size, lengths, seed=9)


def _steps(engine, batch, n):
    gs = GraphedTrainStep(engine, training=True)
    out = []
    for _ in range(n):
        loss = gs.step(*batch)
        torch.cuda.synchronize()
        out.append((loss.detach().cpu().clone(), _graph_grads(engine)))
    return out


def test_full_model_step_properties(full_model):
    cfg, model, batch = full_model
    results = {}
    for name, kw in (("model_keep", dict(stream_unit="model", recompute=False)),
                     ("model_keep_once", dict(stream_unit="model", recompute=False,
                                              dequant_once=True)),
                     ("model_recompute", dict(stream_unit="model", recompute=True)),
                     ("model_recompute_once", dict(stream_unit="model", recompute=True,
                                                   dequant_once=True)),
                     ("layer_keep", dict(stream_unit="layer", recompute=False)),
                     ("resident_keep", dict(resident_weights=True, recompute=False))):
        kw.setdefault("resident_weights", False)
        engine = ops.Qwen2FusedEngine(model, DEV, dropout_seed=1234, **kw)
        results[name] = _steps(engine, batch, 2)
        del engine
        torch.cuda.empty_cache()
    base = results["model_keep"]
    loss0 = float(base[0][0])
    # random init: logits ~ N(0, 0.02 * sqrt(1536)) per vocabulary row, so loss ~ ln V + 0.3
    assert math.isfinite(loss0) and abs(loss0 - math.log(cfg.vocab_size)) < 1.0, loss0
    for name, res in results.items():
        for step in range(2):  # step 2 draws new dropout masks (seed + 2) in every engine
            assert torch.equal(res[step][0], base[step][0]), (name, step)
            for gi, (a, b) in enumerate(zip(res[step][1], base[step][1])):
                assert torch.equal(a, b), (name, step, gi)
    assert not torch.equal(base[0][0], base[1][0])  # different masks per step


def test_full_model_replays_repeat_and_match_eager(full_model):
    cfg, model, batch = full_model
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=True, recompute=False,
                                  dropout_seed=99)
    gs = GraphedTrainStep(engine, training=True)
    seed0 = int(engine.dropout_seed.item())
    loss = gs.step(*batch)
    torch.cuda.synchronize()
    grads = _graph_grads(engine)
    # the same masks again (same seed): bit-identical replay
    engine.dropout_seed.fill_(seed0)
    loss2 = gs.step(*batch)
    torch.cuda.synchronize()
    assert torch.equal(loss.cpu(), loss2.cpu())
    for a, b in zip(grads, _graph_grads(engine)):
        assert torch.equal(a, b)
    # the plain autograd eager step with the replay's masks (seed0 + 1)
    pb = ops.pack_varlen(*(t.to(DEV) for t in batch))
    for p in engine.lora_params:
        p.grad = None
    seed = torch.tensor([seed0 + 1], dtype=torch.int64, device=DEV)
    h = engine.host_head.embed(pb.input_ids)
    loss_e = eager_step_loss(engine, h, pb.pos_ids, pb.shift_labels, pb.row_lengths,
                             training=True, seed=seed)
    loss_e.backward()
    torch.cuda.synchronize()
    assert abs(float(loss) - float(loss_e)) <= 1e-3 * abs(float(loss_e))
    # the gradients of two fp16 paths differ most in the deepest layers (up to ~5% relative on
    # the smallest LoRA-A gradients here); this only guards against gross errors such as other
    # dropout masks (O(1) differences). The bound against the fp32 oracle is the next test's.
    for gi, (g_f, p) in enumerate(zip(grads, engine.lora_params)):
        assert _rel(g_f, p.grad.cpu()) <= 0.1, (gi, _rel(g_f, p.grad.cpu()))


def _oracle_step(model, batch, dropout_seed=None):
    """Loss and LoRA gradients of the fp32 CPU oracle on a host batch."""
    pbc = ops.pack_varlen(*batch)
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pbc.input_ids, pbc.pos_ids,
                                   pbc.shift_labels, pbc.row_lengths, dropout_seed=dropout_seed)
    loss_ref.backward()
    return float(loss_ref), [leaf.grad for leaf in lora]


def _eager_step(engine, batch, training, seed=None):
    pb = ops.pack_varlen(*(t.to(DEV) for t in batch))
    for p in engine.lora_params:
        p.grad = None
    h = engine.host_head.embed(pb.input_ids)
    loss_e = eager_step_loss(engine, h, pb.pos_ids, pb.shift_labels, pb.row_lengths,
                             training=training, seed=seed)
    loss_e.backward()
    torch.cuda.synchronize()
    return float(loss_e), [p.grad.detach().cpu().clone() for p in engine.lora_params]


def _gradient_table(grads, grads_e, grads_ref):
    """[(tensor index, fused distance, eager distance)] relative Frobenius to the oracle."""
    return [(gi, _rel(g_f, g_r), _rel(g_e, g_r))
            for gi, (g_f, g_e, g_r) in enumerate(zip(grads, grads_e, grads_ref))]


# LoRA gradients (index 4 * layer + [q_A, q_B, v_A, v_B]) held to the 1e-2 relative bound against
# the fp32 oracle at these batches; every other one is within 1e-2 of it only up to the fp16
# arithmetic both GPU paths share, and is held to 1.25x the plain fp16 autograd step's own
# distance and to 7.5e-2. The measured distances (fused, eager) of every tensor are tabulated in
# the repository's design notes. At random init the attention is nearly uniform, so the query
# gradients are small against the fp16 rounding of Q, K and P: up to 5.8% (fused) and 6.1%
# (eager) at 695 tokens, 1.07% / 1.07% at 113.
STRICT_SHORT = frozenset(range(112)) - {100, 108}
STRICT_BENCH = frozenset({94, 95, 98, 99, 102, 103, 106, 107, 110, 111})


def _check_gradient_table(table, strict):
    bound = {gi: 1e-2 if gi in strict else max(1e-2, min(1.25 * b, 7.5e-2))
             for gi, _, b in table}
    bad = [(gi, a, b) for gi, a, b in table if a > bound[gi]]
    assert not bad, bad


def test_bench_engine_step_matches_oracle(full_model):
    # The engine exactly as bench.py runs it (whole-model streaming, one dequant per step,
    # activations kept, captured step with buckets of 64, LoRA dropout 0.05 on) on a 4-row
    # lognormal batch, against the fp32 CPU oracle drawing the same Philox masks.
    cfg, model, _ = full_model
    lengths = M.lengths_lognormal(4, seed=3)  # 695 tokens
    batch = _batch(cfg.vocab_size, lengths, seed=17)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                  recompute=False, dequant_once=True, dropout_seed=4321)
    gs = GraphedTrainStep(engine, bucket=64, training=True)
    seed = int(engine.dropout_seed.item()) + 1  # the step advances the seed, then draws
    loss = float(gs.step(*batch))
    torch.cuda.synchronize()
    grads = _graph_grads(engine)
    assert int(engine.dropout_seed.item()) == seed
    loss_e, grads_e = _eager_step(engine, batch, True,
                                  seed=torch.tensor([seed], dtype=torch.int64, device=DEV))
    loss_ref, grads_ref = _oracle_step(model, batch, dropout_seed=seed)
    table = _gradient_table(grads, grads_e, grads_ref)
    print(f"\nbench engine, {sum(lengths)} tokens: loss {loss:.6f} eager {loss_e:.6f} "
          f"oracle {loss_ref:.6f}")
    print("GRADTABLE bench", [(gi, round(a, 5), round(b, 5)) for gi, a, b in table])
    assert abs(loss - loss_ref) <= 2e-3 * abs(loss_ref), (loss, loss_ref)
    _check_gradient_table(table, STRICT_BENCH)


def test_full_model_graph_step_matches_oracle(full_model):
    cfg, model, _ = full_model
    batch = _batch(cfg.vocab_size, [72, 41], seed=13)
    engine = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                  recompute=False)
    gs = GraphedTrainStep(engine, training=False)
    loss = float(gs.step(*batch))
    torch.cuda.synchronize()
    grads = _graph_grads(engine)
    # the unfused fp16 autograd step on the same weights
    pb = ops.pack_varlen(*(t.to(DEV) for t in batch))
    for p in engine.lora_params:
        p.grad = None
    h = engine.host_head.embed(pb.input_ids)
    loss_e = eager_step_loss(engine, h, pb.pos_ids, pb.shift_labels, pb.row_lengths,
                             training=False)
    loss_e.backward()
    torch.cuda.synchronize()
    grads_e = [p.grad.detach().cpu().clone() for p in engine.lora_params]
    # fp32 CPU oracle
    pbc = ops.pack_varlen(*batch)
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    loss_ref, _ = ostack.step_loss(model, deq, lora, pbc.input_ids, pbc.pos_ids,
                                   pbc.shift_labels, pbc.row_lengths)
    loss_ref.backward()
    del deq
    assert abs(loss - float(loss_ref)) <= 2e-3 * abs(float(loss_ref)), (loss, float(loss_ref))
    table = _gradient_table(grads, grads_e, [leaf.grad for leaf in lora])
    print("\nGRADTABLE short", [(gi, round(a, 5), round(b, 5)) for gi, a, b in table])
    _check_gradient_table(table, STRICT_SHORT)


def test_bench_loop_loss_curve_matches_eager_adamw(full_model):
    # The benchmarked loop (captured step with buckets of 64, one dequant per step, whole-model
    # streaming, LoRA dropout, FlatAdamW at lr 2e-4) against the plain fp16 autograd step with
    # torch.optim.AdamW on an identical second model, the same batches and the same dropout
    # masks, for 16 steps. The reference accepts a full run when the first-step loss is within
    # 1% and the mean loss curve within 3% of the base run (harness/check_rules.py:29-30,
    # 372-386); here every step's loss agrees within 2e-3 relative, and after 16 steps every LoRA
    # factor has moved by the same amount within 0.1 relative (Frobenius, per tensor): AdamW
    # normalises each element's step, so the fp16 noise of the small query gradients shows up
    # in the moves (3-7% between the two fp16 paths), while a wrong or missing update is O(1).
    from rus_amd.optim import FlatAdamW

    cfg, model, _ = full_model
    twin = M.build_random_qlora_qwen2(cfg, DEV, seed=0)  # same weights and LoRA init
    batches = [_batch(cfg.vocab_size, M.lengths_lognormal(4, seed=40 + i), seed=50 + i)
               for i in range(4)]
    eng_f = ops.Qwen2FusedEngine(model, DEV, resident_weights=False, stream_unit="model",
                                 recompute=False, dequant_once=True, dropout_seed=777)
    eng_e = ops.Qwen2FusedEngine(twin, DEV, resident_weights=True, dropout_seed=777)
    start = [p.detach().cpu().clone() for p in eng_f.lora_params]
    assert all(torch.equal(a, b.detach().cpu()) for a, b in zip(start, eng_e.lora_params))
    gs = GraphedTrainStep(eng_f, bucket=64, training=True)
    opt_f = FlatAdamW([eng_f.flat_lora_parameter()], lr=2e-4)
    opt_e = torch.optim.AdamW(eng_e.lora_params, lr=2e-4)
    curve_f, curve_e = [], []
    for step in range(16):
        b = batches[step % 4]
        curve_f.append(float(gs.step(*b)))
        opt_f.step()
        seed = torch.tensor([777 + step + 1], dtype=torch.int64, device=DEV)
        loss_e, _ = _eager_step(eng_e, b, True, seed=seed)
        opt_e.step()
        curve_e.append(loss_e)
    torch.cuda.synchronize()
    print("\nloss curves (fused, eager):", [(round(a, 5), round(b, 5)) for a, b in
                                            zip(curve_f, curve_e)])
    assert abs(curve_f[0] - curve_e[0]) <= 0.01 * abs(curve_e[0])
    assert abs(sum(curve_f) - sum(curve_e)) <= 0.03 * abs(sum(curve_e))
    for step, (a, b) in enumerate(zip(curve_f, curve_e)):
        assert abs(a - b) <= 2e-3 * abs(b), (step, a, b)
    moves = []
    for gi, (p0, pf, pe) in enumerate(zip(start, eng_f.lora_params, eng_e.lora_params)):
        d_f, d_e = pf.detach().cpu() - p0, pe.detach().cpu() - p0
        moves.append((gi, _rel(d_f, d_e)))
    print("parameter moves, relative difference, worst 5:",
          sorted(moves, key=lambda m: -m[1])[:5])
    assert all(r <= 0.1 for _, r in moves), [m for m in moves if m[1] > 0.1]
