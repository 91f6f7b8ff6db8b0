#!/usr/bin/env python3
"""Benchmark of the fused QLoRA training step on one MI355X.

Workload: one training step = packed forward + backward of a random-init, NF4 double-quantised
Qwen2.5-1.5B-shaped model (28 layers, LoRA r=16 / alpha=32 / dropout 0.05 on q and v) over a batch
of 4 rows with lognormal lengths (median 140, mean 220, clipped to [16, 512]) of uniform random
token ids, followed by an AdamW step on the LoRA parameters (lr 2e-4). Base layers are streamed
per step from pinned host memory through two device slots (as configured); batches are resident
in HBM before the timed region.

Prints one JSON line: tokens/s over the K timed steps (value), the dominant kernel's roofline
(HIP events around each of its launches inside the timed region), the CPU baseline (the oracle
on a bounded sample, extrapolated), peak HBM per step against the unfused eager step, per-kernel
rates and a resident-weights ablation.

Usage: python bench.py [--gpus 1] [--steps 64] [--warmup 2]
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "train tokens/s (packed 1.5B NF4 QLoRA); lm_head-CE & NF4-dequant HBM GB/s"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
LMHEAD_KERNELS = ("lmhead_ce_fwd", "lmhead_ce_fwd_keep", "lmhead_ce_logits",
                  "lmhead_ce_grad_logits", "lmhead_ce_grad_hidden")
# kernels whose roofline is the fp16 MFMA peak (the rest are bound by HBM bandwidth)
MFMA_KERNELS = LMHEAD_KERNELS + ("gemm_parts", "nf4_gemm", "attn_fwd", "attn_bwd")


def make_batches(cfg, n_batches, rows, max_len, seed, device):
    import torch

    from rus_amd.model import lengths_lognormal

    out = []
    for b in range(n_batches):
        lengths = lengths_lognormal(rows, seed=seed + b, hi=max_len)
        S = max(lengths)
        g = torch.Generator().manual_seed(seed + 1000 + b)
        ids = torch.randint(0, cfg.vocab_size, (rows, S), generator=g)
        mask = torch.zeros(rows, S, dtype=torch.long)
        for r, L in enumerate(lengths):
            mask[r, :L] = 1
        labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
        # Host batches (pinned), as a data loader hands them over: the captured step packs them
        # on the host; the eager step moves them to the device first.
        if device != "cpu":
            ids, mask, labels = ids.pin_memory(), mask.pin_memory(), labels.pin_memory()
        out.append((ids, mask, labels, sum(lengths)))
    return out


def train_step(engine, opt, batch, graph=None):
    """One step: packed forward + backward (eager autograd, or one replay of the bucket's captured
    graph) and the AdamW update of the LoRA parameters."""
    from rus_amd.ops import fused_causal_lm_forward

    ids, mask, labels, _ = batch
    if graph is not None:
        loss = graph.step(ids, mask, labels)
    else:
        ids, mask, labels = (t.to(engine.device, non_blocking=True) for t in (ids, mask, labels))
        loss, _, _, _ = fused_causal_lm_forward(engine, ids, mask, labels, training=True)
        loss.backward()
    opt.step()
    opt.zero_grad(set_to_none=True)
    return loss


def flat_adamw(engine):
    """AdamW (lr 2e-4, torch.optim.AdamW's defaults otherwise) over the engine's flat LoRA
    parameter (every factor is a view of it): one rus_adamw_step launch per step
    (rus_amd.optim.FlatAdamW) instead of a foreach pass over 112 tensors; elementwise, so the
    same update. Returns (optimizer, implementation)."""
    from rus_amd.optim import FlatAdamW

    return FlatAdamW([engine.flat_lora_parameter()], lr=2e-4), "rus_adamw_step"


def timed_run(engine, opt, batches, steps, warmup, kernel_filter=None, graph=None):
    """Runs warmup + timed steps; returns (seconds, tokens, per-step seconds, timer summary)."""
    import torch

    from rus_amd.kernels import KernelTimer

    if graph is not None:
        kernel_filter = set()  # kernels inside a replayed graph cannot be bracketed by events
    for i in range(warmup):
        train_step(engine, opt, batches[i % len(batches)], graph)
    torch.cuda.synchronize()
    timer = KernelTimer(only=kernel_filter)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    step_tokens = []
    tokens = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with timer:
        for i in range(steps):
            marks[i].record()
            b = batches[(warmup + i) % len(batches)]
            train_step(engine, opt, b, graph)
            tokens += b[3]
            step_tokens.append(b[3])
        marks[steps].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # Per-step device time between stream marks (the host runs ahead of the device).
    per_step = [(marks[i].elapsed_time(marks[i + 1]) / 1e3, step_tokens[i]) for i in range(steps)]
    return t1 - t0, tokens, per_step, timer.summary()


def kernel_rates(summary, steps):
    out = {}
    for name, r in summary.items():
        sec = r["ms"] / 1e3
        e = {"launches_per_step": r["launches"] / steps, "ms_per_step": r["ms"] / steps}
        if name in MFMA_KERNELS:
            e["tflops"] = r["flops"] / sec / 1e12 if sec > 0 else None
        e["gbps"] = r["bytes"] / sec / 1e9 if sec > 0 else None
        out[name] = e
    return out


def cpu_baseline(seed=0, batch=None, reps=5):
    """The CPU oracle on a bounded sample of the same workload: one config-5 layer plus the
    lm_head over one of the bench's own batches (its packed tokens and row lengths, ~700 tokens),
    forward + backward including the NF4 dequant of the layer's weights, median of ``reps`` timed
    repetitions after one warm-up; extrapolated to the 28-layer step as tokens/s."""
    import statistics

    import torch

    from oracle import ops as oref
    from oracle import stack as ostack
    from rus_amd import model as M
    from rus_amd.ops import pack_varlen

    # This GPU's share of the box's host cores (its OMP_NUM_THREADS: 16 per GPU on the GPU
    # boxes, which ask that thread pools stay within it), at most the affinity mask.
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    threads = max(1, min(affinity, share))
    torch.set_num_threads(threads)
    cfg = M.qwen2_1p5b()
    cfg1 = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": 1, "lora_dropout": 0.0})
    model = M.build_random_qlora_qwen2(cfg1, "cpu", seed=seed)
    if batch is None:
        batch = make_batches(cfg, 1, 4, 512, seed, "cpu")[0]
    ids, mask, labels = (t.cpu() for t in batch[:3])
    pb = pack_varlen(ids, mask, labels)
    n = pb.input_ids.numel()
    g = torch.Generator().manual_seed(seed)
    d_final = torch.randn(n, cfg.hidden_size, generator=g)
    layer, head = [], []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        deq = ostack.dequant_model(model)
        lora = ostack.lora_leaves(model)
        final = ostack.stack_forward(model, deq, lora, pb.input_ids, pb.pos_ids, pb.row_lengths)
        final.backward(d_final)  # the layer's LoRA gradients
        t1 = time.perf_counter()
        layer.append(t1 - t0)
        if i < 4:  # the head is the slower part: a warm-up and three repetitions
            oref.lm_head_ce(final.detach().half(), model.embed, pb.shift_labels, need_grad=True)
            head.append(time.perf_counter() - t1)
    t_layer, t_head = statistics.median(layer[1:]), statistics.median(head[1:])
    t_step = cfg.num_hidden_layers * t_layer + t_head
    return {"value": n / t_step, "unit": "tokens/s", "cores": threads, "affinity_cores": affinity,
            "kind": "port",
            "sample": (f"oracle (eager fp32 torch + numpy NF4 dequant) on 1 of 28 config-5 layers "
                       f"+ lm_head over the bench's first batch ({n} packed tokens in "
                       f"{len(pb.row_lengths)} rows), fwd+bwd, medians of {reps} (layer) and 3 "
                       f"(lm_head) repetitions after a warm-up; "
                       f"per-step estimate 28*{t_layer:.3f}s + {t_head:.3f}s (lm_head); threads: "
                       f"this GPU's share of the host ({threads} of {affinity} affinity cores)")}


# ---------------------------------------------------------------------------------------------
# Per-configuration kernel records on cold inputs
# ---------------------------------------------------------------------------------------------

COLD_BYTES = 640 << 20  # input sets rotated per launch: > 2x the 256 MB last-level cache


def _n_sets(set_bytes: int, cap: int = 64) -> int:
    return max(2, min(cap, -(-COLD_BYTES // max(set_bytes, 1))))


def _time_rotating(launch, n_sets: int, reps: int) -> float:
    """Average µs per launch of ``launch(i)``, i cycling over the input sets: ``reps`` launches
    captured into one HIP graph (so the host's per-call cost is out of the measurement, as in
    the replayed training step), the graph replayed three times between one pair of HIP events
    on the current stream. Each launch reads a set the previous n_sets - 1 launches did not."""
    import torch

    for i in range(min(n_sets, 4)):
        launch(i)  # warm-up outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(reps):
            launch(i % n_sets)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1e3 / (3 * reps)


def _hbm(name, shape, us, nbytes, **extra):
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"kernel": name, "shape": shape, "gpu_us": us, "bytes": nbytes, "gbps": gbps,
            "bound": "hbm", "frac": gbps / HBM_PEAK_GBS, **extra}


def _mfma(name, shape, us, flops, **extra):
    tf = flops / (us * 1e-6) / 1e12
    return {"kernel": name, "shape": shape, "gpu_us": us, "flops": flops, "tflops": tf,
            "bound": "mfma", "frac": tf / FP16_PEAK_TFLOPS, **extra}


def _nf4_bytes(n: int, n_absmax2: int) -> int:
    return n // 2 + n // 64 + 4 * n_absmax2 + 1024 + 2 * n


def config_batch_lengths(seed: int = 0):
    from rus_amd.model import lengths_lognormal

    return lengths_lognormal(4, seed=seed)


def config_records(seed: int = 0, reps: int = 40) -> dict:
    """GPU time per kernel of BASELINE configs 1-4 at their shapes, each launch reading inputs
    not touched by the previous launches (rotating input sets of > 2x the last-level cache):
    averages over back-to-back launches between one event pair, with the algorithmic bytes or
    FLOPs and the fraction of the roofline."""
    import torch

    from rus_amd import kernels as K
    from rus_amd import ops as O
    from rus_amd import quant

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    out = {}

    def nf4_job(shapes):
        parts = [quant.quantize_nf4((torch.randn(r, c, device=dev, generator=g) * 0.02).half())
                 for r, c in shapes]
        fused, splits, offs, bases = quant.concat_segments(parts)
        return fused, splits, offs, bases

    def dequant_record(name, shapes):
        fused, splits, offs, bases = nf4_job(shapes)
        n = fused.shape[0] * fused.shape[1]
        nb = _nf4_bytes(n, fused.absmax2.numel())
        ns = _n_sets(nb)
        sets = [(fused.packed.clone(), fused.absmax.clone(), fused.absmax2.clone(),
                 torch.empty(n, dtype=torch.float16, device=dev)) for _ in range(ns)]
        code2 = fused.code2.to(dev)

        def launch(i):
            p, a, a2, o = sets[i]
            K.dequant_nf4_tensor(p, a, code2, a2, offs, fused.shape, out_buf=o,
                                 split_bytes=splits, absmax2_bases=bases)
        us = _time_rotating(launch, ns, reps)
        return _hbm(name, list(fused.shape), us, nb, input_sets=ns)

    # config 1: fused q|k|v dequant; residual + RMSNorm forward and backward [880, 1536]
    c1 = [dequant_record("nf4_dequant qkv", [(1536, 1536), (256, 1536), (256, 1536)])]
    N, D = 880, 1536
    w = (1 + 0.05 * torch.randn(D, device=dev, generator=g)).half()
    nbytes = 4 * N * D * 2 + 2 * D + 4 * N
    ns = _n_sets(nbytes)
    xs = [(torch.randn(N, D, device=dev, generator=g).half(),
           torch.randn(N, D, device=dev, generator=g).half()) for _ in range(ns)]
    fw = [K.rms_norm_fwd(x, w, 1e-6, residual=r) for x, r in xs]  # eager: the backward's inputs

    def norm_fwd(i):
        K.rms_norm_fwd(xs[i][0], w, 1e-6, residual=xs[i][1])
    c1.append(_hbm("rmsnorm_fwd residual", [N, D], _time_rotating(norm_fwd, ns, reps), nbytes,
                   input_sets=ns))

    def norm_bwd(i):
        y, h, rstd = fw[i]
        K.rms_norm_bwd(xs[i][0], h, w, rstd, dresidual=xs[i][1])
    # reads dy, h and dresidual, writes dx: four [N, D] arrays, the weight and rstd
    c1.append(_hbm("rmsnorm_bwd dresidual", [N, D], _time_rotating(norm_bwd, ns, reps),
                   4 * N * D * 2 + 2 * D + 4 * N, input_sets=ns))
    out["1"] = c1
    del xs, fw

    # config 2: the lm_head CE forward + backward at N=2048, V=151936 (token blocks of 768, 768
    # and 512: a [768, V] logit buffer)
    n2, V = 2048, 151936
    h = torch.randn(n2, D, device=dev, generator=g).half()
    W = (torch.randn(V, D, device=dev, generator=g) * 0.02).half()
    lab = torch.randint(0, V, (n2,), device=dev, generator=g)
    lab[torch.rand(n2, device=dev, generator=g) < 0.1] = -100
    wt = K.lm_head_weight_t(W)
    for _ in range(2):
        K.lm_head_ce(h, W, lab, weight_t=wt)
    torch.cuda.synchronize()
    timer = K.KernelTimer()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        K.lm_head_ce(h, W, lab, weight_t=wt)
    e1.record()
    torch.cuda.synchronize()
    head_us = e0.elapsed_time(e1) * 1e3 / 3
    with timer:
        for _ in range(3):
            K.lm_head_ce(h, W, lab, weight_t=wt)
    summ = timer.summary()
    flops = 2.0 * n2 * D * V
    c2 = [_mfma("lm_head_ce fwd+bwd (whole head)", [n2, D, V], head_us, 2 * flops,
                note="4*N*D*V over the whole head's time (logits GEMM, row statistics and "
                     "gradient, hidden-gradient GEMM, split-K reduce)")]
    for k in ("lmhead_ce_logits", "lmhead_ce_grad_hidden"):
        r = summ[k]
        us = r["ms"] * 1e3 / r["launches"]
        c2.append(_mfma(k, [r["launches"] // 3, "launches per head"], us,
                        r["flops"] / r["launches"], note="per launch (one token block)"))
    for k in ("lmhead_ce_rows", "lmhead_dh_reduce"):
        r = summ[k]
        us = r["ms"] * 1e3 / r["launches"]
        c2.append(_hbm(k, [r["launches"] // 3, "launches per head"], us, r["bytes"] / r["launches"]))
    # the engine's default layout: one pass over vocabulary chunks (the chunk chosen for the
    # token count), and the config's own V_CHUNK of 8192 rows
    for chunk, what in ((K.lm_head_chunk_cols(n2, V, K.cu_count(dev)), "chosen for N"),
                        (8192, "the config's V_CHUNK")):
        for _ in range(2):
            K.lm_head_ce(h, W, lab, weight_t=wt, v_chunk=chunk)
        e0.record()
        for _ in range(3):
            K.lm_head_ce(h, W, lab, weight_t=wt, v_chunk=chunk)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 3
        c2.append(_mfma(f"lm_head_ce fwd+bwd (single pass, chunks of {chunk} rows: {what})",
                        [n2, D, V], us, 2 * flops,
                        note="4*N*D*V over the whole pass (per chunk: statistics GEMM keeping "
                             "the logits, P = e^{z-M}, hidden-gradient GEMM into rescaled "
                             "partials; then combine and finish)"))
    out["2"] = c2
    del h, W, wt, lab

    # config 3: attention prologue / epilogue on a lognormal 4-row batch
    lens = config_batch_lengths(seed)
    n3 = sum(lens)
    cos, sin = O.rope_cache(2048, 128, 1e6, dev)
    pos = torch.cat([torch.arange(L, device=dev) for L in lens])
    per_tok_f, per_tok_b = 12296, 8712
    ns = _n_sets(n3 * per_tok_f)
    rs = [(torch.randn(n3, 2048, device=dev, generator=g).half(),
           torch.randn(n3, 1536, device=dev, generator=g).half(),
           torch.randn(n3, 256, device=dev, generator=g).half()) for _ in range(ns)]
    qkv_out = [K.qkv_rope_fwd(q, cos, sin, pos, ql, vl) for q, ql, vl in rs]  # eager

    def rope_f(i):
        qkv, ql, vl = rs[i]
        K.qkv_rope_fwd(qkv, cos, sin, pos, ql, vl)
    c3 = [_hbm("rope_fwd lora", [n3, 12, 2, 128], _time_rotating(rope_f, ns, reps),
               n3 * per_tok_f, input_sets=ns)]

    def rope_b(i):
        K.qkv_rope_bwd(*qkv_out[i], cos, sin, pos)
    c3.append(_hbm("rope_bwd", [n3, 12, 2, 128], _time_rotating(rope_b, ns, reps),
                   n3 * per_tok_b, input_sets=ns))
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32,
                      device=dev)
    att_flops = float(sum(2 * L * (L + 1) * 128 * 12 for L in lens))
    att = [K.attn_varlen_fwd(*qkv_out[i], cu) for i in range(ns)]  # eager: the backward's inputs

    def attn_f(i):
        q, k, v = qkv_out[i]
        K.attn_varlen_fwd(q, k, v, cu)
    c3.append(_mfma("attn_varlen_fwd", [n3, 12, 2, 128], _time_rotating(attn_f, ns, reps),
                    att_flops, note="causal FLOPs 4*h*d*sum L(L+1)/2"))

    def attn_b(i):
        q, k, v = qkv_out[i]
        o, lse = att[i]
        K.attn_varlen_bwd(o, q, k, v, o, lse, cu)
    c3.append(_mfma("attn_varlen_bwd", [n3, 12, 2, 128], _time_rotating(attn_b, ns, reps),
                    2.5 * att_flops))
    out["3"] = c3
    del rs, qkv_out, att

    # config 4: MLP block: [gate|up] and down dequant, SwiGLU forward / backward [880, 17920]
    c4 = [dequant_record("nf4_dequant gate|up", [(8960, 1536), (8960, 1536)]),
          dequant_record("nf4_dequant down", [(1536, 8960)])]
    I = 8960
    nbf, nbb = N * 3 * I * 2, N * 5 * I * 2
    ns = _n_sets(nbf)
    gus = [torch.randn(N, 2 * I, device=dev, generator=g).half() for _ in range(ns)]
    douts = [torch.randn(N, I, device=dev, generator=g).half() for _ in range(ns)]
    c4.append(_hbm("swiglu_fwd", [N, 2 * I], _time_rotating(lambda i: K.mlp_glu_fwd(gus[i]), ns, reps),
                   nbf, input_sets=ns))
    c4.append(_hbm("swiglu_bwd in place", [N, 2 * I],
                   _time_rotating(lambda i: K.mlp_glu_bwd(douts[i], gus[i]), ns, reps), nbb,
                   input_sets=ns))
    out["4"] = c4
    out["scaling"] = scaling_records(seed, reps)
    return out


def scaling_records(seed: int = 0, reps: int = 40) -> list:
    """The bandwidth-bound kernels at three sizes each: a launch of one row / token / unit (the
    fixed cost of a launch: dispatch, wave start, first-load latency, drain), the BASELINE
    configuration's shape, and a large shape whose transfer time dwarfs that fixed cost. Timed
    like the configuration records (graph-replayed launches over rotating input sets);
    ``frac_above_floor`` divides the algorithmic bytes by the time above the size-one launch."""
    import torch

    from rus_amd import kernels as K
    from rus_amd import ops as O
    from rus_amd import quant

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + 7)
    recs = []

    def add(name, size, us, nbytes, floor_us, ns):
        r = _hbm(name, size, us, nbytes, input_sets=ns)
        if floor_us is not None and us > floor_us:
            r["floor_us"] = floor_us
            r["frac_above_floor"] = nbytes / ((us - floor_us) * 1e-6) / 1e9 / HBM_PEAK_GBS
        recs.append(r)
        return us

    D = 1536
    w = (1 + 0.05 * torch.randn(D, device=dev, generator=g)).half()
    for tag, N in (("floor", 1), ("config", 880), ("large", 16384)):
        nbytes = 4 * N * D * 2 + 2 * D + 4 * N
        ns = _n_sets(nbytes)
        xs = [(torch.randn(N, D, device=dev, generator=g).half(),
               torch.randn(N, D, device=dev, generator=g).half()) for _ in range(ns)]
        fw = [K.rms_norm_fwd(x, w, 1e-6, residual=r) for x, r in xs]
        us_f = _time_rotating(lambda i: K.rms_norm_fwd(xs[i][0], w, 1e-6, residual=xs[i][1]),
                              ns, reps)
        us_b = _time_rotating(lambda i: K.rms_norm_bwd(xs[i][0], fw[i][1], w, fw[i][2],
                                                       dresidual=xs[i][1]), ns, reps)
        if tag == "floor":
            floor_nf, floor_nb = us_f, us_b
        add(f"rmsnorm_fwd residual ({tag})", [N, D], us_f, nbytes,
            None if tag == "floor" else floor_nf, ns)
        add(f"rmsnorm_bwd dresidual ({tag})", [N, D], us_b, nbytes,
            None if tag == "floor" else floor_nb, ns)
        del xs, fw
    cos, sin = O.rope_cache(2048, 128, 1e6, dev)
    for tag, n in (("floor", 1), ("config", 876), ("large", 16384)):
        pos = (torch.arange(n, device=dev) % 2048)
        ns = _n_sets(n * 12296)
        rs = [(torch.randn(n, 2048, device=dev, generator=g).half(),
               torch.randn(n, 1536, device=dev, generator=g).half(),
               torch.randn(n, 256, device=dev, generator=g).half()) for _ in range(ns)]
        outs = [K.qkv_rope_fwd(q, cos, sin, pos, ql, vl) for q, ql, vl in rs]
        us_f = _time_rotating(lambda i: K.qkv_rope_fwd(rs[i][0], cos, sin, pos, rs[i][1],
                                                       rs[i][2]), ns, reps)
        us_b = _time_rotating(lambda i: K.qkv_rope_bwd(*outs[i], cos, sin, pos), ns, reps)
        if tag == "floor":
            floor_rf, floor_rb = us_f, us_b
        add(f"rope_fwd lora ({tag})", [n, 12, 2, 128], us_f, n * 12296,
            None if tag == "floor" else floor_rf, ns)
        add(f"rope_bwd ({tag})", [n, 12, 2, 128], us_b, n * 8712,
            None if tag == "floor" else floor_rb, ns)
        del rs, outs
    I = 8960
    for tag, N in (("floor", 1), ("config", 880), ("large", 8192)):
        nbf, nbb = N * 3 * I * 2, N * 5 * I * 2
        ns = _n_sets(nbf)
        gus = [torch.randn(N, 2 * I, device=dev, generator=g).half() for _ in range(ns)]
        douts = [torch.randn(N, I, device=dev, generator=g).half() for _ in range(ns)]
        us_f = _time_rotating(lambda i: K.mlp_glu_fwd(gus[i]), ns, reps)
        us_b = _time_rotating(lambda i: K.mlp_glu_bwd(douts[i], gus[i]), ns, reps)
        if tag == "floor":
            floor_sf, floor_sb = us_f, us_b
        add(f"swiglu_fwd ({tag})", [N, 2 * I], us_f, nbf,
            None if tag == "floor" else floor_sf, ns)
        add(f"swiglu_bwd in place ({tag})", [N, 2 * I], us_b, nbb,
            None if tag == "floor" else floor_sb, ns)
        del gus, douts
    for tag, shape in (("floor", (64, 64)), ("config qkv", (2048, 1536)),
                       ("large", (8192, 8192))):
        part = quant.quantize_nf4((torch.randn(*shape, device=dev, generator=g) * 0.02).half())
        n = shape[0] * shape[1]
        nb = _nf4_bytes(n, part.absmax2.numel())
        ns = _n_sets(nb)
        sets = [(part.packed.clone(), part.absmax.clone(), part.absmax2.clone(),
                 torch.empty(n, dtype=torch.float16, device=dev)) for _ in range(ns)]
        code2 = part.code2.to(dev)

        def launch(i):
            p_, a_, a2_, o_ = sets[i]
            K.dequant_nf4_tensor(p_, a_, code2, a2_, part.offset, shape, out_buf=o_)
        us = _time_rotating(launch, ns, reps)
        if tag == "floor":
            floor_dq = us
        add(f"nf4_dequant ({tag})", list(shape), us, nb, None if tag == "floor" else floor_dq, ns)
        del sets
    torch.cuda.empty_cache()
    return recs


def config_cpu_times(seed: int = 0) -> dict:
    """CPU oracle times for the configuration records (bench.py's CPU-baseline leg): the same
    operations on the host cores (fp32 torch / numpy restatement of the reference's arithmetic),
    median of 3, bounded samples where the full shape would take minutes."""
    import numpy as np
    import torch

    from oracle import ops as ref
    from rus_amd import quant

    g = torch.Generator().manual_seed(seed)
    out = {}

    def med(fn, n=3):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts) * 1e6

    def nf4(shapes):
        parts = [quant.quantize_nf4((torch.randn(r, c, generator=g) * 0.02).half()) for r, c in shapes]
        fused, splits, offs, bases = quant.concat_segments(parts)
        args = (fused.packed.numpy(), fused.absmax.numpy(), fused.code2.numpy(),
                fused.absmax2.numpy(), offs, fused.shape)
        return lambda: ref.nf4_dequant(*args, split_bytes=splits, absmax2_bases=bases)

    N, D, I = 880, 1536, 8960
    x, res = torch.randn(N, D, generator=g).half(), torch.randn(N, D, generator=g).half()
    w = (1 + 0.05 * torch.randn(D, generator=g)).half()
    y, h, rstd = ref.rms_norm_fwd(x, w, 1e-6, residual=res)
    out["1"] = {"nf4_dequant qkv": med(nf4([(1536, 1536), (256, 1536), (256, 1536)])),
                "rmsnorm_fwd residual": med(lambda: ref.rms_norm_fwd(x, w, 1e-6, residual=res)),
                "rmsnorm_bwd dresidual": med(lambda: ref.rms_norm_bwd(x, h, w, rstd, dresidual=res))}
    # config 2 on 256 of the 2048 tokens (per-token work; scaled by 8)
    V, n2 = 151936, 256
    hh = torch.randn(n2, D, generator=g).half()
    W = (torch.randn(V, D, generator=g) * 0.02).half()
    lab = torch.randint(0, V, (n2,), generator=g)
    t = med(lambda: ref.lm_head_ce(hh, W, lab, need_grad=True), n=1)
    out["2"] = {"lm_head_ce fwd+bwd (whole head)": t * (2048 / n2)}
    lens = config_batch_lengths(seed)
    n3 = sum(lens)
    cos, sin = ref.rope_tables(2048, 128, 1e6)
    pos = torch.cat([torch.arange(L) for L in lens])
    qkv = torch.randn(n3, 2048, generator=g).half()
    ql, vl = torch.randn(n3, 1536, generator=g).half(), torch.randn(n3, 256, generator=g).half()
    q, k, v = ref.qkv_rope_fwd(qkv, cos, sin, pos, ql, vl)
    cu = [0] + list(np.cumsum(lens))
    out["3"] = {"rope_fwd lora": med(lambda: ref.qkv_rope_fwd(qkv, cos, sin, pos, ql, vl)),
                "rope_bwd": med(lambda: ref.qkv_rope_bwd(q, k, v, cos, sin, pos)),
                "attn_varlen_fwd": med(lambda: ref.attention_varlen_fwd(q, k, v, cu), n=1),
                "attn_varlen_bwd": med(lambda: ref.attention_varlen_bwd(q, q, k, v, cu), n=1)}
    gg, uu = torch.randn(N, I, generator=g).half(), torch.randn(N, I, generator=g).half()
    do = torch.randn(N, I, generator=g).half()
    out["4"] = {"nf4_dequant gate|up": med(nf4([(8960, 1536), (8960, 1536)]), n=1),
                "nf4_dequant down": med(nf4([(1536, 8960)]), n=1),
                "swiglu_fwd": med(lambda: ref.swiglu_fwd(gg, uu)),
                "swiglu_bwd in place": med(lambda: ref.swiglu_bwd(do, gg, uu))}
    return out


def _calibration_copies(dev, reps: int = 5) -> None:
    """Five plain 128 MiB device-to-device copies: what FETCH_SIZE / WRITE_SIZE read for a known
    number of bytes (the first copy kernels of a probe run; ``counter_summary`` scales by them)."""
    import torch

    src = torch.empty(64 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"probe: {reps} copies of {src.numel() * 2} bytes", flush=True)


def elementwise_probe(reps: int = 5) -> None:
    """Fixed launches for counter runs of the bandwidth-bound kernels at their BASELINE shapes,
    each launch on input sets no earlier launch touched (so HBM, not the last-level cache,
    serves them): RMSNorm forward / backward [880, 1536], RoPE forward (LoRA) / backward on the
    config-3 batch, SwiGLU forward / backward [880, 17920]; plus 5 plain 128 MiB device copies
    (the counters' calibration)."""
    import torch

    from rus_amd import kernels as K
    from rus_amd import ops as O

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    src = torch.empty(64 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    N, D, I = 880, 1536, 8960
    w = (1 + 0.05 * torch.randn(D, device=dev, generator=g)).half()
    xs = [(torch.randn(N, D, device=dev, generator=g).half(),
           torch.randn(N, D, device=dev, generator=g).half()) for _ in range(reps)]
    fw = [K.rms_norm_fwd(x, w, 1e-6, residual=r) for x, r in xs]
    for (x, r), (y, h, rstd) in zip(xs, fw):
        K.rms_norm_bwd(x, h, w, rstd, dresidual=r)
    lens = config_batch_lengths(0)
    n3 = sum(lens)
    cos, sin = O.rope_cache(2048, 128, 1e6, dev)
    pos = torch.cat([torch.arange(L, device=dev) for L in lens])
    rs = [(torch.randn(n3, 2048, device=dev, generator=g).half(),
           torch.randn(n3, 1536, device=dev, generator=g).half(),
           torch.randn(n3, 256, device=dev, generator=g).half()) for _ in range(reps)]
    qkvs = [K.qkv_rope_fwd(q, cos, sin, pos, ql, vl) for q, ql, vl in rs]
    for q, k, v in qkvs:
        K.qkv_rope_bwd(q, k, v, cos, sin, pos)
    gus = [torch.randn(N, 2 * I, device=dev, generator=g).half() for _ in range(reps)]
    outs = [K.mlp_glu_fwd(gu) for gu in gus]
    for gu, o in zip(gus, outs):
        K.mlp_glu_bwd(o, gu)
    torch.cuda.synchronize()
    print(f"probe: {reps} launches each of rmsnorm fwd/bwd [{N},{D}], rope fwd/bwd "
          f"[{n3} tokens], swiglu fwd/bwd [{N},{2 * I}] on distinct inputs", flush=True)
    del xs, fw, rs, qkvs, gus, outs
    # the same kernels at large shapes (transfer time >> the launch's fixed cost), 3 launches
    # each over 2 input sets
    NL = 16384
    xs = [(torch.randn(NL, D, device=dev, generator=g).half(),
           torch.randn(NL, D, device=dev, generator=g).half()) for _ in range(2)]
    fw = [K.rms_norm_fwd(xs[i % 2][0], w, 1e-6, residual=xs[i % 2][1]) for i in range(3)]
    for i, (y, h, rstd) in enumerate(fw):
        K.rms_norm_bwd(xs[i % 2][0], h, w, rstd, dresidual=xs[i % 2][1])
    del xs, fw
    posl = torch.arange(NL, device=dev) % 2048
    rs = [(torch.randn(NL, 2048, device=dev, generator=g).half(),
           torch.randn(NL, 1536, device=dev, generator=g).half(),
           torch.randn(NL, 256, device=dev, generator=g).half()) for _ in range(2)]
    qkvs = [K.qkv_rope_fwd(*rs[i % 2][:1], cos, sin, posl, *rs[i % 2][1:]) for i in range(3)]
    for q, k, v in qkvs:
        K.qkv_rope_bwd(q, k, v, cos, sin, posl)
    del rs, qkvs
    NS = 8192
    gus = [torch.randn(NS, 2 * I, device=dev, generator=g).half() for _ in range(2)]
    outs = [K.mlp_glu_fwd(gus[i % 2]) for i in range(3)]
    for i, o in enumerate(outs):
        K.mlp_glu_bwd(o, gus[i % 2])
    torch.cuda.synchronize()
    print(f"probe: 3 launches each of rmsnorm fwd/bwd [{NL},{D}], rope fwd/bwd [{NL} tokens], "
          f"swiglu fwd/bwd [{NS},{2 * I}]", flush=True)


def lmhead_probe(reps: int = 5, single_pass: bool = False) -> None:
    """Fixed launches for counter runs of the lm_head CE kernels at BASELINE config 2: hidden
    [2048, 1536] ~ N(0,1), W [151936, 1536] ~ N(0, 0.02), 10% labels -100, whole vocabulary per
    pass (forward statistics, logit gradient, hidden gradient): the token-blocked head, or with
    ``single_pass`` the engine's default one pass over vocabulary chunks (the chunk chosen for
    N), one pass first under the per-launch timer, which prints each launcher's algorithmic
    bytes / FLOPs per launch."""
    import torch

    from rus_amd import kernels as K
    from rus_amd.kernels import KernelTimer

    dev = torch.device("cuda:0")
    _calibration_copies(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    n, d, v = 2048, 1536, 151936
    h = torch.randn(n, d, device=dev, generator=g).half()
    w = (torch.randn(v, d, device=dev, generator=g) * 0.02).half()
    lab = torch.randint(0, v, (n,), device=dev, generator=g)
    lab[torch.rand(n, device=dev, generator=g) < 0.1] = -100
    wt = K.lm_head_weight_t(w)
    chunk = K.lm_head_chunk_cols(n, v, K.cu_count(dev)) if single_pass else None
    torch.cuda.synchronize()
    if single_pass:
        K.lm_head_ce(h, w, lab, weight_t=wt, v_chunk=chunk)
        torch.cuda.synchronize()
        with KernelTimer() as timer:
            K.lm_head_ce(h, w, lab, weight_t=wt, v_chunk=chunk)
        for name, r in sorted(timer.summary().items()):
            print(json.dumps({"launcher": name, "launches_per_pass": r["launches"],
                              "bytes_per_launch": r["bytes"] / r["launches"],
                              "flops_per_launch": r["flops"] / r["launches"]}), flush=True)
    for _ in range(reps):
        K.lm_head_ce(h, w, lab, weight_t=wt, v_chunk=chunk)
    torch.cuda.synchronize()
    what = f"single passes over {chunk}-row vocabulary chunks" if single_pass else "passes"
    print(f"probe: {reps} lm_head CE forward+gradient {what} at N={n}, V={v}, d={d}", flush=True)


def kernel_probe(reps: int = 5) -> None:
    """Fixed launches for hardware-counter runs: a plain 128 MiB device copy (the calibration for
    the FETCH_SIZE / WRITE_SIZE counters) and one config-5 layer's four-segment NF4 dequant
    carrying a residual + RMSNorm forward of a 707-token batch, as in the train step."""
    import torch

    from rus_amd import model as M
    from rus_amd.hostload import WeightStream

    dev = torch.device("cuda:0")
    _calibration_copies(dev)
    cfg = M.qwen2_1p5b()
    cfg1 = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": 1})
    model = M.build_random_qlora_qwen2(cfg1, dev, seed=0)
    ws = WeightStream(model.layers, dev, resident=True)
    from rus_amd import kernels as K

    x = torch.randn(707, cfg.hidden_size, device=dev).half()
    res = torch.randn_like(x)
    lnw = torch.ones(cfg.hidden_size, device=dev)
    for _ in range(reps):
        *_, pend = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
        ws.dequant_layer(0, norm=pend)
    torch.cuda.synchronize()
    print(f"probe: {reps} four-segment dequants of layer 0 with a riding norm forward", flush=True)
    y, h, rstd = K.rms_norm_fwd(x, lnw, 1e-6, residual=res)
    for _ in range(reps):
        _, pend = K.rms_norm_bwd(x, h, lnw, rstd, dresidual=res, defer=True)
        ws.dequant_layer(0, norm=pend)
    torch.cuda.synchronize()
    print(f"probe: {reps} four-segment dequants of layer 0 with a riding norm backward", flush=True)
    # the step's form: the input norm forward and the q / v LoRA-down (rank 16, dropout 0.05
    # keep bits) ride in the layer's dequant launch
    L0 = model.layers[0]
    a_q, a_v = L0.q_A.detach().half().contiguous(), L0.v_A.detach().half().contiguous()
    seed = torch.tensor([7], dtype=torch.int64, device=dev)
    bits_q, bits_v = K.dropout_keep_bits(seed, 0, 2, x.shape[0], cfg.hidden_size, 0.05, 0.05)
    for _ in range(reps):
        *_, pend = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
        pend.carry_lora_down(a_q, a_v, bits_q, bits_v, 0.05, 0.05)
        ws.dequant_layer(0, norm=pend)
    torch.cuda.synchronize()
    print(f"probe: {reps} four-segment dequants of layer 0 carrying the norm forward and the "
          f"LoRA-down", flush=True)


def gemm_parts_probe(reps: int = 5, n_tok: int = 707) -> None:
    """Fixed launches for hardware-counter runs: the plain 128 MiB device copy (the counters'
    calibration), then the step's split-K MLP input gradient at the bench's mean batch,
    d_gu [707, 17920] x W_gu [17920, 1536] into fp32 partials with the engine's split count,
    each launch reading one of 4 weight sets (cold, as in the step)."""
    import torch

    from rus_amd import ops as O

    dev = torch.device("cuda:0")
    src = torch.empty(64 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"probe: {reps} copies of {src.numel() * 2} bytes", flush=True)
    del src, dst
    g = torch.Generator(device=dev).manual_seed(0)
    ws = [(torch.randn(17920, 1536, device=dev, generator=g) * 0.02).half() for _ in range(4)]
    x = torch.randn(n_tok, 17920, device=dev, generator=g).half()
    parts = None
    for i in range(reps):
        parts = O._input_grad_parts(x, ws[i % 4])
    torch.cuda.synchronize()
    sp = parts.shape[0]
    nbytes = (n_tok * 17920 + 17920 * 1536) * 2 + 4 * sp * n_tok * 1536
    print(f"probe: {reps} split-K products [{n_tok}, 17920] x [17920, 1536], {sp} partials, "
          f"{nbytes} algorithmic bytes per launch", flush=True)
    del ws, x, parts


def step_probe(steps: int = 3) -> None:
    """Fixed work for counter runs of every kernel in its in-step form: 5 plain 128 MiB device
    copies (the FETCH_SIZE / WRITE_SIZE calibration), then eager training steps (the bench's
    engine settings, AdamW) on the bench's first batch. One step runs under the per-launch timer
    first and prints each launcher's launches and algorithmic bytes / FLOPs per step."""
    import torch

    from rus_amd import model as M
    from rus_amd.kernels import KernelTimer
    from rus_amd.ops import Qwen2FusedEngine

    dev = torch.device("cuda:0")
    src = torch.empty(64 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    print(f"probe: 5 copies of {128 << 20} bytes", flush=True)
    cfg = M.qwen2_1p5b()
    model = M.build_random_qlora_qwen2(cfg, dev, seed=0)
    batch = make_batches(cfg, 1, 4, 512, 0, dev)[0]
    engine = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit="model",
                              recompute=False, dequant_once=True)
    opt = flat_adamw(engine)[0]
    train_step(engine, opt, batch)
    torch.cuda.synchronize()
    with KernelTimer() as timer:
        train_step(engine, opt, batch)
    for name, r in sorted(timer.summary().items()):
        print(json.dumps({"launcher": name, "launches_per_step": r["launches"],
                          "bytes_per_launch": r["bytes"] / r["launches"],
                          "flops_per_launch": r["flops"] / r["launches"]}), flush=True)
    for _ in range(steps):
        train_step(engine, opt, batch)
    torch.cuda.synchronize()
    print(f"probe: {steps} eager steps of {batch[3]} tokens after the timed one", flush=True)


def counter_summary(paths: list[str]) -> None:
    """Per-kernel averages of rocprofv3 counter runs (``--pmc ... --output-format csv``
    counter_collection files): dispatches, mean duration under collection, and each counter per
    dispatch. FETCH_SIZE / WRITE_SIZE are also given in MB scaled by what they read for the
    largest plain device copy in the same file (bytes moved / counter), the calibration."""
    import collections
    import csv
    import re

    for path in paths:
        rows = list(csv.DictReader(open(path)))
        agg = collections.defaultdict(lambda: collections.defaultdict(list))
        dur = collections.defaultdict(dict)
        for r in rows:
            k = (_kernel_label(r["Kernel_Name"]), int(r["Grid_Size"]))  # one line per launch shape
            agg[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
            dur[k][r["Dispatch_Id"]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        # calibration: the five plain 128 MiB device copies every probe runs before anything else
        # (the first five copy kernels of the run; later copy kernels also move host data)
        fetch_f = write_f = None
        copies = sorted({int(r["Dispatch_Id"]) for r in rows if "copyBuffer" in r["Kernel_Name"]})
        early = [r for r in rows if int(r["Dispatch_Id"]) in set(copies[:5])]
        if early:
            big = max(int(r["Grid_Size"]) for r in early)
            cal = [(c, [float(r["Counter_Value"]) for r in early
                        if r["Counter_Name"] == c and int(r["Grid_Size"]) == big])
                   for c in ("FETCH_SIZE", "WRITE_SIZE")]
            for c, vals in cal:
                if vals:
                    f = (128 << 20) / 1024 / (sum(vals) / len(vals))
                    if c == "FETCH_SIZE":
                        fetch_f = f
                    else:
                        write_f = f
        print(f"## {path}")
        if fetch_f or write_f:
            print(f"calibration (128 MiB copy): fetch factor {fetch_f}, write factor {write_f}")
        print("| kernel | grid | dispatches | mean us | counter | per dispatch | scaled MB |")
        print("|---|---|---|---|---|---|---|")
        for k, cs in sorted(agg.items(), key=lambda kv: -sum(dur[kv[0]].values())):
            us = sum(dur[k].values()) / len(dur[k]) / 1e3
            for c, v in sorted(cs.items()):
                m = sum(v) / len(v)
                f = fetch_f if c == "FETCH_SIZE" else write_f if c == "WRITE_SIZE" else None
                mb = f"{m * 1024 * f / 1e6:.2f}" if f else ""
                print(f"| {k[0]} | {k[1]} | {len(dur[k])} | {us:.2f} | {c} | {m:.1f} | {mb} |")


def _print_record(rec: dict) -> None:
    print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v) for k, v in rec.items()}),
          flush=True)


def ceilings_probe(reps: int = 40) -> None:
    """Streaming rates of this GPU at the per-layer dequant's traffic (config 5: 23.5 MB of
    packed codes read, 94 MB of fp16 written), each launch on buffers the previous launches did
    not touch: torch ``fill_`` (write only), ``copy_`` (1 byte read per byte written), a 1:4
    broadcast copy (the dequant's read:write ratio) and the dequant launch itself (four segments
    of one layer, no riding norm). Prints one JSON record per measurement."""
    import torch

    from rus_amd import model as M
    from rus_amd.hostload import WeightStream

    dev = torch.device("cuda:0")
    cfg = M.qwen2_1p5b()
    out_bytes = 94_175_232  # one layer's fp16 weights: 2 x 47,087,616 parameters
    n_out = out_bytes // 2
    sets = _n_sets(out_bytes + out_bytes // 4)
    outs = [torch.empty(n_out, dtype=torch.float16, device=dev) for _ in range(sets)]
    ins = [torch.randn(n_out // 4, device=dev).half() for _ in range(sets)]
    recs = [
        _hbm("torch fill_ (write only)", [n_out], _time_rotating(
            lambda i: outs[i].fill_(1.0), sets, reps), out_bytes),
        _hbm("torch copy_ (1:1)", [n_out // 4], _time_rotating(
            lambda i: outs[i][: n_out // 4].copy_(ins[i]), sets, reps), out_bytes // 2),
        _hbm("torch broadcast copy (1:4 read:write)", [n_out // 4, 4], _time_rotating(
            lambda i: outs[i].view(-1, 4).copy_(ins[i].view(-1, 1).expand(-1, 4)), sets, reps),
            out_bytes + out_bytes // 4),
    ]
    del outs, ins
    torch.cuda.empty_cache()
    cfg_n = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": sets})
    model = M.build_random_qlora_qwen2(cfg_n, dev, seed=0)
    ws = WeightStream(model.layers, dev, resident=True)
    spaces = [{k: torch.empty_like(v) for k, v in ws.workspaces.items()} for _ in range(sets)]
    n_abs2 = sum(sg.absmax2_slice.stop - sg.absmax2_slice.start
                 for sg in ws.layer_segments[0].values())
    dq_bytes = _nf4_bytes(n_out, n_abs2)
    recs.append(_hbm("rus nf4 dequant, 4 segments", [n_out], _time_rotating(
        lambda i: ws.dequant_layer(i, workspaces=spaces[i]), sets, reps), dq_bytes))
    for r in recs:
        r["sets"] = sets
        _print_record(r)


def contention_probe(steps: int = 24, warmup: int = 8) -> None:
    """Device time of one captured step's replay (events after its copy wait, mean over whole
    cycles of the bench's 8 batches) for (a) HBM-resident weights; (b) the same resident graph
    while an unrelated host-to-device copy of the model image's size loops on a side stream;
    (c) the resident graph with one such copy per step on the side stream and each step waiting
    (a stream wait) for the previous step's copy; (d) the bench's streamed engine (whose own
    per-step copy runs beside it and gates the next step). Shows which of a concurrent PCIe
    copy and a step tied to the copies lengthens the replay, and (copy events on the side or
    copy stream) how long the copies take meanwhile and how much of the replays' time a copy ran
    beside. Prints JSON records."""
    import torch

    from rus_amd import model as M
    from rus_amd.graph import GraphedTrainStep
    from rus_amd.ops import Qwen2FusedEngine

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = M.qwen2_1p5b()
    model = M.build_random_qlora_qwen2(cfg, dev, seed=0)
    batches = make_batches(cfg, 8, 4, 512, 0, dev)

    copy_marks = []

    def timed_copy(st=None):  # on a side stream (default: ``side``)
        st = side if st is None else st
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        with torch.cuda.stream(st):
            dst.copy_(host, non_blocking=True)
        e1.record(st)
        copy_marks.append((e0, e1))

    def replays(engine, side_copy=None, tied=False):
        g = GraphedTrainStep(engine, bucket=64)
        for b in batches:
            g.prepare(b[0], b[1], b[2])
        opt = flat_adamw(engine)[0]
        copy_marks.clear()
        torch.cuda.synchronize()
        ref = torch.cuda.Event(enable_timing=True)  # time origin of the copy / replay intervals
        ref.record()
        if side_copy is not None:
            side_copy()
        ws = engine.weight_stream
        if ws.unit == "model":
            ws.time_copies()
        begin = ws.begin_step
        if tied:  # each step copies once on the side stream and waits for the previous copy
            done = []

            def begin_tied():
                buf = begin()
                if done:
                    torch.cuda.current_stream(dev).wait_event(done[-1])
                with torch.cuda.stream(side):
                    timed_copy()
                    done.append(torch.cuda.Event())
                    done[-1].record(side)
                return buf

            ws.begin_step = begin_tied
        for i in range(warmup):
            train_step(engine, opt, batches[i % len(batches)], g)
        g.time_replays()
        for i in range(steps):
            train_step(engine, opt, batches[(warmup + i) % len(batches)], g)
        rmarks = list(g.replay_marks)
        ms = g.replay_ms()
        torch.cuda.synchronize()
        ws.begin_step = begin
        cmarks = list(ws.copy_marks or []) if ws.unit == "model" else list(copy_marks)
        if ws.unit == "model":
            ws.time_copies(False)
        # how much of the timed replays' device time a copy ran beside (0 when the copies and the
        # replays were serialised, e.g. by sharing a hardware queue)
        civ = [(ref.elapsed_time(a), ref.elapsed_time(b)) for a, b in cmarks]
        riv = [(ref.elapsed_time(a), ref.elapsed_time(b)) for a, b in rmarks]
        ov = sum(max(0.0, min(r1, c1) - max(r0, c0)) for r0, r1 in riv for c0, c1 in civ)
        overlap = ov / sum(r1 - r0 for r0, r1 in riv) if civ else None
        # the copies that ran beside timed replays: drop the warm-up's and the loop's tail
        cms = [c1 - c0 for c0, c1 in civ][warmup:warmup + steps]
        return (statistics.fmean(ms), [round(x, 3) for x in ms[:8]], [round(x, 3) for x in ms[-8:]],
                statistics.fmean(cms) if cms else None, overlap)

    eng_s = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit="model",
                             recompute=False, dequant_once=True)
    image_bytes = eng_s.weight_stream.model_bytes
    eng_r = Qwen2FusedEngine(model, dev, resident_weights=True, recompute=False,
                             dequant_once=True)
    host = torch.empty(image_bytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(image_bytes, dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream(device=dev)  # default priority

    def copy_loop(st=None):  # enough copies to outlast the warm-up and timed replays
        for _ in range(warmup + steps + 8):
            timed_copy(st)

    # four more side streams created together: HIP maps a process's streams onto a few hardware
    # queues, so one of them may share the replaying stream's queue (copies and replays then
    # serialise: overlap 0)
    fresh = [torch.cuda.Stream(device=dev) for _ in range(4)]
    cases = [("resident weights", eng_r, None, False),
             ("resident weights + side-stream H2D copy loop", eng_r, copy_loop, False),
             ("resident weights + one side-stream H2D copy per step, each step waiting for the "
              "previous step's copy", eng_r, None, True),
             ("streamed weights (bench default)", eng_s, None, False)]
    cases += [(f"resident weights + the H2D copy loop on fresh side stream {k} of 4", eng_r,
               (lambda st=st: copy_loop(st)), False) for k, st in enumerate(fresh)]
    recs = []
    for label, eng, loop, tied in cases:
        mean, first, last, copy_ms, overlap = replays(eng, loop, tied)
        torch.cuda.synchronize()
        recs.append({"probe": "contention", "case": label, "replay_ms_mean": mean,
                     "replay_ms_first8": first, "replay_ms_last8": last, "steps": steps,
                     "warmup": warmup,
                     "copy_bytes": image_bytes if loop or tied or eng is eng_s else 0,
                     "copy_ms_mean": copy_ms, "copy_overlap_of_replay_time": overlap})
    for r in recs:
        _print_record(r)


def gemm_probe(reps: int = 20) -> None:
    """Per-product GPU time of one config-5 layer at the bench batch's token count (the eight
    projections: F.linear / the input-gradient torch.mm on dequantised fp16 weights, i.e.
    hipBLASLt, against the fused NF4 products rus_nf4_gemm), the layer's dequant launch, and the
    lm_head's two GEMMs of one 256-token block against hipBLASLt on the same operands. Weights
    rotate over several layers so each launch reads them from HBM. Prints JSON records."""
    import torch
    import torch.nn.functional as F

    from rus_amd import kernels as K
    from rus_amd import model as M
    from rus_amd import ops as O
    from rus_amd.hostload import SEGMENTS, WeightStream

    dev = torch.device("cuda:0")
    cfg = M.qwen2_1p5b()
    n_tok = sum(config_batch_lengths(0))
    sets = 4
    cfg_n = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": sets})
    model = M.build_random_qlora_qwen2(cfg_n, dev, seed=0)
    ws = WeightStream(model.layers, dev, resident=True)
    w16 = []
    for i in range(sets):
        spaces = {k: torch.empty_like(v) for k, v in ws.workspaces.items()}
        w16.append(ws.dequant_layer(i, workspaces=spaces))
    nf4 = [ws.nf4_layer(i) for i in range(sets)]
    g = torch.Generator(device=dev).manual_seed(0)
    tot = {"hipblaslt": 0.0, "engine": 0.0, "fused": 0.0}
    for name in SEGMENTS:
        rows, cols = w16[0][name].shape
        for trans in (False, True):
            k_in, n_out = (rows, cols) if trans else (cols, rows)
            x = torch.randn(n_tok, k_in, device=dev, generator=g).half()
            if trans:
                lib = lambda i: torch.mm(x, w16[i][name])
                eng = lambda i: O._mm_w(x, w16[i][name])
                fused = lambda i: K.nf4_gemm(x, nf4[i][name], trans=True)
            else:
                lib = lambda i: F.linear(x, w16[i][name])
                eng = lambda i: O._lin(x, w16[i][name])
                fused = lambda i: K.nf4_gemm(x, nf4[i][name])
            flops = 2.0 * n_tok * k_in * n_out
            shape = [n_tok, k_in, n_out]
            label = f"{name} {'input-grad' if trans else 'forward'}"
            split = k_in >= O.SPLIT_K_MIN
            kinds = [("hipblaslt", lib), ("fused", fused)]
            if split:
                kinds.insert(1, ("engine", eng))
            for kind, fn in kinds:
                us = _time_rotating(fn, sets, reps)
                tot[kind] += us
                if kind == "hipblaslt" and not split:
                    tot["engine"] += us  # the engine calls the library GEMM as is
                _print_record(_mfma(f"{label} {kind}", shape, us, flops))
            for sp in (2, 4, 7) if split else ():  # the batched GEMM of sp slices + its reduce
                if k_in % sp:
                    continue
                if trans:
                    part = lambda i: O._split_k_parts(x, w16[i][name], sp)
                else:  # x [M, K] @ W[D, K]^T over K slices
                    wk = lambda i: w16[i][name].view(n_out, sp, k_in // sp).permute(1, 2, 0)
                    part = lambda i: torch.bmm(x.view(n_tok, sp, k_in // sp).permute(1, 0, 2),
                                               wk(i), out_dtype=torch.float32)
                us_p = _time_rotating(part, sets, reps)
                pr = part(0)
                us_r = _time_rotating(lambda i: K.sum_splits(pr, x.dtype), sets, reps)
                _print_record(_mfma(f"{label} split-K {sp}", shape, us_p + us_r, flops,
                                    batched_gemm_us=us_p, reduce_us=us_r))
    dq = _time_rotating(lambda i: ws.dequant_layer(i), sets, reps)
    _print_record({"kernel": "layer dequant (4 segments)", "gpu_us": dq})
    _print_record({"kernel": "layer total", "dequant_plus_hipblaslt_us": tot["hipblaslt"] + 2 * dq,
                   "dequant_plus_engine_products_us": tot["engine"] + 2 * dq,
                   "fused_us": tot["fused"], "note": "dequant once per pass (forward, backward)"})
    del w16, nf4, ws, model
    torch.cuda.empty_cache()
    # lm_head: one 256-token block against the whole vocabulary
    nb, d, V = 256, cfg.hidden_size, cfg.vocab_size
    h = torch.randn(nb, d, device=dev, generator=g).half()
    w = (torch.randn(V, d, device=dev, generator=g) * 0.02).half()
    wt = K.lm_head_weight_t(w)
    kp = _round_up(V, 64)
    z = torch.empty((nb, kp), dtype=torch.float16, device=dev)
    zl = torch.empty((nb, V), dtype=torch.float16, device=dev)
    splits = K.lm_head_split_count(nb, d, V, K.cu_count(dev))
    parts = torch.empty((splits, nb, d), dtype=torch.float32, device=dev)
    dh = torch.empty((nb, d), dtype=torch.float16, device=dev)
    fl = 2.0 * nb * d * V
    for kind, fn in (("rus lmhead_ce_logits", lambda i: K.lm_head_ce_logits(h, w, z)),
                     ("hipblaslt h W^T", lambda i: torch.mm(h, w.t(), out=zl))):
        _print_record(_mfma(f"lm_head logits {kind}", [nb, d, V], _time_rotating(fn, 1, reps), fl))
    for kind, fn in (("rus lmhead_ce_grad_hidden", lambda i: K.lm_head_ce_grad_hidden(
                         z, wt, V, parts, accumulate=False)),
                     ("hipblaslt G W", lambda i: torch.mm(zl, w, out=dh))):
        _print_record(_mfma(f"lm_head hidden grad {kind}", [nb, V, d],
                            _time_rotating(fn, 1, reps), fl, splits=splits))


def _kernel_label(name: str) -> str:
    """Short label of a kernel-trace name: hipBLASLt kernels as one label; demangled names cut at
    their argument list; mangled ones (the profiler leaves templates over _Float16 mangled) as
    name<template arguments, still mangled>, so instantiations stay apart."""
    import re

    if name.startswith(("Cijk", "Custom_Cijk")):
        return "hipBLASLt GEMMs"
    m = re.match(r"_ZN3rus12_GLOBAL__N_1(\d+)", name)
    if m:
        rest = name[m.end():]
        ident, rest = rest[:int(m.group(1))], rest[int(m.group(1)):]
        if rest.startswith("I") and "EE" in rest:
            return f"{ident}<{rest[1:rest.index('EE')]}>"
        return ident
    k = re.sub(r"^void |rus::|\(anonymous namespace\)::", "", name)
    return k.split("(")[0][:60]


def trace_summary(path: str, steps: int) -> None:
    """Per-step kernel time of the last ``steps`` graph replays in a ``rocprofv3 --kernel-trace``
    CSV of a bench run: the replays are the kernels between the last steps + 1 launches of the
    once-per-step dropout-bits kernel. hipBLASLt kernels are summed as one line."""
    import csv
    import re

    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "keep_bits_kernel" in r["Kernel_Name"]]
    if len(marks) < steps + 1:
        raise SystemExit(f"{path}: {len(marks)} step markers, need {steps + 1}")
    sel = rows[marks[-steps - 1] + 1: marks[-1] + 1]
    dur = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in sel]
    wall = int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])
    print(f"{steps} replayed steps: {len(sel) / steps:.0f} kernels/step, "
          f"{wall / 1e6 / steps:.2f} ms/step from first start to last end, "
          f"{sum(dur) / 1e6 / steps:.2f} ms/step of kernels")
    agg: dict = {}
    for r, d in zip(sel, dur):
        n = r["Kernel_Name"]
        a = agg.setdefault(_kernel_label(n), [0, 0])
        a[0] += d
        a[1] += 1
    print(" ms/step  launches/step  us/launch  kernel")
    for k, (t, c) in sorted(agg.items(), key=lambda kv: -kv[1][0]):
        print(f"{t / 1e6 / steps:8.3f}  {c / steps:13.1f}  {t / c / 1e3:9.2f}  {k}")


def _round_up(x: int, m: int) -> int:
    return -(-x // m) * m


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed counter summary, if there is one."""
    path = os.path.join(REPO, "profiles", f"{kernel}_traffic_config5.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch"):
                return float(line.split("=")[1])
    return None


def _graph_run(engine, model_opt, batches, steps, warmup, bucket=64):
    """Captures the step's graphs for every batch bucket and times ``steps`` replays + AdamW
    (each replay's device time is kept: ``g.replay_ms()[warmup:]``)."""
    from rus_amd.graph import GraphedTrainStep

    g = GraphedTrainStep(engine, bucket=bucket)
    for b in batches:
        g.prepare(b[0], b[1], b[2])
    g.time_replays()
    opt = flat_adamw(engine)[0]
    secs, tokens, _, _ = timed_run(engine, opt, batches, steps, warmup, graph=g)
    return tokens / secs, g


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--rows", type=int, default=4)
    ap.add_argument("--max-len", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-eager", action="store_true")
    ap.add_argument("--no-resident", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-configuration kernel records (BASELINE configs 1-4)")
    ap.add_argument("--no-graph", action="store_true",
                    help="time eager autograd steps instead of captured-graph replays")
    ap.add_argument("--roofline-steps", type=int, default=8)
    ap.add_argument("--stream-unit", choices=("model", "layer"), default="model",
                    help="per step, copy the packed model once (model) or each layer per pass "
                         "through two one-layer slots (layer, the reference's policy); the other "
                         "is timed as an ablation")
    ap.add_argument("--recompute", choices=("off", "on"), default="off",
                    help="off: the forward keeps every layer's activations for the backward; on: "
                         "the backward recomputes them from the saved layer inputs (the "
                         "reference's checkpointing); the other setting is timed as an ablation")
    ap.add_argument("--overlap", choices=("on", "off"), default="off",
                    help="on: each layer's NF4 dequant runs one layer ahead on a second stream "
                         "and LoRA-down beside the q/k/v GEMM (measured slower on this stack: "
                         "cross-stream joins inside a replayed graph cost more than they hide)")
    ap.add_argument("--gemm", choices=("dequant", "fused"), default="dequant",
                    help="dequant: NF4 -> fp16 workspace, then the library GEMM; fused: the "
                         "products decode NF4 inside their MFMA loop (rus_nf4_gemm)")
    ap.add_argument("--dequant-once", choices=("on", "off"), default="on",
                    help="on: each layer is dequantised once per step, into fp16 weights of its "
                         "own that the backward reads (2.6 GB); off: again in the backward, as "
                         "the reference does; the other setting is timed as an ablation")
    ap.add_argument("--bucket", type=int, default=64,
                    help="captured-graph bucket: each batch's packed token count is padded to a "
                         "multiple of this (one graph per bucket and weight buffer; 64 pads the "
                         "bench's 707.5 tokens per step to 744 on average, 256 to 864)")
    ap.add_argument("--lm-block", type=int, default=0,
                    help="most tokens per block of the token-blocked lm_head (whole 256-token "
                         "tiles; 0: the tiles whose fp16 logits fit 256 MiB, 768 at V=151936)")
    ap.add_argument("--lm-chunk", type=int, default=-1,
                    help="lm_head layout: vocabulary rows per chunk of the single pass over "
                         "the vocabulary (a multiple of 256; W read once, an [N, chunk] logit "
                         "buffer); -1 (default): chunk chosen per token count (128 MiB of "
                         "logits at most); 0: the token-blocked head ([block, V] logits)")
    ap.add_argument("--no-ablation", action="store_true",
                    help="skip the timing of the other --recompute, --dequant-once and "
                         "--stream-unit settings")
    ap.add_argument("--counter-summary", nargs="+", metavar="COUNTER_CSV",
                    help="summarise rocprofv3 --pmc counter_collection CSVs per kernel")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the per-step kernel time of the last --steps replays in a "
                         "rocprofv3 --kernel-trace CSV of a bench run, and exit")
    ap.add_argument("--probe", nargs="?", const="dequant",
                    choices=("dequant", "lmhead", "lmhead_pass", "elementwise", "ceilings",
                             "gemm", "gemm_parts", "step", "contention"),
                    help="only fixed launches for counter runs: copy + dequant (default), the "
                         "lm_head CE kernels at config 2 (token blocks; lmhead_pass: the single "
                         "pass over vocabulary chunks), the elementwise kernels on cold "
                         "inputs, the split-K MLP input gradient (gemm_parts), or eager "
                         "training steps with every kernel in its in-step form (step); or printed "
                         "timings: streaming ceilings at the dequant's traffic (ceilings), "
                         "per-product GEMM times (gemm), a step's replay with and without a "
                         "concurrent host-to-device copy (contention)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs and measures one GPU only (asked for --gpus "
              f"{args.gpus}); a sharded run over several GPUs is not implemented", file=sys.stderr)
        return 2
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps)
        return 0
    if args.probe in ("lmhead", "lmhead_pass"):
        lmhead_probe(single_pass=args.probe == "lmhead_pass")
        return 0
    if args.probe == "elementwise":
        elementwise_probe()
        return 0
    if args.probe == "ceilings":
        ceilings_probe()
        return 0
    if args.probe == "gemm":
        gemm_probe()
        return 0
    if args.probe == "gemm_parts":
        gemm_parts_probe()
        return 0
    if args.probe == "step":
        step_probe()
        return 0
    if args.probe == "contention":
        contention_probe(args.steps, max(args.warmup, 8))
        return 0
    if args.counter_summary:
        counter_summary(args.counter_summary)
        return 0
    if args.probe:
        kernel_probe()
        return 0

    import torch

    from rus_amd import model as M
    from rus_amd.eager_reference import eager_step_loss
    from rus_amd import kernels as K
    from rus_amd.kernels import KernelTimer
    from rus_amd.ops import Qwen2FusedEngine, pack_varlen

    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    cfg = M.qwen2_1p5b()
    model = M.build_random_qlora_qwen2(cfg, dev, seed=args.seed)
    batches = make_batches(cfg, 8, args.rows, args.max_len, args.seed, dev)
    params = model.lora_parameters()
    opt = torch.optim.AdamW(params, lr=2e-4)
    model_mib = torch.cuda.memory_allocated(dev) / 2**20  # the random model's device tensors

    # Configured engine: NF4 layers streamed per step from pinned host memory.
    recompute = args.recompute == "on"
    overlap = args.overlap == "on" and args.stream_unit == "model" and args.gemm == "dequant"
    once = (args.dequant_once == "on" and args.stream_unit == "model" and args.gemm == "dequant"
            and not overlap)
    engine = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=args.stream_unit,
                              recompute=recompute, overlap=overlap, gemm=args.gemm,
                              dequant_once=once)
    engine.lm_block_tokens = args.lm_block or None
    engine.lm_v_chunk = args.lm_chunk
    lm_block = args.lm_block or K.lm_head_block_tokens(engine.host_head.gpu_weight.shape[0])
    # Calibration pass (eager): every kernel timed, to name the dominant one.
    _, _, _, calib = timed_run(engine, opt, batches, 2, args.warmup, kernel_filter=None)
    dominant = max(calib, key=lambda k: calib[k]["ms"])
    # Roofline pass (eager, same steps): the dominant kernel's launches bracketed by HIP events on
    # the stream they run on (events cannot time single kernels inside a replayed graph). Its
    # peak allocation above the engine's resident buffers is the step's working set.
    torch.cuda.reset_peak_memory_stats(dev)
    base_alloc = torch.cuda.memory_allocated(dev)
    r_secs, r_tokens, _, summary = timed_run(engine, opt, batches, args.roofline_steps, 0,
                                             kernel_filter={dominant})
    peak = torch.cuda.max_memory_allocated(dev)
    # Timed region: captured-graph steps (one replay + AdamW per step) unless --no-graph.
    graph = None
    reserved0 = torch.cuda.memory_reserved(dev)
    if not args.no_graph:
        from rus_amd.graph import GraphedTrainStep

        graph = GraphedTrainStep(engine, bucket=args.bucket)
        for b in batches:
            graph.prepare(b[0], b[1], b[2])
    graph_pool_mib = (torch.cuda.memory_reserved(dev) - reserved0) / 2**20
    opt_t, opt_kind = (opt, "foreach") if graph is None else flat_adamw(engine)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    ws = engine.weight_stream
    if ws.unit == "model":
        ws.time_copies()
    if graph is not None:
        graph.time_replays()
    secs, tokens, per_step, _ = timed_run(engine, opt_t, batches, args.steps, args.warmup,
                                          graph=graph)
    replay_ms = None
    if graph is not None:
        rms = graph.replay_ms()[args.warmup:]
        graph.time_replays(False)
        replay_ms = statistics.fmean(rms) if rms else None
    h2d = None
    if ws.unit == "model":
        # the per-step copy of the packed model over PCIe, timed on the copy stream while the
        # steps run; its rate bounds tokens/s whatever the kernels do
        cms = ws.copy_ms()[args.warmup:]
        ws.time_copies(False)
        if cms:
            c_ms = statistics.median(cms)
            h2d = {"bytes_per_step": ws.model_bytes, "ms_per_copy": c_ms,
                   "gbps": ws.model_bytes / (c_ms / 1e3) / 1e9,
                   "tokens_per_s_ceiling": tokens / args.steps / (c_ms / 1e3),
                   "note": "median duration of the per-step whole-model copy (pinned host -> "
                           "HBM, copy stream) during the timed steps; tokens/s ceiling = "
                           "tokens per step / copy time. Splitting the copy over 2 or 4 "
                           "streams gives the same 57.5 GB/s (PCIe link bound)"}
    del ws  # the engine's buffers must go with the engine (the eager step's memory is measured later)
    device_peak = {"max_allocated_mib": torch.cuda.max_memory_allocated(dev) / 2**20,
                   "max_reserved_mib": torch.cuda.max_memory_reserved(dev) / 2**20,
                   "model_tensors_mib": model_mib,
                   "note": "whole process during the timed replays: the random model's device "
                           "tensors, the engine's two whole-model NF4 buffers, workspaces "
                           "(with dequant-once: every layer's fp16 weights), the embedding / "
                           "lm_head and its transpose, graph pools"}
    value = tokens / secs
    d = summary[dominant]
    avg_ms = d["ms"] / d["launches"]
    # The roofline that bounds the kernel: MFMA kernels whose algorithmic bytes take longer at
    # 8 TB/s than their flops at the fp16 peak (a split-K product's fp32 partials) are HBM-bound.
    mfma_frac = d["flops"] / (d["ms"] / 1e3) / 1e12 / FP16_PEAK_TFLOPS
    hbm_frac = d["bytes"] / (d["ms"] / 1e3) / 1e9 / HBM_PEAK_GBS
    mfma_bound = dominant in MFMA_KERNELS and mfma_frac >= hbm_frac
    if mfma_bound:
        achieved = d["flops"] / (d["ms"] / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": mfma_frac, "traffic": measured_traffic(dominant)}
    else:
        achieved = d["bytes"] / (d["ms"] / 1e3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": hbm_frac, "traffic": measured_traffic(dominant)}
    if dominant in MFMA_KERNELS:
        roof["mfma_frac"] = mfma_frac
        roof["tflops"] = mfma_frac * FP16_PEAK_TFLOPS
    roof["traffic_source"] = (f"profiles/{dominant}_traffic_config5.txt (FETCH_SIZE / WRITE_SIZE "
                              "counter runs of bench.py --probe, scaled by a plain copy's "
                              "counters)")
    roof.update({"kernel": dominant, "avg_launch_ms": avg_ms, "launches": d["launches"],
                 "event_pair_overhead_ms": KernelTimer.pair_overhead_ms(),
                 "per_launch": d["flops"] / d["launches"] if mfma_bound
                 else d["bytes"] / d["launches"],
                 "per_launch_bytes": d["bytes"] / d["launches"],
                 "per_launch_flops": d["flops"] / d["launches"],
                 "timed_in": f"eager pass of {args.roofline_steps} steps of the same workload"})

    out = {
        "metric": METRIC, "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": secs / args.steps * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: uniform random token ids, lognormal row lengths; random-init NF4 model",
        "config": {"workload": "BASELINE config 5: 28-layer packed QLoRA train step + AdamW, "
                               "Qwen2.5-1.5B shapes, NF4 layers streamed from pinned host memory",
                   "rows": args.rows, "max_len": args.max_len,
                   "tokens_per_step": tokens / args.steps, "lora": "r16 alpha32 dropout0.05 q,v",
                   "stream_unit": args.stream_unit, "recompute": args.recompute,
                   "overlap": "on" if overlap else "off", "gemm": args.gemm,
                   "dequant_once": "on" if once else "off", "graph_bucket": args.bucket,
                   "lm_head": (f"vocabulary chunks of {args.lm_chunk} rows, [N, chunk] logits"
                               if args.lm_chunk > 0 else
                               "one pass over vocabulary chunks chosen per token count (at most "
                               "128 MiB of logits, never [N, V]; online max / sum-exp)"
                               if args.lm_chunk < 0 else
                               f"token blocks of whole 256-token tiles, <= {lm_block} tokens and "
                               "at least two per batch: a [block, V] logits buffer, never "
                               "[N, V]"),
                   "optimizer": f"AdamW lr 2e-4 ({opt_kind}"
                                + (", one flat LoRA buffer)" if graph is not None else ")")},
        "roofline": roof,
        "median_step_tokens_per_s": statistics.median(n / sec for sec, n in per_step),
        "h2d": h2d,
        "peak_hbm_mib": (peak - base_alloc) / 2**20,
        "peak_hbm_mib_note": "working set of one step above the resident buffers (eager pass)",
        "device_peak": device_peak,
        "kernels_calibration": kernel_rates(calib, 2),
        "step_mode": "hip_graph" if graph is not None else "eager",
        "eager_fused_tokens_per_s": r_tokens / r_secs,
        "graph_pool_reserved_mib": graph_pool_mib,
        "graph_buckets": len(graph.graphs) if graph is not None else 0,
    }
    lm = [calib[k] for k in LMHEAD_KERNELS if k in calib]
    if lm:
        out["lm_head_ce_tflops"] = sum(r["flops"] for r in lm) / (sum(r["ms"] for r in lm) / 1e3) / 1e12
    if "nf4_dequant" in calib:
        r = calib["nf4_dequant"]
        out["nf4_dequant_gbps"] = r["bytes"] / (r["ms"] / 1e3) / 1e9
    del graph
    torch.cuda.empty_cache()

    if not args.no_ablation and not args.no_graph:
        # The other activation policy and the other streaming unit: same batches, graphs.
        other = "on" if not recompute else "off"
        eng_a = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=args.stream_unit,
                                 recompute=not recompute, overlap=overlap, gemm=args.gemm,
                                 dequant_once=once)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base_a = torch.cuda.memory_allocated(dev)
        timed_run(eng_a, opt, batches, 1, 0)
        out[f"recompute_{other}_peak_hbm_mib"] = (torch.cuda.max_memory_allocated(dev) - base_a) / 2**20
        out[f"recompute_{other}_tokens_per_s"], g_a = _graph_run(eng_a, None, batches,
                                                                 min(args.steps, 16), 1,
                                                                 args.bucket)
        del eng_a, g_a
        if args.stream_unit == "model" and args.gemm == "dequant" and not overlap:
            eng_d = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit="model",
                                     recompute=recompute, gemm=args.gemm, dequant_once=not once)
            out[f"dequant_once_{'off' if once else 'on'}_tokens_per_s"], g_d = _graph_run(
                eng_d, None, batches, min(args.steps, 16), 1, args.bucket)
            del eng_d, g_d
            torch.cuda.empty_cache()
        # The other lm_head layout: the token-blocked head ([block, V] logit buffers) against
        # the single pass over vocabulary chunks (W read once, an [N, chunk] buffer).
        eng_c = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=args.stream_unit,
                                 recompute=recompute, overlap=overlap, gemm=args.gemm,
                                 dequant_once=once)
        eng_c.lm_block_tokens = engine.lm_block_tokens
        eng_c.lm_v_chunk = 0 if args.lm_chunk else -1
        out[f"lm_head_{'token_blocked' if args.lm_chunk else 'vocab_chunked'}_tokens_per_s"], \
            g_c = _graph_run(eng_c, None, batches, min(args.steps, 16), 1, args.bucket)
        del eng_c, g_c
        torch.cuda.empty_cache()
        unit = "layer" if args.stream_unit == "model" else "model"
        eng_u = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=unit,
                                 recompute=recompute, overlap=False, gemm=args.gemm)
        out[f"stream_unit_{unit}_tokens_per_s"], g_u = _graph_run(eng_u, None, batches,
                                                                   min(args.steps, 16), 1,
                                                                   args.bucket)
        del eng_u, g_u
        torch.cuda.empty_cache()

    if not args.no_resident and not args.no_graph:
        eng_r = Qwen2FusedEngine(model, dev, resident_weights=True, recompute=recompute,
                                 overlap=overlap, gemm=args.gemm, dequant_once=once)
        out["resident_weights_tokens_per_s"], g_r = _graph_run(eng_r, None, batches,
                                                                min(args.steps, 16), 1,
                                                                args.bucket)
        r_ms = g_r.replay_ms()[1:]
        if replay_ms is not None and r_ms and h2d is not None:
            # same batches, whole cycles of the 8 in both runs: the replays' mean device time
            out["step_replay"] = {
                "streamed_ms": replay_ms, "resident_ms": statistics.fmean(r_ms),
                "copy_ms": h2d["ms_per_copy"],
                "note": "mean device time of one captured step's replay (events after its copy "
                        "wait), streamed weights vs HBM-resident weights, same batches. The "
                        "replay itself is the same kernels either way; while the next step's "
                        "model copy saturates the PCIe link, the streamed replay runs longer "
                        "(small kernels and the gaps between launches grow), so the streamed "
                        "step is bounded by max(copy, streamed replay)"}
        del eng_r, g_r
        torch.cuda.empty_cache()

    if not args.no_eager:
        # Unfused eager autograd step (transformers-style stack, fp16 [N, V] logits): with every
        # fused engine and graph of this run freed, its device peak is comparable with the timed
        # run's (both include the random model's own tensors).
        del engine
        gc.collect()  # the engines and captured graphs above hold reference cycles
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        eng_e = Qwen2FusedEngine(model, dev, resident_weights=True)
        b = batches[0]
        pb = pack_varlen(*(t.to(dev) for t in b[:3]))
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base_e = torch.cuda.memory_allocated(dev)
        t0 = time.perf_counter()
        for _ in range(2):
            h = eng_e.host_head.embed(pb.input_ids)
            loss = eager_step_loss(eng_e, h, pb.pos_ids, pb.shift_labels, pb.row_lengths, training=True)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
        torch.cuda.synchronize()
        out["eager_ms_per_step"] = (time.perf_counter() - t0) / 2 * 1e3
        out["eager_tokens_per_s"] = b[3] / (out["eager_ms_per_step"] / 1e3)
        out["eager_peak_hbm_mib"] = (torch.cuda.max_memory_allocated(dev) - base_e) / 2**20
        out["eager_device_peak_mib"] = torch.cuda.max_memory_allocated(dev) / 2**20
        out["eager_base_mib"] = base_e / 2**20
        del eng_e
        torch.cuda.empty_cache()

    records = None
    if not args.no_configs:
        records = config_records(args.seed)
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.seed, batches[0])
        if records is not None:
            cpu = config_cpu_times(args.seed)
            for c, recs in records.items():
                for r in recs:
                    t = cpu.get(c, {}).get(r["kernel"])
                    if t is not None:
                        r["cpu_us"] = t
                        r["cpu_cores"] = out["cpu_baseline"]["cores"]
                        r["speedup"] = t / r["gpu_us"]
    else:
        out["cpu_baseline"] = None
    if records is not None:
        out["configs"] = records
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
