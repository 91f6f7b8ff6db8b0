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
MFMA_KERNELS = ("lmhead_ce_fwd", "lmhead_ce_fwd_keep", "lmhead_ce_logits", "lmhead_ce_grad_logits",
                "lmhead_ce_grad_hidden")


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
        out.append((ids.pin_memory(), mask.pin_memory(), labels.pin_memory(), sum(lengths)))
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
    """AdamW (lr 2e-4) over the engine's flat LoRA parameter (every factor is a view of it): one
    fused update launch per step instead of a foreach pass over 112 tensors; elementwise, so the
    same values. Returns (optimizer, implementation)."""
    import torch

    p = engine.flat_lora_parameter()
    try:
        return torch.optim.AdamW([p], lr=2e-4, fused=True), "fused"
    except (RuntimeError, ValueError):
        return torch.optim.AdamW([p], lr=2e-4, foreach=True), "foreach"


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


def cpu_baseline(seed=0):
    """The CPU oracle on a bounded sample of the same workload: one config-5 layer plus the
    lm_head over one packed row of 128 tokens, forward + backward including the NF4 dequant of
    the layer's weights; extrapolated to the 28-layer step as tokens/s."""
    import torch

    from oracle import ops as oref
    from oracle import stack as ostack
    from rus_amd import model as M

    threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    torch.set_num_threads(threads)
    cfg = M.qwen2_1p5b()
    cfg1 = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": 1, "lora_dropout": 0.0})
    model = M.build_random_qlora_qwen2(cfg1, "cpu", seed=seed)
    n = 128
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg.vocab_size, (n,), generator=g)
    pos = torch.arange(n)
    labels = torch.cat([ids[1:], torch.tensor([-100])])
    reps = []
    for _ in range(2):
        t0 = time.perf_counter()
        deq = ostack.dequant_model(model)
        t1 = time.perf_counter()
        lora = ostack.lora_leaves(model)
        loss, final = ostack.step_loss(model, deq, lora, ids, pos, labels, [n])
        loss.backward()
        t2 = time.perf_counter()
        oref.lm_head_ce(final.detach().half(), model.embed, labels, need_grad=True)
        t3 = time.perf_counter()
        reps.append((t1 - t0, t2 - t1, t3 - t2))
    t_deq, t_fb, t_head = (min(r[i] for r in reps) for i in range(3))
    t_layer = t_deq + max(t_fb - t_head, 0.0)
    t_step = cfg.num_hidden_layers * t_layer + t_head
    return {"value": n / t_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle (eager fp32 torch + numpy NF4 dequant) on 1 of 28 config-5 layers "
                       f"+ lm_head, one packed row of {n} tokens, fwd+bwd; per-step estimate "
                       f"28*{t_layer:.3f}s + {t_head:.3f}s (lm_head)")}


def lmhead_probe(reps: int = 5) -> None:
    """Fixed launches for counter runs of the lm_head CE kernels at BASELINE config 2: hidden
    [2048, 1536] ~ N(0,1), W [151936, 1536] ~ N(0, 0.02), 10% labels -100, whole vocabulary per
    pass (forward statistics, logit gradient, hidden gradient)."""
    import torch

    from rus_amd import kernels as K

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    n, d, v = 2048, 1536, 151936
    h = torch.randn(n, d, device=dev, generator=g).half()
    w = (torch.randn(v, d, device=dev, generator=g) * 0.02).half()
    lab = torch.randint(0, v, (n,), device=dev, generator=g)
    lab[torch.rand(n, device=dev, generator=g) < 0.1] = -100
    wt = K.lm_head_weight_t(w)
    torch.cuda.synchronize()
    for _ in range(reps):
        K.lm_head_ce(h, w, lab, weight_t=wt)
    torch.cuda.synchronize()
    print(f"probe: {reps} lm_head CE forward+gradient passes at N={n}, V={v}, d={d}", flush=True)


def kernel_probe(reps: int = 5) -> None:
    """Fixed launches for hardware-counter runs: a plain 128 MiB device copy (the calibration for
    the FETCH_SIZE / WRITE_SIZE counters) and one config-5 layer's four-segment NF4 dequant
    carrying a residual + RMSNorm forward of a 707-token batch, as in the train step."""
    import torch

    from rus_amd import model as M
    from rus_amd.hostload import WeightStream

    dev = torch.device("cuda:0")
    cfg = M.qwen2_1p5b()
    cfg1 = M.Qwen2Config(**{**cfg.__dict__, "num_hidden_layers": 1})
    model = M.build_random_qlora_qwen2(cfg1, dev, seed=0)
    ws = WeightStream(model.layers, dev, resident=True)
    src = torch.empty(64 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"probe: {reps} copies of {src.numel() * 2} bytes", flush=True)
    from rus_amd import kernels as K

    x = torch.randn(707, cfg.hidden_size, device=dev).half()
    res = torch.randn_like(x)
    lnw = torch.ones(cfg.hidden_size, device=dev)
    for _ in range(reps):
        *_, pend = K.rms_norm_fwd(x, lnw, 1e-6, residual=res, defer=True)
        ws.dequant_layer(0, norm=pend)
    torch.cuda.synchronize()
    print(f"probe: {reps} four-segment dequants of layer 0 with a riding norm", flush=True)


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
    ap.add_argument("--no-graph", action="store_true",
                    help="time eager autograd steps instead of captured-graph replays")
    ap.add_argument("--roofline-steps", type=int, default=8)
    ap.add_argument("--stream-unit", choices=("model", "layer"), default="model",
                    help="per step, copy the packed model once (model) or each layer per pass "
                         "through two one-layer slots (layer, the reference's policy)")
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
    ap.add_argument("--no-ablation", action="store_true",
                    help="skip the timing of the other --recompute setting")
    ap.add_argument("--probe", nargs="?", const="dequant", choices=("dequant", "lmhead"),
                    help="only fixed launches for counter runs: copy + dequant (default) or the "
                         "lm_head CE kernels at config 2")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs and measures one GPU only (asked for --gpus "
              f"{args.gpus}); a sharded run over several GPUs is not implemented", file=sys.stderr)
        return 2
    if args.probe == "lmhead":
        lmhead_probe()
        return 0
    if args.probe:
        kernel_probe()
        return 0

    import torch

    from rus_amd import model as M
    from rus_amd.eager_reference import eager_step_loss
    from rus_amd.ops import Qwen2FusedEngine, pack_varlen

    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    cfg = M.qwen2_1p5b()
    model = M.build_random_qlora_qwen2(cfg, dev, seed=args.seed)
    batches = make_batches(cfg, 8, args.rows, args.max_len, args.seed, dev)
    params = model.lora_parameters()
    opt = torch.optim.AdamW(params, lr=2e-4)

    # Configured engine: NF4 layers streamed per step from pinned host memory.
    recompute = args.recompute == "on"
    overlap = args.overlap == "on" and args.stream_unit == "model" and args.gemm == "dequant"
    engine = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=args.stream_unit,
                              recompute=recompute, overlap=overlap, gemm=args.gemm)
    # Calibration pass (eager): every kernel timed, to name the dominant one.
    _, _, _, calib = timed_run(engine, opt, batches, 2, args.warmup, kernel_filter=None)
    dominant = max(calib, key=lambda k: calib[k]["ms"])
    # Roofline pass (eager, same steps): the dominant kernel's launches bracketed by HIP events on
    # the stream they run on (events cannot time single kernels inside a replayed graph). Its
    # peak allocation is the step's working set.
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

        graph = GraphedTrainStep(engine)
        for b in batches:
            graph.prepare(b[0], b[1], b[2])
    graph_pool_mib = (torch.cuda.memory_reserved(dev) - reserved0) / 2**20
    opt_t, opt_kind = (opt, "foreach") if graph is None else flat_adamw(engine)
    secs, tokens, per_step, _ = timed_run(engine, opt_t, batches, args.steps, args.warmup,
                                          graph=graph)
    value = tokens / secs
    d = summary[dominant]
    avg_ms = d["ms"] / d["launches"]
    if dominant in MFMA_KERNELS:
        achieved = d["flops"] / (d["ms"] / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / FP16_PEAK_TFLOPS, "traffic": None}
    else:
        achieved = d["bytes"] / (d["ms"] / 1e3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": measured_traffic(dominant)}
    from rus_amd.kernels import KernelTimer

    roof.update({"kernel": dominant, "avg_launch_ms": avg_ms, "launches": d["launches"],
                 "event_pair_overhead_ms": KernelTimer.pair_overhead_ms(),
                 "per_launch": d["flops"] / d["launches"] if dominant in MFMA_KERNELS
                 else d["bytes"] / d["launches"],
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
                   "optimizer": f"AdamW lr 2e-4 ({opt_kind}"
                                + (", one flat LoRA buffer)" if graph is not None else ")")},
        "roofline": roof,
        "median_step_tokens_per_s": statistics.median(n / sec for sec, n in per_step),
        "peak_hbm_mib": (peak - base_alloc) / 2**20,
        "kernels_calibration": kernel_rates(calib, 2),
        "step_mode": "hip_graph" if graph is not None else "eager",
        "eager_fused_tokens_per_s": r_tokens / r_secs,
        "graph_pool_reserved_mib": graph_pool_mib,
        "graph_buckets": len(graph.graphs) if graph is not None else 0,
    }
    lm = [calib[k] for k in MFMA_KERNELS if k in calib]
    if lm:
        # rate of the head's MFMA launches; and 4*N*D*V (one forward and one backward product)
        # over the whole head's kernel time, the in-place gradient pass included
        out["lm_head_ce_tflops"] = sum(r["flops"] for r in lm) / (sum(r["ms"] for r in lm) / 1e3) / 1e12
        fwd = sum(calib[k]["flops"] for k in ("lmhead_ce_fwd", "lmhead_ce_fwd_keep") if k in calib)
        head_ms = sum(r["ms"] for r in lm) + sum(
            calib[k]["ms"] for k in ("lmhead_ce_grad_from_logits",) if k in calib)
        out["lm_head_ce_tflops_credited_4NDV"] = 2.0 * fwd / (head_ms / 1e3) / 1e12
    if "nf4_dequant" in calib:
        r = calib["nf4_dequant"]
        out["nf4_dequant_gbps"] = r["bytes"] / (r["ms"] / 1e3) / 1e9

    if not args.no_ablation:
        # The other activation policy: same streamed weights, graphs, batches; its throughput
        # and its working set (peak allocation of one eager step, as for the headline engine).
        eng_a = Qwen2FusedEngine(model, dev, resident_weights=False, stream_unit=args.stream_unit,
                                 recompute=not recompute, overlap=overlap, gemm=args.gemm)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base_a = torch.cuda.memory_allocated(dev)
        timed_run(eng_a, opt, batches, 1, 0)
        peak_a = (torch.cuda.max_memory_allocated(dev) - base_a) / 2**20
        g_a = None
        if graph is not None:
            g_a = GraphedTrainStep(eng_a)
            for b in batches:
                g_a.prepare(b[0], b[1], b[2])
        opt_a = opt if g_a is None else flat_adamw(eng_a)[0]
        s_a, t_a, _, _ = timed_run(eng_a, opt_a, batches, min(args.steps, 16), 1, graph=g_a)
        other = "on" if not recompute else "off"
        out[f"recompute_{other}_tokens_per_s"] = t_a / s_a
        out[f"recompute_{other}_peak_hbm_mib"] = peak_a
        del eng_a, g_a

    if not args.no_resident:
        eng_r = Qwen2FusedEngine(model, dev, resident_weights=True, recompute=recompute,
                                 overlap=overlap, gemm=args.gemm)
        g_r = None
        if graph is not None:
            g_r = GraphedTrainStep(eng_r)
            for b in batches:
                g_r.prepare(b[0], b[1], b[2])
        opt_r = opt if g_r is None else flat_adamw(eng_r)[0]
        s_r, t_r, _, _ = timed_run(eng_r, opt_r, batches, min(args.steps, 16), 1, graph=g_r)
        out["resident_weights_tokens_per_s"] = t_r / s_r
        del eng_r

    if not args.no_eager:
        eng_e = Qwen2FusedEngine(model, dev, resident_weights=False)
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
        del eng_e

    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.seed)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
