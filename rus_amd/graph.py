"""A whole training step (embedding, 28-layer stack forward, lm_head cross-entropy and gradient,
stack backward) captured once per packed-shape bucket as a HIP graph and replayed.

The reference runs this step eagerly from Python (solution/ops.py:1097-1164 calling the stack and
lm_head autograd functions), which on MI355X leaves the GPU waiting on the host: a step is ~1,800
small launches. Here the host only packs the batch, copies it into the bucket's static buffers
and launches one graph; the optimizer step stays outside (it updates the LoRA parameters in place,
which the graph reads through their flat buffer on every replay).

Buckets: the packed token count N is padded to Np = round_up(N + 1, bucket) with one extra packed
row of Np - N padding tokens (labels -100, positions 0..), which attends only to itself and adds
nothing to the loss or to any gradient. A graph is keyed by (Np, number of rows, longest row
rounded up to a power of two); the first batch of a key captures it.

Semantics of ``step``: it overwrites (does not accumulate) each LoRA parameter's ``.grad``, which
are views of one fp32 buffer; the loss is the reference's sum(nll) / denom; dropout masks change
every replay (the graph advances the engine's device seed).
"""

from __future__ import annotations

import torch

from . import kernels as K
from .ops import (PRESCALE_GRAD, Qwen2FusedEngine, VarlenMeta, pack_varlen, stack_backward,
                  stack_forward)


GRAPH_NODE_TYPES = ("kernel", "memcpy", "memset", "host", "graph", "empty", "wait_event",
                    "event_record", "other")


def graph_node_counts(g: torch.cuda.CUDAGraph) -> dict[str, int]:
    """Node census of a captured graph (needs ``CUDAGraph(keep_graph=True)``, before replay)."""
    import ctypes

    from . import _lib

    counts = (ctypes.c_int64 * len(GRAPH_NODE_TYPES))()
    _lib.call("rus_graph_node_counts", g.raw_cuda_graph(), counts, len(GRAPH_NODE_TYPES))
    return {name: int(c) for name, c in zip(GRAPH_NODE_TYPES, counts)}


def _pow2_at_least(x: int) -> int:
    p = 1
    while p < x:
        p *= 2
    return p


class _Captured:
    """Static buffers and the graph of one bucket."""

    def __init__(self, n_pad: int, n_rows: int, max_len: int, device):
        self.n_pad, self.n_rows, self.max_len = n_pad, n_rows, max_len
        self.ids = torch.zeros(n_pad, dtype=torch.int64, device=device)
        self.pos = torch.zeros(n_pad, dtype=torch.int64, device=device)
        self.labels = torch.full((n_pad,), -100, dtype=torch.int64, device=device)
        self.cu = torch.zeros(n_rows + 1, dtype=torch.int32, device=device)
        self.cu_host = torch.zeros(n_rows + 1, dtype=torch.int32).pin_memory()
        self.pad_pos = torch.arange(n_pad, dtype=torch.int64, device=device)
        self.vm = VarlenMeta.from_device(self.cu, max_len)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}  # per whole-model weight buffer
        self.outputs: dict[int, tuple] = {}  # (loss, nll, entropy, argmax) static tensors
        self.node_counts: dict[int, dict] = {}

    def load(self, pb, lens: list[int]) -> None:
        n = pb.input_ids.numel()
        self.ids[:n].copy_(pb.input_ids)
        self.ids[n:].zero_()
        self.pos[:n].copy_(pb.pos_ids)
        self.pos[n:].copy_(self.pad_pos[: self.n_pad - n])
        self.labels[:n].copy_(pb.shift_labels)
        self.labels[n:].fill_(-100)
        cu = [0]
        for L in lens:
            cu.append(cu[-1] + L)
        # The previous replay's copy from cu_host is complete: pack_varlen synchronised.
        self.cu_host.copy_(torch.tensor(cu, dtype=torch.int32))
        self.cu.copy_(self.cu_host, non_blocking=True)


class GraphedTrainStep:
    """``step(input_ids, attention_mask, labels)`` -> loss (device scalar), with the LoRA
    gradients left in the parameters' ``.grad``. One captured graph per bucket."""

    def __init__(self, engine: Qwen2FusedEngine, bucket: int = 256, training: bool = True,
                 num_items_in_batch=None, census: bool = False):
        if not engine.host_head.resident:
            raise ValueError("GraphedTrainStep needs an HBM-resident lm_head (resident_head=True)")
        if engine.input_stream.offload:
            raise ValueError("GraphedTrainStep keeps layer inputs in HBM (offload_inputs=False)")
        if engine.attention not in ("varlen", "varlen_aten"):
            raise ValueError("GraphedTrainStep needs one launch over all packed rows "
                             "(attention='varlen' or 'varlen_aten')")
        self.engine = engine
        self.bucket = int(bucket)
        self.training = training
        self.num_items = num_items_in_batch
        self.graphs: dict[tuple[int, int, int], _Captured] = {}
        self.pool = torch.cuda.graph_pool_handle()
        dev = engine.device
        self.grad16 = torch.zeros(engine.lora_numel, dtype=torch.float16, device=dev)
        self.grad32 = torch.zeros(engine.lora_numel, dtype=torch.float32, device=dev)
        self.grad_views = engine.lora_views(self.grad32)
        self.last = None
        self.census = census  # count each captured graph's node types (node_counts per bucket)

    # -- the captured body -----------------------------------------------------------------------
    def _body(self, cap: _Captured):
        eng = self.engine
        seed = eng.dropout_seed
        if self.training:
            seed.add_(1)
        h = eng.host_head.embed(cap.ids)
        lora16 = eng.lora_fp16()
        final, st = stack_forward(eng, h, cap.pos, None, self.training, lora16, seed, vm=cap.vm,
                                  save=not eng.recompute)
        head = eng.host_head
        nll, _lse, ent, amax, _denom, d_final, loss = K.lm_head_ce(
            final, head.gpu_weight, cap.labels, num_items_in_batch=self.num_items,
            need_grad=True, weight_t=head.gpu_weight_t, dh_scale=1.0 / PRESCALE_GRAD,
            dh_dtype=final.dtype)
        del final
        stack_backward(eng, st, d_final, self.grad16)
        self.grad32.copy_(self.grad16)
        return loss, nll, ent, amax

    def _key(self, pb):
        n = pb.input_ids.numel()
        n_pad = -(-(n + 1) // self.bucket) * self.bucket
        lens = [int(L) for L in pb.row_lengths if L > 0] + [n_pad - n]
        return (n_pad, len(lens), _pow2_at_least(max(max(lens), 16))), lens

    def _capture(self, key, pb, lens) -> _Captured:
        cap = self.graphs.get(key)
        if cap is None:
            cap = _Captured(*key, self.engine.device)
            self.graphs[key] = cap
        ws = self.engine.weight_stream
        for buf in ((0, 1) if ws.unit == "model" else (0,)):
            if buf not in cap.graphs:
                self._capture_one(cap, buf, pb, lens)
        return cap

    def _capture_one(self, cap: _Captured, buf: int, pb, lens) -> None:
        """Warm-up and capture of the step reading whole-model weight buffer ``buf``."""
        eng = self.engine
        ws = eng.weight_stream
        cap.load(pb, lens)
        if ws.unit == "model":  # the buffer's contents must be valid for the warm-up run
            ws.stage(buf)
            torch.cuda.current_stream(eng.device).wait_event(ws.ready_events[buf])
            ws.staged[buf] = False
            ws.use_buffer(buf)
        seed0 = eng.dropout_seed.clone()
        # Warm-up outside the graph on a side stream (library handles, allocator, autotuning).
        side = torch.cuda.Stream(device=eng.device)
        side.wait_stream(torch.cuda.current_stream(eng.device))
        with torch.cuda.stream(side):
            eng.weight_stream.after_replay()
            self._body(cap)
            eng.weight_stream.after_replay()
        torch.cuda.current_stream(eng.device).wait_stream(side)
        torch.cuda.synchronize(eng.device)
        eng.dropout_seed.copy_(seed0)  # the warm-up does not consume a step's masks
        g = torch.cuda.CUDAGraph(keep_graph=self.census)
        with torch.cuda.graph(g, pool=self.pool):
            ws.begin_capture()
            cap.outputs[buf] = self._body(cap)
        ws.after_replay()
        ws.end_step(buf)
        if self.census:
            cap.node_counts[buf] = graph_node_counts(g)
            g.instantiate()
        cap.graphs[buf] = g

    def prepare(self, input_ids, attention_mask=None, labels=None) -> None:
        """Captures the graph for this batch's bucket if it does not exist yet (no step taken)."""
        pb = pack_varlen(input_ids, attention_mask, labels)
        key, lens = self._key(pb)
        self._capture(key, pb, lens)

    def step(self, input_ids, attention_mask=None, labels=None) -> torch.Tensor:
        self.engine.sync_lora_storage()  # the graphs read the parameters' flat buffer
        pb = pack_varlen(input_ids, attention_mask, labels)
        key, lens = self._key(pb)
        cap = self._capture(key, pb, lens)
        cap.load(pb, lens)
        ws = self.engine.weight_stream
        buf = ws.begin_step()  # waits for this step's whole-model copy (unit="model")
        cap.graphs[buf].replay()
        ws.after_replay()
        ws.end_step(buf)
        for p, v in zip(self.engine.lora_params, self.grad_views):
            if p.grad is None or p.grad.data_ptr() != v.data_ptr():
                p.grad = v
        self.last = (cap, buf, pb)
        return cap.outputs[buf][0][0]

    def last_token_outputs(self):
        """(nll, entropy, argmax) of the last step's real tokens, packed order."""
        cap, buf, pb = self.last
        n = pb.input_ids.numel()
        out = cap.outputs[buf]
        return out[1][:n], out[2][:n], out[3][:n]


__all__ = ["GraphedTrainStep"]
