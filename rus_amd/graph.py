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
are views of one fp32 buffer (also the ``.grad`` of ``engine.flat_lora_parameter()`` when that
exists); the loss is the reference's sum(nll) / denom; dropout masks change every replay (the
graph advances the engine's device seed). The first batch fixes where inputs are packed: host
(CPU) batches on the host, into the next of a ring of pinned images that one kernel copies into
the bucket's device image right before the replay (no copy-engine transfer for the step to wait
on, and the host waits only when the ring wraps onto a copy that has not run); device batches on
the device.
"""

from __future__ import annotations

import torch

from . import kernels as K
from .ops import (PRESCALE_GRAD, Qwen2FusedEngine, VarlenMeta, lm_head_layout, pack_varlen,
                  stack_backward, stack_forward)


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


HOST_RING = 4  # pinned host images per bucket, used in turn


class _Stage:
    """One device image of a bucket's inputs: ids | positions | labels (int64, n_pad each) |
    cu_seqlens (int32), and the views a captured graph reads."""

    def __init__(self, n_pad: int, n_rows: int, max_len: int, device):
        cu_words = (n_rows + 2) // 2
        words = 3 * n_pad + cu_words
        words += words % 2  # whole 16-byte units for the host-image copy kernel
        self.buf = torch.zeros(words, dtype=torch.int64, device=device)
        self.ids = self.buf[:n_pad]
        self.pos = self.buf[n_pad: 2 * n_pad]
        self.labels = self.buf[2 * n_pad: 3 * n_pad]
        self.labels.fill_(-100)
        self.cu = self.buf[3 * n_pad:].view(torch.int32)[: n_rows + 1]
        self.vm = VarlenMeta.from_device(self.cu, max_len)


class _Captured:
    """Static buffers and graphs of one bucket: one input image and one graph per whole-model
    weight buffer (otherwise one of each), and a ring of pinned host images."""

    def __init__(self, n_pad: int, n_rows: int, max_len: int, device, host: bool,
                 n_images: int):
        self.n_pad, self.n_rows, self.max_len = n_pad, n_rows, max_len
        self.stages = [_Stage(n_pad, n_rows, max_len, device) for _ in range(n_images)]
        self.cu_host = torch.zeros(n_rows + 1, dtype=torch.int32).pin_memory()
        self.pad_pos = torch.arange(n_pad, dtype=torch.int64, device=device)
        n_words = self.stages[0].buf.numel()
        self.ring = [torch.zeros(n_words, dtype=torch.int64).pin_memory()
                     for _ in range(HOST_RING if host else 0)]
        self.ring_done: list[torch.cuda.Event | None] = [None] * len(self.ring)
        self.ring_turn = 0
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}  # per whole-model weight buffer
        self.outputs: dict[int, tuple] = {}  # (loss, nll, entropy, argmax) static tensors
        self.node_counts: dict[int, dict] = {}

    def load(self, pb, lens: list[int], j: int) -> None:
        """Batch -> device image ``j``, enqueued on the current stream: a host batch through the
        next pinned image of the ring and one copy kernel (waiting on the host only if that
        image's previous copy has not run yet); a device batch by device copies."""
        st = self.stages[j]
        cu = [0]
        for L in lens:
            cu.append(cu[-1] + L)
        n, P = pb.input_ids.numel(), self.n_pad
        if pb.input_ids.device.type == "cpu":
            r = self.ring_turn
            self.ring_turn = (r + 1) % len(self.ring)
            done = self.ring_done[r]
            if done is not None and not done.query():
                done.synchronize()
            hb = self.ring[r]
            hb[:n] = pb.input_ids
            hb[n:P] = 0
            hb[P: P + n] = pb.pos_ids
            hb[P + n: 2 * P] = torch.arange(P - n, dtype=torch.int64)
            hb[2 * P: 2 * P + n] = pb.shift_labels
            hb[2 * P + n: 3 * P] = -100
            hb[3 * P:].view(torch.int32)[: len(cu)] = torch.tensor(cu, dtype=torch.int32)
            K.copy_from_host(st.buf, hb)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(st.buf.device))
            self.ring_done[r] = ev
            return
        st.ids[:n].copy_(pb.input_ids)
        st.ids[n:].zero_()
        st.pos[:n].copy_(pb.pos_ids)
        st.pos[n:].copy_(self.pad_pos[: P - n])
        st.labels[:n].copy_(pb.shift_labels)
        st.labels[n:].fill_(-100)
        # The previous replay's copy from cu_host is complete: pack_varlen synchronised.
        self.cu_host.copy_(torch.tensor(cu, dtype=torch.int32))
        st.cu.copy_(self.cu_host, non_blocking=True)


class GraphedTrainStep:
    """``step(input_ids, attention_mask, labels)`` -> loss (device scalar), with the LoRA
    gradients left in the parameters' ``.grad``. One captured graph per bucket."""

    def __init__(self, engine: Qwen2FusedEngine, bucket: int = 64, training: bool = True,
                 num_items_in_batch=None, census: bool = False):
        if not engine.host_head.resident:
            raise ValueError("GraphedTrainStep needs an HBM-resident lm_head (resident_head=True)")
        if engine.input_stream.offload:
            raise ValueError("GraphedTrainStep keeps layer inputs in HBM (offload_inputs=False)")
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
        self.replay_marks: list | None = None  # (start, end) timing events per replay, when timing
        self.host_inputs: bool | None = None  # fixed by the first batch: host or device tensors

    # -- the captured body -----------------------------------------------------------------------
    def _body(self, img: _Stage):
        eng = self.engine
        seed = eng.dropout_seed
        if self.training:
            seed.add_(1)
        h = eng.host_head.embed(img.ids)
        lora16 = eng.lora_fp16()
        final, st = stack_forward(eng, h, img.pos, None, self.training, lora16, seed, vm=img.vm,
                                  save=not eng.recompute)
        head = eng.host_head
        # the engine's head layout; the single pass's chunk chosen for the bucket's token count
        v_chunk = lm_head_layout(eng.lm_v_chunk, final.shape[0], head.gpu_weight.shape[0],
                                 final.device)
        nll, _lse, ent, amax, _denom, d_final, loss = K.lm_head_ce(
            final, head.gpu_weight, img.labels, num_items_in_batch=self.num_items,
            need_grad=True, weight_t=head.gpu_weight_t, dh_scale=1.0 / PRESCALE_GRAD,
            dh_dtype=final.dtype, block_tokens=eng.lm_block_tokens, v_chunk=v_chunk)
        del final
        stack_backward(eng, st, d_final, self.grad16)
        self.grad32.copy_(self.grad16)
        return loss, nll, ent, amax

    def _key(self, pb):
        n = pb.input_ids.numel()
        n_pad = -(-(n + 1) // self.bucket) * self.bucket
        lens = [int(L) for L in pb.row_lengths if L > 0] + [n_pad - n]
        return (n_pad, len(lens), _pow2_at_least(max(max(lens), 16))), lens

    def _images(self) -> tuple[int, ...]:
        """Input images (and graphs) per bucket: one per whole-model weight buffer, else one."""
        return tuple(range(self.engine.weight_stream.n_buffers))

    def _pack(self, input_ids, attention_mask, labels):
        """Packs a batch where this step's inputs live (fixed by the first batch): host tensors
        are packed on the host, device tensors on the device."""
        if self.host_inputs is None:
            self.host_inputs = input_ids.device.type == "cpu"
        dev = self.engine.device
        if self.host_inputs:
            ts = [None if t is None else t.cpu() for t in (input_ids, attention_mask, labels)]
        else:
            ts = [None if t is None else t.to(dev) for t in (input_ids, attention_mask, labels)]
        return pack_varlen(*ts, vocab_size=self.engine.host_head.vocab_size)

    def _capture(self, key, pb, lens) -> _Captured:
        cap = self.graphs.get(key)
        if cap is None:
            cap = _Captured(*key, self.engine.device, bool(self.host_inputs),
                            len(self._images()))
            self.graphs[key] = cap
        for buf in self._images():
            if buf not in cap.graphs:
                self._capture_one(cap, buf, pb, lens)
        return cap

    def _capture_one(self, cap: _Captured, buf: int, pb, lens) -> None:
        """Warm-up and capture of the step reading input image ``buf`` (and, with whole-model
        streaming, weight buffer ``buf``)."""
        eng = self.engine
        ws = eng.weight_stream
        img = cap.stages[buf]
        cap.load(pb, lens, buf)
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
            self._body(img)
            eng.weight_stream.after_replay()
        torch.cuda.current_stream(eng.device).wait_stream(side)
        torch.cuda.synchronize(eng.device)
        eng.dropout_seed.copy_(seed0)  # the warm-up does not consume a step's masks
        g = torch.cuda.CUDAGraph(keep_graph=self.census)
        with torch.cuda.graph(g, pool=self.pool):
            ws.begin_capture()
            cap.outputs[buf] = self._body(img)
        ws.after_replay()
        ws.end_step(buf)
        if self.census:
            cap.node_counts[buf] = graph_node_counts(g)
            g.instantiate()
        cap.graphs[buf] = g

    def time_replays(self, on: bool = True) -> None:
        """Starts (or stops) recording a pair of timing events around every replay."""
        self.replay_marks = [] if on else None

    def replay_ms(self) -> list[float]:
        """Device time (ms) of each replay recorded since ``time_replays()`` (synchronises)."""
        out = []
        for e0, e1 in self.replay_marks or []:
            e1.synchronize()
            out.append(e0.elapsed_time(e1))
        return out

    def prepare(self, input_ids, attention_mask=None, labels=None) -> None:
        """Captures the graph for this batch's bucket if it does not exist yet (no step taken)."""
        pb = self._pack(input_ids, attention_mask, labels)
        key, lens = self._key(pb)
        self._capture(key, pb, lens)

    def step(self, input_ids, attention_mask=None, labels=None) -> torch.Tensor:
        self.engine.sync_lora_storage()  # the graphs read the parameters' flat buffer
        pb = self._pack(input_ids, attention_mask, labels)
        key, lens = self._key(pb)
        cap = self._capture(key, pb, lens)
        ws = self.engine.weight_stream
        j = ws.next_buffer if ws.unit == "model" else 0  # the image paired with the weights
        cap.load(pb, lens, j)
        buf = ws.begin_step()  # waits for this step's whole-model copy (unit="model")
        marks = self.replay_marks
        if marks is not None:  # recorded after the copy wait: the events bracket the replay only
            marks.append((torch.cuda.Event(enable_timing=True),
                          torch.cuda.Event(enable_timing=True)))
            marks[-1][0].record()
        cap.graphs[buf].replay()
        if marks is not None:
            marks[-1][1].record()
        ws.after_replay()
        ws.end_step(buf)
        for p, v in zip(self.engine.lora_params, self.grad_views):
            if p.grad is None or p.grad.data_ptr() != v.data_ptr():
                p.grad = v
        flat = self.engine.flat_param
        if flat is not None and (flat.grad is None or flat.grad.data_ptr() != self.grad32.data_ptr()):
            flat.grad = self.grad32
        self.last = (cap, buf, pb)
        return cap.outputs[buf][0][0]

    def last_token_outputs(self):
        """(nll, entropy, argmax) of the last step's real tokens, packed order."""
        cap, buf, pb = self.last
        n = pb.input_ids.numel()
        out = cap.outputs[buf]
        return out[1][:n], out[2][:n], out[3][:n]


__all__ = ["GraphedTrainStep"]
