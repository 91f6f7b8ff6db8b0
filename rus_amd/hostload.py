"""Weight, lm_head and activation residency for the fused Qwen2 stack (solution/hostload.py).

* ``WeightStream`` packs each layer's seven NF4 projections into four fused segments
  ([q|k|v], o, [gate|up], down; solution/hostload.py:159-258) in one byte buffer per layer and
  serves fp16 weights through the gfx950 dequant kernel. Two residencies:
    - ``resident=False`` (the reference's policy): packed layers live in pinned
      host memory and are copied per step into two device slots on a side stream, ordered by
      events (prefetch / wait_slot / release_slot, hostload.py:297-323);
    - ``resident=True`` (MI355X: 28 packed layers are 0.65 GB of 288 GB HBM): packed layers stay in
      HBM and prefetch / wait_slot / release_slot do nothing.
  Each segment dequantises into its own fp16 workspace, so the stack dequantises a segment once
  per layer per pass instead of re-dequantising a single shared workspace (the reference does 17
  dequants per layer per step, hostload.py:295, 325-342; this layout needs 8).
* ``HostHead`` holds the tied embedding / lm_head: HBM-resident with its W^T for the gradient GEMM
  (default), or in pinned host memory streamed in vocabulary chunks through two device slots
  (hostload.py:345-408).
* ``InputStream`` keeps each layer's input for the backward recompute: in HBM (default) or
  offloaded to pinned host memory with a one-ahead reverse prefetch (hostload.py:411-488, whose
  three-ahead prefetch into a two-slot ring is always overwritten before use).
"""

from __future__ import annotations

import torch

from . import kernels as K
from .quant import NF4Weight, concat_segments

MAX_MLP_TOKENS = 1 << 30  # the reference chunks the MLP at 512 tokens for a 15 GB T4; not needed
V_CHUNK_DEFAULT = 8192  # vocabulary rows per streamed lm_head chunk (hostload.py:24)
SEGMENTS = ("qkv", "o", "gu", "down")


class PackedNF4Segment:
    """One fused segment of a layer's packed buffer (hostload.py:27-62), plus the absmax2 base of
    each sub-segment (the reference assumes global super-block indexing)."""

    __slots__ = ("out_features", "in_features", "packed_slice", "absmax_slice", "absmax2_slice",
                 "offsets", "split_bytes", "absmax2_bases", "blocksize", "super_blocksize")

    def __init__(self, out_features, in_features, packed_slice, absmax_slice, absmax2_slice,
                 offsets, split_bytes, absmax2_bases, blocksize=64, super_blocksize=256):
        self.out_features = out_features
        self.in_features = in_features
        self.packed_slice = packed_slice
        self.absmax_slice = absmax_slice
        self.absmax2_slice = absmax2_slice
        self.offsets = offsets
        self.split_bytes = split_bytes
        self.absmax2_bases = absmax2_bases
        self.blocksize = blocksize
        self.super_blocksize = super_blocksize


def _pinned(t: torch.Tensor) -> torch.Tensor:
    cpu = t.detach().contiguous().cpu()
    return cpu.pin_memory() if torch.cuda.is_available() else cpu


class WeightStream:
    """Packed NF4 layers served as fp16 weights through the dequant kernel.

    ``unit`` (when not resident) sets what is streamed from pinned host memory:
      * "layer": two one-layer device slots refilled per layer per pass (the reference's policy,
        hostload.py:286-323; 2 x 28 layer copies per step);
      * "model": ``model_buffers`` (default 2) whole-model device buffers used in turn; each
        step copies the packed model once (one 645 MiB H2D copy at Qwen2.5-1.5B) into the
        buffer of the next step, on the copy stream, overlapping the current step; the step
        waits for its own copy (``begin_step``), uses that buffer for forward and backward and
        releases it (``end_step``). A copy does not wait for the last reader of its buffer: the
        base weights are frozen, so it rewrites the bytes that reader sees. (A copy stream
        holding a wait on a running step delays, on this runtime, the completion of the copies
        ahead of it, which idles the start of the next step.)"""

    def __init__(self, layers, device, resident: bool = False, unit: str = "layer",
                 model_buffers: int = 2):
        if unit not in ("layer", "model"):
            raise ValueError("unit must be 'layer' or 'model'")
        if model_buffers < 2:
            raise ValueError("model_buffers must be at least 2")
        self.n_buffers = model_buffers if (unit == "model" and not resident) else 1
        self.device = torch.device(device)
        self.num_layers = len(layers)
        self.resident = resident
        self.unit = "resident" if resident else unit
        self.layer_segments: list[dict[str, PackedNF4Segment]] = []
        self.layer_biases: list[torch.Tensor | None] = []
        self.code2_gpu: torch.Tensor | None = None
        packed_l, absmax_l, absmax2_l = [], [], []
        ws_elems = {s: 0 for s in SEGMENTS}
        for L in layers:
            parts = {"qkv": [L.q, L.k, L.v], "o": [L.o], "gu": [L.gate, L.up], "down": [L.down]}
            if self.code2_gpu is None:
                self.code2_gpu = L.q.code2.to(self.device, torch.float32).contiguous()
            biases = [L.q_bias, L.k_bias, L.v_bias]
            self.layer_biases.append(
                torch.cat([b.to(self.device, torch.float16) for b in biases]).contiguous()
                if all(b is not None for b in biases) else None)
            segs = {}
            pb, ab, a2b = [], [], []
            p_cur = a_cur = a2_cur = 0
            for name in SEGMENTS:
                fused, splits, offs, bases = concat_segments(parts[name])
                nb, na, na2 = fused.packed.numel(), fused.absmax.numel(), fused.absmax2.numel()
                segs[name] = PackedNF4Segment(
                    fused.shape[0], fused.shape[1], slice(p_cur, p_cur + nb),
                    slice(a_cur, a_cur + na), slice(a2_cur, a2_cur + na2), offs, splits, bases,
                    fused.blocksize, fused.super_blocksize)
                pb.append(fused.packed)
                ab.append(fused.absmax)
                a2b.append(fused.absmax2)
                p_cur, a_cur, a2_cur = p_cur + nb, a_cur + na, a2_cur + na2
                ws_elems[name] = max(ws_elems[name], fused.shape[0] * fused.shape[1])
            self.layer_segments.append(segs)
            packed_l.append(torch.cat([t.reshape(-1).cpu() for t in pb]))
            absmax_l.append(torch.cat([t.reshape(-1).cpu() for t in ab]))
            absmax2_l.append(torch.cat([t.reshape(-1).float().cpu() for t in a2b]))
        self.layer_bytes = [int(p.numel() + a.numel() + 4 * a2.numel())
                            for p, a, a2 in zip(packed_l, absmax_l, absmax2_l)]
        if resident:
            self.gpu_layers = [(p.to(self.device), a.to(self.device), a2.to(self.device))
                               for p, a, a2 in zip(packed_l, absmax_l, absmax2_l)]
        elif self.unit == "model":
            self._init_model_buffers(packed_l, absmax_l, absmax2_l)
        else:
            self.cpu_packed = [_pinned(p) for p in packed_l]
            self.cpu_absmax = [_pinned(a) for a in absmax_l]
            self.cpu_absmax2 = [_pinned(a) for a in absmax2_l]
            mp = max(p.numel() for p in packed_l)
            ma = max(a.numel() for a in absmax_l)
            ma2 = max(a.numel() for a in absmax2_l)
            self.gpu_packed_slots = [torch.empty(mp, dtype=torch.uint8, device=self.device) for _ in range(2)]
            self.gpu_absmax_slots = [torch.empty(ma, dtype=torch.uint8, device=self.device) for _ in range(2)]
            self.gpu_absmax2_slots = [torch.empty(ma2, dtype=torch.float32, device=self.device) for _ in range(2)]
            self.stream = torch.cuda.Stream(device=self.device)
            self.slot_events = [torch.cuda.Event() for _ in range(2)]
            self.compute_done_events = [torch.cuda.Event() for _ in range(2)]
            self.slot_layer = [-1, -1]
        self.workspaces = {s: torch.empty(n, dtype=torch.float16, device=self.device)
                           for s, n in ws_elems.items()}

    def _init_model_buffers(self, packed_l, absmax_l, absmax2_l) -> None:
        """One pinned host blob holding every layer (packed | absmax | absmax2, each 256-byte
        aligned) and n_buffers device blobs of the same layout."""
        def up(x):
            return (x + 255) // 256 * 256

        offs, cur = [], 0
        for p, a, a2 in zip(packed_l, absmax_l, absmax2_l):
            po = cur
            ao = up(po + p.numel())
            a2o = up(ao + a.numel())
            cur = up(a2o + 4 * a2.numel())
            offs.append((po, ao, a2o))
        self.model_bytes = cur
        blob = torch.zeros(cur, dtype=torch.uint8)
        for (po, ao, a2o), p, a, a2 in zip(offs, packed_l, absmax_l, absmax2_l):
            blob[po: po + p.numel()] = p
            blob[ao: ao + a.numel()] = a
            blob[a2o: a2o + 4 * a2.numel()] = a2.contiguous().view(torch.uint8)
        self.host_blob = _pinned(blob)
        nb = self.n_buffers
        self.dev_blobs = [torch.empty(cur, dtype=torch.uint8, device=self.device)
                          for _ in range(nb)]
        self.blob_views = []
        for b in self.dev_blobs:
            views = []
            for (po, ao, a2o), p, a, a2 in zip(offs, packed_l, absmax_l, absmax2_l):
                views.append((b[po: po + p.numel()], b[ao: ao + a.numel()],
                              b[a2o: a2o + 4 * a2.numel()].view(torch.float32)))
            self.blob_views.append(views)
        self.stream = torch.cuda.Stream(device=self.device)
        self.ready_events = [torch.cuda.Event() for _ in range(nb)]
        self.staged = [False] * nb
        self.active = 0
        self.next_buffer = 0

    # -- whole-model streaming (unit="model") --------------------------------------------------
    def stage(self, buf: int) -> None:
        """Copies the packed model into device buffer ``buf`` on the copy stream. Only a buffer's
        first copy precedes every read of it; later copies rewrite identical bytes, so they do
        not wait for the buffer's readers."""
        with torch.cuda.stream(self.stream):
            self.dev_blobs[buf].copy_(self.host_blob, non_blocking=True)
            self.ready_events[buf].record(self.stream)
        self.staged[buf] = True

    def begin_step(self) -> int:
        """Starts a step on the next buffer (staging it if the previous step did not) and stages
        the other buffer for the following step. Returns the buffer index; no-op (0) unless
        unit="model"."""
        if self.unit != "model":
            return 0
        buf = self.next_buffer
        if not self.staged[buf]:
            self.stage(buf)
        torch.cuda.current_stream(self.device).wait_event(self.ready_events[buf])
        self.staged[buf] = False
        self.active = buf
        self.next_buffer = (buf + 1) % self.n_buffers
        self.stage(self.next_buffer)
        return buf

    def use_buffer(self, buf: int) -> None:
        """Reads of the following dequants come from device buffer ``buf`` (a backward pass
        resuming the buffer its forward used)."""
        if self.unit == "model":
            self.active = buf

    def end_step(self, buf: int) -> None:
        """Ends a step's use of ``buf``. Nothing to record: the next copy into ``buf`` rewrites
        the bytes its readers see, so it does not wait for them."""
        del buf

    # -- streaming protocol (hostload.py:297-323) ------------------------------------------------
    def prefetch(self, layer_idx: int) -> None:
        if self.unit != "layer" or layer_idx < 0 or layer_idx >= self.num_layers:
            return
        slot = layer_idx % 2
        if self.slot_layer[slot] == layer_idx:
            return
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(self.compute_done_events[slot])
            for dst, src in ((self.gpu_packed_slots, self.cpu_packed),
                             (self.gpu_absmax_slots, self.cpu_absmax),
                             (self.gpu_absmax2_slots, self.cpu_absmax2)):
                s = src[layer_idx]
                dst[slot][: s.numel()].copy_(s, non_blocking=True)
            self.slot_events[slot].record(self.stream)
            self.slot_layer[slot] = layer_idx

    def wait_slot(self, layer_idx: int) -> int:
        if self.unit != "layer":
            return 0
        slot = layer_idx % 2
        if self.slot_layer[slot] != layer_idx:
            self.prefetch(layer_idx)
        torch.cuda.current_stream(self.device).wait_event(self.slot_events[slot])
        return slot

    def begin_capture(self) -> None:
        """Before capturing a step into a HIP graph: the side stream's first waits depend on an
        event recorded in the capturing stream, and the slots are taken as empty so that the
        graph copies every layer it uses (unit="layer"; nothing to do otherwise)."""
        if self.unit != "layer":
            return
        cur = torch.cuda.current_stream(self.device)
        self.compute_done_events = [torch.cuda.Event() for _ in range(2)]
        for ev in self.compute_done_events:
            ev.record(cur)
        self.slot_events = [torch.cuda.Event() for _ in range(2)]
        self.slot_layer = [-1, -1]

    def after_replay(self) -> None:
        """After a graph replay (or capture) on the current stream: later eager prefetches wait
        for it before overwriting the slots, and take the slots as empty (unit="layer")."""
        if self.unit != "layer":
            return
        cur = torch.cuda.current_stream(self.device)
        self.compute_done_events = [torch.cuda.Event() for _ in range(2)]
        for ev in self.compute_done_events:
            ev.record(cur)
        self.slot_events = [torch.cuda.Event() for _ in range(2)]
        self.slot_layer = [-1, -1]

    def release_slot(self, layer_idx: int) -> None:
        if self.unit != "layer":
            return
        self.compute_done_events[layer_idx % 2].record(torch.cuda.current_stream(self.device))

    def _arrays(self, layer_idx: int):
        if self.unit == "resident":
            return self.gpu_layers[layer_idx]
        if self.unit == "model":
            return self.blob_views[self.active][layer_idx]
        slot = layer_idx % 2
        return self.gpu_packed_slots[slot], self.gpu_absmax_slots[slot], self.gpu_absmax2_slots[slot]

    def dequant(self, layer_idx: int, seg_name: str) -> torch.Tensor:
        """fp16 [out, in] weight of one segment (a view of that segment's workspace, valid until
        the same segment is dequantised again)."""
        seg = self.layer_segments[layer_idx][seg_name]
        packed, absmax, absmax2 = self._arrays(layer_idx)
        return K.dequant_nf4_tensor(
            packed[seg.packed_slice], absmax[seg.absmax_slice], self.code2_gpu,
            absmax2[seg.absmax2_slice], seg.offsets, (seg.out_features, seg.in_features),
            out_buf=self.workspaces[seg_name], split_bytes=seg.split_bytes,
            blocksize=seg.blocksize, super_blocksize=seg.super_blocksize,
            absmax2_bases=seg.absmax2_bases)

    def dequant_layer(self, layer_idx: int, workspaces=None, norm=None) -> dict[str, torch.Tensor]:
        """All four segments of a layer in one dequant launch: {"qkv", "o", "gu", "down"} ->
        fp16 weights (views of the per-segment workspaces, or of ``workspaces``). ``norm``: a
        deferred RMSNorm (``K.DeferredNorm``) that runs in the same launch."""
        packed, absmax, absmax2 = self._arrays(layer_idx)
        segs = self.layer_segments[layer_idx]
        first = segs[SEGMENTS[0]]
        wsp = self.workspaces if workspaces is None else workspaces
        jobs = [{"packed": packed[sg.packed_slice], "absmax": absmax[sg.absmax_slice],
                 "absmax2": absmax2[sg.absmax2_slice], "offset": sg.offsets,
                 "out_shape": (sg.out_features, sg.in_features), "out_buf": wsp[name],
                 "split_bytes": sg.split_bytes, "absmax2_bases": sg.absmax2_bases}
                for name, sg in ((n, segs[n]) for n in SEGMENTS)]
        outs = K.dequant_nf4_segments(jobs, self.code2_gpu, first.blocksize, first.super_blocksize,
                                      norm=norm)
        return dict(zip(SEGMENTS, outs))

    def nf4_layer(self, layer_idx: int) -> dict[str, "K.NF4Operand"]:
        """The four segments of a layer as NF4 operands of the fused products (``K.nf4_gemm``):
        no dequantisation; the kernels read the packed bytes where they lie (slot, whole-model
        buffer or resident copy), so a streamed slot must stay unreleased until the layer's last
        product is enqueued. Operands are cached per (buffer, layer)."""
        key = (self.unit, getattr(self, "active", 0) if self.unit == "model" else 0, layer_idx)
        cache = self.__dict__.setdefault("_nf4_ops", {})
        got = cache.get(key)
        if got is None:
            packed, absmax, absmax2 = self._arrays(layer_idx)
            got = {}
            for name, sg in self.layer_segments[layer_idx].items():
                got[name] = K.NF4Operand(
                    packed[sg.packed_slice], absmax[sg.absmax_slice], absmax2[sg.absmax2_slice],
                    self.code2_gpu, sg.offsets, (sg.out_features, sg.in_features),
                    split_bytes=sg.split_bytes, absmax2_bases=sg.absmax2_bases,
                    blocksize=sg.blocksize, super_blocksize=sg.super_blocksize)
            cache[key] = got
        return got

    # -- dequantisation one layer ahead on a second stream ---------------------------------------
    @property
    def dequant_ahead(self) -> bool:
        return getattr(self, "_ahead", False)

    def enable_dequant_ahead(self) -> None:
        """Dequantises each layer on a second stream into one of two workspace sets while the
        previous layer computes (HBM-bound dequant beside MFMA-bound GEMMs). Whole-model and
        resident units only: their packed bytes are on the device for the whole step."""
        if self.unit == "layer":
            raise ValueError("dequant-ahead needs stream_unit='model' or resident weights")
        self._ahead = True
        self.workspace_sets = [self.workspaces,
                               {k: torch.empty_like(t) for k, t in self.workspaces.items()}]
        self.dq_stream = torch.cuda.Stream(device=self.device)
        self.dq_events = [torch.cuda.Event() for _ in range(2)]
        self.dq_out: list = [None, None]

    def issue_dequant(self, layer_idx: int) -> None:
        """Enqueues the dequant of ``layer_idx`` into workspace set ``layer_idx % 2`` on the
        dequant stream, after all work enqueued so far on the current stream (which holds the
        last use of that set, two layers back in either direction)."""
        k = layer_idx % 2
        main = torch.cuda.current_stream(self.device)
        self.dq_stream.wait_stream(main)
        with torch.cuda.stream(self.dq_stream):
            w = self.dequant_layer(layer_idx, self.workspace_sets[k])
            self.dq_events[k].record(self.dq_stream)
        self.dq_out[k] = (layer_idx, w)

    def take_dequant(self, layer_idx: int) -> dict[str, torch.Tensor]:
        """The weights of ``layer_idx`` from issue_dequant; the current stream waits for them."""
        k = layer_idx % 2
        got = self.dq_out[k]
        if got is None or got[0] != layer_idx:
            raise RuntimeError(f"dequant of layer {layer_idx} was not issued")
        torch.cuda.current_stream(self.device).wait_event(self.dq_events[k])
        return got[1]


class HostHead:
    """Tied embedding / lm_head: HBM-resident (with W^T for the gradient GEMM) or streamed from
    pinned host memory in ``v_chunk``-row chunks through two device slots."""

    def __init__(self, weight: torch.Tensor, device, v_chunk: int = V_CHUNK_DEFAULT,
                 resident: bool = True):
        self.device = torch.device(device)
        self.v_chunk = v_chunk
        self.resident = resident
        self.vocab_size, self.hidden_size = weight.shape
        if resident:
            self.gpu_weight = weight.detach().to(self.device, torch.float16).contiguous()
            self.gpu_weight_t = K.lm_head_weight_t(self.gpu_weight)
        else:
            self.cpu_weight = _pinned(weight.detach().to(torch.float16))
            self.stream = torch.cuda.Stream(device=self.device)
            self.slot_events = [torch.cuda.Event() for _ in range(2)]
            self.compute_done_events = [torch.cuda.Event() for _ in range(2)]
            self.slot_chunk = [-1, -1]
            self.gpu_slots = [torch.empty((v_chunk, self.hidden_size), dtype=torch.float16,
                                          device=self.device) for _ in range(2)]

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        ids = input_ids.reshape(-1)
        if self.resident:
            out = torch.nn.functional.embedding(ids.to(self.device), self.gpu_weight)
        else:  # host gather + async copy, as hostload.py:381-386
            emb = self.cpu_weight.index_select(0, ids.cpu())
            out = emb.pin_memory().to(self.device, non_blocking=True)
        return out.view(*input_ids.shape, self.hidden_size)

    def prefetch_chunk(self, chunk_idx: int, start_v: int, end_v: int) -> None:
        slot = chunk_idx % 2
        if self.slot_chunk[slot] == start_v:
            return
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(self.compute_done_events[slot])
            self.gpu_slots[slot][: end_v - start_v].copy_(self.cpu_weight[start_v:end_v], non_blocking=True)
            self.slot_events[slot].record(self.stream)
            self.slot_chunk[slot] = start_v

    def get_chunk(self, chunk_idx: int, start_v: int, end_v: int) -> torch.Tensor:
        slot = chunk_idx % 2
        if self.slot_chunk[slot] != start_v:
            self.prefetch_chunk(chunk_idx, start_v, end_v)
        torch.cuda.current_stream(self.device).wait_event(self.slot_events[slot])
        return self.gpu_slots[slot][: end_v - start_v]

    def release_chunk(self, chunk_idx: int) -> None:
        self.compute_done_events[chunk_idx % 2].record(torch.cuda.current_stream(self.device))


class InputStream:
    """Per-layer inputs kept for the backward recompute (solution/hostload.py:411-488)."""

    def __init__(self, num_layers: int, hidden_size: int, max_tokens: int, device,
                 offload: bool = False):
        self.num_layers = num_layers
        self.hidden_size = hidden_size
        self.max_tokens = max_tokens
        self.device = torch.device(device)
        self.offload = offload
        self.gpu_saved: dict[int, torch.Tensor] = {}
        if offload:
            self.stream = torch.cuda.Stream(device=self.device)
            self.d2h_events = [torch.cuda.Event() for _ in range(num_layers)]
            self.h2d_events = [torch.cuda.Event() for _ in range(2)]
            self.slot_ready_events = [torch.cuda.Event() for _ in range(2)]
            self.slot_layer = [-1, -1]
            self._alloc(max_tokens)

    def _alloc(self, n: int) -> None:
        self.max_tokens = n
        self.cpu_buffers = [torch.empty((n, self.hidden_size), dtype=torch.float16, pin_memory=True)
                            for _ in range(self.num_layers)]
        self.gpu_slots = [torch.empty((n, self.hidden_size), dtype=torch.float16, device=self.device)
                          for _ in range(2)]

    def save(self, layer_idx: int, x: torch.Tensor) -> None:
        if not self.offload or layer_idx >= self.num_layers - 2:
            self.gpu_saved[layer_idx] = x.detach()  # the stack never modifies a layer input
            return
        n = x.shape[0]
        if n > self.max_tokens:
            torch.cuda.current_stream(self.device).synchronize()
            self._alloc(max(n, 2 * self.max_tokens))
            self.slot_layer = [-1, -1]
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(ev)
            self.cpu_buffers[layer_idx][:n].copy_(x.detach(), non_blocking=True)
            self.d2h_events[layer_idx].record(self.stream)

    def prefetch(self, layer_idx: int, n_tokens: int) -> None:
        if not self.offload or layer_idx < 0 or layer_idx in self.gpu_saved:
            return
        slot = layer_idx % 2
        if self.slot_layer[slot] == layer_idx:
            return
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(self.d2h_events[layer_idx])
            self.stream.wait_event(self.slot_ready_events[slot])
            self.gpu_slots[slot][:n_tokens].copy_(self.cpu_buffers[layer_idx][:n_tokens], non_blocking=True)
            self.h2d_events[slot].record(self.stream)
            self.slot_layer[slot] = layer_idx

    def load(self, layer_idx: int, n_tokens: int) -> torch.Tensor:
        if layer_idx in self.gpu_saved:
            return self.gpu_saved.pop(layer_idx)
        slot = layer_idx % 2
        if self.slot_layer[slot] != layer_idx:
            self.prefetch(layer_idx, n_tokens)
        torch.cuda.current_stream(self.device).wait_event(self.h2d_events[slot])
        return self.gpu_slots[slot][:n_tokens]

    def release(self, layer_idx: int) -> None:
        if self.offload and layer_idx < self.num_layers - 2:
            slot = layer_idx % 2
            self.slot_ready_events[slot].record(torch.cuda.current_stream(self.device))
            self.slot_layer[slot] = -1
