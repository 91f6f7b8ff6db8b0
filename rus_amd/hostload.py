"""Weight, lm_head and activation residency for the fused Qwen2 stack (solution/hostload.py).

Everything that moves between pinned host memory and HBM goes through one mechanism here, a
``SlotRing``: a few device buffers ("slots") that a copy stream refills from the host while the
compute stream reads the others, ordered only by events (no host synchronisation). The three
reference classes keep their public protocol on top of it:

* ``WeightStream`` packs each layer's seven NF4 projections into four fused segments
  ([q|k|v], o, [gate|up], down; solution/hostload.py:159-258) and lays all layers out in one
  byte image (per layer: packed | absmax | absmax2, 256-byte aligned). Placements:
    - ``resident=True``: the image lives in HBM (0.65 GB at Qwen2.5-1.5B; prefetch / wait_slot /
      release_slot do nothing);
    - ``unit="layer"`` (the reference's policy, hostload.py:286-323): the image is pinned on the
      host and a two-slot ring receives one layer at a time (prefetch / wait_slot /
      release_slot);
    - ``unit="model"``: the whole image is copied once per step into one of two device buffers
      while the previous step runs (begin_step / end_step).
  Each segment dequantises into its own fp16 workspace, so a layer needs one dequant launch per
  pass instead of the reference's 17 per step (hostload.py:295, 325-342).
* ``HostHead`` holds the tied embedding / lm_head: HBM-resident with W^T for the gradient GEMM
  (default), or pinned on the host with vocabulary chunks streamed through a two-slot ring
  (hostload.py:345-408). Embedding rows of a host head are gathered on the device by a kernel
  that reads them over the bus (the reference gathers on the host after synchronising).
* ``InputStream`` keeps each layer's input for the backward recompute: in HBM (default), or
  offloaded to pinned host memory and brought back one layer ahead through a two-slot ring
  (hostload.py:411-488, whose three-ahead prefetch into a two-slot ring is always overwritten
  before use).
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch

from . import kernels as K
from .quant import concat_segments

MAX_MLP_TOKENS = 1 << 30  # the reference chunks the MLP at 512 tokens for a 15 GB T4; not needed
V_CHUNK_DEFAULT = 8192  # vocabulary rows per streamed lm_head chunk (hostload.py:24)
SEGMENTS = ("qkv", "o", "gu", "down")
_ALIGN = 256


def _align(x: int) -> int:
    return (x + _ALIGN - 1) // _ALIGN * _ALIGN


def _pinned(t: torch.Tensor) -> torch.Tensor:
    cpu = t.detach().contiguous().cpu()
    return cpu.pin_memory() if torch.cuda.is_available() else cpu


class SlotRing:
    """Device slots refilled from pinned host memory on a copy stream.

    Item ``i`` always uses slot ``i % len(slots)``. Per slot the ring remembers which tag it
    holds, an event that completes when its last fill has landed and an event that completes when
    its last reader is done. ``fill`` enqueues a copy behind that reader event (so a copy never
    overwrites bytes a kernel still reads) unless the slot already holds the tag; ``take`` fills
    if needed and makes the current stream wait for the fill; ``give_back`` marks the reader
    event on the current stream. Copies of one ring run in the order they are enqueued."""

    def __init__(self, device, slots: Sequence):
        self.device = torch.device(device)
        self.slots = list(slots)
        n = len(self.slots)
        self.copy_stream = torch.cuda.Stream(device=self.device)  # default priority
        self._holds: list = [None] * n
        self._landed = [torch.cuda.Event() for _ in range(n)]
        self._read_done = [torch.cuda.Event() for _ in range(n)]
        self._read_marked = [False] * n

    def slot(self, item: int) -> int:
        return item % len(self.slots)

    def holds(self, item: int, tag) -> bool:
        return self._holds[self.slot(item)] == tag

    def fill(self, item: int, tag, copy: Callable) -> int:
        """Enqueues ``copy(slot_buffers)`` on the copy stream (after the slot's last reader) unless
        the slot already holds ``tag``; returns the slot index."""
        s = self.slot(item)
        if self._holds[s] == tag:
            return s
        cs = self.copy_stream
        with torch.cuda.stream(cs):
            if self._read_marked[s]:
                cs.wait_event(self._read_done[s])
            copy(self.slots[s])
            self._landed[s].record(cs)
        self._holds[s] = tag
        return s

    def take(self, item: int, tag, copy: Callable):
        """The slot buffers holding ``tag`` (filled now if they do not), ready for the current
        stream."""
        s = self.fill(item, tag, copy)
        torch.cuda.current_stream(self.device).wait_event(self._landed[s])
        return self.slots[s]

    def give_back(self, item: int, forget: bool = False) -> None:
        """The current stream's reads of ``item``'s slot are all enqueued; ``forget`` drops the tag
        (the next ``fill`` copies again)."""
        s = self.slot(item)
        self._read_done[s].record(torch.cuda.current_stream(self.device))
        self._read_marked[s] = True
        if forget:
            self._holds[s] = None

    def restart(self) -> None:
        """Every slot empty, and idle once the current stream's work so far is done. Used around
        graph capture and replay: the copy stream's first waits then depend on an event recorded
        in the same stream as the capture, and a captured step copies every item it reads."""
        cur = torch.cuda.current_stream(self.device)
        n = len(self.slots)
        self._landed = [torch.cuda.Event() for _ in range(n)]
        self._read_done = [torch.cuda.Event() for _ in range(n)]
        for ev in self._read_done:
            ev.record(cur)
        self._read_marked = [True] * n
        self._holds = [None] * n


class PackedNF4Segment:
    """One fused segment of a layer's packed bytes (hostload.py:27-62), plus the absmax2 base of
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


class _LayerImage:
    """Byte layout of the packed model: per layer [packed | absmax | absmax2 (fp32)], each part
    256-byte aligned, layers back to back. ``views(buf, l, base)`` cuts one layer's three arrays out
    of a byte buffer holding that layer at byte ``base``."""

    def __init__(self, packed_l, absmax_l, absmax2_l):
        self.parts = []  # per layer (start, packed_off, absmax_off, absmax2_off, n_p, n_a, n_a2)
        cur = 0
        for p, a, a2 in zip(packed_l, absmax_l, absmax2_l):
            start = cur
            ao = _align(p.numel())
            a2o = _align(ao + a.numel())
            size = _align(a2o + 4 * a2.numel())
            self.parts.append((start, 0, ao, a2o, p.numel(), a.numel(), a2.numel(), size))
            cur += size
        self.total = cur
        self.max_layer = max((q[-1] for q in self.parts), default=0)

    def build(self, packed_l, absmax_l, absmax2_l) -> torch.Tensor:
        img = torch.zeros(self.total, dtype=torch.uint8)
        for (start, po, ao, a2o, *_), p, a, a2 in zip(self.parts, packed_l, absmax_l, absmax2_l):
            img[start + po: start + po + p.numel()] = p
            img[start + ao: start + ao + a.numel()] = a
            img[start + a2o: start + a2o + 4 * a2.numel()] = a2.contiguous().view(torch.uint8)
        return img

    def layer_range(self, l: int) -> tuple[int, int]:
        start, *_, size = self.parts[l]
        return start, start + size

    def views(self, buf: torch.Tensor, l: int, base: int):
        _, po, ao, a2o, n_p, n_a, n_a2, _ = self.parts[l]
        return (buf[base + po: base + po + n_p], buf[base + ao: base + ao + n_a],
                buf[base + a2o: base + a2o + 4 * n_a2].view(torch.float32))


class WeightStream:
    """Packed NF4 layers served as fp16 weights through the dequant kernel.

    ``unit`` (when not resident) sets what is streamed from pinned host memory per step:
      * "layer": a two-slot ring refilled one layer at a time in each pass (the reference's
        policy, hostload.py:286-323; 2 x 28 layer copies per step);
      * "model": ``model_buffers`` (default 2) whole-model device buffers used in turn; each step
        copies the packed model once (645 MiB at Qwen2.5-1.5B) into the buffer of the next step,
        on the copy stream, while the current step runs. Such a copy does not wait for the
        buffer's last reader while the host image is unchanged (it rewrites the same bytes; a
        copy stream holding a wait on a running step delays, on this runtime, the completion of
        the copies queued before it). After ``host_image_changed()`` the next copy into each
        buffer waits for that buffer's last step."""

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
        self.image = _LayerImage(packed_l, absmax_l, absmax2_l)
        self.model_bytes = self.image.total
        host = self.image.build(packed_l, absmax_l, absmax2_l)
        del packed_l, absmax_l, absmax2_l
        self.active = 0
        if resident:
            self.dev_blobs = [host.to(self.device)]
        else:
            self.host_blob = _pinned(host)
            if self.unit == "model":
                self._init_model_buffers()
            else:
                self._ring = SlotRing(self.device, [
                    torch.empty(self.image.max_layer, dtype=torch.uint8, device=self.device)
                    for _ in range(2)])
        del host
        self.workspaces = {s: torch.empty(n, dtype=torch.float16, device=self.device)
                           for s, n in ws_elems.items()}

    # -- whole-model streaming (unit="model") --------------------------------------------------
    def _init_model_buffers(self) -> None:
        nb = self.n_buffers
        self.dev_blobs = [torch.empty(self.image.total, dtype=torch.uint8, device=self.device)
                          for _ in range(nb)]
        self.stream = torch.cuda.Stream(device=self.device)  # default priority
        self.ready_events = [torch.cuda.Event() for _ in range(nb)]
        self._last_step = [torch.cuda.Event() for _ in range(nb)]
        self._stepped = [False] * nb
        self._image_version = 0
        self._buf_version = [-1] * nb
        self.staged = [False] * nb
        self.next_buffer = 0
        self.copy_marks: list | None = None  # (start, end) timing events per copy, when timing

    def time_copies(self, on: bool = True) -> None:
        """Starts (or stops) recording a pair of timing events around every whole-model copy."""
        self.copy_marks = [] if on else None

    def copy_ms(self) -> list[float]:
        """Durations (ms) of the copies recorded since ``time_copies()`` (synchronises)."""
        out = []
        for e0, e1 in self.copy_marks or []:
            e1.synchronize()
            out.append(e0.elapsed_time(e1))
        return out

    def host_image_changed(self) -> None:
        """Call after modifying ``host_blob``: the next copy into each device buffer then waits
        for the last step that read that buffer."""
        if self.unit == "model":
            self._image_version += 1

    def stage(self, buf: int) -> None:
        """Copies the packed model into device buffer ``buf`` on the copy stream."""
        with torch.cuda.stream(self.stream):
            stale = self._buf_version[buf] not in (-1, self._image_version)
            if stale and self._stepped[buf]:
                self.stream.wait_event(self._last_step[buf])
            if self.copy_marks is not None:
                e0 = torch.cuda.Event(enable_timing=True)
                e0.record(self.stream)
            self.dev_blobs[buf].copy_(self.host_blob, non_blocking=True)
            self.ready_events[buf].record(self.stream)
            if self.copy_marks is not None:
                e1 = torch.cuda.Event(enable_timing=True)
                e1.record(self.stream)
                self.copy_marks.append((e0, e1))
        self._buf_version[buf] = self._image_version
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
        """The current stream's reads of ``buf`` for this step are enqueued."""
        if self.unit == "model":
            self._last_step[buf].record(torch.cuda.current_stream(self.device))
            self._stepped[buf] = True

    # -- per-layer streaming protocol (hostload.py:297-323) ---------------------------------------
    def _layer_copy(self, layer_idx: int):
        lo, hi = self.image.layer_range(layer_idx)
        src = self.host_blob[lo:hi]

        def copy(slot: torch.Tensor) -> None:
            slot[: hi - lo].copy_(src, non_blocking=True)

        return copy

    def prefetch(self, layer_idx: int) -> None:
        """Starts copying ``layer_idx`` into its slot (unit="layer"; otherwise nothing)."""
        if self.unit != "layer" or not 0 <= layer_idx < self.num_layers:
            return
        self._ring.fill(layer_idx, layer_idx, self._layer_copy(layer_idx))

    def wait_slot(self, layer_idx: int) -> int:
        """Makes the current stream wait until ``layer_idx`` is in its slot; returns the slot."""
        if self.unit != "layer":
            return 0
        self._ring.take(layer_idx, layer_idx, self._layer_copy(layer_idx))
        return self._ring.slot(layer_idx)

    def release_slot(self, layer_idx: int) -> None:
        """Every read of ``layer_idx``'s slot is enqueued on the current stream."""
        if self.unit == "layer":
            self._ring.give_back(layer_idx)

    def begin_capture(self) -> None:
        """Before capturing a step into a HIP graph (unit="layer"): the ring restarts empty, so
        the graph copies every layer it reads, behind an event of the capturing stream."""
        if self.unit == "layer":
            self._ring.restart()

    def after_replay(self) -> None:
        """After a graph replay (or capture) on the current stream: later eager prefetches wait
        for it, and take the slots as empty (unit="layer")."""
        if self.unit == "layer":
            self._ring.restart()

    def _arrays(self, layer_idx: int):
        if self.unit == "layer":
            return self.image.views(self._ring.slots[self._ring.slot(layer_idx)], layer_idx, 0)
        buf = self.dev_blobs[self.active if self.unit == "model" else 0]
        return self.image.views(buf, layer_idx, self.image.layer_range(layer_idx)[0])

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
        where = self._ring.slot(layer_idx) if self.unit == "layer" else self.active
        key = (self.unit, where, layer_idx)
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

    # -- one dequant per layer and step: the backward reads the forward's fp16 weights ------------
    @property
    def dequant_once(self) -> bool:
        return getattr(self, "_once", False)

    def enable_dequant_once(self) -> None:
        """Gives every layer fp16 weights of its own (one device allocation holding all layers'
        segments, 2 x the model's weight count in bytes: 2.6 GB for Qwen2.5-1.5B). The forward
        dequantises each layer into its own set and the backward reads that set instead of
        dequantising again. The base weights are frozen, so the set holds the values a second
        dequant of the same packed bytes would write. Whole-model and resident units only."""
        if self.unit == "layer":
            raise ValueError("dequant-once needs stream_unit='model' or resident weights")
        if self.dequant_once:
            return
        sizes = [{n: sg.out_features * sg.in_features for n, sg in segs.items()}
                 for segs in self.layer_segments]
        store = torch.empty(sum(sum(s.values()) for s in sizes), dtype=torch.float16,
                            device=self.device)
        sets, off = [], 0
        for s in sizes:
            d = {}
            for name in SEGMENTS:
                d[name] = store[off: off + s[name]]
                off += s[name]
            sets.append(d)
        self.layer_store, self.layer_sets = store, sets
        self._once = True

    def forward_weights(self, layer_idx: int, norm=None) -> dict[str, torch.Tensor]:
        """The forward's dequant of ``layer_idx`` (with ``norm`` riding in its launch), into the
        layer's own set when dequant-once is on."""
        sets = self.layer_sets[layer_idx] if self.dequant_once else None
        return self.dequant_layer(layer_idx, workspaces=sets, norm=norm)

    def stored_weights(self, layer_idx: int) -> dict[str, torch.Tensor]:
        """The fp16 weights the forward left in ``layer_idx``'s set (dequant-once)."""
        segs = self.layer_segments[layer_idx]
        return {n: self.layer_sets[layer_idx][n].view(sg.out_features, sg.in_features)
                for n, sg in segs.items()}

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
    """Tied embedding / lm_head: HBM-resident (with W^T for the gradient GEMM) or pinned on the
    host and streamed in ``v_chunk``-row vocabulary chunks through a two-slot ring. A chunk slot
    holds the rows [start, end) and, for the gradient GEMM, their transpose (built on the device
    from the rows just copied, so the host is read once per chunk and pass)."""

    def __init__(self, weight: torch.Tensor, device, v_chunk: int = V_CHUNK_DEFAULT,
                 resident: bool = True):
        self.device = torch.device(device)
        self.v_chunk = int(v_chunk)
        self.resident = resident
        self.vocab_size, self.hidden_size = weight.shape
        if self.v_chunk <= 0 or self.v_chunk % K.LM_TILE:
            raise ValueError(f"v_chunk must be a positive multiple of {K.LM_TILE}")
        if resident:
            self.gpu_weight = weight.detach().to(self.device, torch.float16).contiguous()
            self.gpu_weight_t = K.lm_head_weight_t(self.gpu_weight)
        else:
            self.cpu_weight = _pinned(weight.detach().to(torch.float16))
            rows = min(self.v_chunk, self.vocab_size)
            self._ring = SlotRing(self.device, [
                (torch.empty((rows, self.hidden_size), dtype=torch.float16, device=self.device),
                 torch.zeros((self.hidden_size, K._round_up(rows, K.LM_K)), dtype=torch.float16,
                             device=self.device))
                for _ in range(2)])
            self.embed_error = torch.zeros(1, dtype=torch.int32, device=self.device)

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Embedding rows of ``input_ids`` (any shape) as fp16 [*shape, hidden] on the device.

        An id outside [0, vocab) raises IndexError: on the host for host ids, and for device ids
        through ``F.embedding`` (resident) or, streamed, through the packing step's check
        (``ops.pack_varlen(vocab_size=...)``, which every engine path runs first); the streamed
        gather itself reads nothing out of range (such a row becomes zeros and sets
        ``embed_error``)."""
        ids = input_ids.reshape(-1)
        if ids.device.type == "cpu" and ids.numel() and (
                int(ids.min()) < 0 or int(ids.max()) >= self.vocab_size):
            raise IndexError(f"embed: a token id lies outside [0, {self.vocab_size})")
        if self.resident:
            out = torch.nn.functional.embedding(ids.to(self.device), self.gpu_weight)
        else:
            out = K.gather_rows_from_host(self.cpu_weight, ids.to(self.device, torch.int64),
                                          err_flag=self.embed_error)
        return out.view(*input_ids.shape, self.hidden_size)

    def _chunk_copy(self, start_v: int, end_v: int):
        src = self.cpu_weight[start_v:end_v]

        def copy(slot) -> None:
            rows, rows_t = slot
            rows[: end_v - start_v].copy_(src, non_blocking=True)

        return copy

    def prefetch_chunk(self, chunk_idx: int, start_v: int, end_v: int) -> None:
        """Starts copying vocabulary rows [start_v, end_v) into chunk ``chunk_idx``'s slot."""
        self._ring.fill(chunk_idx, (start_v, end_v), self._chunk_copy(start_v, end_v))

    def get_chunk(self, chunk_idx: int, start_v: int, end_v: int) -> torch.Tensor:
        """W[start_v:end_v] on the device, ready for the current stream."""
        rows, _ = self._ring.take(chunk_idx, (start_v, end_v), self._chunk_copy(start_v, end_v))
        return rows[: end_v - start_v]

    def get_chunk_t(self, chunk_idx: int, start_v: int, end_v: int) -> torch.Tensor:
        """W[start_v:end_v]^T [hidden, round_up(rows, 64)] (zero padding columns), formed on the
        current stream from the chunk's rows (which must be in the slot: ``get_chunk`` first)."""
        s = self._ring.slot(chunk_idx)
        if not self._ring.holds(chunk_idx, (start_v, end_v)):
            raise RuntimeError("get_chunk_t: the chunk is not in its slot")
        rows, rows_t = self._ring.slots[s]
        n = end_v - start_v
        K.transpose_rows(rows[:n], rows_t)
        return rows_t

    def release_chunk(self, chunk_idx: int) -> None:
        """Every read of chunk ``chunk_idx``'s slot is enqueued on the current stream."""
        self._ring.give_back(chunk_idx)


class InputStream:
    """Per-layer inputs kept for the backward recompute (solution/hostload.py:411-488).

    In HBM by default. With ``offload=True`` every layer but the last two goes to pinned host
    memory on the ring's copy stream (after the producing stream's work), and ``prefetch`` /
    ``load`` bring it back through a two-slot ring one layer ahead; a layer's host copy and its
    return trip run on the same copy stream, so the return waits for the copy by stream order."""

    def __init__(self, num_layers: int, hidden_size: int, max_tokens: int, device,
                 offload: bool = False):
        self.num_layers = num_layers
        self.hidden_size = hidden_size
        self.max_tokens = max_tokens
        self.device = torch.device(device)
        self.offload = offload
        self.gpu_saved: dict[int, torch.Tensor] = {}
        if offload:
            self._alloc(max_tokens)

    def _alloc(self, n: int) -> None:
        self.max_tokens = n
        self.cpu_buffers = [torch.empty((n, self.hidden_size), dtype=torch.float16, pin_memory=True)
                            for _ in range(self.num_layers)]
        self._ring = SlotRing(self.device, [
            torch.empty((n, self.hidden_size), dtype=torch.float16, device=self.device)
            for _ in range(2)])
        self._saved_n = [0] * self.num_layers

    def _on_host(self, layer_idx: int) -> bool:
        return self.offload and layer_idx < self.num_layers - 2

    def save(self, layer_idx: int, x: torch.Tensor) -> None:
        """Keeps layer ``layer_idx``'s input (the stack never modifies it afterwards)."""
        if not self._on_host(layer_idx):
            self.gpu_saved[layer_idx] = x.detach()
            return
        n = x.shape[0]
        if n > self.max_tokens:
            torch.cuda.current_stream(self.device).synchronize()
            self._ring.copy_stream.synchronize()
            self._alloc(max(n, 2 * self.max_tokens))
        cur = torch.cuda.current_stream(self.device)
        cs = self._ring.copy_stream
        cs.wait_stream(cur)
        with torch.cuda.stream(cs):
            self.cpu_buffers[layer_idx][:n].copy_(x.detach(), non_blocking=True)
        x.record_stream(cs)
        self._saved_n[layer_idx] = n

    def _copy_back(self, layer_idx: int, n: int):
        src = self.cpu_buffers[layer_idx][:n]

        def copy(slot: torch.Tensor) -> None:
            slot[:n].copy_(src, non_blocking=True)

        return copy

    def prefetch(self, layer_idx: int, n_tokens: int) -> None:
        """Starts bringing layer ``layer_idx``'s input back into its slot."""
        if not self._on_host(layer_idx) or layer_idx < 0:
            return
        self._ring.fill(layer_idx, layer_idx, self._copy_back(layer_idx, n_tokens))

    def load(self, layer_idx: int, n_tokens: int) -> torch.Tensor:
        """Layer ``layer_idx``'s input [n_tokens, hidden], ready for the current stream."""
        if layer_idx in self.gpu_saved:
            return self.gpu_saved.pop(layer_idx)
        slot = self._ring.take(layer_idx, layer_idx, self._copy_back(layer_idx, n_tokens))
        return slot[:n_tokens]

    def release(self, layer_idx: int) -> None:
        """The current stream's reads of layer ``layer_idx``'s input are enqueued."""
        if self._on_host(layer_idx):
            self._ring.give_back(layer_idx, forget=True)
