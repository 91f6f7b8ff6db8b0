"""Kernel launchers with the names and signatures of ``solution/kernels.py`` (the reference).

Each launcher validates its tensors, allocates outputs with ``torch.empty`` on the input's device
(as the reference does, kernels.py:588, 633-634, 684, 732-734, 778, 810, 892-893) and enqueues one
gfx950 kernel from ``librus_amd.so`` on the current HIP stream through the C ABI
(``include/rus_amd.h``). Nothing here computes on the host: a CPU tensor or a missing library
raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import DTYPE_F16, DTYPE_F32

__all__ = [
    "adamw_step",
    "lora_cast_t",
    "dequant_nf4_tensor",
    "dequant_nf4_segments",
    "NF4Operand",
    "nf4_gemm_plan",
    "nf4_gemm",
    "nf4_absmax2_bases",
    "rms_norm_fwd",
    "rms_norm_bwd",
    "DeferredNorm",
    "copy_from_host",
    "gather_rows_from_host",
    "rms_norm_bwd_parts",
    "qkv_rope_fwd",
    "qkv_rope_bwd",
    "qkv_rope_bwd_lora",
    "qkv_rope_bwd_lora_mid",
    "qkv_rope_bwd_lora_mid_parts",
    "rope_bwd_mid_supported",
    "lora_dropout_fwd",
    "lora_dropout_bwd_add",
    "dropout_keep_bits",
    "lora_workspace_size",
    "lora_down_rows",
    "LORA_ROWS_RANKS",
    "lora_down_fwd",
    "qkv_rope_fwd_mid",
    "lora_bwd_x",
    "lora_bwd_w",
    "mlp_glu_fwd",
    "mlp_glu_bwd",
    "lm_head_ce",
    "lm_head_ce_loss",
    "lm_head_ce_chunk_scale",
    "lm_head_ce_grad_hidden_scaled",
    "lm_head_ce_dh_finish",
    "lm_head_chunk_cols",
    "lm_head_token_blocks",
    "lm_head_block_tokens",
    "lm_head_ce_denom",
    "lm_head_ce_logits",
    "lm_head_ce_rows",
    "LMHeadPass",
    "lm_head_ce_fwd_chunk",
    "lm_head_ce_combine",
    "lm_head_ce_grad_logits",
    "lm_head_ce_grad_from_logits",
    "lm_head_ce_grad_hidden",
    "lm_head_dh_reduce",
    "lm_head_weight_t",
    "transpose_rows",
    "attn_varlen_fwd",
    "attn_varlen_bwd",
    "attn_varlen_bwd_parts",
    "gemm_parts",
    "gemm_parts_count",
]


def _require_device(fn: str, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{fn}: rus_amd kernels need HIP device tensors, got {t.device}")


def _dtype_code(fn: str, dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DTYPE_F16
    if dtype == torch.float32:
        return DTYPE_F32
    raise TypeError(f"{fn}: unsupported dtype {dtype} (fp16 or fp32)")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class KernelTimer:
    """Per-launch device timing for the launchers in this module: while active, every launch is
    bracketed by two HIP events recorded on the stream it is enqueued on (the current stream) and
    tagged with its algorithmic bytes and FLOPs. ``summary()`` synchronises and aggregates."""

    active: "KernelTimer | None" = None

    def __init__(self, only: set[str] | None = None):
        self.only = only  # record only these kernels (None: all)
        self.records: list[tuple[str, torch.cuda.Event, torch.cuda.Event, float, float]] = []

    def __enter__(self):
        KernelTimer.active = self
        return self

    def __exit__(self, *exc):
        KernelTimer.active = None
        return False

    @staticmethod
    def pair_overhead_ms(n: int = 64) -> float:
        """Median elapsed time of an empty event pair on the current stream (the floor under
        every per-launch figure)."""
        pairs = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            e1.record()
            pairs.append((e0, e1))
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) for a, b in pairs)
        return ts[len(ts) // 2]

    def summary(self) -> dict[str, dict]:
        torch.cuda.synchronize()
        out: dict[str, dict] = {}
        for name, e0, e1, nbytes, flops in self.records:
            r = out.setdefault(name, {"launches": 0, "ms": 0.0, "bytes": 0.0, "flops": 0.0})
            r["launches"] += 1
            r["ms"] += e0.elapsed_time(e1)
            r["bytes"] += nbytes
            r["flops"] += flops
        return out


def _launch(kernel: str, nbytes: float, flops: float, fn: str, *args) -> None:
    """Calls C entry point ``fn``; under an active KernelTimer also records its duration."""
    t = KernelTimer.active
    if t is None or (t.only is not None and kernel not in t.only):
        _lib.call(fn, *args)
        return
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    _lib.call(fn, *args)
    e1.record()
    t.records.append((kernel, e0, e1, float(nbytes), float(flops)))


# ---------------------------------------------------------------------------------------------
# NF4 double-quant dequantisation (reference: kernels.py:27-118, launcher kernels.py:572-619)
# ---------------------------------------------------------------------------------------------


def nf4_absmax2_bases(
    n_bytes: int, split_bytes: tuple[int, int] | None, blocksize: int, super_blocksize: int
) -> tuple[int, int]:
    """absmax2 index at which segments 1 and 2 start when each segment was double-quantised on
    its own (ceil(blocks / super_blocksize) entries per segment, concatenated)."""
    if split_bytes is None:
        return 0, 0
    hb = blocksize // 2
    s1, s2 = int(split_bytes[0]), int(split_bytes[1])
    n0 = -(-(s1 // hb) // super_blocksize) if s1 > 0 else 0
    n1 = -(-((s2 - s1) // hb) // super_blocksize) if s2 > s1 else 0
    return n0, n0 + n1


def dequant_nf4_tensor(
    packed: torch.Tensor,
    absmax: torch.Tensor,
    code2: torch.Tensor,
    absmax2: torch.Tensor,
    offset: float | tuple[float, float, float],
    out_shape: tuple[int, int],
    out_buf: torch.Tensor | None = None,
    split_bytes: tuple[int, int] | None = None,
    blocksize: int = 64,
    super_blocksize: int = 256,
    absmax2_bases: tuple[int, int] | None = None,
) -> torch.Tensor:
    """Dequantise packed NF4 (2 codes per byte, high nibble first) with double-quantised absmax
    into fp16 ``out_shape`` (a new tensor, or a view at the start of ``out_buf``).

    ``offset`` is one float or one per segment; ``split_bytes`` gives the byte offsets where
    segments 1 and 2 start (fused [q|k|v] or [gate|up]). ``absmax2_bases`` (an extension of the
    reference signature) gives where each segment's absmax2 entries start; by default each segment
    is taken to have been double-quantised on its own, which equals the reference's global
    super-block indexing whenever segment block counts are multiples of ``super_blocksize``.
    """
    fn = "dequant_nf4_tensor"
    _require_device(fn, packed, absmax, code2, absmax2, out_buf)
    n_elements = int(out_shape[0]) * int(out_shape[1])
    if n_elements % 2:
        raise ValueError(f"{fn}: element count {n_elements} must be even (2 codes per byte)")
    n_bytes = n_elements // 2
    if packed.dtype != torch.uint8 or absmax.dtype != torch.uint8:
        raise TypeError(f"{fn}: packed and absmax must be uint8")
    if code2.dtype != torch.float32 or absmax2.dtype != torch.float32:
        raise TypeError(f"{fn}: code2 and absmax2 must be float32")
    packed = packed.reshape(-1)
    absmax = absmax.reshape(-1)
    code2 = code2.reshape(-1)
    absmax2 = absmax2.reshape(-1)
    for name, t in (("packed", packed), ("absmax", absmax), ("code2", code2), ("absmax2", absmax2)):
        if not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous")
    if packed.numel() < n_bytes:
        raise ValueError(f"{fn}: packed has {packed.numel()} bytes, need {n_bytes}")
    if code2.numel() != 256:
        raise ValueError(f"{fn}: code2 must have 256 entries, got {code2.numel()}")
    if out_buf is None:
        out = torch.empty(out_shape, dtype=torch.float16, device=packed.device)
    else:
        if out_buf.dtype != torch.float16 or out_buf.numel() < n_elements:
            raise ValueError(f"{fn}: out_buf must be fp16 with at least {n_elements} elements")
        out = out_buf.view(-1)[:n_elements].view(out_shape)
    if isinstance(offset, (tuple, list)):
        off0, off1, off2 = float(offset[0]), float(offset[1]), float(offset[2])
    else:
        off0 = off1 = off2 = float(offset)
    if split_bytes is not None:
        sb1, sb2 = int(split_bytes[0]), int(split_bytes[1])
    else:
        sb1 = sb2 = n_bytes
    if absmax2_bases is None:
        absmax2_bases = nf4_absmax2_bases(n_bytes, (sb1, sb2), blocksize, super_blocksize)
    _launch(
        "nf4_dequant", n_bytes + absmax.numel() + 4 * absmax2.numel() + 1024 + 2 * n_elements, 0,
        "rus_nf4_dequant",
        packed.data_ptr(), absmax.data_ptr(), code2.data_ptr(), absmax2.data_ptr(),
        off0, off1, off2, sb1, sb2, int(absmax2_bases[0]), int(absmax2_bases[1]),
        n_bytes, absmax.numel(), absmax2.numel(), int(blocksize), int(super_blocksize),
        out.data_ptr(), _stream(out),
    )
    return out


def dequant_nf4_segments(segments: list[dict], code2: torch.Tensor, blocksize: int = 64,
                         super_blocksize: int = 256,
                         norm: DeferredNorm | None = None) -> list[torch.Tensor]:
    """Dequantise 1..4 NF4 segments in one launch (one layer's [q|k|v], o, [gate|up], down).

    Each entry: packed, absmax, absmax2 (device tensors), offset (float or 3-tuple), out_shape,
    out_buf (fp16, optional), split_bytes and absmax2_bases (optional), as for
    ``dequant_nf4_tensor``. ``norm``: a deferred RMSNorm run inside the same launch (or just
    before it, when its shape does not fit the combined kernel). Returns the fp16 weights in
    order."""
    fn = "dequant_nf4_segments"
    if not 1 <= len(segments) <= 4:
        raise ValueError(f"{fn}: 1..4 segments")
    _require_device(fn, code2)
    if code2.dtype != torch.float32 or code2.numel() != 256:
        raise ValueError(f"{fn}: code2 must be 256 float32 values")
    code2 = code2.reshape(-1).contiguous()
    jobs = (_lib.Nf4Job * len(segments))()
    outs = []
    total_bytes = 1024
    for j, sg in enumerate(segments):
        packed, absmax, absmax2 = (sg[k].reshape(-1) for k in ("packed", "absmax", "absmax2"))
        _require_device(fn, packed, absmax, absmax2, sg.get("out_buf"))
        if packed.dtype != torch.uint8 or absmax.dtype != torch.uint8 or absmax2.dtype != torch.float32:
            raise TypeError(f"{fn}: packed/absmax must be uint8 and absmax2 float32")
        for t in (packed, absmax, absmax2):
            if not t.is_contiguous():
                raise ValueError(f"{fn}: segment arrays must be contiguous")
        shape = sg["out_shape"]
        n_el = int(shape[0]) * int(shape[1])
        if n_el % 2 or n_el == 0:
            raise ValueError(f"{fn}: element count {n_el} must be even and positive")
        nb = n_el // 2
        if packed.numel() < nb:
            raise ValueError(f"{fn}: packed has {packed.numel()} bytes, need {nb}")
        ob = sg.get("out_buf")
        if ob is None:
            out = torch.empty(shape, dtype=torch.float16, device=packed.device)
        else:
            if ob.dtype != torch.float16 or ob.numel() < n_el:
                raise ValueError(f"{fn}: out_buf must be fp16 with at least {n_el} elements")
            out = ob.view(-1)[:n_el].view(shape)
        off = sg["offset"]
        offs = (off, off, off) if not isinstance(off, (tuple, list)) else tuple(off)
        sp = sg.get("split_bytes") or (nb, nb)
        bases = sg.get("absmax2_bases") or nf4_absmax2_bases(nb, sp, blocksize, super_blocksize)
        jb = jobs[j]
        jb.packed, jb.absmax, jb.absmax2 = packed.data_ptr(), absmax.data_ptr(), absmax2.data_ptr()
        jb.off0, jb.off1, jb.off2 = (float(o) for o in offs)
        jb.split_byte_1, jb.split_byte_2 = int(sp[0]), int(sp[1])
        jb.absmax2_base_1, jb.absmax2_base_2 = int(bases[0]), int(bases[1])
        jb.n_bytes, jb.n_absmax, jb.n_absmax2 = nb, absmax.numel(), absmax2.numel()
        jb.out_u32 = out.data_ptr()
        outs.append(out)
        total_bytes += nb + absmax.numel() + 4 * absmax2.numel() + 2 * n_el
    if norm is not None and not norm.done and norm.side is not None:
        down = None if norm.down is None else ctypes.byref(norm.down)
        extra = 0 if norm.down is None else _down_rows_bytes(norm.down)
        _launch("nf4_dequant", total_bytes + norm.nbytes + extra, 0, "rus_nf4_dequant_multi_norm",
                jobs, len(segments), code2.data_ptr(), int(blocksize), int(super_blocksize),
                ctypes.byref(norm.side), down, _stream(code2))
        norm.done = True
        return outs
    if norm is not None:
        norm.run()
    _launch("nf4_dequant", total_bytes, 0, "rus_nf4_dequant_multi", jobs, len(segments),
            code2.data_ptr(), int(blocksize), int(super_blocksize), _stream(code2))
    return outs


# ---------------------------------------------------------------------------------------------
# NF4 W4A16 products: dequantisation inside the GEMM main loop (replaces dequant_nf4_tensor +
# F.linear / torch.mm on its output, solution/ops.py:710-724, 771, 810, 873-993)
# ---------------------------------------------------------------------------------------------


class NF4Operand:
    """A device NF4 double-quant weight [out_features, in_features] (one segment job: up to
    three row segments with their own offsets and absmax2 bases) for ``nf4_gemm``. Holds the
    device arrays it points into."""

    __slots__ = ("job", "code2", "shape", "blocksize", "super_blocksize", "_keep")

    def __init__(self, packed, absmax, absmax2, code2, offset, shape, split_bytes=None,
                 absmax2_bases=None, blocksize: int = 64, super_blocksize: int = 256):
        fn = "NF4Operand"
        packed, absmax, absmax2 = (t.reshape(-1) for t in (packed, absmax, absmax2))
        _require_device(fn, packed, absmax, absmax2, code2)
        if packed.dtype != torch.uint8 or absmax.dtype != torch.uint8 or \
                absmax2.dtype != torch.float32 or code2.dtype != torch.float32:
            raise TypeError(f"{fn}: packed/absmax must be uint8, absmax2/code2 float32")
        if not (packed.is_contiguous() and absmax.is_contiguous() and absmax2.is_contiguous()):
            raise ValueError(f"{fn}: arrays must be contiguous")
        rows, cols = int(shape[0]), int(shape[1])
        nb = rows * cols // 2
        if packed.numel() < nb:
            raise ValueError(f"{fn}: packed has {packed.numel()} bytes, need {nb}")
        offs = (offset,) * 3 if not isinstance(offset, (tuple, list)) else tuple(offset)
        sp = split_bytes or (nb, nb)
        bases = absmax2_bases or nf4_absmax2_bases(nb, sp, blocksize, super_blocksize)
        jb = _lib.Nf4Job()
        jb.packed, jb.absmax, jb.absmax2 = packed.data_ptr(), absmax.data_ptr(), absmax2.data_ptr()
        jb.off0, jb.off1, jb.off2 = (float(o) for o in offs)
        jb.split_byte_1, jb.split_byte_2 = int(sp[0]), int(sp[1])
        jb.absmax2_base_1, jb.absmax2_base_2 = int(bases[0]), int(bases[1])
        jb.n_bytes, jb.n_absmax, jb.n_absmax2 = nb, absmax.numel(), absmax2.numel()
        jb.out_u32 = None
        self.job = jb
        self.code2 = code2.reshape(-1).contiguous()
        self.shape = (rows, cols)
        self.blocksize = int(blocksize)
        self.super_blocksize = int(super_blocksize)
        self._keep = (packed, absmax, absmax2)

    @property
    def device(self) -> torch.device:
        return self.code2.device


_gemm_plans: dict[tuple[int, int, int, int, int], tuple[int, int, int]] = {}
_gemm_counters: dict[tuple[int, int], torch.Tensor] = {}
_attn_counters: dict[tuple[int, int], torch.Tensor] = {}


def nf4_gemm_plan(m: int, w_rows: int, w_cols: int, trans: bool, split: int = 0):
    """(split, fp32 workspace elements, counters) that ``nf4_gemm`` uses for this shape."""
    key = (int(m), int(w_rows), int(w_cols), int(bool(trans)), int(split))
    got = _gemm_plans.get(key)
    if got is None:
        sp, fl, ct = ctypes.c_int32(int(split)), ctypes.c_int64(), ctypes.c_int64()
        _lib.call("rus_nf4_gemm_plan", int(m), int(w_rows), int(w_cols), int(bool(trans)),
                  ctypes.byref(sp), ctypes.byref(fl), ctypes.byref(ct))
        got = _gemm_plans[key] = (sp.value, fl.value, ct.value)
    return got


def nf4_gemm(x: torch.Tensor, w: NF4Operand, trans: bool = False,
             bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
             split: int = 0) -> torch.Tensor:
    """trans=False: x [m, in] @ W^T (+ bias) -> [m, out] (F.linear); trans=True: x [m, out] @ W
    -> [m, in] (the input-gradient product). W is decoded from NF4 inside the kernel; fp32 sums,
    one fp16 rounding. ``out``: optional fp16 destination with unit column stride."""
    fn = "nf4_gemm"
    _require_device(fn, x, bias, out)
    rows, cols = w.shape
    n_in, n_out = (rows, cols) if trans else (cols, rows)
    x2 = _rows(fn, x, n_in, "x")
    if x2.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 activations only")
    m = x2.shape[0]
    if bias is not None:
        if trans or bias.dtype != torch.float16 or bias.numel() != n_out:
            raise ValueError(f"{fn}: bias must be fp16 [{n_out}] (forward product only)")
        bias = bias.reshape(-1).contiguous()
    if out is None:
        out = torch.empty((m, n_out), dtype=torch.float16, device=x2.device)
    elif out.dtype != torch.float16 or tuple(out.shape) != (m, n_out) or out.stride(1) != 1:
        raise ValueError(f"{fn}: out must be fp16 [{m}, {n_out}] with unit column stride")
    ks, floats, counters = nf4_gemm_plan(m, rows, cols, trans, split)
    ws = cnt = None
    if ks > 1:
        ws = torch.empty(floats, dtype=torch.float32, device=x2.device)
        cnt = _counter_buffer(_gemm_counters, x2.device, counters)
    _launch("nf4_gemm", m * n_in * 2 + rows * cols * 33 // 64 + m * n_out * 2, 2 * m * rows * cols,
            "rus_nf4_gemm", x2.data_ptr(), m, x2.stride(0), ctypes.byref(w.job),
            w.code2.data_ptr(), rows, cols, w.blocksize, w.super_blocksize, int(bool(trans)),
            _ptr(bias), out.data_ptr(), out.stride(0), ks, _ptr(ws),
            0 if ws is None else ws.numel(), _ptr(cnt), 0 if cnt is None else cnt.numel(),
            _stream(x2))
    return out


def _counter_buffer(cache: dict, dev: torch.device, need: int) -> torch.Tensor:
    """A zeroed int32 arrival-counter buffer for kernels that leave their counters at zero, one
    per (device, stream) (launches on one stream never overlap), kept for the life of the process
    (captured graphs hold its address)."""
    if need > LORA_MAX_COUNTERS:
        raise RuntimeError(f"kernel needs {need} arrival counters (at most {LORA_MAX_COUNTERS})")
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    cnt = cache.get(key)
    if cnt is None:
        cnt = cache[key] = torch.zeros(LORA_MAX_COUNTERS, dtype=torch.int32, device=dev)
    return cnt


# ---------------------------------------------------------------------------------------------
# Residual + RMSNorm (reference: kernels.py:125-199, launchers kernels.py:622-714)
# ---------------------------------------------------------------------------------------------


def copy_from_host(dst: torch.Tensor, host_src: torch.Tensor) -> None:
    """dst <- host_src, where host_src is a pinned CPU tensor of the same byte size (a multiple of
    16): read by a kernel on the current stream (no copy-engine transfer), so a captured graph can
    take its inputs from a host staging image."""
    fn = "copy_from_host"
    _require_device(fn, dst)
    if host_src.device.type != "cpu" or not host_src.is_pinned():
        raise ValueError(f"{fn}: the source must be a pinned CPU tensor")
    nb = dst.numel() * dst.element_size()
    if not dst.is_contiguous() or not host_src.is_contiguous() or \
            host_src.numel() * host_src.element_size() != nb:
        raise ValueError(f"{fn}: contiguous tensors of equal byte size required")
    _launch("copy_from_host", 2 * nb, 0, "rus_copy_from_host", dst.data_ptr(),
            host_src.data_ptr(), nb, _stream(dst))


def gather_rows_from_host(host_rows: torch.Tensor, ids: torch.Tensor,
                          err_flag: torch.Tensor | None = None) -> torch.Tensor:
    """host_rows[ids] as a new device tensor, where host_rows is a pinned 2-D CPU tensor and ids
    an int64 device tensor: a kernel on the current stream reads the selected rows over the bus
    (no host synchronisation). Ids out of range give zero rows and set ``err_flag`` (a device
    int32 tensor) when one is passed."""
    fn = "gather_rows_from_host"
    _require_device(fn, ids, err_flag)
    if host_rows.device.type != "cpu" or not host_rows.is_pinned() or host_rows.dim() != 2 \
            or not host_rows.is_contiguous():
        raise ValueError(f"{fn}: the source must be a contiguous pinned 2-D CPU tensor")
    row_bytes = host_rows.shape[1] * host_rows.element_size()
    if row_bytes % 16:
        raise ValueError(f"{fn}: rows must be a multiple of 16 bytes")
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64:
        raise TypeError(f"{fn}: ids must be int64")
    flat = flat.contiguous()
    out = torch.empty((flat.numel(), host_rows.shape[1]), dtype=host_rows.dtype, device=ids.device)
    if err_flag is not None and (err_flag.dtype != torch.int32 or err_flag.numel() < 1):
        raise ValueError(f"{fn}: err_flag must be a device int32 tensor")
    _launch("gather_rows_from_host", 2 * out.numel() * out.element_size() + 8 * flat.numel(), 0,
            "rus_gather_rows_from_host", host_rows.data_ptr(), host_rows.shape[0], row_bytes,
            flat.data_ptr(), flat.numel(), out.data_ptr(), _ptr(err_flag), _stream(out))
    return out


class DeferredNorm:
    """An RMSNorm launch held back (``rms_norm_fwd`` / ``rms_norm_bwd`` with ``defer=True``): its
    outputs exist, its kernel runs either inside the next layer dequant launch
    (``dequant_nf4_segments(..., norm=...)``, when ``side`` is set) or alone (``run``). Nothing
    may read the outputs before one of the two has been enqueued. Holds its operands alive."""

    __slots__ = ("kernel", "nbytes", "fn", "args", "side", "keep", "done", "out", "down",
                 "down_keep")

    def __init__(self, kernel, nbytes, fn, args, side, keep, out=None):
        self.kernel, self.nbytes, self.fn, self.args = kernel, nbytes, fn, args
        self.side, self.keep, self.done, self.out = side, keep, False, out
        self.down = self.down_keep = None

    def carry_lora_down(self, a_q: torch.Tensor, a_v: torch.Tensor,
                        bits_q: torch.Tensor | None = None, bits_v: torch.Tensor | None = None,
                        p_q: float = 0.0, p_v: float = 0.0):
        """Attaches the LoRA-down of this (forward) norm's output, ``lora_down_rows`` on it, to
        the norm's launch: the dequant launch that carries the norm forms it in the same blocks,
        ``run`` right after the norm. Returns (mid_q, mid_v), valid once the norm is enqueued."""
        if self.out is None or self.done or self.down is not None:
            raise RuntimeError("carry_lora_down: needs a forward norm not yet enqueued")
        mid_q, mid_v, args, keep = _lora_rows(self.out, a_q, a_v, bits_q, bits_v, p_q, p_v)
        self.down, self.down_keep = args, keep
        return mid_q, mid_v

    def run(self) -> None:
        """Launches the norm (and a carried LoRA-down) on its own (no-op once enqueued)."""
        if not self.done:
            _launch(self.kernel, self.nbytes, 0, self.fn, *self.args)
            if self.down is not None:
                _launch_down_rows(self.down, self.out)
            self.done = True


def _norm_side(kind, n_rows, n_cols, stride, eps, wdt, x, res, h, w, rstd, sum_out, out):
    """The rus_norm_side of a norm the dequant launch can carry (None when it cannot: fp16
    rows of at most 2048 columns, widths and strides multiples of 8, 16-byte aligned)."""
    ptrs = [t for t in (x, res, h, w, sum_out, out) if t is not None]
    if n_rows == 0 or n_cols > 2048 or n_cols % 8 or stride % 8 or \
            any(t.data_ptr() % 16 for t in ptrs) or x.dtype != torch.float16:
        return None
    sd = _lib.NormSide()
    sd.kind, sd.w_dtype = kind, wdt
    sd.n_rows, sd.n_cols, sd.stride_row, sd.eps = n_rows, n_cols, stride, float(eps)
    sd.x, sd.residual, sd.h, sd.weight = (_ptr(t) for t in (x, res, h, w))
    sd.rstd, sd.sum_out, sd.out = _ptr(rstd), _ptr(sum_out), _ptr(out)
    return sd


def rms_norm_fwd(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    residual: torch.Tensor | None = None,
    defer: bool = False,
):
    """Fused residual add + RMSNorm forward. Returns (norm_out, sum_out_or_x, rstd), plus a
    ``DeferredNorm`` (not yet launched) when ``defer``."""
    fn = "rms_norm_fwd"
    _require_device(fn, x, weight, residual)
    dt = _dtype_code(fn, x.dtype)
    wdt = _dtype_code(fn, weight.dtype)
    orig_shape = x.shape
    n_cols = orig_shape[-1]
    x_2d = x.contiguous().view(-1, n_cols)
    n_rows = x_2d.shape[0]
    w = weight.contiguous()
    if w.numel() != n_cols:
        raise ValueError(f"{fn}: weight has {w.numel()} entries, rows have {n_cols}")
    norm_out = torch.empty_like(x_2d)
    rstd = torch.empty((n_rows,), dtype=torch.float32, device=x.device)
    if residual is not None:
        if residual.dtype != x.dtype or residual.shape != orig_shape:
            raise ValueError(f"{fn}: residual must match x in shape and dtype")
        res_2d = residual.contiguous().view(-1, n_cols)
        sum_out = torch.empty_like(x_2d)
    else:
        res_2d = sum_out = None
    nbytes = (4 if res_2d is not None else 2) * n_rows * n_cols * x_2d.element_size() + \
        w.numel() * w.element_size() + 4 * n_rows
    args = (x_2d.data_ptr(), _ptr(res_2d), w.data_ptr(), wdt, _ptr(sum_out), norm_out.data_ptr(),
            rstd.data_ptr(), n_rows, n_cols, x_2d.stride(0), float(eps), dt, _stream(x))
    outs = (norm_out.view(orig_shape), x if sum_out is None else sum_out.view(orig_shape), rstd)
    if defer:
        side = _norm_side(_lib.NORM_FWD, n_rows, n_cols, x_2d.stride(0), eps, wdt, x_2d, res_2d,
                          None, w, rstd, sum_out, norm_out)
        return outs + (DeferredNorm("rmsnorm_fwd", nbytes, "rus_rmsnorm_fwd", args, side,
                                    (x_2d, res_2d, w, sum_out, norm_out, rstd), out=norm_out),)
    _launch("rmsnorm_fwd", nbytes, 0, "rus_rmsnorm_fwd", *args)
    return outs


def rms_norm_bwd(
    dy: torch.Tensor,
    h: torch.Tensor,
    weight: torch.Tensor,
    rstd: torch.Tensor,
    dresidual: torch.Tensor | None = None,
    defer: bool = False,
):
    """RMSNorm backward with optional residual-gradient accumulation (no weight gradient).
    Returns dx, or (dx, ``DeferredNorm``) when ``defer`` (not yet launched)."""
    fn = "rms_norm_bwd"
    _require_device(fn, dy, h, weight, rstd, dresidual)
    dt = _dtype_code(fn, h.dtype)
    wdt = _dtype_code(fn, weight.dtype)
    orig_shape = dy.shape
    n_cols = orig_shape[-1]
    dy_2d = dy.contiguous().view(-1, n_cols)
    h_2d = h.contiguous().view(-1, n_cols)
    if dy_2d.dtype != h_2d.dtype or dy_2d.shape != h_2d.shape:
        raise ValueError(f"{fn}: dy and h must match in shape and dtype")
    n_rows = dy_2d.shape[0]
    w = weight.contiguous()
    rs = rstd.contiguous()
    if rs.dtype != torch.float32 or rs.numel() != n_rows:
        raise ValueError(f"{fn}: rstd must be float32 with {n_rows} entries")
    dx = torch.empty_like(h_2d)
    dres_ptr = dres_2d = None
    if dresidual is not None:
        dres_2d = dresidual.contiguous().view(-1, n_cols)
        if dres_2d.dtype != h_2d.dtype or dres_2d.shape != h_2d.shape:
            raise ValueError(f"{fn}: dresidual must match h in shape and dtype")
        dres_ptr = dres_2d.data_ptr()
    nbytes = (4 if dres_ptr is not None else 3) * n_rows * n_cols * h_2d.element_size() + \
        w.numel() * w.element_size() + 4 * n_rows
    args = (dy_2d.data_ptr(), h_2d.data_ptr(), w.data_ptr(), wdt, rs.data_ptr(), dres_ptr,
            dx.data_ptr(), n_rows, n_cols, dy_2d.stride(0), dt, _stream(dy))
    if defer:
        side = None
        if dy_2d.stride(0) == h_2d.stride(0) == dx.stride(0) and \
                (dres_2d is None or dres_2d.stride(0) == dx.stride(0)):
            side = _norm_side(_lib.NORM_BWD, n_rows, n_cols, dx.stride(0), 0.0, wdt, dy_2d,
                              dres_2d, h_2d, w, rs, None, dx)
        return dx.view(orig_shape), DeferredNorm("rmsnorm_bwd", nbytes, "rus_rmsnorm_bwd", args,
                                                 side, (dy_2d, h_2d, w, rs, dres_2d, dx))
    _launch("rmsnorm_bwd", nbytes, 0, "rus_rmsnorm_bwd", *args)
    return dx.view(orig_shape)


def gemm_parts_count(k: int, n_split: int) -> int:
    """Number of pieces rus_gemm_parts cuts a K-long reduction into when asked for ``n_split``:
    pieces of round_up(ceil(k / n_split), 64) columns."""
    per = _round_up(-(-k // n_split), LM_K)
    return -(-k // per)


def gemm_parts(a: torch.Tensor, b: torch.Tensor, b_kn: bool, n_split: int,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 split-K partials [S, M, N] of a . b (``b_kn``: b is [K, N]) or a . b^T (b is [N, K]),
    S = gemm_parts_count(K, n_split); the split-K form of torch.mm(d_gu, W_gu)
    (solution/ops.py:939) whose partials rms_norm_bwd_parts consumes."""
    fn = "gemm_parts"
    _require_device(fn, a, b, out)
    for name, t in (("a", a), ("b", b)):
        if t.dtype != torch.float16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"{fn}: {name} must be a 2-D fp16 tensor with contiguous rows")
    m, k = a.shape
    n = b.shape[1] if b_kn else b.shape[0]
    if (b.shape[0] if b_kn else b.shape[1]) != k:
        raise ValueError(f"{fn}: inner dimensions differ: a {tuple(a.shape)}, b {tuple(b.shape)}")
    sp = gemm_parts_count(k, n_split)
    if out is None:
        out = torch.empty(sp, m, n, dtype=torch.float32, device=a.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (sp, m, n) or not out.is_contiguous():
        raise ValueError(f"{fn}: out must be contiguous float32 [{sp}, {m}, {n}]")
    _launch("gemm_parts", (m * k + k * n) * 2 + 4 * sp * m * n, 2.0 * m * n * k,
            "rus_gemm_parts", a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
            1 if b_kn else 0, m, n, k, out.data_ptr(), sp, _stream(a))
    return out


def rms_norm_bwd_parts(dy_parts: torch.Tensor, h: torch.Tensor, weight: torch.Tensor,
                       rstd: torch.Tensor, dresidual: torch.Tensor | None = None) -> torch.Tensor:
    """``rms_norm_bwd`` whose dy is fp16(sum over the leading axis of the fp32 partials
    dy_parts [S, n_rows, n_cols], in order): a split-K product consumed without a reduce
    launch; equal bit for bit to ``rms_norm_bwd(sum_splits(dy_parts), ...)``."""
    fn = "rms_norm_bwd_parts"
    _require_device(fn, dy_parts, h, weight, rstd, dresidual)
    if h.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 activations only")
    n_cols = h.shape[-1]
    h_2d = h.contiguous().view(-1, n_cols)
    n_rows = h_2d.shape[0]
    if dy_parts.dtype != torch.float32 or dy_parts.dim() != 3 or \
            tuple(dy_parts.shape[1:]) != (n_rows, n_cols) or not dy_parts.is_contiguous():
        raise ValueError(f"{fn}: dy_parts must be contiguous float32 [S, {n_rows}, {n_cols}]")
    if not 1 <= dy_parts.shape[0] <= 64:
        raise ValueError(f"{fn}: 1 to 64 partials, got {dy_parts.shape[0]}")
    wdt = _dtype_code(fn, weight.dtype)
    w = weight.contiguous()
    rs = rstd.contiguous()
    if rs.dtype != torch.float32 or rs.numel() != n_rows:
        raise ValueError(f"{fn}: rstd must be float32 with {n_rows} entries")
    dx = torch.empty_like(h_2d)
    dres_ptr = None
    if dresidual is not None:
        dres_2d = dresidual.contiguous().view(-1, n_cols)
        if dres_2d.dtype != h_2d.dtype or dres_2d.shape != h_2d.shape:
            raise ValueError(f"{fn}: dresidual must match h in shape and dtype")
        dres_ptr = dres_2d.data_ptr()
    n_parts = dy_parts.shape[0]
    _launch("rmsnorm_bwd", (4 * n_parts + (3 if dres_ptr is not None else 2)) * n_rows * n_cols
            + w.numel() * w.element_size() + 4 * n_rows, 0, "rus_rmsnorm_bwd_parts",
            dy_parts.data_ptr(), n_parts, h_2d.data_ptr(), w.data_ptr(), wdt, rs.data_ptr(),
            dres_ptr, dx.data_ptr(), n_rows, n_cols, h_2d.stride(0), _stream(h_2d))
    return dx.view(h.shape)


# ---------------------------------------------------------------------------------------------
# LoRA-delta + NeoX RoPE (reference: kernels.py:206-348, launchers kernels.py:717-798)
# ---------------------------------------------------------------------------------------------


def _rows(fn: str, t: torch.Tensor, width: int, name: str) -> torch.Tensor:
    if t.dim() != 2 or t.shape[1] < width:
        raise ValueError(f"{fn}: {name} must be 2-D with at least {width} columns, got {tuple(t.shape)}")
    return t if t.stride(1) == 1 else t.contiguous()


def qkv_rope_fwd(
    qkv: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos_ids: torch.Tensor,
    q_lora: torch.Tensor | None = None,
    v_lora: torch.Tensor | None = None,
    scale_q: float = 2.0,
    scale_v: float = 2.0,
    h_q: int = 12,
    h_kv: int = 2,
    head_dim: int = 128,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Q = rope(q + scale_q*q_lora), K = rope(k), V = v + scale_v*v_lora; returns (q, k, v) as
    contiguous [n_tokens, heads, head_dim]. LoRA is applied only when both deltas are given."""
    fn = "qkv_rope_fwd"
    _require_device(fn, qkv, cos, sin, pos_ids, q_lora, v_lora)
    dt = _dtype_code(fn, qkv.dtype)
    n_tokens = qkv.shape[0]
    q_dim, kv_dim = h_q * head_dim, h_kv * head_dim
    qkv = _rows(fn, qkv, q_dim + 2 * kv_dim, "qkv")
    cos = _rows(fn, cos, head_dim, "cos")
    sin = _rows(fn, sin, head_dim, "sin")
    if cos.dtype != qkv.dtype or sin.dtype != qkv.dtype or sin.stride(0) != cos.stride(0):
        raise ValueError(f"{fn}: cos/sin must share qkv's dtype and a row stride")
    if sin.shape[0] != cos.shape[0]:
        raise ValueError(f"{fn}: cos and sin tables differ in length")
    pos = pos_ids.reshape(-1)
    if pos.dtype != torch.int64 or pos.numel() != n_tokens:
        raise ValueError(f"{fn}: pos_ids must be int64 with {n_tokens} entries")
    pos = pos.contiguous()
    has_lora = q_lora is not None and v_lora is not None
    ql = vl = None
    if has_lora:
        ql = _rows(fn, q_lora, q_dim, "q_lora")
        vl = _rows(fn, v_lora, kv_dim, "v_lora")
        if ql.dtype != qkv.dtype or vl.dtype != qkv.dtype:
            raise ValueError(f"{fn}: LoRA deltas must share qkv's dtype")
        if ql.shape[0] != n_tokens or vl.shape[0] != n_tokens:
            raise ValueError(f"{fn}: LoRA deltas must have {n_tokens} rows")
    q_out = torch.empty((n_tokens, h_q, head_dim), dtype=qkv.dtype, device=qkv.device)
    k_out = torch.empty((n_tokens, h_kv, head_dim), dtype=qkv.dtype, device=qkv.device)
    v_out = torch.empty((n_tokens, h_kv, head_dim), dtype=qkv.dtype, device=qkv.device)
    es = qkv.element_size()
    width = q_dim + 2 * kv_dim
    _launch(
        "rope_fwd", n_tokens * (es * (2 * width + (q_dim + kv_dim if has_lora else 0) + 2 * head_dim) + 8),
        0, "rus_qkv_lora_rope_fwd",
        qkv.data_ptr(), _ptr(ql), _ptr(vl), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
        q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), n_tokens, qkv.stride(0),
        ql.stride(0) if has_lora else 0, vl.stride(0) if has_lora else 0, cos.stride(0),
        cos.shape[0], float(scale_q), float(scale_v), h_q, h_kv, head_dim, None, dt, _stream(qkv),
    )
    return q_out, k_out, v_out


def _rope_bwd(fn, dq_rot, dk_rot, dv_out, cos, sin, pos_ids, h_q, h_kv, head_dim, scale_q,
              scale_v, with_lora, mid=None, parts=False):
    _require_device(fn, dq_rot, dk_rot, dv_out, cos, sin, pos_ids)
    dt = _dtype_code(fn, dq_rot.dtype)
    n_tokens = dq_rot.shape[0]
    q_dim, kv_dim = h_q * head_dim, h_kv * head_dim
    dq_c = dq_rot.contiguous()
    dk_c = dk_rot.contiguous()
    dv_c = dv_out.contiguous()
    checks = [("dq_rot", dq_c, q_dim, dq_c.dtype)]
    if parts:  # per-query-head fp32 partials [h_q, n_tokens, head_dim]
        checks += [("dk_part", dk_c, q_dim, torch.float32), ("dv_part", dv_c, q_dim, torch.float32)]
    else:
        checks += [("dk_rot", dk_c, kv_dim, dq_c.dtype), ("dv_out", dv_c, kv_dim, dq_c.dtype)]
    for name, t, width, dtype in checks:
        if t.numel() != n_tokens * width or t.dtype != dtype:
            raise ValueError(f"{fn}: {name} must hold [{n_tokens}, {width}] of {dtype}")
    cos = _rows(fn, cos, head_dim, "cos")
    sin = _rows(fn, sin, head_dim, "sin")
    if cos.dtype != dq_c.dtype or sin.dtype != dq_c.dtype or sin.stride(0) != cos.stride(0):
        raise ValueError(f"{fn}: cos/sin must share the gradient dtype and a row stride")
    pos = pos_ids.reshape(-1).contiguous()
    if pos.dtype != torch.int64 or pos.numel() != n_tokens:
        raise ValueError(f"{fn}: pos_ids must be int64 with {n_tokens} entries")
    dqkv = torch.empty((n_tokens, q_dim + 2 * kv_dim), dtype=dq_c.dtype, device=dq_c.device)
    dql = dvl = None
    if with_lora:
        dql = torch.empty((n_tokens, q_dim), dtype=dq_c.dtype, device=dq_c.device)
        dvl = torch.empty((n_tokens, kv_dim), dtype=dq_c.dtype, device=dq_c.device)
    es = dq_c.element_size()
    width = q_dim + 2 * kv_dim
    if mid is not None:
        bt_q, bt_v = mid
        r = bt_q.shape[0]
        dmq = torch.empty((n_tokens, r), dtype=dq_c.dtype, device=dq_c.device)
        dmv = torch.empty((n_tokens, r), dtype=dq_c.dtype, device=dq_c.device)
        extra = n_tokens * (8 * q_dim - 4 * kv_dim) if parts else 0  # fp32 partials read
        _launch(
            "rope_bwd", n_tokens * (es * (2 * width + 2 * head_dim + q_dim + kv_dim + 2 * r) + 8)
            + es * r * (q_dim + kv_dim) + extra, 2 * n_tokens * r * (q_dim + kv_dim),
            "rus_qkv_rope_bwd_mid_parts" if parts else "rus_qkv_rope_bwd_mid",
            dq_c.data_ptr(), dk_c.data_ptr(), dv_c.data_ptr(),
            cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), dqkv.data_ptr(), dql.data_ptr(),
            dvl.data_ptr(), bt_q.data_ptr(), bt_v.data_ptr(), r, dmq.data_ptr(), dmv.data_ptr(),
            n_tokens, dqkv.stride(0), cos.stride(0), cos.shape[0], float(scale_q),
            float(scale_v), h_q, h_kv, head_dim, None, _stream(dq_c))
        return dqkv, dql, dvl, dmq, dmv
    _launch(
        "rope_bwd", n_tokens * (es * (2 * width + 2 * head_dim + (q_dim + kv_dim if with_lora else 0)) + 8),
        0, "rus_qkv_rope_bwd",
        dq_c.data_ptr(), dk_c.data_ptr(), dv_c.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        pos.data_ptr(), dqkv.data_ptr(), _ptr(dql), _ptr(dvl), n_tokens, dqkv.stride(0),
        cos.stride(0), cos.shape[0], float(scale_q), float(scale_v), h_q, h_kv, head_dim, None,
        dt, _stream(dq_c),
    )
    return dqkv, dql, dvl


def rope_bwd_mid_supported(h_q: int, h_kv: int, head_dim: int, r: int) -> bool:
    """Whether ``qkv_rope_bwd_lora_mid`` covers this head layout and rank: rank 16, and a
    token's (h_q + 2 h_kv) * head_dim / 16 thread slots divide 256 with each head kind's slots a
    multiple of 16 (so one block holds whole tokens and every 16-lane group one head kind)."""
    if r != 16 or head_dim % 16:
        return False
    per_head = head_dim // 16
    slots = (h_q + 2 * h_kv) * per_head
    return 256 % slots == 0 and slots % 16 == 0 and (h_q * per_head) % 16 == 0 and \
        (h_kv * per_head) % 16 == 0


def qkv_rope_bwd_lora_mid(dq_rot, dk_rot, dv_out, cos, sin, pos_ids, scale_q: float,
                          scale_v: float, bt_q: torch.Tensor, bt_v: torch.Tensor, h_q: int = 12,
                          h_kv: int = 2, head_dim: int = 128):
    """``qkv_rope_bwd_lora`` that also returns the LoRA products d_mid_q = fp16(dq_lora B_q) and
    d_mid_v = fp16(dv_lora B_v) [n_tokens, 16] from the same launch (solution/ops.py:975-992,
    d_mid = dq @ B). bt_q / bt_v are B^T [16, h * head_dim]. fp16 only. Returns
    (dqkv, dq_lora, dv_lora, d_mid_q, d_mid_v)."""
    fn = "qkv_rope_bwd_lora_mid"
    _require_device(fn, dq_rot, dk_rot, dv_out, cos, sin, pos_ids, bt_q, bt_v)
    if dq_rot.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 gradients only")
    r = bt_q.shape[0]
    if not rope_bwd_mid_supported(h_q, h_kv, head_dim, r):
        raise ValueError(f"{fn}: unsupported layout h_q={h_q} h_kv={h_kv} head_dim={head_dim} "
                         f"rank={r}")
    _lora_operand(fn, bt_q, (r, h_q * head_dim), "bt_q")
    _lora_operand(fn, bt_v, (r, h_kv * head_dim), "bt_v")
    return _rope_bwd(fn, dq_rot, dk_rot, dv_out, cos, sin, pos_ids, h_q, h_kv, head_dim, scale_q,
                     scale_v, True, mid=(bt_q, bt_v))


def qkv_rope_bwd_lora_mid_parts(dq_rot, dk_part, dv_part, cos, sin, pos_ids, scale_q: float,
                                scale_v: float, bt_q: torch.Tensor, bt_v: torch.Tensor,
                                h_q: int = 12, h_kv: int = 2, head_dim: int = 128):
    """``qkv_rope_bwd_lora_mid`` fed by ``attn_varlen_bwd_parts``: dK and dV are the fp32
    per-query-head partials [h_q, N, head_dim], summed over each KV group in head order and
    rounded once inside the launch (the same values as the attention's own group sum)."""
    fn = "qkv_rope_bwd_lora_mid_parts"
    _require_device(fn, dq_rot, dk_part, dv_part, cos, sin, pos_ids, bt_q, bt_v)
    if dq_rot.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 gradients only")
    r = bt_q.shape[0]
    if not rope_bwd_mid_supported(h_q, h_kv, head_dim, r) or h_q // h_kv > 8:
        raise ValueError(f"{fn}: unsupported layout h_q={h_q} h_kv={h_kv} head_dim={head_dim} "
                         f"rank={r}")
    _lora_operand(fn, bt_q, (r, h_q * head_dim), "bt_q")
    _lora_operand(fn, bt_v, (r, h_kv * head_dim), "bt_v")
    return _rope_bwd(fn, dq_rot, dk_part, dv_part, cos, sin, pos_ids, h_q, h_kv, head_dim,
                     scale_q, scale_v, True, mid=(bt_q, bt_v), parts=True)


def qkv_rope_bwd(
    dq_rot: torch.Tensor,
    dk_rot: torch.Tensor,
    dv_out: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos_ids: torch.Tensor,
    h_q: int = 12,
    h_kv: int = 2,
    head_dim: int = 128,
) -> torch.Tensor:
    """Adjoint RoPE on dQ/dK, copy of dV, packed into dqkv [n_tokens, (h_q + 2 h_kv) * head_dim]."""
    dqkv, _, _ = _rope_bwd("qkv_rope_bwd", dq_rot, dk_rot, dv_out, cos, sin, pos_ids, h_q, h_kv,
                           head_dim, 1.0, 1.0, False)
    return dqkv


def qkv_rope_bwd_lora(
    dq_rot: torch.Tensor,
    dk_rot: torch.Tensor,
    dv_out: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    pos_ids: torch.Tensor,
    scale_q: float,
    scale_v: float,
    h_q: int = 12,
    h_kv: int = 2,
    head_dim: int = 128,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``qkv_rope_bwd`` that also returns the LoRA-delta gradients dq_lora = T(dQ*scale_q) and
    dv_lora = T(dV*scale_v) from the same launch (the reference computes them with two torch
    elementwise ops, ops.py:144-147 and ops.py:972-973)."""
    return _rope_bwd("qkv_rope_bwd_lora", dq_rot, dk_rot, dv_out, cos, sin, pos_ids, h_q, h_kv,
                     head_dim, scale_q, scale_v, True)


# ---------------------------------------------------------------------------------------------
# SwiGLU (reference: kernels.py:355-446, launchers kernels.py:801-912)
# ---------------------------------------------------------------------------------------------


def mlp_glu_fwd(gate_or_gu: torch.Tensor, up: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up over a fused [gate | up] tensor (up=None) or separate gate and up."""
    fn = "mlp_glu_fwd"
    _require_device(fn, gate_or_gu, up)
    dt = _dtype_code(fn, gate_or_gu.dtype)
    if up is None:
        orig_shape = gate_or_gu.shape
        if orig_shape[-1] % 2:
            raise ValueError(f"{fn}: fused [gate|up] width {orig_shape[-1]} must be even")
        n_cols = orig_shape[-1] // 2
        gu_2d = gate_or_gu.contiguous().view(-1, 2 * n_cols)
        n_rows = gu_2d.shape[0]
        out_2d = torch.empty((n_rows, n_cols), dtype=gate_or_gu.dtype, device=gate_or_gu.device)
        base = gu_2d.data_ptr()
        _launch("swiglu_fwd", 3 * n_rows * n_cols * gu_2d.element_size(), 0,
                "rus_swiglu_fwd", base, base + n_cols * gu_2d.element_size(), out_2d.data_ptr(),
                  n_rows, n_cols, gu_2d.stride(0), gu_2d.stride(0), out_2d.stride(0), dt,
                  _stream(gu_2d))
        return out_2d.view(*orig_shape[:-1], n_cols)
    orig_shape = gate_or_gu.shape
    if up.shape != orig_shape or up.dtype != gate_or_gu.dtype:
        raise ValueError(f"{fn}: gate and up must match in shape and dtype")
    n_cols = orig_shape[-1]
    gate_2d = gate_or_gu.contiguous().view(-1, n_cols)
    up_2d = up.contiguous().view(-1, n_cols)
    n_rows = gate_2d.shape[0]
    out_2d = torch.empty((n_rows, n_cols), dtype=gate_or_gu.dtype, device=gate_or_gu.device)
    _launch("swiglu_fwd", 3 * n_rows * n_cols * gate_2d.element_size(), 0,
            "rus_swiglu_fwd", gate_2d.data_ptr(), up_2d.data_ptr(), out_2d.data_ptr(), n_rows,
              n_cols, gate_2d.stride(0), up_2d.stride(0), out_2d.stride(0), dt, _stream(gate_2d))
    return out_2d.view(orig_shape)


def mlp_glu_bwd(
    dout: torch.Tensor,
    gate_or_gu: torch.Tensor,
    up: torch.Tensor | None = None,
    dgu_out: torch.Tensor | None = None,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """SwiGLU backward. Fused (up=None): writes [d_gate | d_up] into ``dgu_out``, or in place over
    ``gate_or_gu`` when ``dgu_out`` is None, and returns it as [rows, 2*n_cols]. Separate: returns
    (d_gate, d_up) as new tensors."""
    fn = "mlp_glu_bwd"
    _require_device(fn, dout, gate_or_gu, up, dgu_out)
    dt = _dtype_code(fn, gate_or_gu.dtype)
    if dout.dtype != gate_or_gu.dtype:
        raise ValueError(f"{fn}: dout dtype {dout.dtype} != activations {gate_or_gu.dtype}")
    if up is None:
        n_cols = dout.shape[-1]
        dout_2d = dout.contiguous().view(-1, n_cols)
        gu_2d = gate_or_gu.view(-1, 2 * n_cols)  # in place needs the caller's own storage
        n_rows = gu_2d.shape[0]
        if dout_2d.shape[0] != n_rows:
            raise ValueError(f"{fn}: dout has {dout_2d.shape[0]} rows, [gate|up] has {n_rows}")
        dgu_2d = gu_2d if dgu_out is None else dgu_out.view(-1, 2 * n_cols)
        if dgu_2d.dtype != gu_2d.dtype or dgu_2d.shape != gu_2d.shape:
            raise ValueError(f"{fn}: dgu_out must match [gate|up] in shape and dtype")
        es = gu_2d.element_size()
        g, d = gu_2d.data_ptr(), dgu_2d.data_ptr()
        _launch("swiglu_bwd", 5 * n_rows * n_cols * es, 0,
                "rus_swiglu_bwd", dout_2d.data_ptr(), g, g + n_cols * es, d, d + n_cols * es,
                  n_rows, n_cols, dout_2d.stride(0), gu_2d.stride(0), gu_2d.stride(0),
                  dgu_2d.stride(0), dgu_2d.stride(0), dt, _stream(dout_2d))
        return dgu_2d
    orig_shape = gate_or_gu.shape
    n_cols = orig_shape[-1]
    dout_2d = dout.contiguous().view(-1, n_cols)
    gate_2d = gate_or_gu.contiguous().view(-1, n_cols)
    up_2d = up.contiguous().view(-1, n_cols)
    n_rows = gate_2d.shape[0]
    if up_2d.shape != gate_2d.shape or dout_2d.shape != gate_2d.shape:
        raise ValueError(f"{fn}: dout, gate and up must match in shape")
    dg_2d = torch.empty_like(dout_2d)
    du_2d = torch.empty_like(dout_2d)
    _launch("swiglu_bwd", 5 * n_rows * n_cols * gate_2d.element_size(), 0,
            "rus_swiglu_bwd", dout_2d.data_ptr(), gate_2d.data_ptr(), up_2d.data_ptr(),
              dg_2d.data_ptr(), du_2d.data_ptr(), n_rows, n_cols, dout_2d.stride(0),
              gate_2d.stride(0), up_2d.stride(0), dg_2d.stride(0), du_2d.stride(0), dt,
              _stream(dout_2d))
    return dg_2d.view(orig_shape), du_2d.view(orig_shape)


# ---------------------------------------------------------------------------------------------
# LoRA-input dropout with a counter-based mask (reference: ops.py:775-777, 882-886, 986-992)
# ---------------------------------------------------------------------------------------------


def _drop_rows(fn: str, t: torch.Tensor, n_cols: int, name: str) -> torch.Tensor:
    t2 = t.view(-1, n_cols) if t.is_contiguous() else t
    if t2.dim() != 2 or t2.shape[1] != n_cols or t2.stride(1) != 1:
        raise ValueError(f"{fn}: {name} must be [rows, {n_cols}] with unit column stride")
    return t2


def lora_dropout_fwd(x: torch.Tensor, seed: torch.Tensor, stream_a: int, stream_b: int,
                     p_a: float, p_b: float, out_a: torch.Tensor | None = None,
                     out_b: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(dropout(x; stream_a, p_a), dropout(x; stream_b, p_b)) in one pass. ``seed`` is a one-element
    int64 device tensor read by the kernel (so a captured graph sees its current value)."""
    fn = "lora_dropout_fwd"
    _require_device(fn, x, seed, out_a, out_b)
    dt = _dtype_code(fn, x.dtype)
    if seed.dtype != torch.int64 or seed.numel() != 1:
        raise ValueError(f"{fn}: seed must be one int64 element")
    n_cols = x.shape[-1]
    x2 = _drop_rows(fn, x, n_cols, "x")
    shape = (x2.shape[0], n_cols)
    oa = torch.empty(shape, dtype=x.dtype, device=x.device) if out_a is None else _drop_rows(fn, out_a, n_cols, "out_a")
    ob = torch.empty(shape, dtype=x.dtype, device=x.device) if out_b is None else _drop_rows(fn, out_b, n_cols, "out_b")
    for o in (oa, ob):
        if o.shape[0] != shape[0] or o.dtype != x.dtype:
            raise ValueError(f"{fn}: outputs must be {shape} {x.dtype}")
    n = shape[0] * n_cols
    _launch("lora_dropout_fwd", 3 * n * x.element_size(), 0, "rus_lora_dropout_fwd",
            x2.data_ptr(), oa.data_ptr(), ob.data_ptr(), shape[0], n_cols, x2.stride(0),
            oa.stride(0), ob.stride(0), seed.data_ptr(), int(stream_a), int(stream_b), float(p_a),
            float(p_b), dt, _stream(x2))
    return oa.view(x.shape), ob.view(x.shape)


def lora_dropout_bwd_add(acc: torch.Tensor, grad_a: torch.Tensor, grad_b: torch.Tensor,
                         seed: torch.Tensor, stream_a: int, stream_b: int, p_a: float,
                         p_b: float) -> torch.Tensor:
    """acc += dropout(grad_a) then += dropout(grad_b), in place, with the forward's masks."""
    fn = "lora_dropout_bwd_add"
    _require_device(fn, acc, grad_a, grad_b, seed)
    dt = _dtype_code(fn, acc.dtype)
    if seed.dtype != torch.int64 or seed.numel() != 1:
        raise ValueError(f"{fn}: seed must be one int64 element")
    n_cols = acc.shape[-1]
    a2 = _drop_rows(fn, acc, n_cols, "acc")
    ga = _drop_rows(fn, grad_a, n_cols, "grad_a")
    gb = _drop_rows(fn, grad_b, n_cols, "grad_b")
    if not (ga.shape == gb.shape == a2.shape) or not (ga.dtype == gb.dtype == acc.dtype):
        raise ValueError(f"{fn}: acc, grad_a and grad_b must match in shape and dtype")
    n = a2.shape[0] * n_cols
    _launch("lora_dropout_bwd", 4 * n * acc.element_size(), 0, "rus_lora_dropout_bwd_add",
            a2.data_ptr(), ga.data_ptr(), gb.data_ptr(), a2.shape[0], n_cols, a2.stride(0),
            ga.stride(0), gb.stride(0), seed.data_ptr(), int(stream_a), int(stream_b), float(p_a),
            float(p_b), dt, _stream(a2))
    return acc


# ---------------------------------------------------------------------------------------------
# Fused rank-r LoRA branches (reference: ops.py:775-778, 882-888, 975-992)
# ---------------------------------------------------------------------------------------------

LORA_RANKS = (4, 8, 16, 32)


def _lora_operand(fn, t, shape, name):
    if t.dtype != torch.float16 or not t.is_contiguous() or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{fn}: {name} must be contiguous fp16 {tuple(shape)}, got "
                         f"{t.dtype} {tuple(t.shape)}")
    return t


def dropout_keep_bits(seed: torch.Tensor, stream0: int, n_streams: int, n_rows: int, n_cols: int,
                      p_even: float, p_odd: float) -> torch.Tensor:
    """Packed keep bits of the LoRA dropout masks of streams stream0 .. stream0 + n_streams - 1
    (the masks of ``lora_dropout_fwd``): int32 [n_streams, n_rows, ceil(n_cols / 32)], bit i of
    word w of row t set when element (t, 32 w + i) is kept; even streams use p_even, odd p_odd.
    One launch for all layers of a step (streams 2l / 2l + 1: q / v of layer l)."""
    fn = "dropout_keep_bits"
    _require_device(fn, seed)
    if seed.dtype != torch.int64 or seed.numel() != 1:
        raise ValueError(f"{fn}: seed must be one int64 element")
    words = (n_cols + 31) // 32
    out = torch.empty((n_streams, n_rows, words), dtype=torch.int32, device=seed.device)
    _launch("dropout_bits", out.numel() * 4, 0, "rus_dropout_keep_bits", seed.data_ptr(),
            int(stream0), int(n_streams), int(n_rows), int(n_cols), float(p_even), float(p_odd),
            out.data_ptr(), _stream(seed))
    return out


def _bits(fn, bits, n, d, name):
    """Device pointer of one branch's keep bits [n, ceil(d / 32)] (None: no dropout)."""
    if bits is None:
        return None
    _require_device(fn, bits)
    if bits.dtype != torch.int32 or tuple(bits.shape) != (n, (d + 31) // 32) or \
            not bits.is_contiguous():
        raise ValueError(f"{fn}: {name} must be contiguous int32 [{n}, {(d + 31) // 32}]")
    return bits.data_ptr()


LORA_DOWN, LORA_BWD_X, LORA_BWD_W = 0, 1, 2  # RUS_LORA_* of include/rus_amd.h
LORA_MAX_COUNTERS = 65536  # arrival counters per buffer (the library's bound)
_lora_counters: dict[tuple[int, int, int], torch.Tensor] = {}


def lora_workspace_size(which: int, n: int, d: int, d_q: int, d_v: int, r: int) -> tuple[int, int]:
    """(fp32 workspace elements, arrival counters) that LoRA entry point ``which``
    (LORA_DOWN / LORA_BWD_X / LORA_BWD_W) needs for these sizes."""
    floats, counters = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("rus_lora_workspace_size", int(which), int(n), int(d), int(d_q), int(d_v), int(r),
              ctypes.byref(floats), ctypes.byref(counters))
    return floats.value, counters.value


def _lora_scratch(which: int, n: int, d: int, d_q: int, d_v: int, r: int, dev: torch.device):
    """Workspace (stream-ordered, from torch's caching allocator) and the arrival counters of one
    LoRA launch. Counters start at zero and every launch leaves them zero, so one buffer serves
    every launch of an entry point on a stream (launches on one stream never overlap); buffers
    are kept for the life of the process (captured graphs hold their addresses)."""
    floats, counters = lora_workspace_size(which, n, d, d_q, d_v, r)
    ws = torch.empty(max(floats, 4), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), which, stream)
    cnt = _lora_counters.get(key)
    if cnt is None:
        cnt = torch.zeros(LORA_MAX_COUNTERS, dtype=torch.int32, device=dev)
        _lora_counters[key] = cnt
    return ws, cnt


def lora_down_fwd(x: torch.Tensor, a_q: torch.Tensor, a_v: torch.Tensor,
                  bits_q: torch.Tensor | None = None, bits_v: torch.Tensor | None = None,
                  p_q: float = 0.0, p_v: float = 0.0, out=None):
    """(mid_q, mid_v) = (drop_q(x) A_q^T, drop_v(x) A_v^T) in fp16, one launch; drop_* applies
    the keep bits of ``dropout_keep_bits`` with scale 1 / (1 - p) (None: no dropout). ``out``:
    preallocated (mid_q, mid_v) [n, r] fp16 (e.g. allocated on another stream than the one
    the kernel runs on)."""
    fn = "lora_down_fwd"
    _require_device(fn, x, a_q, a_v)
    r, d = a_q.shape
    if r not in LORA_RANKS:
        raise ValueError(f"{fn}: rank {r} not in {LORA_RANKS}")
    x2 = _rows(fn, x, d, "x")
    if x2.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 activations only")
    _lora_operand(fn, a_q, (r, d), "a_q")
    _lora_operand(fn, a_v, (r, d), "a_v")
    n = x2.shape[0]
    bq = _bits(fn, bits_q, n, d, "bits_q")
    bv = _bits(fn, bits_v, n, d, "bits_v")
    dev = x.device
    if out is None:
        mid_q = torch.empty((n, r), dtype=torch.float16, device=dev)
        mid_v = torch.empty((n, r), dtype=torch.float16, device=dev)
    else:
        mid_q, mid_v = out
        _lora_operand(fn, mid_q, (n, r), "mid_q")
        _lora_operand(fn, mid_v, (n, r), "mid_v")
    ws, cnt = _lora_scratch(LORA_DOWN, n, d, 16, 16, r, dev)
    _launch("lora_down", n * d * 2 + 4 * r * d + 4 * n * r + n * d // 4, 4 * n * d * r,
            "rus_lora_down_fwd", x2.data_ptr(), n, d, x2.stride(0), a_q.data_ptr(),
            a_v.data_ptr(), r, mid_q.data_ptr(), mid_v.data_ptr(), bq, bv, float(p_q), float(p_v),
            ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), _stream(x2))
    return mid_q, mid_v


LORA_ROWS_RANKS = (4, 8, 16)  # ranks of rus_lora_down_rows


def _lora_rows(x: torch.Tensor, a_q, a_v, bits_q, bits_v, p_q, p_v, out=None):
    """(mid_q, mid_v, rus_lora_rows, tensors it points at) of lora_down_rows."""
    fn = "lora_down_rows"
    _require_device(fn, x, a_q, a_v, bits_q, bits_v)
    r, d = a_q.shape
    if r not in LORA_ROWS_RANKS or d % 64:
        raise ValueError(f"{fn}: rank {r} not in {LORA_ROWS_RANKS} or d = {d} not a multiple "
                         f"of 64")
    x2 = _rows(fn, x, d, "x")
    if x2.dtype != torch.float16:
        raise ValueError(f"{fn}: fp16 activations only")
    _lora_operand(fn, a_q, (r, d), "a_q")
    _lora_operand(fn, a_v, (r, d), "a_v")
    n = x2.shape[0]
    bq = _bits(fn, bits_q, n, d, "bits_q")
    bv = _bits(fn, bits_v, n, d, "bits_v")
    if out is None:
        mid_q = torch.empty((n, r), dtype=torch.float16, device=x.device)
        mid_v = torch.empty((n, r), dtype=torch.float16, device=x.device)
    else:
        mid_q, mid_v = out
        _lora_operand(fn, mid_q, (n, r), "mid_q")
        _lora_operand(fn, mid_v, (n, r), "mid_v")
    a = _lib.LoraRows()
    a.x, a.stride_x, a.n_tokens, a.d, a.r = x2.data_ptr(), x2.stride(0), n, d, r
    a.a_q, a.a_v, a.bits_q, a.bits_v = a_q.data_ptr(), a_v.data_ptr(), bq, bv
    a.p_q, a.p_v = float(p_q), float(p_v)
    a.mid_q, a.mid_v = mid_q.data_ptr(), mid_v.data_ptr()
    return mid_q, mid_v, a, (x2, a_q, a_v, bits_q, bits_v, mid_q, mid_v)


def _down_rows_bytes(a) -> int:
    n, d, r = a.n_tokens, a.d, a.r
    return n * d * 2 + 4 * r * d + 4 * n * r + (n * d // 4 if a.bits_q else 0)


def _launch_down_rows(a, like: torch.Tensor) -> None:
    _launch("lora_down", _down_rows_bytes(a), 4 * a.n_tokens * a.d * a.r, "rus_lora_down_rows",
            ctypes.byref(a), _stream(like))


def lora_down_rows(x: torch.Tensor, a_q: torch.Tensor, a_v: torch.Tensor,
                   bits_q: torch.Tensor | None = None, bits_v: torch.Tensor | None = None,
                   p_q: float = 0.0, p_v: float = 0.0, out=None):
    """(mid_q, mid_v) = (drop_q(x) A_q^T, drop_v(x) A_v^T) in fp16 as ``lora_down_fwd``, by
    blocks of four token rows without workspace (ranks 4, 8, 16, d a multiple of 64): the
    arithmetic of the LoRA-down a dequant launch carries beside the input norm
    (``DeferredNorm.carry_lora_down``), so both give the same bits."""
    mid_q, mid_v, a, keep = _lora_rows(x, a_q, a_v, bits_q, bits_v, p_q, p_v, out)
    _launch_down_rows(a, keep[0])
    return mid_q, mid_v


def qkv_rope_fwd_mid(qkv: torch.Tensor, mid_q: torch.Tensor, mid_v: torch.Tensor,
                     b_q: torch.Tensor, b_v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     pos_ids: torch.Tensor, scale_q: float = 2.0, scale_v: float = 2.0,
                     h_q: int = 12, h_kv: int = 2, head_dim: int = 128):
    """qkv_rope_fwd with q_lora = mid_q B_q^T and v_lora = mid_v B_v^T formed in the kernel."""
    fn = "qkv_rope_fwd_mid"
    _require_device(fn, qkv, mid_q, mid_v, b_q, b_v, cos, sin, pos_ids)
    n_tokens = qkv.shape[0]
    q_dim, kv_dim = h_q * head_dim, h_kv * head_dim
    r = mid_q.shape[1]
    if qkv.dtype != torch.float16 or r not in LORA_RANKS:
        raise ValueError(f"{fn}: fp16 and rank in {LORA_RANKS} only")
    qkv = _rows(fn, qkv, q_dim + 2 * kv_dim, "qkv")
    cos = _rows(fn, cos, head_dim, "cos")
    sin = _rows(fn, sin, head_dim, "sin")
    if cos.dtype != qkv.dtype or sin.dtype != qkv.dtype or sin.stride(0) != cos.stride(0):
        raise ValueError(f"{fn}: cos/sin must share qkv's dtype and a row stride")
    for t, shp, nm in ((mid_q, (n_tokens, r), "mid_q"), (mid_v, (n_tokens, r), "mid_v"),
                       (b_q, (q_dim, r), "b_q"), (b_v, (kv_dim, r), "b_v")):
        _lora_operand(fn, t, shp, nm)
    pos = pos_ids.reshape(-1)
    if pos.dtype != torch.int64 or pos.numel() != n_tokens:
        raise ValueError(f"{fn}: pos_ids must be int64 with {n_tokens} entries")
    pos = pos.contiguous()
    q_out = torch.empty((n_tokens, h_q, head_dim), dtype=qkv.dtype, device=qkv.device)
    k_out = torch.empty((n_tokens, h_kv, head_dim), dtype=qkv.dtype, device=qkv.device)
    v_out = torch.empty((n_tokens, h_kv, head_dim), dtype=qkv.dtype, device=qkv.device)
    width = q_dim + 2 * kv_dim
    _launch("rope_fwd", n_tokens * (2 * (2 * width + 2 * head_dim + 2 * r) + 8), 0,
            "rus_qkv_lora_rope_fwd_mid", qkv.data_ptr(), mid_q.data_ptr(), mid_v.data_ptr(),
            b_q.data_ptr(), b_v.data_ptr(), r, cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
            q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), n_tokens, qkv.stride(0),
            cos.stride(0), cos.shape[0], float(scale_q), float(scale_v), h_q, h_kv, head_dim,
            None, _stream(qkv))
    return q_out, k_out, v_out


def lora_bwd_x(dq_lora: torch.Tensor, dv_lora: torch.Tensor, a_t_q: torch.Tensor,
               a_t_v: torch.Tensor, b_t_q: torch.Tensor, b_t_v: torch.Tensor, dx: torch.Tensor,
               bits_q: torch.Tensor | None = None, bits_v: torch.Tensor | None = None,
               p_q: float = 0.0, p_v: float = 0.0):
    """d_mid = dq B per branch; dx += drop_q(d_mid_q A_q), then += drop_v(d_mid_v A_v), in
    place, with the forward's keep bits. The factors come rank-major: a_t = A^T [d, r],
    b_t = B^T [r, d_q]. Returns (d_mid_q, d_mid_v)."""
    fn = "lora_bwd_x"
    _require_device(fn, dq_lora, dv_lora, a_t_q, a_t_v, b_t_q, b_t_v, dx)
    d, r = a_t_q.shape
    if r not in LORA_RANKS:
        raise ValueError(f"{fn}: rank {r} not in {LORA_RANKS}")
    n = dq_lora.shape[0]
    d_q, d_v = dq_lora.shape[1], dv_lora.shape[1]
    for t, shp, nm in ((dq_lora, (n, d_q), "dq_lora"), (dv_lora, (n, d_v), "dv_lora"),
                       (a_t_q, (d, r), "a_t_q"), (a_t_v, (d, r), "a_t_v"),
                       (b_t_q, (r, d_q), "b_t_q"), (b_t_v, (r, d_v), "b_t_v")):
        _lora_operand(fn, t, shp, nm)
    dx2 = _rows(fn, dx, d, "dx")
    if dx2.dtype != torch.float16 or dx2.shape[0] != n:
        raise ValueError(f"{fn}: dx must be fp16 [{n}, {d}]")
    bq = _bits(fn, bits_q, n, d, "bits_q")
    bv = _bits(fn, bits_v, n, d, "bits_v")
    dmq = torch.empty((n, r), dtype=torch.float16, device=dx.device)
    dmv = torch.empty((n, r), dtype=torch.float16, device=dx.device)
    ws, cnt = _lora_scratch(LORA_BWD_X, n, d, d_q, d_v, r, dx.device)
    _launch("lora_bwd_x", 2 * n * (d_q + d_v + 2 * d + 2 * r) + 4 * r * (d + d_q) + n * d // 4,
            2 * n * r * (d_q + d_v + 2 * d), "rus_lora_bwd_x", dq_lora.data_ptr(),
            dv_lora.data_ptr(), n, d_q, d_v, a_t_q.data_ptr(), a_t_v.data_ptr(),
            b_t_q.data_ptr(), b_t_v.data_ptr(), r, d, dmq.data_ptr(), dmv.data_ptr(),
            dx2.data_ptr(), dx2.stride(0), bq, bv, float(p_q), float(p_v), ws.data_ptr(),
            ws.numel(), cnt.data_ptr(), cnt.numel(), _stream(dx2))
    return dmq, dmv


def lora_bwd_w(x: torch.Tensor, dq_lora: torch.Tensor, dv_lora: torch.Tensor,
               mid_q: torch.Tensor, mid_v: torch.Tensor, d_mid_q: torch.Tensor,
               d_mid_v: torch.Tensor, g_a_q: torch.Tensor, g_b_q: torch.Tensor,
               g_a_v: torch.Tensor, g_b_v: torch.Tensor, bits_q: torch.Tensor | None = None,
               bits_v: torch.Tensor | None = None, p_q: float = 0.0, p_v: float = 0.0,
               expand=None) -> None:
    """g_a = d_mid^T drop(x) [r, d], g_b = dq^T mid [d_q, r] for both branches (the dropped
    inputs formed from x and the forward's keep bits), fp16 outputs written in place (e.g. views
    of a flat gradient buffer). With ``expand = (a_t_q, a_t_v, dx)`` the same launch also adds
    the input gradients drop_q(d_mid_q A_q), then drop_v(d_mid_v A_v), into dx in place
    (``lora_bwd_x`` without its d_mid products; a_t = A^T [d, r])."""
    fn = "lora_bwd_w" if expand is None else "lora_bwd_xw"
    _require_device(fn, x, dq_lora, dv_lora, mid_q, mid_v, d_mid_q, d_mid_v, g_a_q, g_b_q,
                    g_a_v, g_b_v)
    n, r = mid_q.shape
    d = x.shape[1]
    d_q, d_v = dq_lora.shape[1], dv_lora.shape[1]
    if r not in LORA_RANKS:
        raise ValueError(f"{fn}: rank {r} not in {LORA_RANKS}")
    x2 = _rows(fn, x, d, "x")
    if x2.dtype != torch.float16 or x2.shape[0] != n:
        raise ValueError(f"{fn}: x must be fp16 [{n}, {d}]")
    for t, shp, nm in ((dq_lora, (n, d_q), "dq_lora"), (dv_lora, (n, d_v), "dv_lora"),
                       (mid_q, (n, r), "mid_q"), (mid_v, (n, r), "mid_v"),
                       (d_mid_q, (n, r), "d_mid_q"), (d_mid_v, (n, r), "d_mid_v"),
                       (g_a_q, (r, d), "g_a_q"), (g_b_q, (d_q, r), "g_b_q"),
                       (g_a_v, (r, d), "g_a_v"), (g_b_v, (d_v, r), "g_b_v")):
        _lora_operand(fn, t, shp, nm)
    bq = _bits(fn, bits_q, n, d, "bits_q")
    bv = _bits(fn, bits_v, n, d, "bits_v")
    ws, cnt = _lora_scratch(LORA_BWD_W, n, d, d_q, d_v, r, x.device)
    args = (x2.data_ptr(), x2.stride(0), bq, bv, float(p_q), float(p_v), dq_lora.data_ptr(),
            dv_lora.data_ptr(), mid_q.data_ptr(), mid_v.data_ptr(), d_mid_q.data_ptr(),
            d_mid_v.data_ptr(), n, d, d_q, d_v, r, g_a_q.data_ptr(), g_b_q.data_ptr(),
            g_a_v.data_ptr(), g_b_v.data_ptr())
    scratch = (ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), _stream(mid_q))
    nbytes = 2 * n * (d + d_q + d_v + 4 * r) + n * d // 4
    flops = 2 * n * r * (2 * d + d_q + d_v)
    if expand is None:
        _launch("lora_bwd_w", nbytes, flops, "rus_lora_bwd_w", *args, *scratch)
        return
    a_t_q, a_t_v, dx = expand
    _require_device(fn, a_t_q, a_t_v, dx)
    _lora_operand(fn, a_t_q, (d, r), "a_t_q")
    _lora_operand(fn, a_t_v, (d, r), "a_t_v")
    dx2 = _rows(fn, dx, d, "dx")
    if dx2.data_ptr() != dx.data_ptr() or dx2.dtype != torch.float16 or dx2.shape[0] != n:
        raise ValueError(f"{fn}: dx must be fp16 [{n}, {d}] with unit column stride")
    _launch("lora_bwd_w", nbytes + 4 * n * d + 4 * r * d, flops + 4 * n * r * d,
            "rus_lora_bwd_xw", *args, a_t_q.data_ptr(), a_t_v.data_ptr(), dx2.data_ptr(),
            dx2.stride(0), *scratch)


# ---------------------------------------------------------------------------------------------
# Vocab-tiled lm_head cross-entropy on fp16 MFMA (reference: lm_head_piece_kernel /
# lm_head_finish_kernel, kernels.py:453-565, and the chunk loops of ops.py:174-349)
# ---------------------------------------------------------------------------------------------

LM_TILE = 256  # vocabulary rows per forward partial (the kernels' block tile)
LM_K = 64  # K granularity of the MFMA mainloop


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def lm_head_num_parts(vocab_size: int) -> int:
    """Partial rows the forward writes for ``vocab_size`` vocabulary rows."""
    return (vocab_size + LM_TILE - 1) // LM_TILE


_CU_COUNT: dict = {}


def cu_count(device=None) -> int:
    """Compute units of ``device`` (256 on MI355X; also the value used without a GPU)."""
    if device is None or not torch.cuda.is_available():
        return 256
    dev = torch.device(device)
    if dev.type != "cuda":
        return 256
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _CU_COUNT[idx]


def _round_fill(blocks: int, n_cu: int) -> float:
    """Share of the CU slots used by a grid of ``blocks`` one-per-CU workgroups, with the grid
    rounded up to a multiple of 8 as the GEMM launches do (whole rounds of n_cu blocks)."""
    launched = -(-blocks // 8) * 8
    return blocks / (n_cu * -(-launched // n_cu))


def lm_head_split_count(n_tok: int, d: int, n_vocab: int, n_cu: int = 256,
                        max_split: int = 64) -> int:
    """Split-K count for the hidden-gradient GEMM. One of its workgroups fills a CU (128 KiB of
    LDS, 512 registers per lane), so the grid runs in rounds of ``n_cu`` blocks: of the split
    counts the C ABI accepts (each split a multiple of 64 vocabulary columns) up to ``max_split``,
    take the one whose (token, hidden) tiles x splits fill their last round best (the share of the
    CUs used when under one round), the smallest on ties (fewer fp32 partials to write and sum)."""
    kpad = _round_up(n_vocab, LM_K)
    if kpad == 0:
        return 1
    tiles = max(1, -(-n_tok // 256) * -(-d // 256))
    best, best_key = 1, None
    for want in range(1, max(1, min(64, max_split, kpad // LM_K)) + 1):
        per = _round_up(-(-kpad // want), LM_K)
        n_split = -(-kpad // per)
        key = (_round_fill(tiles * n_split, n_cu), -n_split)
        if best_key is None or key > best_key:
            best, best_key = n_split, key
    return best


LM_CHUNK_BUDGET = 128 << 20  # bytes of fp16 logits one chunk of the single-pass head may hold


def lm_head_chunk_cols(n_tok: int, n_vocab: int, n_cu: int = 256,
                       budget: int = LM_CHUNK_BUDGET) -> int:
    """Vocabulary rows per chunk of the single-pass head: a multiple of 256 whose fp16 logits
    [n_tok, cols] fit ``budget``, chosen to minimise an estimate of the statistics GEMM time
    (whole rounds of one-per-CU 256x256 tiles, ~50 us each) plus a per-chunk cost for the three
    launches of a chunk (~15 us)."""
    tiles_v = -(-n_vocab // LM_TILE)
    if tiles_v <= 1 or n_tok <= 0:
        return max(LM_TILE, tiles_v * LM_TILE)
    tt = -(-n_tok // 256)
    cap = max(1, min(tiles_v, budget // (2 * LM_TILE * n_tok)))
    best, best_cost = 1, None
    for k in range(1, cap + 1):
        full, rest = divmod(tiles_v, k)
        rounds = full * -(-(-(-k * tt // 8) * 8) // n_cu)
        if rest:
            rounds += -(-(-(-rest * tt // 8) * 8) // n_cu)
        cost = 50.0 * rounds + 15.0 * (full + (1 if rest else 0))
        if best_cost is None or cost < best_cost or (cost == best_cost and k > best):
            best, best_cost = k, cost
    return best * LM_TILE


class LMHeadPartials:
    """Device buffers for the forward partial statistics: [n_parts, n_tok] m, s, w, idx."""

    def __init__(self, n_parts: int, n_tok: int, device):
        self.n_parts, self.n_tok = n_parts, n_tok
        self.m = torch.empty((n_parts, n_tok), dtype=torch.float32, device=device)
        self.s = torch.empty((n_parts, n_tok), dtype=torch.float32, device=device)
        self.w = torch.empty((n_parts, n_tok), dtype=torch.float32, device=device)
        self.idx = torch.empty((n_parts, n_tok), dtype=torch.int32, device=device)


def _lm_operand(fn: str, t: torch.Tensor, d: int, name: str) -> torch.Tensor:
    if t.dtype != torch.float16:
        raise TypeError(f"{fn}: {name} must be fp16, got {t.dtype}")
    if t.dim() != 2 or t.shape[1] < d:
        raise ValueError(f"{fn}: {name} must be 2-D with {d} columns")
    if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    if t.shape[0] * t.stride(0) * 2 >= 1 << 32:
        raise ValueError(f"{fn}: {name} exceeds the 4 GiB operand limit of the MFMA kernels")
    return t


def lm_head_ce_fwd_chunk(hidden: torch.Tensor, weight_rows: torch.Tensor, labels: torch.Tensor,
                         vocab_start: int, parts: LMHeadPartials, target: torch.Tensor,
                         logits_out: torch.Tensor | None = None) -> None:
    """Forward partial statistics of vocabulary rows [vocab_start, vocab_start + len(weight_rows))
    (replaces one iteration of the reference's forward chunk loop, ops.py:217-251). With
    ``logits_out`` ([n_tok, >= round_up(n, 64)] fp16) the rounded logits are kept there too, for
    ``lm_head_ce_grad_from_logits``."""
    fn = "lm_head_ce_fwd_chunk"
    _require_device(fn, hidden, weight_rows, labels, target, logits_out)
    if vocab_start % LM_TILE:
        raise ValueError(f"{fn}: vocab_start must be a multiple of {LM_TILE}")
    d = hidden.shape[1]
    h = _lm_operand(fn, hidden, d, "hidden")
    w = _lm_operand(fn, weight_rows, d, "weight")
    n_tok, n_vocab = h.shape[0], w.shape[0]
    part_base = vocab_start // LM_TILE
    if part_base + lm_head_num_parts(n_vocab) > parts.n_parts or parts.n_tok != n_tok:
        raise ValueError(f"{fn}: partial buffers too small for this chunk")
    lab = labels.reshape(-1)
    if lab.dtype != torch.int64 or lab.numel() != n_tok:
        raise ValueError(f"{fn}: labels must be int64 with {n_tok} entries")
    lab = lab.contiguous()
    nbytes = (n_tok + n_vocab) * d * 2 + 16 * n_tok * lm_head_num_parts(n_vocab)
    args = (h.data_ptr(), w.data_ptr(), lab.data_ptr(), n_tok, d, h.stride(0), w.stride(0),
            n_vocab, vocab_start, parts.m.data_ptr(), parts.s.data_ptr(), parts.w.data_ptr(),
            parts.idx.data_ptr(), part_base, n_tok, target.data_ptr())
    if logits_out is None:
        _launch("lmhead_ce_fwd", nbytes, 2.0 * n_tok * d * n_vocab, "rus_lmhead_ce_fwd", *args,
                _stream(h))
        return
    kp = _round_up(n_vocab, LM_K)
    z = logits_out
    if z.dtype != torch.float16 or z.dim() != 2 or z.shape[0] != n_tok or z.shape[1] < kp \
            or z.stride(1) != 1:
        raise ValueError(f"{fn}: logits_out must be fp16 [{n_tok}, >= {kp}] with contiguous rows")
    if z.shape[0] * z.stride(0) * 2 >= 1 << 32:
        raise ValueError(f"{fn}: logits_out exceeds the 4 GiB operand limit of the MFMA kernels")
    _launch("lmhead_ce_fwd_keep", nbytes + n_tok * kp * 2, 2.0 * n_tok * d * n_vocab,
            "rus_lmhead_ce_fwd_keep", *args, z.data_ptr(), z.stride(0), _stream(h))


def lm_head_ce_combine(parts: LMHeadPartials, target: torch.Tensor, labels: torch.Tensor):
    """(lse, nll, entropy, argmax) per token from the partials (replaces lm_head_finish_kernel,
    kernels.py:534-565)."""
    fn = "lm_head_ce_combine"
    _require_device(fn, target, labels)
    n = parts.n_tok
    dev = target.device
    lse = torch.empty(n, dtype=torch.float32, device=dev)
    nll = torch.empty(n, dtype=torch.float32, device=dev)
    ent = torch.empty(n, dtype=torch.float32, device=dev)
    amax = torch.empty(n, dtype=torch.int64, device=dev)
    lab = labels.reshape(-1).contiguous()
    _launch("lmhead_ce_combine", 16 * n * parts.n_parts + 32 * n, 0,
            "rus_lmhead_ce_combine", parts.m.data_ptr(), parts.s.data_ptr(), parts.w.data_ptr(),
              parts.idx.data_ptr(), parts.n_parts, n, target.data_ptr(), lab.data_ptr(), n,
              lse.data_ptr(), nll.data_ptr(), ent.data_ptr(), amax.data_ptr(), _stream(target))
    return lse, nll, ent, amax


def lm_head_ce_grad_logits(hidden: torch.Tensor, weight_rows: torch.Tensor, labels: torch.Tensor,
                           lse: torch.Tensor, denom: torch.Tensor, vocab_start: int,
                           out: torch.Tensor) -> torch.Tensor:
    """fp16 logit gradient of one vocabulary range into ``out`` [n_tok, >= round_up(n, 64)]
    (replaces lm_head_piece_kernel MODE 1 and its recompute GEMM, ops.py:287-319)."""
    fn = "lm_head_ce_grad_logits"
    _require_device(fn, hidden, weight_rows, labels, lse, denom, out)
    d = hidden.shape[1]
    h = _lm_operand(fn, hidden, d, "hidden")
    w = _lm_operand(fn, weight_rows, d, "weight")
    n_tok, n_vocab = h.shape[0], w.shape[0]
    if out.dtype != torch.float16 or out.shape[0] != n_tok or out.stride(1) != 1:
        raise ValueError(f"{fn}: out must be fp16 [n_tok, *] with contiguous rows")
    if denom.dtype != torch.float32 or denom.numel() != 1:
        raise ValueError(f"{fn}: denom must be a one-element float32 device tensor")
    lab = labels.reshape(-1).contiguous()
    _launch("lmhead_ce_grad_logits", (n_tok + n_vocab) * d * 2 + n_tok * _round_up(n_vocab, LM_K) * 2,
            2.0 * n_tok * d * n_vocab,
            "rus_lmhead_ce_grad_logits", h.data_ptr(), w.data_ptr(), lab.data_ptr(),
              lse.data_ptr(), denom.data_ptr(), n_tok, d, h.stride(0), w.stride(0), n_vocab,
              vocab_start, out.data_ptr(), out.stride(0), _stream(h))
    return out


def lm_head_ce_grad_from_logits(logits: torch.Tensor, labels: torch.Tensor, lse: torch.Tensor,
                                denom: torch.Tensor, n_vocab: int, vocab_start: int = 0) -> torch.Tensor:
    """Turn the fp16 logits kept by ``lm_head_ce_fwd_chunk(..., logits_out=)`` into the logit
    gradient in place, element for element the value ``lm_head_ce_grad_logits`` computes
    (replaces lm_head_piece_kernel MODE 1, kernels.py:517-531, without its recompute GEMM)."""
    fn = "lm_head_ce_grad_from_logits"
    _require_device(fn, logits, labels, lse, denom)
    n_tok = logits.shape[0]
    kp = _round_up(n_vocab, LM_K)
    if logits.dtype != torch.float16 or logits.dim() != 2 or logits.shape[1] < kp \
            or logits.stride(1) != 1:
        raise ValueError(f"{fn}: logits must be fp16 [n_tok, >= {kp}] with contiguous rows")
    if denom.dtype != torch.float32 or denom.numel() != 1:
        raise ValueError(f"{fn}: denom must be a one-element float32 device tensor")
    lab = labels.reshape(-1)
    if lab.dtype != torch.int64 or lab.numel() != n_tok or lse.numel() != n_tok:
        raise ValueError(f"{fn}: labels (int64) and lse need {n_tok} entries")
    lab = lab.contiguous()
    _launch("lmhead_ce_grad_from_logits", 2 * n_tok * kp * 2 + 12 * n_tok, 0,
            "rus_lmhead_ce_grad_from_logits", logits.data_ptr(), logits.stride(0), lab.data_ptr(),
              lse.data_ptr(), denom.data_ptr(), n_tok, n_vocab, vocab_start, _stream(logits))
    return logits


def lm_head_ce_grad_hidden(grad_logits: torch.Tensor, weight_t_cols: torch.Tensor, n_vocab: int,
                           parts: torch.Tensor, accumulate: bool) -> None:
    """parts[s] (+)= grad_logits . (W^T cols)^T split over vocabulary (replaces the fp16
    ``addmm_`` accumulation of ops.py:320 with fp32 split-K partials)."""
    fn = "lm_head_ce_grad_hidden"
    _require_device(fn, grad_logits, weight_t_cols, parts)
    n_tok = grad_logits.shape[0]
    d = weight_t_cols.shape[0]
    n_split = parts.shape[0]
    if parts.dtype != torch.float32 or tuple(parts.shape[1:]) != (n_tok, d) or not parts.is_contiguous():
        raise ValueError(f"{fn}: parts must be contiguous float32 [n_split, {n_tok}, {d}]")
    for name, t in (("grad_logits", grad_logits), ("weight_t", weight_t_cols)):
        if t.dtype != torch.float16 or t.stride(1) != 1:
            raise ValueError(f"{fn}: {name} must be fp16 with contiguous rows")
        if t.shape[0] * t.stride(0) * 2 >= 1 << 32:
            raise ValueError(f"{fn}: {name} exceeds the 4 GiB operand limit of the MFMA kernels")
    kp = _round_up(n_vocab, LM_K)
    _launch("lmhead_ce_grad_hidden", (n_tok + d) * kp * 2 + 4 * n_split * n_tok * d * (2 if accumulate else 1),
            2.0 * n_tok * d * n_vocab,
            "rus_lmhead_ce_grad_hidden", grad_logits.data_ptr(), grad_logits.stride(0),
              weight_t_cols.data_ptr(), weight_t_cols.stride(0), n_tok, d, n_vocab,
              parts.data_ptr(), n_split, 1 if accumulate else 0, _stream(grad_logits))


def lm_head_dh_reduce(parts: torch.Tensor, scale: float, out_dtype=torch.float16,
                      scale_dev: torch.Tensor | None = None,
                      _tag: str = "lmhead_dh_reduce", out: torch.Tensor | None = None) -> torch.Tensor:
    """out = out_dtype(scale * scale_dev * sum over the leading split dimension of ``parts``);
    ``scale_dev`` is an optional one-element float32 device tensor (read on the device); ``out``
    (contiguous, ``parts.shape[1:]``, 16-byte aligned) receives the result when given."""
    fn = "lm_head_dh_reduce"
    _require_device(fn, parts, scale_dev, out)
    if parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError(f"{fn}: parts must be contiguous float32")
    if scale_dev is not None and (scale_dev.dtype != torch.float32 or scale_dev.numel() != 1):
        raise ValueError(f"{fn}: scale_dev must be a one-element float32 tensor")
    if out is None:
        out = torch.empty(parts.shape[1:], dtype=out_dtype, device=parts.device)
    elif out.shape != parts.shape[1:] or not out.is_contiguous():
        raise ValueError(f"{fn}: out must be contiguous {tuple(parts.shape[1:])}")
    out_dtype = out.dtype
    _launch(_tag, parts.numel() * 4 + out.numel() * out.element_size(), 0,
            "rus_lmhead_dh_reduce", parts.data_ptr(), parts.shape[0], out.numel(), float(scale),
              _ptr(scale_dev), out.data_ptr(), _dtype_code(fn, out_dtype), _stream(parts))
    return out


def sum_splits(parts: torch.Tensor, out_dtype=torch.float16) -> torch.Tensor:
    """out_dtype(sum over the leading dimension of fp32 ``parts``): the reduce of a split-K GEMM."""
    return lm_head_dh_reduce(parts, 1.0, out_dtype, _tag="splitk_reduce")


# ---------------------------------------------------------------------------------------------
# Varlen causal GQA attention (reference: ops.py:669-696, torch SDPA per packed row)
# ---------------------------------------------------------------------------------------------

ATTN_HEAD_DIM = 128
ATTN_BLOCK = 32


def attn_max_blocks(n_tokens: int, n_rows: int) -> int:
    """Upper bound of sum_i ceil(len_i / 32) over rows that cover n_tokens tokens."""
    return -(-n_tokens // ATTN_BLOCK) + n_rows


def _attn_operands(fn, q, k, v, cu):
    _require_device(fn, q, k, v, cu)
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape or q.shape[0] != k.shape[0]:
        raise ValueError(f"{fn}: q [N, h_q, 128], k/v [N, h_kv, 128] expected, got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if q.shape[2] != ATTN_HEAD_DIM or k.shape[2] != ATTN_HEAD_DIM:
        raise ValueError(f"{fn}: head_dim must be {ATTN_HEAD_DIM}")
    if q.shape[1] % k.shape[1]:
        raise ValueError(f"{fn}: h_q={q.shape[1]} is not a multiple of h_kv={k.shape[1]}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous fp16")
    if cu.dtype != torch.int32 or cu.dim() != 1 or cu.numel() < 2 or not cu.is_contiguous():
        raise ValueError(f"{fn}: cu_seqlens must be a contiguous int32 [n_rows + 1] tensor")


def _attn_flops(lens, hq):
    # 2 products of 2 * L(L+1)/2 * 128 multiply-adds each per head (causal half).
    return 0.0 if lens is None else float(sum(2 * L * (L + 1) * ATTN_HEAD_DIM * hq for L in lens))


def attn_varlen_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                    max_blocks: int | None = None, scale: float | None = None, lens=None):
    """(out [N, h_q, 128] fp16, lse [h_q, N] fp32): causal softmax(scale q k^T) v per packed row
    [cu[i], cu[i+1]) with K/V head h // (h_q / h_kv); cu_seqlens (device int32) must cover all
    N tokens. ``lens`` (host row lengths) only feeds the timer's FLOP count."""
    fn = "attn_varlen_fwd"
    _attn_operands(fn, q, k, v, cu_seqlens)
    n, hq, d = q.shape
    n_rows = cu_seqlens.numel() - 1
    mb = attn_max_blocks(n, n_rows) if max_blocks is None else int(max_blocks)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out = torch.empty_like(q)
    lse = torch.empty((hq, n), dtype=torch.float32, device=q.device)
    nbytes = 2 * (q.numel() * 2 + k.numel() * 2) + lse.numel() * 4
    _launch("attn_fwd", nbytes, _attn_flops(lens, hq), "rus_attn_varlen_fwd", q.data_ptr(),
            k.data_ptr(), v.data_ptr(), cu_seqlens.data_ptr(), n_rows, n, mb, hq, k.shape[1], d,
            scale, out.data_ptr(), lse.data_ptr(), _stream(q))
    return out, lse


def attn_varlen_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    out: torch.Tensor, lse: torch.Tensor, cu_seqlens: torch.Tensor,
                    max_blocks: int | None = None, scale: float | None = None, lens=None):
    """(dq, dk, dv) fp16 for ``attn_varlen_fwd``'s inputs, given its (out, lse); dk / dv sum the
    query heads of each KV group in fp32 and are rounded once."""
    fn = "attn_varlen_bwd"
    _attn_operands(fn, q, k, v, cu_seqlens)
    n, hq, d = q.shape
    for name, t in (("dout", dout), ("out", out)):
        if t.shape != q.shape or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous fp16 like q")
    if lse.shape != (hq, n) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError(f"{fn}: lse must be contiguous fp32 [h_q, N]")
    _require_device(fn, dout, out, lse)
    n_rows = cu_seqlens.numel() - 1
    mb = attn_max_blocks(n, n_rows) if max_blocks is None else int(max_blocks)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    ws = torch.empty(2 * hq * n * d, dtype=torch.float32, device=q.device)
    # q, dO, O, dQ; k, v, dK, dV; the partials written and read back; lse
    nbytes = 2 * (4 * q.numel() + 4 * k.numel()) + 4 * 2 * hq * n * d * 2 + lse.numel() * 4
    cnt = _counter_buffer(_attn_counters, q.device, mb * k.shape[1])
    _launch("attn_bwd", nbytes, 2.5 * _attn_flops(lens, hq), "rus_attn_varlen_bwd",
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr(),
            lse.data_ptr(), cu_seqlens.data_ptr(), n_rows, n, mb, hq, k.shape[1], d, scale,
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), cnt.data_ptr(),
            cnt.numel(), _stream(q))
    return dq, dk, dv


def attn_varlen_bwd_parts(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          out: torch.Tensor, lse: torch.Tensor, cu_seqlens: torch.Tensor,
                          max_blocks: int | None = None, scale: float | None = None, lens=None):
    """``attn_varlen_bwd`` without the sum over each KV group's query heads: (dq, dk_part,
    dv_part), the partials fp32 [h_q, N, 128] (dk_part scaled), for
    ``qkv_rope_bwd_lora_mid_parts`` to sum."""
    fn = "attn_varlen_bwd_parts"
    _attn_operands(fn, q, k, v, cu_seqlens)
    n, hq, d = q.shape
    for name, t in (("dout", dout), ("out", out)):
        if t.shape != q.shape or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous fp16 like q")
    if lse.shape != (hq, n) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError(f"{fn}: lse must be contiguous fp32 [h_q, N]")
    _require_device(fn, dout, out, lse)
    n_rows = cu_seqlens.numel() - 1
    mb = attn_max_blocks(n, n_rows) if max_blocks is None else int(max_blocks)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    dq = torch.empty_like(q)
    ws = torch.empty(2 * hq * n * d, dtype=torch.float32, device=q.device)
    # q, dO, O, dQ; k, v; the partials written; lse
    nbytes = 2 * (4 * q.numel() + 2 * k.numel()) + 4 * 2 * hq * n * d + lse.numel() * 4
    _launch("attn_bwd", nbytes, 2.5 * _attn_flops(lens, hq), "rus_attn_varlen_bwd_parts",
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr(),
            lse.data_ptr(), cu_seqlens.data_ptr(), n_rows, n, mb, hq, k.shape[1], d, scale,
            dq.data_ptr(), ws.data_ptr(), _stream(q))
    dk_part = ws[: hq * n * d].view(hq, n, d)
    dv_part = ws[hq * n * d:].view(hq, n, d)
    return dq, dk_part, dv_part


def transpose_rows(rows: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[:, :n] = rows^T and out[:, n:] = 0 for fp16 rows [n, d] and out [d, >= n] (both with
    contiguous rows): the K-contiguous W^T operand of the hidden-gradient GEMM, on the device."""
    fn = "transpose_rows"
    _require_device(fn, rows, out)
    if rows.dtype != torch.float16 or out.dtype != torch.float16 or rows.dim() != 2 \
            or out.dim() != 2 or rows.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError(f"{fn}: fp16 2-D tensors with contiguous rows expected")
    n, d = rows.shape
    if out.shape[0] != d or out.shape[1] < n:
        raise ValueError(f"{fn}: out must be [{d}, >= {n}]")
    _launch("transpose_f16", 2 * (n * d + out.shape[0] * out.shape[1]), 0, "rus_transpose_f16",
            rows.data_ptr(), n, d, rows.stride(0), out.data_ptr(), out.stride(0), out.shape[1],
            _stream(rows))
    return out


def lm_head_weight_t(weight: torch.Tensor) -> torch.Tensor:
    """W^T [d, round_up(V, 64)] fp16 with zero padding columns, cached on the weight tensor (the
    lm_head is frozen in QLoRA, so this is built once; rebuilt if the weight is modified)."""
    hit = getattr(weight, "_rus_weight_t", None)
    if hit is not None and hit[0] == weight._version and hit[1].device == weight.device:
        return hit[1]
    V, d = weight.shape
    wt = torch.empty((d, _round_up(V, LM_K)), dtype=torch.float16, device=weight.device)
    transpose_rows(weight.detach(), wt)
    weight._rus_weight_t = (weight._version, wt)
    return wt


def lm_head_ce_loss(nll: torch.Tensor, labels: torch.Tensor, num_items_in_batch=None):
    """(loss, denom) as one-element float32 device tensors: denom = max(num_items_in_batch, 1)
    if given, else max(#(labels != -100), 1); loss = sum(nll) / denom (no host read)."""
    fn = "lm_head_ce_loss"
    _require_device(fn, nll, labels)
    dev = nll.device
    n = nll.numel()
    if labels.numel() != n or nll.dtype != torch.float32 or labels.dtype != torch.int64:
        raise ValueError(f"{fn}: nll float32 [n] and labels int64 [n] expected")
    ni = None
    if isinstance(num_items_in_batch, torch.Tensor):
        ni = num_items_in_batch.detach().to(device=dev, dtype=torch.float32).reshape(1)
    elif num_items_in_batch is not None:
        ni = torch.full((1,), float(num_items_in_batch), dtype=torch.float32, device=dev)
    out = torch.empty(2, dtype=torch.float32, device=dev)
    _launch("lmhead_ce_loss", n * 12, 0, "rus_lmhead_ce_loss", nll.contiguous().data_ptr(),
            labels.contiguous().data_ptr(), n, _ptr(ni), out.data_ptr(), out.data_ptr() + 4,
            _stream(nll))
    return out[0:1], out[1:2]


def lm_head_ce_chunk_scale(logits: torch.Tensor, n_vocab: int, parts: LMHeadPartials,
                           part_base: int, m_run: torch.Tensor, alpha: torch.Tensor,
                           first: bool) -> torch.Tensor:
    """In place over one chunk's kept fp16 logits [n_tok, >= round_up(n_vocab, 64)]: P =
    fp16(e^{z - M}) with M = max(running max, the chunk's max from partial rows part_base ...);
    updates ``m_run`` and writes ``alpha`` = e^{M_old - M} (replaces the logit recompute and
    lm_head_piece_kernel MODE 1, kernels.py:517-531)."""
    fn = "lm_head_ce_chunk_scale"
    _require_device(fn, logits, m_run, alpha)
    n_tok = logits.shape[0]
    kp = _round_up(n_vocab, LM_K)
    if logits.dtype != torch.float16 or logits.dim() != 2 or logits.shape[1] < kp \
            or logits.stride(1) != 1:
        raise ValueError(f"{fn}: logits must be fp16 [n_tok, >= {kp}] with contiguous rows")
    for name, t in (("m_run", m_run), ("alpha", alpha)):
        if t.dtype != torch.float32 or t.numel() < n_tok or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous float32 with {n_tok} entries")
    if part_base < 0 or part_base + lm_head_num_parts(n_vocab) > parts.n_parts \
            or parts.n_tok != n_tok:
        raise ValueError(f"{fn}: partial rows out of range")
    _launch("lmhead_ce_chunk_scale", 2 * n_tok * kp * 2 + 4 * n_tok * lm_head_num_parts(n_vocab),
            0, "rus_lmhead_ce_chunk_scale", logits.data_ptr(), logits.stride(0), n_tok, n_vocab,
            parts.m.data_ptr(), parts.m.stride(0), part_base, m_run.data_ptr(), alpha.data_ptr(),
            1 if first else 0, _stream(logits))
    return logits


def lm_head_ce_grad_hidden_scaled(probs: torch.Tensor, weight_t_cols: torch.Tensor, n_vocab: int,
                                  parts: torch.Tensor, accumulate: bool,
                                  alpha: torch.Tensor) -> None:
    """parts[s] = parts[s] * alpha[row] + (P . W_chunk)[split s] (or = without ``accumulate``):
    the hidden-gradient GEMM of one chunk of the single-pass head (replaces the per-chunk
    ``addmm_`` of ops.py:320). Every split of ``parts`` is written, empty ones only rescaled."""
    fn = "lm_head_ce_grad_hidden_scaled"
    _require_device(fn, probs, weight_t_cols, parts, alpha)
    n_tok = probs.shape[0]
    d = weight_t_cols.shape[0]
    n_split = parts.shape[0]
    if parts.dtype != torch.float32 or tuple(parts.shape[1:]) != (n_tok, d) or not parts.is_contiguous():
        raise ValueError(f"{fn}: parts must be contiguous float32 [n_split, {n_tok}, {d}]")
    if alpha.dtype != torch.float32 or alpha.numel() < n_tok:
        raise ValueError(f"{fn}: alpha must be float32 with {n_tok} entries")
    for name, t in (("probs", probs), ("weight_t", weight_t_cols)):
        if t.dtype != torch.float16 or t.stride(1) != 1:
            raise ValueError(f"{fn}: {name} must be fp16 with contiguous rows")
        if t.shape[0] * t.stride(0) * 2 >= 1 << 32:
            raise ValueError(f"{fn}: {name} exceeds the 4 GiB operand limit of the MFMA kernels")
    kp = _round_up(n_vocab, LM_K)
    _launch("lmhead_ce_grad_hidden", (n_tok + d) * kp * 2 + 4 * n_split * n_tok * d * (2 if accumulate else 1),
            2.0 * n_tok * d * n_vocab, "rus_lmhead_ce_grad_hidden_scaled", probs.data_ptr(),
            probs.stride(0), weight_t_cols.data_ptr(), weight_t_cols.stride(0), n_tok, d,
            n_vocab, parts.data_ptr(), n_split, 1 if accumulate else 0, alpha.data_ptr(),
            _stream(probs))


def lm_head_ce_dh_finish(parts: torch.Tensor, m_run: torch.Tensor, lse: torch.Tensor,
                         labels: torch.Tensor, w_rows: torch.Tensor, denom: torch.Tensor,
                         scale: float = 1.0, scale_dev: torch.Tensor | None = None,
                         out_dtype=torch.float32) -> torch.Tensor:
    """Hidden gradient (x 2^16 / denom x scale) of the single-pass head: (sum_s parts[s] *
    e^{m_run - lse} - W[y]) per labelled token, 0 for label -100. ``w_rows`` is the lm_head
    weight [V, d] on the device or pinned on the host (its label rows are then read over the
    bus)."""
    fn = "lm_head_ce_dh_finish"
    _require_device(fn, parts, m_run, lse, labels, denom, scale_dev)
    n_split, n_tok, d = parts.shape
    if parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError(f"{fn}: parts must be contiguous float32")
    on_host = w_rows.device.type == "cpu"
    if on_host and not w_rows.is_pinned():
        raise ValueError(f"{fn}: a host weight must be pinned")
    if not on_host:
        _require_device(fn, w_rows)
    if w_rows.dtype != torch.float16 or w_rows.dim() != 2 or w_rows.shape[1] != d \
            or w_rows.stride(1) != 1:
        raise ValueError(f"{fn}: w_rows must be fp16 [V, {d}] with contiguous rows")
    lab = labels.reshape(-1)
    if lab.dtype != torch.int64 or lab.numel() != n_tok:
        raise ValueError(f"{fn}: labels must be int64 with {n_tok} entries")
    out = torch.empty((n_tok, d), dtype=out_dtype, device=parts.device)
    _launch("lmhead_ce_dh_finish", parts.numel() * 4 + out.numel() * out.element_size(), 0,
            "rus_lmhead_ce_dh_finish", parts.data_ptr(), n_split, n_tok, d, m_run.data_ptr(),
            lse.data_ptr(), lab.contiguous().data_ptr(), w_rows.data_ptr(), w_rows.stride(0),
            w_rows.shape[0], 1 if on_host else 0, denom.data_ptr(), float(scale),
            _ptr(scale_dev), out.data_ptr(), _dtype_code(fn, out_dtype), _stream(parts))
    return out


class LMHeadPass:
    """One single pass of the lm_head cross-entropy over vocabulary chunks (in order).

    Per chunk: the statistics GEMM (partial m, s, w, argmax and the target logit per 256 rows)
    and, when the hidden gradient is wanted, its fp16 logits kept in a [n_tok, chunk] buffer,
    turned in place into P = e^{z - M} (M the running maximum) and accumulated as P . W_chunk into
    fp32 split-K partials rescaled whenever M grows. ``finish`` combines the statistics (lse,
    nll, entropy, argmax, loss) and forms dH = sum_v (softmax - onehot) W_v x 2^16 / denom. W is
    read once, and no [n_tok, V] array exists (the reference reads W twice and recomputes the
    logits, solution/ops.py:217-322)."""

    def __init__(self, n_tok: int, d: int, n_vocab: int, chunk: int, device, need_grad: bool):
        self.n_tok, self.d, self.n_vocab, self.chunk = n_tok, d, n_vocab, int(chunk)
        self.need_grad = need_grad
        self.parts = LMHeadPartials(lm_head_num_parts(n_vocab), n_tok, device)
        self.target = torch.zeros(n_tok, dtype=torch.float32, device=device)
        self.first = True
        if need_grad:
            self.z = torch.empty((n_tok, _round_up(min(self.chunk, n_vocab), LM_K)),
                                 dtype=torch.float16, device=device)
            self.m_run = torch.empty(n_tok, dtype=torch.float32, device=device)
            self.alpha = torch.empty(n_tok, dtype=torch.float32, device=device)
            # every chunk's GEMM reads and rewrites all the fp32 partials (the rescaled
            # accumulation), so splits beyond one round of CUs cost a partial pass per chunk for
            # a few percent of mainloop: at most one round
            n_cu = cu_count(device)
            tiles = -(-n_tok // 256) * -(-d // 256)
            self.n_split = lm_head_split_count(n_tok, d, min(self.chunk, n_vocab), n_cu,
                                               max_split=max(1, n_cu // tiles))
            self.dparts = torch.empty((self.n_split, n_tok, d), dtype=torch.float32, device=device)

    def add_chunk(self, hidden: torch.Tensor, w_rows: torch.Tensor, w_t: torch.Tensor | None,
                  start: int, labels: torch.Tensor) -> None:
        """Vocabulary rows [start, start + len(w_rows)) with their transpose ``w_t`` [d, >= rows]
        (needed with the gradient only)."""
        n = w_rows.shape[0]
        if not self.need_grad:
            lm_head_ce_fwd_chunk(hidden, w_rows, labels, start, self.parts, self.target)
            return
        lm_head_ce_fwd_chunk(hidden, w_rows, labels, start, self.parts, self.target,
                             logits_out=self.z)
        lm_head_ce_chunk_scale(self.z, n, self.parts, start // LM_TILE, self.m_run, self.alpha,
                               self.first)
        lm_head_ce_grad_hidden_scaled(self.z, w_t, n, self.dparts, not self.first, self.alpha)
        self.first = False

    def finish(self, labels: torch.Tensor, num_items_in_batch, w_rows_all: torch.Tensor,
               dh_scale: float = 1.0, dh_dtype=torch.float32, scale_dev=None):
        """(nll, lse, entropy, argmax, denom, dh, loss); dh None without the gradient."""
        lse, nll, ent, amax = lm_head_ce_combine(self.parts, self.target, labels)
        loss, denom = lm_head_ce_loss(nll, labels, num_items_in_batch)
        dh = None
        if self.need_grad:
            dh = lm_head_ce_dh_finish(self.dparts, self.m_run, lse, labels, w_rows_all, denom,
                                      dh_scale, scale_dev, dh_dtype)
        return nll, lse, ent, amax, denom, dh, loss


def lm_head_ce_logits(hidden: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[t, v] = fp16(hidden[t] . weight[v]) for the vocabulary rows of ``weight``, zeros in
    ``out``'s columns up to round_up(V, 64) (out [n_tok, >= that] fp16, contiguous rows)."""
    fn = "lm_head_ce_logits"
    _require_device(fn, hidden, weight, out)
    d = hidden.shape[1]
    h = _lm_operand(fn, hidden, d, "hidden")
    w = _lm_operand(fn, weight, d, "weight")
    n_tok, V = h.shape[0], w.shape[0]
    kp = _round_up(V, LM_K)
    if out.dtype != torch.float16 or out.dim() != 2 or out.shape[0] != n_tok \
            or out.shape[1] < kp or out.stride(1) != 1:
        raise ValueError(f"{fn}: out must be fp16 [{n_tok}, >= {kp}] with contiguous rows")
    if out.shape[0] * out.stride(0) * 2 >= 1 << 32:
        raise ValueError(f"{fn}: out exceeds the 4 GiB operand limit of the MFMA kernels")
    _launch("lmhead_ce_logits", (n_tok + V) * d * 2 + n_tok * kp * 2, 2.0 * n_tok * d * V,
            "rus_lmhead_ce_logits", h.data_ptr(), w.data_ptr(), n_tok, d, h.stride(0),
            w.stride(0), V, out.data_ptr(), out.stride(0), _stream(h))
    return out


def lm_head_ce_rows(logits: torch.Tensor, n_vocab: int, labels: torch.Tensor,
                    denom: torch.Tensor | None, lse: torch.Tensor, nll: torch.Tensor,
                    ent: torch.Tensor, amax: torch.Tensor) -> None:
    """Per-token lse / nll / entropy / argmax of kept logit rows into the given tensors (one
    entry per row) and, with ``denom``, the rows turned into the fp16 logit gradient in place
    (replaces lm_head_piece_kernel MODE 0 / 1 and lm_head_finish_kernel, kernels.py:453-565)."""
    fn = "lm_head_ce_rows"
    _require_device(fn, logits, labels, denom, lse, nll, ent, amax)
    n_tok = logits.shape[0]
    kp = _round_up(n_vocab, LM_K)
    if logits.dtype != torch.float16 or logits.dim() != 2 or logits.shape[1] < kp \
            or logits.stride(1) != 1:
        raise ValueError(f"{fn}: logits must be fp16 [n_tok, >= {kp}] with contiguous rows")
    lab = labels.reshape(-1)
    if lab.dtype != torch.int64 or lab.numel() != n_tok or not lab.is_contiguous():
        raise ValueError(f"{fn}: labels must be contiguous int64 with {n_tok} entries")
    for name, t, dt in (("lse", lse, torch.float32), ("nll", nll, torch.float32),
                        ("entropy", ent, torch.float32), ("argmax", amax, torch.int64)):
        if t.dtype != dt or t.numel() != n_tok or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be contiguous {dt} with {n_tok} entries")
    if denom is not None and (denom.dtype != torch.float32 or denom.numel() != 1):
        raise ValueError(f"{fn}: denom must be a one-element float32 device tensor")
    grad = denom is not None
    _launch("lmhead_ce_rows", n_tok * kp * 2 * (3 if grad else 1) + 28 * n_tok, 0,
            "rus_lmhead_ce_rows", logits.data_ptr(), logits.stride(0), n_tok, n_vocab,
            lab.data_ptr(), _ptr(denom), lse.data_ptr(), nll.data_ptr(), ent.data_ptr(),
            amax.data_ptr(), _stream(logits))


def lm_head_ce_denom(labels: torch.Tensor, num_items_in_batch=None) -> torch.Tensor:
    """The loss denominator alone, as a one-element float32 device tensor (what ``lm_head_ce_loss``
    will use): max(num_items_in_batch, 1) if given, else max(#(labels != -100), 1)."""
    fn = "lm_head_ce_denom"
    _require_device(fn, labels)
    dev = labels.device
    lab = labels.reshape(-1)
    if lab.dtype != torch.int64:
        raise ValueError(f"{fn}: labels must be int64")
    ni = None
    if isinstance(num_items_in_batch, torch.Tensor):
        ni = num_items_in_batch.detach().to(device=dev, dtype=torch.float32).reshape(1)
    elif num_items_in_batch is not None:
        ni = torch.full((1,), float(num_items_in_batch), dtype=torch.float32, device=dev)
    denom = torch.empty(1, dtype=torch.float32, device=dev)
    _launch("lmhead_ce_loss", lab.numel() * 8, 0, "rus_lmhead_ce_loss", None,
            lab.contiguous().data_ptr(), lab.numel(), _ptr(ni), None, denom.data_ptr(),
            _stream(lab))
    return denom


LM_BLOCK_BUDGET = 256 << 20  # bytes of fp16 logits one token block of the blocked head may hold


def lm_head_block_tokens(n_vocab: int, budget: int = LM_BLOCK_BUDGET) -> int:
    """Most tokens one block of the token-blocked head takes: the whole 256-token tiles whose fp16
    logits [tokens, round_up(V, 64)] fit ``budget`` (at least one tile)."""
    kp = max(LM_K, _round_up(n_vocab, LM_K))
    return max(1, budget // (2 * kp * LM_TILE)) * LM_TILE


def lm_head_token_blocks(n_tok: int, max_block: int = LM_TILE) -> list[tuple[int, int]]:
    """Token ranges [t0, t1) of the token-blocked head. No block holds every token of a batch of
    two or more, so the logits of all N tokens never exist at once: a batch of more than one
    256-token MFMA tile goes in at least two blocks of whole tiles (the last one partial), its
    tiles spread evenly over the fewest blocks of at most ``max_block`` tokens (rounded down to
    whole tiles, at least one) — no block adds a partly filled tile; a batch within one tile
    goes in two halves."""
    if n_tok <= 0:
        return []
    tiles = -(-n_tok // LM_TILE)
    if tiles == 1:
        half = (n_tok + 1) // 2
        return [(0, half), (half, n_tok)] if n_tok > 1 else [(0, n_tok)]
    max_tiles = max(1, min(max_block // LM_TILE, tiles - 1))
    nb = -(-tiles // max_tiles)
    base, extra = divmod(tiles, nb)
    out, t = [], 0
    for b in range(nb):
        t1 = min(n_tok, t + (base + (1 if b < extra else 0)) * LM_TILE)
        out.append((t, t1))
        t = t1
    return out


def _fwd_rows(hidden, weight, labels, parts: LMHeadPartials, target, t0: int, t1: int,
              logits: torch.Tensor | None) -> None:
    """Statistics (and kept logits) of tokens [t0, t1) over the whole vocabulary: the token
    columns t0 .. of the partial arrays."""
    n, d = t1 - t0, hidden.shape[1]
    V = weight.shape[0]
    h = hidden[t0:t1]
    args = (h.data_ptr(), weight.data_ptr(), labels.data_ptr() + 8 * t0, n, d, h.stride(0),
            weight.stride(0), V, 0, parts.m.data_ptr() + 4 * t0, parts.s.data_ptr() + 4 * t0,
            parts.w.data_ptr() + 4 * t0, parts.idx.data_ptr() + 4 * t0, 0, parts.n_tok,
            target.data_ptr() + 4 * t0)
    nbytes = (n + V) * d * 2 + 16 * n * parts.n_parts
    if logits is None:
        _launch("lmhead_ce_fwd", nbytes, 2.0 * n * d * V, "rus_lmhead_ce_fwd", *args, _stream(h))
    else:
        _launch("lmhead_ce_fwd_keep", nbytes + n * logits.shape[1] * 2, 2.0 * n * d * V,
                "rus_lmhead_ce_fwd_keep", *args, logits.data_ptr(), logits.stride(0), _stream(h))


def lm_head_ce(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
               num_items_in_batch=None, v_chunk: int | None = None, need_grad: bool = True,
               weight_t: torch.Tensor | None = None, dh_scale: float = 1.0,
               dh_dtype: torch.dtype = torch.float32, block_tokens: int | None = None):
    """Whole cross-entropy head on a device-resident fp16 lm_head weight [V, d].

    Returns (nll, lse, entropy, argmax, denom, dh, loss) where denom is a float32 device scalar
    (num_items_in_batch, else the count of labels != -100, clamped to >= 1), loss = sum(nll) /
    denom (device scalar) and dh the hidden gradient of loss times 2^16, scaled by ``dh_scale``
    and stored as ``dh_dtype`` (None without need_grad).

    With the gradient, the tokens go in blocks (``lm_head_token_blocks``: whole 256-token MFMA
    tiles, at least two blocks for two or more tokens, at most ``block_tokens`` each; default:
    the tiles whose fp16 logits fit 256 MiB, 768 tokens at V = 151936; 744 tokens go as 512 +
    232; a batch within one tile takes the single pass below over at least two vocabulary
    chunks). For each block one GEMM over the whole vocabulary stores its fp16 logits in a
    [block, V] buffer; one kernel per token row forms the statistics and turns the row into the
    reference's fp16 gradient G = fp16((softmax - onehot) 2^16 / denom) in place (the denominator
    is known up front); and a split-K GEMM G . W writes the block's dH partials, summed once. W
    (and W^T) is read once per block; the logit buffer stays bounded at any token count and no
    logit is recomputed (the reference holds [N, 8192] chunks and
    recomputes every logit, solution/ops.py:209-322). ``v_chunk`` (a multiple of 256) selects
    the single pass over vocabulary chunks instead (``LMHeadPass``: W read once in total, an
    [N, v_chunk] buffer), the engine's default layout (``ops.lm_head_layout``) and that of a
    head streamed from the host. ``weight_t`` is W^T
    [d, >= round_up(V, 64)] (built and cached on the weight when not given).
    """
    fn = "lm_head_ce"
    _require_device(fn, hidden, weight, labels)
    n_tok, d = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    lab = labels.reshape(-1).to(torch.int64).contiguous()
    h = _lm_operand(fn, hidden, d, "hidden")
    w = _lm_operand(fn, weight, d, "weight")
    if lab.numel() != n_tok:
        raise ValueError(f"{fn}: labels must have {n_tok} entries")
    if v_chunk is None and need_grad and 1 < n_tok <= LM_TILE:
        # A batch within one 256-token tile: split into token blocks, each block's GEMMs would
        # read all of W on a half-empty tile (twice the cost of one pass); the pass over at
        # least two vocabulary chunks reads W once and still never holds [N, V] logits.
        v_chunk = min(lm_head_chunk_cols(n_tok, V, cu_count(dev)),
                      _round_up(-(-V // 2), LM_TILE))
    if v_chunk is not None:
        chunk = int(v_chunk)
        if chunk <= 0 or (chunk < V and chunk % LM_TILE):
            raise ValueError(f"{fn}: v_chunk must be a positive multiple of {LM_TILE}")
        wt = None
        if need_grad:
            wt = weight_t if weight_t is not None else lm_head_weight_t(weight)
        hp = LMHeadPass(n_tok, d, V, chunk, dev, need_grad)
        for start in range(0, V, chunk):
            end = min(start + chunk, V)
            hp.add_chunk(h, w[start:end], None if wt is None else wt[:, start:], start, lab)
        return hp.finish(lab, num_items_in_batch, w, dh_scale, dh_dtype)

    if not need_grad or n_tok == 0:
        parts = LMHeadPartials(lm_head_num_parts(V), n_tok, dev)
        target = torch.zeros(n_tok, dtype=torch.float32, device=dev)
        if n_tok:
            _fwd_rows(h, w, lab, parts, target, 0, n_tok, None)
        lse, nll, ent, amax = lm_head_ce_combine(parts, target, lab)
        loss, denom = lm_head_ce_loss(nll, lab, num_items_in_batch)
        dh = torch.zeros((n_tok, d), dtype=dh_dtype, device=dev) if need_grad else None
        return nll, lse, ent, amax, denom, dh, loss
    wt = weight_t if weight_t is not None else lm_head_weight_t(weight)
    kp = _round_up(V, LM_K)
    if wt.dtype != torch.float16 or wt.shape[0] != d or wt.shape[1] < kp or wt.stride(1) != 1:
        raise ValueError(f"{fn}: weight_t must be fp16 [{d}, >= {kp}] with contiguous rows")
    blocks = lm_head_token_blocks(n_tok, block_tokens if block_tokens else lm_head_block_tokens(V))
    nb_max = max(t1 - t0 for t0, t1 in blocks)
    ncu = cu_count(dev)
    splits = {nb: lm_head_split_count(nb, d, V, ncu) for nb in {t1 - t0 for t0, t1 in blocks}}
    z = torch.empty((nb_max, kp), dtype=torch.float16, device=dev)
    if z.numel() * 2 >= 1 << 32:
        raise ValueError(f"{fn}: a {nb_max}-token block of logits exceeds the 4 GiB operand limit")
    dflat = torch.empty(max(splits.values()) * nb_max * d, dtype=torch.float32, device=dev)
    denom = lm_head_ce_denom(lab, num_items_in_batch)
    lse = torch.empty(n_tok, dtype=torch.float32, device=dev)
    nll = torch.empty(n_tok, dtype=torch.float32, device=dev)
    ent = torch.empty(n_tok, dtype=torch.float32, device=dev)
    amax = torch.empty(n_tok, dtype=torch.int64, device=dev)
    dh = torch.empty((n_tok, d), dtype=dh_dtype, device=dev)
    for t0, t1 in blocks:
        nb = t1 - t0
        zb = z[:nb]
        lm_head_ce_logits(h[t0:t1], w, zb)
        lm_head_ce_rows(zb, V, lab[t0:t1], denom, lse[t0:t1], nll[t0:t1], ent[t0:t1],
                        amax[t0:t1])
        s = splits[nb]
        dparts = dflat[: s * nb * d].view(s, nb, d)
        lm_head_ce_grad_hidden(zb, wt, V, dparts, accumulate=False)
        lm_head_dh_reduce(dparts, dh_scale, dh_dtype, out=dh[t0:t1])
    loss, _ = lm_head_ce_loss(nll, lab, num_items_in_batch)
    return nll, lse, ent, amax, denom, dh, loss


# ---------------------------------------------------------------------------------------------
# AdamW over a flat fp32 buffer (the trainer's torch.optim.AdamW, HF "adamw_torch";
# reference harness/_train.py:30)
# ---------------------------------------------------------------------------------------------


def adamw_step(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
               exp_avg_sq: torch.Tensor, lr: float, beta1: float, beta2: float, eps: float,
               weight_decay: float, step: int) -> None:
    """One AdamW step (torch.optim.AdamW's update, amsgrad and maximize off) of step number
    ``step`` (>= 1) over contiguous fp32 device tensors of one size, in place, one launch."""
    fn = "adamw_step"
    _require_device(fn, param, grad, exp_avg, exp_avg_sq)
    n = param.numel()
    for name, t in (("param", param), ("grad", grad), ("exp_avg", exp_avg),
                    ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != n:
            raise ValueError(f"{fn}: {name} must be contiguous float32 with {n} values")
    if int(step) < 1:
        raise ValueError(f"{fn}: step must be >= 1")
    _launch("adamw", 28 * n, 0, "rus_adamw_step", param.data_ptr(), grad.data_ptr(),
            exp_avg.data_ptr(), exp_avg_sq.data_ptr(), n, float(lr), float(beta1), float(beta2),
            float(eps), float(weight_decay), int(step), _stream(param))


def lora_cast_t(flat: torch.Tensor, n_layers: int, shapes, out: torch.Tensor,
                out_t: torch.Tensor | None = None) -> None:
    """One launch: ``out`` = fp16(flat) (same layout: n_layers x the segments of ``shapes``, each
    row-major [rows, cols]) and, when given, ``out_t`` = every layer's segments transposed,
    region j = [n_layers, cols_j, rows_j] (regions back to back in segment order)."""
    fn = "lora_cast_t"
    _require_device(fn, flat, out, out_t)
    shapes = [(int(r), int(c)) for r, c in shapes]
    if not 1 <= len(shapes) <= 4:
        raise ValueError(f"{fn}: 1 to 4 segments per layer")
    n = int(n_layers) * sum(r * c for r, c in shapes)
    if flat.dtype != torch.float32 or not flat.is_contiguous() or flat.numel() != n:
        raise ValueError(f"{fn}: flat must be contiguous float32 with {n} values")
    for name, t in (("out", out), ("out_t", out_t)):
        if t is not None and (t.dtype != torch.float16 or not t.is_contiguous() or t.numel() != n):
            raise ValueError(f"{fn}: {name} must be contiguous float16 with {n} values")
    rows = (ctypes.c_int64 * len(shapes))(*[r for r, _ in shapes])
    cols = (ctypes.c_int64 * len(shapes))(*[c for _, c in shapes])
    _launch("lora_cast_t", n * (4 + 2 + (2 if out_t is not None else 0)), 0, "rus_lora_cast_t",
            flat.data_ptr(), int(n_layers), len(shapes), rows, cols, out.data_ptr(), _ptr(out_t),
            _stream(flat))
