"""Loader for the gfx950 kernel library (``librus_amd.so``) and its C ABI (``include/rus_amd.h``).

The library must be built (``python -m rus_amd.build``) before any kernel is called; there is no
CPU or Python fallback, so a missing library or a non-HIP tensor raises immediately.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librus_amd.so"
ABI_VERSION = 17

DTYPE_F16 = 0
DTYPE_F32 = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_u64 = ctypes.c_uint64

class Nf4Job(ctypes.Structure):
    """struct rus_nf4_job of include/rus_amd.h."""

    _fields_ = [
        ("packed", ctypes.c_void_p), ("absmax", ctypes.c_void_p), ("absmax2", ctypes.c_void_p),
        ("off0", ctypes.c_float), ("off1", ctypes.c_float), ("off2", ctypes.c_float),
        ("split_byte_1", ctypes.c_int64), ("split_byte_2", ctypes.c_int64),
        ("absmax2_base_1", ctypes.c_int64), ("absmax2_base_2", ctypes.c_int64),
        ("n_bytes", ctypes.c_int64), ("n_absmax", ctypes.c_int64), ("n_absmax2", ctypes.c_int64),
        ("out_u32", ctypes.c_void_p),
    ]


class NormSide(ctypes.Structure):
    """struct rus_norm_side of include/rus_amd.h."""

    _fields_ = [
        ("kind", ctypes.c_int32), ("w_dtype", ctypes.c_int32), ("n_rows", ctypes.c_int64),
        ("n_cols", ctypes.c_int64), ("stride_row", ctypes.c_int64), ("eps", ctypes.c_float),
        ("x", ctypes.c_void_p), ("residual", ctypes.c_void_p), ("h", ctypes.c_void_p),
        ("weight", ctypes.c_void_p), ("rstd", ctypes.c_void_p), ("sum_out", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
    ]


NORM_FWD, NORM_BWD = 1, 2


class LoraRows(ctypes.Structure):
    """struct rus_lora_rows of include/rus_amd.h."""

    _fields_ = [
        ("x", ctypes.c_void_p), ("stride_x", ctypes.c_int64), ("n_tokens", ctypes.c_int64),
        ("d", ctypes.c_int64), ("r", ctypes.c_int32), ("a_q", ctypes.c_void_p),
        ("a_v", ctypes.c_void_p), ("bits_q", ctypes.c_void_p), ("bits_v", ctypes.c_void_p),
        ("p_q", ctypes.c_float), ("p_v", ctypes.c_float), ("mid_q", ctypes.c_void_p),
        ("mid_v", ctypes.c_void_p),
    ]

# name -> argtypes, in the order of include/rus_amd.h. Every entry point returns int.
SIGNATURES: dict[str, list] = {
    "rus_copy_from_host": [_vp, _vp, _i64, _vp],
    "rus_gather_rows_from_host": [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp],
    "rus_nf4_dequant": [_vp, _vp, _vp, _vp, _f32, _f32, _f32, _i64, _i64, _i64, _i64, _i64, _i64,
                        _i64, _i32, _i32, _vp, _vp],
    "rus_nf4_dequant_multi": [ctypes.POINTER(Nf4Job), _i32, _vp, _i32, _i32, _vp],
    "rus_lora_down_rows": [ctypes.POINTER(LoraRows), _vp],
    "rus_lora_cast_t": [_vp, _i64, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _vp, _vp,
                        _vp],
    "rus_adamw_step": [_vp, _vp, _vp, _vp, _i64, _f64, _f64, _f64, _f64, _f64, _i64, _vp],
    "rus_nf4_dequant_multi_norm": [ctypes.POINTER(Nf4Job), _i32, _vp, _i32, _i32,
                                   ctypes.POINTER(NormSide), ctypes.POINTER(LoraRows), _vp],
    "rus_nf4_gemm_plan": [_i64, _i64, _i64, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i64),
                          ctypes.POINTER(_i64)],
    "rus_nf4_gemm": [_vp, _i64, _i64, ctypes.POINTER(Nf4Job), _vp, _i64, _i64, _i32, _i32, _i32,
                     _vp, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp],
    "rus_gemm_parts": [_vp, _i64, _vp, _i64, _i32, _i64, _i64, _i64, _vp, _i32, _vp],
    "rus_lora_dropout_fwd": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _u64, _u64, _f32, _f32, _i32, _vp],
    "rus_lora_dropout_bwd_add": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _u64, _u64, _f32, _f32, _i32, _vp],
    "rus_graph_node_counts": [_vp, _vp, _i32],
    "rus_dropout_keep_bits": [_vp, _u64, _i32, _i64, _i64, _f32, _f32, _vp, _vp],
    "rus_lora_workspace_size": [_i32, _i64, _i64, _i64, _i64, _i32, ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64)],
    "rus_lora_down_fwd": [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _f32, _f32,
                          _vp, _i64, _vp, _i64, _vp],
    "rus_lora_down_fwd_noalloc": [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _vp, _vp,
                                  _f32, _f32, _vp],
    "rus_qkv_lora_rope_fwd_mid": [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _i64, _i64, _i64, _i64, _f32, _f32, _i32, _i32, _i32, _vp, _vp],
    "rus_lora_bwd_x": [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _i64, _vp, _vp, _vp,
                       _i64, _vp, _vp, _f32, _f32, _vp, _i64, _vp, _i64, _vp],
    "rus_lora_bwd_w": [_vp, _i64, _vp, _vp, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                       _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp],
    "rus_lora_bwd_xw": [_vp, _i64, _vp, _vp, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                        _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                        _i64, _vp],
    "rus_lmhead_ce_loss": [_vp, _vp, _i64, _vp, _vp, _vp, _vp],
    "rus_attn_varlen_fwd": [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _f32, _vp, _vp,
                            _vp],
    "rus_attn_varlen_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _i32,
                            _f32, _vp, _vp, _vp, _vp, _vp, _i64, _vp],
    "rus_attn_varlen_bwd_parts": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32,
                                  _i32, _i32, _f32, _vp, _vp, _vp],
    "rus_rmsnorm_fwd": [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _i32, _vp],
    "rus_rmsnorm_bwd": [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "rus_rmsnorm_bwd_parts": [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rus_qkv_rope_bwd_mid": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
                             _i64, _i64, _i64, _i64, _f32, _f32, _i32, _i32, _i32, _vp, _vp],
    "rus_qkv_rope_bwd_mid_parts": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _i32, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _f32,
                                   _i32, _i32, _i32, _vp, _vp],
    "rus_qkv_lora_rope_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                              _i64, _i64, _f32, _f32, _i32, _i32, _i32, _vp, _i32, _vp],
    "rus_qkv_rope_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32,
                         _f32, _i32, _i32, _i32, _vp, _i32, _vp],
    "rus_swiglu_fwd": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _vp],
    "rus_swiglu_bwd": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                       _vp],
    "rus_lmhead_ce_fwd": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                          _i64, _i64, _vp, _vp],
    "rus_lmhead_ce_fwd_keep": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp,
                               _vp, _i64, _i64, _vp, _vp, _i64, _vp],
    "rus_lmhead_ce_grad_from_logits": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "rus_lmhead_ce_combine": [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                              _vp],
    "rus_lmhead_ce_grad_logits": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _vp, _i64, _vp],
    "rus_lmhead_ce_grad_hidden": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _i32, _vp],
    "rus_lmhead_dh_reduce": [_vp, _i32, _i64, _f32, _vp, _vp, _i32, _vp],
    "rus_transpose_f16": [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp],
    "rus_lmhead_ce_logits": [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp],
    "rus_lmhead_ce_rows": [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "rus_lmhead_ce_grad_hidden_scaled": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _i32,
                                         _vp, _vp],
    "rus_lmhead_ce_chunk_scale": [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _vp],
    "rus_lmhead_ce_dh_finish": [_vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp,
                                _f32, _vp, _vp, _i32, _vp],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Returns the loaded library, loading it on first use (after torch, to share its HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (torch's libamdhip64.so.7 must be the one this library binds)

        if not LIB_PATH.exists():
            raise RuntimeError(
                f"rus_amd: {LIB_PATH.name} is not built; run `python -m rus_amd.build` "
                "(there is no fallback path)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.rus_last_error.restype = ctypes.c_char_p
        lib.rus_last_error.argtypes = []
        lib.rus_abi_version.restype = ctypes.c_int
        lib.rus_abi_version.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        got = lib.rus_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"rus_amd: library ABI {got} != expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Calls one C entry point and raises RuntimeError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.rus_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")
