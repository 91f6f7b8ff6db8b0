"""rus_amd — MI355X (gfx950) implementation of the fused QLoRA training hot path of
fokyso82002-rgb/rus (its ``solution/`` package).

Modules mirror the reference's layout so they can be used as a drop-in:

* ``rus_amd.kernels``  — launchers with the reference's names (kernels.py), backed by hand-written
  HIP kernels in ``librus_amd.so`` through the C ABI of ``include/rus_amd.h``;
* ``rus_amd.ops``      — the autograd functions, the fused Qwen2 engine and the runtime patches
  (ops.py);
* ``rus_amd.hostload`` — host-pinned weight / head / input streaming (hostload.py);
* ``rus_amd.quant``    — NF4 double-quant quantisation (model-load step);
* ``apply()``          — the one-call installer (solution/__init__.py:111-125).
"""

from __future__ import annotations

__version__ = "0.1.0"

_ACTIVE: dict | None = None  # the patches apply() installed, once it has run


def _warm_up(device) -> None:
    """One launch of every kernel family on tiny inputs, so that a broken library or device fails
    here rather than in the first training step (the reference pre-compiles its Triton kernels the
    same way, solution/__init__.py:41-108, but swallows errors; here they raise)."""
    import torch

    from . import kernels as K

    dev = torch.device(device)
    # NF4 dequant: 32 x 64 weight, one absmax block per 64 codes, one super block
    packed = torch.zeros(1024, dtype=torch.uint8, device=dev)
    absmax = torch.zeros(32, dtype=torch.uint8, device=dev)
    code2 = torch.zeros(256, dtype=torch.float32, device=dev)
    absmax2 = torch.zeros(1, dtype=torch.float32, device=dev)
    K.dequant_nf4_tensor(packed, absmax, code2, absmax2, (0.0, 0.0, 0.0), (32, 64))
    # RMSNorm with and without the residual, forward and backward
    x = torch.zeros(4, 1536, dtype=torch.float16, device=dev)
    w = torch.ones(1536, dtype=torch.float16, device=dev)
    y, h, rstd = K.rms_norm_fwd(x, w, eps=1e-6, residual=x)
    K.rms_norm_bwd(y, h, w, rstd, dresidual=x)
    y, h, rstd = K.rms_norm_fwd(x, w, eps=1e-6)
    K.rms_norm_bwd(y, h, w, rstd)
    # LoRA delta + RoPE forward and backward (12 / 2 heads of 128)
    qkv = torch.zeros(4, 2048, dtype=torch.float16, device=dev)
    q_l = torch.zeros(4, 1536, dtype=torch.float16, device=dev)
    v_l = torch.zeros(4, 256, dtype=torch.float16, device=dev)
    cos = torch.ones(8, 128, dtype=torch.float16, device=dev)
    sin = torch.zeros(8, 128, dtype=torch.float16, device=dev)
    pos = torch.arange(4, dtype=torch.int64, device=dev)
    q, k, v = K.qkv_rope_fwd(qkv, cos, sin, pos, q_lora=q_l, v_lora=v_l)
    K.qkv_rope_bwd(q, k, v, cos, sin, pos)
    # SwiGLU forward and in-place backward over a fused [gate | up]
    gu = torch.zeros(4, 17920, dtype=torch.float16, device=dev)
    K.mlp_glu_bwd(K.mlp_glu_fwd(gu), gu)
    # lm_head cross-entropy, forward and backward
    hid = torch.zeros(4, 1536, dtype=torch.float16, device=dev)
    head = torch.zeros(1024, 1536, dtype=torch.float16, device=dev)
    lab = torch.zeros(4, dtype=torch.int64, device=dev)
    K.lm_head_ce(hid, head, lab)
    torch.cuda.synchronize(dev)


def apply(device=None) -> dict[str, bool]:
    """Installs the fused path once per process (solution/__init__.py:111-125): loads the kernel
    library (raising if it is missing or was built for another ABI), launches every kernel family
    once on ``device`` (default: the current HIP device) when a GPU is visible, and installs the
    runtime patches of ``rus_amd.ops.install_runtime_patches`` — the fused ``Qwen2ForCausalLM``
    training forward, ``Qwen2MLP`` / ``Qwen2RMSNorm`` on the kernels, TRL's entropy helper.
    Returns which patches are active. A second call does nothing and returns the same answer.

    The reference's model-loading hooks (bitsandbytes ``Params4bit._quantize`` and accelerate's
    ``set_module_tensor_to_device``, solution/hostload.py:491-560) are not installed: this build
    reads an already loaded model (``rus_amd.adapters``) and keeps the packed NF4 image in pinned
    host memory itself (``rus_amd.hostload.WeightStream``)."""
    global _ACTIVE
    if _ACTIVE is not None:
        return dict(_ACTIVE)
    import torch

    from . import _lib
    from .ops import install_runtime_patches

    _lib.load()
    if torch.cuda.is_available():
        _warm_up(device if device is not None else torch.cuda.current_device())
    active = install_runtime_patches()
    _ACTIVE = dict(active)
    return active
