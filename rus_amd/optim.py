"""AdamW on the gfx950 kernel library: torch.optim.AdamW's update (decoupled weight decay,
amsgrad and maximize off) with one ``rus_adamw_step`` launch per parameter and step.

The reference's trainer steps the LoRA factors with torch.optim.AdamW (HF "adamw_torch";
harness/_train.py:30 forwards the trainer's optim settings). Over the engine's flat LoRA
parameter (``Qwen2FusedEngine.flat_lora_parameter``) a step is a single launch of 2,128 blocks
reading the fp32 parameter, gradient and both moments once, where torch's fused AdamW covers the
same 2.2 M values with 34 blocks and adds a launch for its device step count. The step count and
the bias corrections stay on the host (a plain int per parameter in ``state``).
"""

from __future__ import annotations

import torch

from . import kernels as K


class FlatAdamW(torch.optim.Optimizer):
    """AdamW over contiguous fp32 CUDA parameters, same hyperparameters and defaults as
    torch.optim.AdamW (lr 1e-3, betas (0.9, 0.999), eps 1e-8, weight_decay 1e-2)."""

    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2):
        if not lr >= 0.0 or not eps >= 0.0 or not weight_decay >= 0.0:
            raise ValueError("FlatAdamW: lr, eps and weight_decay must be >= 0")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError("FlatAdamW: betas must lie in [0, 1)")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps,
                                      weight_decay=weight_decay))
        for group in self.param_groups:
            for p in group["params"]:
                if p.dtype != torch.float32 or not p.is_contiguous() or p.device.type != "cuda":
                    raise ValueError("FlatAdamW: parameters must be contiguous float32 on the GPU")

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("FlatAdamW: sparse gradients are not supported")
                st = self.state[p]
                if not st:
                    st["step"] = 0
                    st["exp_avg"] = torch.zeros_like(p)
                    st["exp_avg_sq"] = torch.zeros_like(p)
                st["step"] += 1
                K.adamw_step(p, p.grad.contiguous(), st["exp_avg"], st["exp_avg_sq"],
                             group["lr"], beta1, beta2, group["eps"], group["weight_decay"],
                             st["step"])
        return loss
