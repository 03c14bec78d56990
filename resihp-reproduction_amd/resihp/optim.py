"""Parameter updates on the HIP kernels: AdamW (the reference's one optimizer) and SGD.

``AdamW`` restates ``torch.optim.AdamW`` as configured by
``resihp.reference.adamw`` (resihp/reference.py:20-38): decoupled weight decay,
then the Adam moments, then the bias-corrected step.  Its per-parameter state
keeps the names and types torch uses (``exp_avg``, ``exp_avg_sq`` in the
parameter's dtype, ``step`` as a CPU float32 scalar tensor), so state digests
and checkpoints read it the same way.  ``SGD`` is the plain update used by the
one-step tiny-model configuration.
"""

import torch

from . import _hip as H


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        if lr < 0 or eps < 0 or not (0 <= betas[0] < 1 and 0 <= betas[1] < 1) or weight_decay < 0:
            raise ValueError("invalid AdamW hyperparameters")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

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
                H.require_gpu(p, p.grad)
                if p.grad.is_sparse:
                    raise RuntimeError("AdamW does not support sparse gradients")
                state = self.state[p]
                if not state:
                    state["step"] = torch.tensor(0.0, dtype=torch.float32)
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                state["step"] += 1
                step = float(state["step"])
                grad = p.grad.contiguous()
                H.call("rh_adamw_step", H.dtype_code(p), p.numel(), p.data_ptr(), grad.data_ptr(),
                       state["exp_avg"].data_ptr(), state["exp_avg_sq"].data_ptr(), group["lr"], beta1, beta2,
                       group["eps"], group["weight_decay"], 1.0 - beta1 ** step, 1.0 - beta2 ** step,
                       H.stream_of(p))
        return loss


class SGD(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, weight_decay=0.0):
        if lr < 0 or weight_decay < 0:
            raise ValueError("invalid SGD hyperparameters")
        super().__init__(params, dict(lr=lr, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                H.require_gpu(p, p.grad)
                grad = p.grad.contiguous()
                H.call("rh_sgd_step", H.dtype_code(p), p.numel(), p.data_ptr(), grad.data_ptr(), group["lr"],
                       group["weight_decay"], H.stream_of(p))
        return loss
