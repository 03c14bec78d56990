"""Parameter updates on the HIP kernels: AdamW (the reference's one optimizer) and SGD.

``AdamW`` restates ``torch.optim.AdamW`` as configured by
``resihp.reference.adamw`` (resihp/reference.py:20-38): decoupled weight decay,
then the Adam moments, then the bias-corrected step, for every parameter in one
multi-tensor launch.  Its per-parameter state keeps the names and types torch
uses (``exp_avg``, ``exp_avg_sq`` in the parameter's dtype, ``step`` as a
float32 scalar tensor -- on the device, as torch's capturable AdamW keeps it),
so state digests and checkpoints read it the same way.  ``SGD`` is the plain update used by the
one-step tiny-model configuration.
"""

import torch

from . import _hip as H


class AdamW(torch.optim.Optimizer):
    """torch.optim.AdamW on the GPU: every parameter of a dtype updated by one rh_adamw_multi call
    (one launch per 64 tensors), with each parameter's step count kept on the device."""

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
            by_dtype: dict = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                H.require_gpu(p, p.grad)
                if p.grad.is_sparse:
                    raise RuntimeError("AdamW does not support sparse gradients")
                if not p.is_contiguous():
                    raise ValueError("AdamW updates contiguous parameters only")
                state = self.state[p]
                if not state:
                    # device step count (torch's capturable form), moments in the parameter's dtype
                    state["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                grad = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
                entry = H.rh_adamw_tensor(p.data_ptr(), grad.data_ptr(), state["exp_avg"].data_ptr(),
                                          state["exp_avg_sq"].data_ptr(), state["step"].data_ptr(), p.numel())
                by_dtype.setdefault((H.dtype_code(p), p.device), []).append((entry, grad))
            for (code, dev), items in by_dtype.items():
                arr = (H.rh_adamw_tensor * len(items))(*[e for e, _ in items])
                H.call("rh_adamw_multi", code, len(items), arr, group["lr"], beta1, beta2, group["eps"],
                       group["weight_decay"], torch.cuda.current_stream(dev).cuda_stream)
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
