"""Drop-in NorMuon for the weight matrices (reference: training/optimizer.py:11-58).

Same constructor (params, lr, betas, eps, weight_decay, cautious_wd), the
same per-parameter state ("step", "exp_avg", "exp_avg_sq", so optimizer
checkpoints (training/checkpoint.py:19-40) load either way) and the same
update.  ``step()`` runs the update as fused kernels
(``fmoe_normuon_step``): one launch per 32 tensors of one dtype and step
count reads grad, param, exp_avg and exp_avg_sq once and writes the three
updated tensors once, where the reference issues about fifteen tensor
operations per parameter.  Parameters must be ROCm tensors in bf16 or fp32
with a last dimension that is a multiple of 4 and at most 4096 (every weight
matrix of the reference model); anything else raises.
"""
from __future__ import annotations

import torch
from torch.optim import Optimizer

from . import _kernels as K


class NorMuon(Optimizer):
    """NorMuon: Adam moments, per-row RMS normalisation of the update and
    cautious weight decay (reference: training/optimizer.py:11-58)."""

    def __init__(self, params, lr: float = 0.02, betas: tuple[float, float] = (0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.1, cautious_wd: bool = True):
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, cautious_wd=cautious_wd)
        super().__init__(params, defaults)

    @torch.no_grad()
    def step(self, closure=None):
        loss = closure() if closure is not None else None
        for group in self.param_groups:
            lr, (beta1, beta2) = group["lr"], group["betas"]
            eps, wd, cautious = group["eps"], group["weight_decay"], group["cautious_wd"]
            batches: dict = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                grad = p.grad
                if not p.is_cuda:
                    raise RuntimeError("fusionllm_amd.optim.NorMuon runs on a ROCm device only")
                if p.dtype not in (torch.bfloat16, torch.float32) or grad.dtype != p.dtype:
                    raise NotImplementedError(f"NorMuon step for {p.dtype} parameters with {grad.dtype} grads")
                if not (p.is_contiguous() and grad.is_contiguous()):
                    raise NotImplementedError("NorMuon step needs contiguous parameters and gradients")
                c = p.shape[-1] if p.dim() >= 1 else 1
                if c % 4 != 0 or c > 4096:
                    raise NotImplementedError(f"NorMuon step for last dimension {c} (needs a multiple of 4, <= 4096)")
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = 0
                    state["exp_avg"] = torch.zeros_like(grad)
                    state["exp_avg_sq"] = torch.zeros_like(grad)
                state["step"] += 1
                key = (p.device, p.dtype, state["step"])
                batches.setdefault(key, []).append((p, grad, state["exp_avg"], state["exp_avg_sq"]))
            for (dev, _dtype, step), items in batches.items():
                bias_corr1 = 1.0 - beta1 ** step
                bias_corr2 = 1.0 - beta2 ** step
                with torch.cuda.device(dev):
                    for i in range(0, len(items), K.NORMUON_MAX_TENSORS):
                        chunk = items[i:i + K.NORMUON_MAX_TENSORS]
                        K.normuon_step([t[0] for t in chunk], [t[1] for t in chunk], [t[2] for t in chunk],
                                       [t[3] for t in chunk], lr, beta1, beta2, eps, wd, cautious,
                                       bias_corr1, bias_corr2)
        return loss
