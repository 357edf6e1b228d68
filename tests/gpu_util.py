"""Helpers shared by the GPU tests (not collected: no test_ prefix)."""
from __future__ import annotations

import torch

from fusionllm_amd import DeepSeekMoE, configs


def build_module(cfg: configs.BlockConfig, data: configs.BlockData, device, dtype=torch.bfloat16):
    m = DeepSeekMoE(cfg.moe_config())
    m.load_state_dict({k: v.to(dtype) for k, v in data.state_dict().items()})
    return m.to(device=device, dtype=dtype)


def f32_bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int32)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def close(a, b, rtol, atol):
    """allclose with a readable failure message."""
    a, b = a.double().cpu(), b.double().cpu()
    err = (a - b).abs()
    bad = err > atol + rtol * b.abs()
    assert not bad.any(), (f"{int(bad.sum())}/{bad.numel()} elements out of tolerance "
                           f"(rtol={rtol}, atol={atol}); max abs err {float(err.max()):.3e}")
