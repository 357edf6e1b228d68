"""Workload definitions: the MoE block shapes the benchmark and the parity
tests use (C1-C5 below) and a seeded synthetic generator (random-init
weights of the reference architecture; there are no checkpoints or
datasets).

Shapes follow FusionLLM's benchmark config (training/benchmark.py:10-45:
dim 768, 8 routed experts, top-2, 1 shared, moe_inter_dim 2048) and the
DeepSeekMoE constructor keys (models/moe.py:29-34).

Draw order of ``make_block`` (one torch CPU generator, fp32 draws, then cast):
x, gate.weight, for each routed expert (w1, w3, w2), shared (w1, w3, w2),
gate.bias, dy.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class BlockConfig:
    name: str
    tokens: int
    dim: int = 768
    inter: int = 2048
    n_experts: int = 8
    topk: int = 2
    n_shared: int = 1
    route_scale: float = 1.0
    weight_std: float = 0.02
    bias: str = "zero"          # "zero" | "skew" (U(-.1,.1) + 1.5 on e0, e1) | "uniform:<a>"
    x_shape: tuple = ()
    layers: int = 1             # > 1: stack of RMSNorm + MoE + residual blocks

    def moe_config(self) -> dict:
        return {
            "dim": self.dim,
            "n_routed_experts": self.n_experts,
            "n_shared_experts": self.n_shared,
            "n_activated_experts": self.topk,
            "moe_inter_dim": self.inter,
            "route_scale": self.route_scale,
        }

    def flops_fwd_bwd(self) -> float:
        """Algorithmic GEMM FLOPs of one forward + backward (3x forward)."""
        per_tok = 6 * self.dim * self.inter * (self.topk + (1 if self.n_shared else 0))
        return 3.0 * per_tok * self.tokens * self.layers


C1 = BlockConfig("C1-cpu-fp32-fwd", 16384, x_shape=(8, 2048, 768))
C2 = BlockConfig("C2-bf16-fwdbwd-skewed", 16384, bias="skew", x_shape=(8, 2048, 768))
C3 = tuple(BlockConfig(f"C3-decode-M{m}", m, x_shape=(m, 768)) for m in (1, 8, 32, 128))
C4 = BlockConfig("C4-16x(RMSNorm+MoE)", 16384, bias="uniform:0.05", x_shape=(4, 4096, 768), layers=16)
C5 = BlockConfig("C5-d2048-E64-k6", 32768, dim=2048, inter=1408, n_experts=64, topk=6, n_shared=2,
                 bias="uniform:0.1", x_shape=(32768, 2048))
ALL = {c.name: c for c in (C1, C2, *C3, C4, C5)}


@dataclass
class BlockData:
    x: torch.Tensor
    gate_w: torch.Tensor
    gate_b: torch.Tensor
    experts: list = field(default_factory=list)  # [(w1, w3, w2)]
    shared: tuple | None = None
    dy: torch.Tensor | None = None

    def to(self, device=None, dtype=None) -> "BlockData":
        f = lambda t: None if t is None else t.to(device=device, dtype=dtype)
        return BlockData(f(self.x), f(self.gate_w), f(self.gate_b),
                         [tuple(f(w) for w in e) for e in self.experts],
                         tuple(f(w) for w in self.shared) if self.shared is not None else None,
                         f(self.dy))

    def state_dict(self) -> dict:
        """Parameters under the reference's names (models/moe.py:36-40)."""
        sd = {"gate.weight": self.gate_w, "gate.bias": self.gate_b}
        for e, (w1, w3, w2) in enumerate(self.experts):
            sd[f"experts.{e}.w1.weight"] = w1
            sd[f"experts.{e}.w3.weight"] = w3
            sd[f"experts.{e}.w2.weight"] = w2
        if self.shared is not None:
            w1, w3, w2 = self.shared
            sd["shared_expert.w1.weight"] = w1
            sd["shared_expert.w3.weight"] = w3
            sd["shared_expert.w2.weight"] = w2
        return sd


def _bias(cfg: BlockConfig, g: torch.Generator) -> torch.Tensor:
    E = cfg.n_experts
    if cfg.bias == "zero":
        return torch.zeros(E)
    if cfg.bias == "skew":
        b = torch.rand(E, generator=g) * 0.2 - 0.1
        b[:2] += 1.5
        return b
    if cfg.bias.startswith("uniform:"):
        a = float(cfg.bias.split(":")[1])
        return torch.rand(E, generator=g) * (2 * a) - a
    raise ValueError(cfg.bias)


def make_block(cfg: BlockConfig, seed: int = 0, tokens: int | None = None, with_dy: bool = True,
               experts: bool = True) -> BlockData:
    """Seeded synthetic block (fp32 CPU tensors); ``tokens`` overrides the token count."""
    g = torch.Generator().manual_seed(seed)
    T = cfg.tokens if tokens is None else tokens
    d, I, E, s = cfg.dim, cfg.inter, cfg.n_experts, cfg.weight_std
    x = torch.randn(T, d, generator=g)
    gate_w = torch.randn(E, d, generator=g) * s
    ex = []
    if experts:
        for _ in range(E):
            w1 = torch.randn(I, d, generator=g) * s
            w3 = torch.randn(I, d, generator=g) * s
            w2 = torch.randn(d, I, generator=g) * s
            ex.append((w1, w3, w2))
    shared = None
    if cfg.n_shared > 0 and experts:
        shared = (torch.randn(I, d, generator=g) * s, torch.randn(I, d, generator=g) * s,
                  torch.randn(d, I, generator=g) * s)
    gate_b = _bias(cfg, g)
    dy = torch.randn(T, d, generator=g) if with_dy else None
    return BlockData(x, gate_w, gate_b, ex, shared, dy)
