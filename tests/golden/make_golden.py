"""Write tests/golden/moe_golden.npz: input/output vectors of FusionLLM's own
DeepSeekMoE (models/moe.py) on tiny shapes, forward and backward.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden.py /root/reference

Why an import: the bitwise bf16 composition of DeepSeekMoE.forward
(moe.py:76-77,87 rounding points) and of its autograd backward are fixed by
nothing but the reference code itself; every other part of the CPU oracle is
pinned by closed forms, torch ops and brute force (tests/test_oracle.py).
Only models/moe.py is loaded (it imports torch alone), by file path.

Fixture layout: one npz, keys "<case>/<name>".  bf16 tensors are stored as
uint16 bit patterns, fp32 as float32, indices as int64.  Every case records
its inputs (x, dy, parameters under the reference's state_dict names) and the
reference's outputs: y, _last_indices, _last_weights, x.grad and each
parameter's .grad ("none" marker array when the reference leaves it None),
and, from the same module after that forward, the aux outputs:
get_load_balance_loss() (moe.py:100-109) as "aux/loss" and gate.bias after
update_gate_bias(AUX_SPEED) (moe.py:89-98) as "aux/bias_after".
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "moe_golden.npz"
AUX_SPEED = 0.01  # update_gate_bias step recorded by every case

# name: (dtype, T, dim, inter, E, k, n_shared, route_scale, bias mode, seed)
CASES = {
    "bf16_e4k2_shared": (torch.bfloat16, 24, 32, 32, 4, 2, 1, 1.0, "uniform", 1),
    "fp32_e4k2_shared": (torch.float32, 24, 32, 32, 4, 2, 1, 1.0, "uniform", 2),
    "bf16_e6k3_noshared_rs2.5": (torch.bfloat16, 20, 32, 48, 6, 3, 0, 2.5, "skew", 3),
    "bf16_zero_gate_ties": (torch.bfloat16, 8, 32, 32, 8, 2, 1, 1.0, "zero_gate", 4),
}


def load_reference_moe(ref_root: Path):
    path = ref_root / "models" / "moe.py"
    spec = importlib.util.spec_from_file_location("fusionllm_reference_moe", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def make_case(ref, dtype, T, d, I, E, k, n_shared, rs, bias, seed):
    g = torch.Generator().manual_seed(seed)
    cfg = {"dim": d, "n_routed_experts": E, "n_shared_experts": n_shared,
           "n_activated_experts": k, "moe_inter_dim": I, "route_scale": rs}
    m = ref.DeepSeekMoE(cfg)
    sd = {}
    for name, p in m.state_dict().items():
        sd[name] = torch.randn(p.shape, generator=g) * (0.2 if name.startswith("gate") else 0.1)
    if bias == "uniform":
        sd["gate.bias"] = torch.rand(E, generator=g) * 0.2 - 0.1
    elif bias == "skew":
        sd["gate.bias"] = torch.rand(E, generator=g) * 0.2 - 0.1
        sd["gate.bias"][0] += 0.5
    elif bias == "zero_gate":
        sd["gate.weight"] = torch.zeros(E, d)  # muP init zeroes the gate: every score is 0.5
        sd["gate.bias"] = torch.zeros(E)
    m.load_state_dict(sd)
    m = m.to(dtype)
    x = torch.randn(T, d, generator=g).to(dtype).requires_grad_(True)
    dy = torch.randn(T, d, generator=g).to(dtype)
    y = m(x)
    y.backward(dy)
    out = {"x": x, "dy": dy, "y": y, "indices": m._last_indices, "weights": m._last_weights, "dx": x.grad}
    for name, p in m.named_parameters():
        out[f"param/{name}"] = p.detach().clone()  # before update_gate_bias below
        out[f"grad/{name}"] = p.grad if p.grad is not None else torch.zeros(0)
        out[f"gradnone/{name}"] = torch.tensor([p.grad is None])
    # aux outputs from the routing of this forward (models/moe.py:89-109)
    out["aux/loss"] = m.get_load_balance_loss().detach()
    m.update_gate_bias(speed=AUX_SPEED)
    out["aux/bias_after"] = m.gate.bias.detach().clone()
    meta = torch.tensor([T, d, I, E, k, n_shared], dtype=torch.int64)
    out["meta"] = meta
    out["route_scale"] = torch.tensor([rs], dtype=torch.float64)
    return out


def main(argv):
    ref_root = Path(argv[1]) if len(argv) > 1 else Path("/root/reference")
    ref = load_reference_moe(ref_root)
    arrays = {}
    for case, spec in CASES.items():
        for name, t in make_case(ref, *spec).items():
            arrays[f"{case}/{name}"] = to_np(t)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main(sys.argv)
