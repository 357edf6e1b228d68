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


def bf16_ulp(t: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at the magnitude of each element (fp64)."""
    m = t.double().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(m)) - 7)




def close_block_output(y, y_ref, y_truth, terms_fn, k, rtol, atol, max_frac=1e-5, label=""):
    """The block output against the reference's bf16 composition y_ref:
    within rtol/atol elementwise, except where the terms of an output element
    cancel.  The reference rounds each expert's output and its weighted copy,
    the routed sum and the shared output to bf16 before the final bf16 add
    (models/moe.py:75-77,86-87); a last-bit difference in a term of magnitude
    ~1 survives a cancellation to a result of magnitude ~0.01.  Such elements
    (at most max_frac of them) must lie within the rounding bound of that
    composition from the exact result y_truth (fp32 arithmetic on the same
    bf16 operands and routing): rtol/atol plus (k + 3) / 2 bf16 ulps of the
    largest term (k weighted expert outputs, the routed sum, the shared
    output, the sum: half an ulp each).  terms_fn(rows) returns, for those
    token rows, the fp32 terms [rows, k + 1, d]: the k weighted expert
    outputs and the shared output.  Prints and returns the number of
    elements that needed that bound."""
    a, b, t = y.double().cpu(), y_ref.double().cpu(), y_truth.double().cpu()
    err = (a - b).abs()
    bad = err > atol + rtol * b.abs()
    n_bad = int(bad.sum())
    # how many elements needed the cancellation bound (reported for every call)
    print(f"[close_block_output] {label}: {n_bad} of {bad.numel()} elements outside rtol {rtol} / atol {atol} "
          f"of the bf16 reference ({n_bad / max(bad.numel(), 1):.2e}; limit {max_frac:.0e})", flush=True)
    if not bad.any():
        return 0
    assert float(bad.double().mean()) <= max_frac, (f"{int(bad.sum())}/{bad.numel()} elements out of tolerance "
                                                    f"(rtol={rtol}, atol={atol}); max abs err {float(err.max()):.3e}")
    rows = bad.any(-1).nonzero().flatten()
    terms = terms_fn(rows).double()
    big = torch.maximum(terms.abs().amax(1), terms[:, :k].sum(1).abs())
    bound = atol + rtol * t[rows].abs() + (k + 3) / 2 * bf16_ulp(big)
    e = (a[rows] - t[rows]).abs()
    over = bad[rows] & (e > bound)
    detail = [(float(a[rows][over][i]), float(b[rows][over][i]), float(t[rows][over][i]), float(big[over][i]))
              for i in range(min(4, int(over.sum())))]
    assert not over.any(), (f"{int(over.sum())} of {int(bad.sum())} elements out of tolerance exceed the rounding "
                            f"bound of the composition; (gpu, ref, truth, largest term): {detail}")
    return n_bad
