"""CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Torch-CPU restatement of FusionLLM's DeepSeekMoE (models/moe.py) and of the
block wiring used by config C4 (models/fusionllm.py:50-53), plus wrappers of
the C restatement of the router and dispatch (router_ref.c).

Every function follows the reference op by op, in the reference's dtypes:
  swiglu          moe.py:20-21   w2(silu(w1 x) * w3 x), bias-free Linears
  route           moe.py:44-50   gate -> sigmoid -> topk -> normalise
  dispatch_combine moe.py:52-77  argsort, unique_consecutive, cumsum, per-expert
                                 loop in ascending expert order, fp32 index_add_,
                                 .to(x.dtype)
  moe_forward     moe.py:79-87   view, route, routed + shared, view back
  block_forward   fusionllm.py:50-53 (ffn half) x + moe(RMSNorm(x)), eps 1e-6
  gate_bias_step  moe.py:89-98   bincount, 1.10/0.90 x mean thresholds, masked +-speed
  load_balance_loss moe.py:100-109 E * sum(f * P) with one-hot P
  normuon_step    training/optimizer.py:18-58 NorMuon.step on one parameter
  router_dlogits  autograd of moe.py:46-49 for the selected scores, fp32 numpy
                  in the order the router backward kernel computes it
Router modes:
  "module" — the reference exactly: logits and scores in the module dtype,
             torch.topk (its own tie order);
  "fp32"   — the build's router: fp32 logits from the same (bf16) operands,
             exact ties to the lowest index (stable descending sort), fp32
             weights.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch
import torch.nn.functional as F

from . import c_oracle


def swiglu(x, w1, w3, w2):
    """SwiGLUExpert.forward, models/moe.py:20-21."""
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w3), w2)


def topk_lowest_index(scores: torch.Tensor, k: int):
    """Top-k, descending, exact ties (and NaNs) to the lowest index."""
    vals, order = torch.sort(scores, dim=-1, descending=True, stable=True)
    return vals[..., :k], order[..., :k]


def route(x, gate_w, gate_b, k: int, route_scale: float = 1.0, mode: str = "fp32", indices=None):
    """DeepSeekMoE._route, models/moe.py:44-50.

    ``indices`` (mode "fp32" only) fixes the selection — e.g. to the GPU's —
    and keeps the weights differentiable: topk's backward scatters into the
    selected scores, which is what gathering them does.
    """
    wide = torch.float64 if x.dtype == torch.float64 else torch.float32  # fp64 ground truth stays fp64
    if indices is not None:
        if mode != "fp32":
            raise ValueError("indices= needs mode='fp32'")
        scores = torch.sigmoid(F.linear(x.to(wide), gate_w.to(wide), gate_b.to(wide)))
        weights = scores.gather(-1, indices.long())
        weights = weights / (weights.sum(dim=-1, keepdim=True) + 1e-10) * route_scale
        return weights, indices.long()
    if mode == "module":
        logits = F.linear(x, gate_w, gate_b)                     # moe.py:46
        scores = torch.sigmoid(logits)                            # moe.py:47
        weights, indices = torch.topk(scores, k=k, dim=-1)        # moe.py:48
    elif mode == "fp32":
        logits = F.linear(x.to(wide), gate_w.to(wide), gate_b.to(wide))
        scores = torch.sigmoid(logits)
        weights, indices = topk_lowest_index(scores, k)
    else:
        raise ValueError(mode)
    weights = weights / (weights.sum(dim=-1, keepdim=True) + 1e-10) * route_scale  # moe.py:49
    return weights, indices


def dispatch_combine(x, weights, indices, experts, n_experts: int, acc_dtype=torch.float32):
    """DeepSeekMoE._dispatch_scatter_gather, models/moe.py:52-77.

    ``experts`` is a list of (w1, w3, w2).  The sort is torch.argsort
    (stable above 32768 slots on CPU, as in the reference); outputs do not
    depend on the order inside an expert because each token appears at most
    once per expert.  ``acc_dtype`` is the reference's fp32 accumulator
    (moe.py:65); fp64 is used only for gradcheck.
    """
    T, topk = x.size(0), weights.size(1)
    flat_indices = indices.flatten()
    flat_weights = weights.flatten().unsqueeze(-1)
    flat_token_ids = torch.arange(T, device=x.device).repeat_interleave(topk)
    sort_idx = flat_indices.argsort()
    flat_indices_sorted = flat_indices[sort_idx]
    flat_weights_sorted = flat_weights[sort_idx]
    flat_token_ids_sorted = flat_token_ids[sort_idx]
    unique_experts, counts = torch.unique_consecutive(flat_indices_sorted, return_counts=True)
    starts = torch.zeros_like(counts)
    starts[1:] = counts.cumsum(0)[:-1]
    y = torch.zeros(T, x.size(1), dtype=acc_dtype, device=x.device)
    for i in range(unique_experts.size(0)):
        e = int(unique_experts[i])
        if e >= n_experts:
            continue
        start, count = int(starts[i]), int(counts[i])
        if count == 0:
            continue
        tok = flat_token_ids_sorted[start:start + count]
        w = flat_weights_sorted[start:start + count]
        out = swiglu(x[tok], *experts[e])
        y.index_add_(0, tok, (out * w).to(y.dtype))
    return y.to(x.dtype)


def moe_forward(x, gate_w, gate_b, experts, shared, k: int, route_scale: float = 1.0,
                mode: str = "fp32", routing=None, acc_dtype=torch.float32):
    """DeepSeekMoE.forward, models/moe.py:79-87.

    Returns (y, weights, indices).  ``routing=(weights, indices)`` replaces
    the router (used to run the expert and combine stages on exactly the
    routing the GPU produced).
    """
    shape = x.shape
    flat = x.reshape(-1, x.shape[-1])
    if routing is None:
        weights, indices = route(flat, gate_w, gate_b, k, route_scale, mode)
    else:
        weights, indices = routing
    y_routed = dispatch_combine(flat, weights, indices, experts, len(experts), acc_dtype)
    y_shared = swiglu(flat, *shared) if shared is not None else 0.0
    return (y_routed + y_shared).view(shape), weights, indices


def rms_norm(x, weight, eps: float = 1e-6):
    """nn.RMSNorm(dim, eps=1e-6) of models/fusionllm.py:48."""
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


def block_forward(x, norm_w, moe_args: dict):
    """FFN half of FusionLLMBlock.forward, models/fusionllm.py:52."""
    y, _, _ = moe_forward(rms_norm(x, norm_w), **moe_args)
    return x + y


def gate_bias_step(bias, indices, n_experts: int, speed: float = 0.001):
    """DeepSeekMoE.update_gate_bias, models/moe.py:89-98; returns the new bias."""
    b = bias.detach().clone()
    load = torch.bincount(indices.flatten(), minlength=n_experts).float()
    mean = load.mean()
    b[load > mean * 1.10] -= speed
    b[load < mean * 0.90] += speed
    return b


def load_balance_loss(indices, weights, n_experts: int):
    """DeepSeekMoE.get_load_balance_loss, models/moe.py:100-109."""
    T, k = weights.shape
    flat = indices.flatten()
    load = torch.bincount(flat, minlength=n_experts).float()
    frac = load / (load.sum() + 1e-10)
    onehot = F.one_hot(flat, num_classes=n_experts).float()
    prob = (onehot * weights.flatten().unsqueeze(-1)).view(T, k, n_experts).sum(dim=1).mean(dim=0)
    return (frac * prob).sum() * n_experts


@torch.no_grad()
def normuon_step(p, grad, state: dict, lr: float = 0.02, betas=(0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.1, cautious_wd: bool = True, ops: bool = False):
    """NorMuon.step for one parameter, training/optimizer.py:18-58, op by op;
    updates p and state in place.

    fp32 (and ``ops=True`` for any dtype and device): the reference's tensor
    operations as written.  bf16: the same operations as torch runs them on
    the GPU (where the reference trains): fp32 arithmetic with the Python
    scalars in fp32, each result rounded to bf16, "a + s*b" as one fused
    multiply-add, and a tensor divided by a Python number as a product with
    the number's fp32 reciprocal (torch's CUDA div_true kernel does that for a
    CPU-scalar divisor: inv = 1.0f / float(b)).  (torch's CPU kernels instead
    round the alpha/value scalars of add_/addcmul_ to bf16, which changes
    about a fifth of the first step's exp_avg elements.)
    """
    beta1, beta2 = betas
    if len(state) == 0:
        state["step"] = 0
        state["exp_avg"] = torch.zeros_like(grad)
        state["exp_avg_sq"] = torch.zeros_like(grad)
    exp_avg, exp_avg_sq = state["exp_avg"], state["exp_avg_sq"]
    state["step"] += 1
    step_count = state["step"]
    bias_corr1 = 1.0 - beta1 ** step_count
    bias_corr2 = 1.0 - beta2 ** step_count
    if p.dtype == torch.bfloat16 and not ops:
        _normuon_bf16(p, grad, exp_avg, exp_avg_sq, lr, beta1, beta2, eps, weight_decay, cautious_wd,
                      bias_corr1, bias_corr2)
        return
    exp_avg.mul_(beta1).add_(grad, alpha=1.0 - beta1)
    exp_avg_sq.mul_(beta2).addcmul_(grad, grad, value=1.0 - beta2)
    denom = (exp_avg_sq.sqrt() / (bias_corr2 ** 0.5)).add_(eps)
    update = exp_avg / bias_corr1 / denom
    if p.ndim >= 2:
        row_norm = update.norm(p=2, dim=-1, keepdim=True)
        row_rms = row_norm / (update.size(-1) ** 0.5 + eps)
        update = update / (row_rms + eps)
    if weight_decay > 0:
        if cautious_wd and p.ndim >= 2:
            mask = (grad * p).sign() == 1.0
            p.mul_(1.0 - lr * weight_decay * mask.to(p.dtype))
        else:
            p.mul_(1.0 - lr * weight_decay)
    p.add_(update, alpha=-lr)


def _normuon_bf16(p, grad, exp_avg, exp_avg_sq, lr, beta1, beta2, eps, weight_decay, cautious_wd,
                  bias_corr1, bias_corr2):
    f32 = lambda v: torch.tensor(v, dtype=torch.float32)  # a Python scalar as the GPU kernels see it
    inv = lambda v: f32(1.0) / f32(v)  # a Python divisor: its fp32 reciprocal, then a product
    r = lambda t: t.to(torch.bfloat16).float()             # round an operation's result to bf16
    fma = lambda a, b, c: (a.double() * b.double() + c.double()).float()
    g, w = grad.float(), p.float()
    m = r(fma(f32(1.0 - beta1), g, r(exp_avg.float() * f32(beta1))))
    v = r(fma(f32(1.0 - beta2) * g, g, r(exp_avg_sq.float() * f32(beta2))))
    denom = r(r(r(v.sqrt()) * inv(bias_corr2 ** 0.5)) + f32(eps))
    update = r(r(m * inv(bias_corr1)) / denom)
    if p.ndim >= 2:
        row_norm = r(update.double().pow(2).sum(-1, keepdim=True).sqrt().float())
        row_rms = r(row_norm * inv(update.size(-1) ** 0.5 + eps))
        update = r(update / r(row_rms + f32(eps)))
    if weight_decay > 0:
        if cautious_wd and p.ndim >= 2:
            mask = (r(g * w) > 0).float()
            w = r(w * r(1.0 - r(f32(lr * weight_decay) * mask)))
        else:
            w = r(w * f32(1.0 - lr * weight_decay))
    w = r(fma(f32(-lr), update, w))
    exp_avg.copy_(m)
    exp_avg_sq.copy_(v)
    p.copy_(w)


# ---- C restatement wrappers -------------------------------------------------------

def _u16(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))


def router_c(x, gate_w, gate_b, k: int, route_scale: float = 1.0, want_scores: bool = False):
    """Bit-exact CPU model of the gfx950 router (router_ref.c) on bf16 operands.

    Returns int32 idx [T,k], fp32 weights [T,k], fp32 topv [T,k] and, if
    asked, fp32 logits and scores [T,E].
    """
    lib = c_oracle()
    xs, ws, bs = _u16(x), _u16(gate_w), _u16(gate_b)
    T, d = x.shape
    E = gate_w.shape[0]
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    v = np.empty((T, k), np.float32)
    lg = np.empty((T, E), np.float32) if want_scores else None
    sc = np.empty((T, E), np.float32) if want_scores else None
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p) if a is not None else None
    rc = lib.oracle_router_fwd(P(xs), P(ws), P(bs), T, d, E, k, float(route_scale), P(idx), P(w), P(v),
                               P(lg), P(sc))
    if rc != 0:
        raise ValueError("oracle_router_fwd: unsupported shape")
    out = [torch.from_numpy(idx), torch.from_numpy(w), torch.from_numpy(v)]
    if want_scores:
        out += [torch.from_numpy(lg), torch.from_numpy(sc)]
    return tuple(out)


def dispatch_c(idx: torch.Tensor, n_experts: int):
    """Counting-sort dispatch (router_ref.c): counts, offsets, perm, pos_of_slot (int32)."""
    lib = c_oracle()
    a = np.ascontiguousarray(idx.to(torch.int32).numpy())
    T, k = a.shape
    counts = np.empty(n_experts, np.int32)
    offsets = np.empty(n_experts + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    pos = np.empty(T * k, np.int32)
    P = lambda z: z.ctypes.data_as(ctypes.c_void_p)
    if lib.oracle_dispatch(P(a), T, n_experts, k, P(counts), P(offsets), P(perm), P(pos)) != 0:
        raise ValueError("expert index out of range")
    return tuple(torch.from_numpy(z) for z in (counts, offsets, perm, pos))


def router_dlogits(d_w: np.ndarray, topv: np.ndarray, route_scale: float) -> np.ndarray:
    """dL/dlogit for each selected expert, fp32 [T, k]: the autograd of
    w = v / (sum_j v_j + 1e-10) * route_scale (moe.py:49) followed by the
    top-k scatter (moe.py:48) and the sigmoid backward (moe.py:47) of the
    selected logits, per token with the sums over j in ascending order:
      D = (v_0 + v_1 + ...) + 1e-10,   dq_j = dw_j * rs,
      dS = 0 - (dq_0 v_0)/(D D) - (dq_1 v_1)/(D D) - ...,
      dv_j = dq_j / D + dS,   dlogit_j = (dv_j * (1 - v_j)) * v_j.
    Every operation is a single IEEE fp32 operation (no fused multiply-add)."""
    dw = np.asarray(d_w, np.float32)
    v = np.asarray(topv, np.float32)
    k = v.shape[1]
    rs = np.float32(route_scale)
    s = v[:, 0].copy()
    for j in range(1, k):
        s = (s + v[:, j]).astype(np.float32)
    D = (s + np.float32(1e-10)).astype(np.float32)
    DD = (D * D).astype(np.float32)
    dS = np.zeros_like(D)
    for j in range(k):
        dq = (dw[:, j] * rs).astype(np.float32)
        dS = (dS - ((dq * v[:, j]).astype(np.float32) / DD).astype(np.float32)).astype(np.float32)
    out = np.empty_like(v)
    for j in range(k):
        dq = (dw[:, j] * rs).astype(np.float32)
        dv = ((dq / D).astype(np.float32) + dS).astype(np.float32)
        out[:, j] = ((dv * (np.float32(1.0) - v[:, j]).astype(np.float32)).astype(np.float32) * v[:, j]).astype(np.float32)
    return out


def expf_c(x: float) -> float:
    return float(c_oracle().oracle_expf(float(x)))


def sigmoid_c_vec(x: np.ndarray) -> np.ndarray:
    lib = c_oracle()
    return np.array([lib.oracle_sigmoid(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))
