"""Drop-in DeepSeekMoE for MI355X: the reference module's interface over the
gfx950 kernels of libfusionmoe.so.

Mirrors FusionLLM ``models/moe.py``:
  * ``SwiGLUExpert`` (moe.py:11-21) — same parameters (w1, w2, w3, bias-free
    nn.Linear) and the same forward; it is a parameter container for
    ``DeepSeekMoE`` and is also imported on its own by the reference's MTP
    module (models/mtp.py:11,28), where its forward runs the one-group
    kernels (``dense_swiglu``), as does ``DenseFFN`` (models/fusionllm.py:17-27).
  * ``DeepSeekMoE`` (moe.py:24-109) — same constructor and config keys
    (moe.py:27-42), parameter names and init, ``forward`` (moe.py:79-87),
    ``update_gate_bias`` (moe.py:89-98), ``get_load_balance_loss``
    (moe.py:100-109), and the ``_last_indices`` / ``_last_weights``
    attributes (moe.py:41-42,83-84).

``DeepSeekMoE.forward`` runs only on a ROCm device, through the kernels; it
raises on CPU tensors (there is no CPU fallback).  Numerics follow the
reference composition with one deliberate change: the router accumulates the
gate logits in fp32 from the bf16 operands (instead of rounding logits and
scores to bf16) and breaks exact score ties toward the lowest expert index.
The combine uses the router's fp32 weights; ``_last_weights`` reports them in
the dtype the reference's scores have (bf16 under autocast or for a bf16
module).

Dtypes (the products always run on bf16 operands with fp32 accumulation):
  * a bf16 module with bf16 input: bf16 output;
  * any module under ``torch.autocast("cuda", dtype=torch.bfloat16)`` (the
    reference trainer's mode, training/trainer.py:158): output in the input's
    dtype (bf16 or fp32), as the reference's ``y_routed.to(x.dtype) +
    y_shared`` promotes there;
  * an fp32 module with fp32 input outside autocast (the trainer's
    ``dtype: fp32`` mode, trainer.py:31,158, and its evaluation,
    trainer.py:332 -> validation.py:53): the operands are cast to bf16 in one
    launch, and the output and every gradient come back in fp32.
Gradients always come back in each parameter's own dtype.  A module and
input of different dtypes outside autocast raise, as the reference's
``nn.Linear`` does.
"""
from __future__ import annotations

import collections
import contextlib

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _kernels as K


def _as_bf16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


def _bf16_operands(ts: list) -> list:
    """Contiguous bf16 versions of the block's operands: bf16 ones as they
    are, contiguous fp32 ones converted together in one launch (the casts
    autocast would make one nn.Linear at a time), anything else by .to()."""
    out = list(ts)
    idx = []
    for i, t in enumerate(ts):
        if t.dtype == torch.bfloat16:
            out[i] = t.contiguous()
        elif t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0:
            idx.append(i)
        else:
            out[i] = t.to(torch.bfloat16).contiguous()
    if idx:
        for i, c in zip(idx, K.cast_bf16([ts[i] for i in idx])):
            out[i] = c
    return out


_DENSE_OFFSETS: dict = {}


def _dense_offsets(T: int, device: torch.device) -> torch.Tensor:
    """Group offsets [0, T] (int32, on the device) of a one-group product."""
    key = (T, device)
    off = _DENSE_OFFSETS.get(key)
    if off is None:
        if len(_DENSE_OFFSETS) > 256:
            _DENSE_OFFSETS.clear()
        off = torch.tensor([0, T], dtype=torch.int32, device=device)
        _DENSE_OFFSETS[key] = off
    return off


class _DenseSwiGLUFunction(torch.autograd.Function):
    """w2(silu(w1 x) * w3 x) on the grouped kernels with one group of all T
    rows (the dense FFN of models/fusionllm.py:17-27 and the SwiGLU of
    models/moe.py:11-21 used on its own, models/mtp.py:28): the gate/up product
    with the SiLU*up epilogue, the down product, and their backward (dX with
    the SwiGLU backward fused, dW1/dW3/dW2).  Output in out_dtype (bf16 as
    the bf16 Linears give, fp32 for an fp32 module outside autocast); input
    and weight gradients in their own dtypes."""

    @staticmethod
    def forward(ctx, x, w1, w3, w2, out_dtype):
        T, d = x.shape
        inter = w1.shape[0]
        xb, w1b, w3b, w2b = _bf16_operands([x, w1, w3, w2])
        off = _dense_offsets(T, x.device)
        ab, h = K.gateup_fwd(xb, None, off, 1, [w1b], [w3b], inter)
        y = K.down_fwd(h, off, 1, T, 0, [w2b], d)
        ctx.save_for_backward(xb, ab, h, w1b, w3b, w2b, off)
        ctx.dtypes = (x.dtype, w1.dtype, w3.dtype, w2.dtype)
        return y if out_dtype == torch.bfloat16 else y.to(out_dtype)

    @staticmethod
    def backward(ctx, dy):
        xb, ab, h, w1b, w3b, w2b, off = ctx.saved_tensors
        return (*_dense_backward(dy, xb, ab, h, w1b, w3b, w2b, off, ctx.dtypes, ctx.needs_input_grad[0]), None)


def _dense_backward(dy, xb, ab, h, w1b, w3b, w2b, off, dtypes, need_dx):
    """Backward kernels of the one-group SwiGLU: (dx or None, dw1, dw3, dw2)
    in the dtypes (x, w1, w3, w2) of dtypes."""
    x_dtype, w1_dtype, w3_dtype, w2_dtype = dtypes
    T, d = xb.shape
    inter = w1b.shape[0]
    dyb = _as_bf16(dy).contiguous()
    d_ab = K.down_bwd_dx(dyb, None, off, 1, [w2b], ab, inter)
    dw2 = torch.empty(d, inter, dtype=w2_dtype, device=xb.device)
    K.weight_grad(dyb, None, h, None, off, 1, T, 0, d, [dw2], None, w2_dtype, tag="w2")
    dx = None
    if need_dx:
        dx = K.gateup_bwd_dx(d_ab, off, 1, T, 0, [w1b], [w3b], d)
        if dx.dtype != x_dtype:
            dx = dx.to(x_dtype)
    dw1 = torch.empty(inter, d, dtype=w1_dtype, device=xb.device)
    dw3 = torch.empty(inter, d, dtype=w1_dtype, device=xb.device)
    K.weight_grad(d_ab, None, xb, None, off, 1, T, 0, inter, [dw1], [dw3], w1_dtype, tag="w13")
    if w3_dtype != w1_dtype:
        dw3 = dw3.to(w3_dtype)
    return dx, dw1, dw3, dw2


def _uniform_dtype(what: str, tensors) -> torch.dtype:
    """Outside autocast: the one dtype (bf16 or fp32) of the input and every
    parameter.  Mixed dtypes raise, as the reference's nn.Linear does
    ("expected mat1 and mat2 to have the same dtype")."""
    dts = {t.dtype for t in tensors}
    if len(dts) != 1:
        names = ", ".join(sorted(str(d) for d in dts))
        raise RuntimeError(f"{what}: input and parameters must have the same dtype outside autocast (got {names})")
    dt = dts.pop()
    if dt not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f"{what} supports bf16 and fp32 tensors (got {dt})")
    return dt


def _autocast_check(what: str, x: torch.Tensor) -> None:
    if torch.get_autocast_dtype("cuda") != torch.bfloat16:
        raise NotImplementedError(f"{what} supports bf16 autocast only")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f"unsupported input dtype {x.dtype}")


def dense_swiglu(x: torch.Tensor, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """``w2(silu(w1 x) * w3 x)`` for bias-free nn.Linear weights (w1, w3
    [inter, dim], w2 [dim, inter]) on the kernels; any leading shape of x.

    Under ``torch.autocast("cuda", dtype=torch.bfloat16)`` the output is bf16,
    as the reference's Linears give there.  Outside autocast the input and
    weights share one dtype: bf16 gives bf16; fp32 runs the same bf16 kernels
    on bf16 copies and returns fp32 (output and gradients).  ROCm tensors only.
    """
    dim = w1.shape[1]
    shape = x.shape
    flat = x.reshape(-1, dim)
    if not flat.is_cuda:
        raise RuntimeError("fusionllm_amd SwiGLU runs on a ROCm device only (got a CPU tensor)")
    if torch.is_autocast_enabled("cuda"):
        _autocast_check("fusionllm_amd SwiGLU", flat)
        out_dtype = torch.bfloat16
    else:
        out_dtype = _uniform_dtype("fusionllm_amd SwiGLU", (flat, w1, w3, w2))
    if flat.shape[0] == 0:
        y = flat.new_zeros(0, dim, dtype=out_dtype)
        return (y + (w1.sum() + w3.sum() + w2.sum()).to(y.dtype) * 0 + flat.sum().to(y.dtype) * 0).view(shape)
    switch = flat.device.index != torch._C._cuda_getDevice()
    with torch.cuda.device(flat.device) if switch else contextlib.nullcontext():
        y = _DenseSwiGLUFunction.apply(flat, w1, w3, w2, out_dtype)
    return y.view(*shape[:-1], w2.shape[0])


class SwiGLUExpert(nn.Module):
    """SwiGLU expert w2(silu(w1 x) * w3 x) (reference: models/moe.py:11-21).

    Inside ``DeepSeekMoE`` it only holds the expert's parameters (the block
    runs all experts in grouped kernels).  Called on its own (the reference's
    MTP module does, models/mtp.py:28), its forward runs the one-group
    kernels of ``dense_swiglu``.
    """

    def __init__(self, dim: int, inter_dim: int):
        super().__init__()
        self.w1 = nn.Linear(dim, inter_dim, bias=False)
        self.w2 = nn.Linear(inter_dim, dim, bias=False)
        self.w3 = nn.Linear(dim, inter_dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w1, w3, w2 = self.w1.weight, self.w3.weight, self.w2.weight
        if torch.compiler.is_compiling():
            # traced (torch.compile): the fusionllm::swiglu_fwd operator
            flat = x.reshape(-1, w1.shape[1])
            y = torch.ops.fusionllm.swiglu_fwd(flat, w1, w3, w2)[0]
            if not torch.is_autocast_enabled("cuda") and x.dtype == torch.float32:
                y = y.float()  # fp32 module outside autocast: fp32 output
            return y.view(*x.shape[:-1], w2.shape[0])
        return dense_swiglu(x, w1, w3, w2)


class DenseFFN(SwiGLUExpert):
    """Dense SwiGLU FFN of the GDN layers (reference: models/fusionllm.py:17-27),
    same parameters (w1, w2, w3) and forward as the reference, on the
    one-group kernels."""


# Whether the training forward reads the routed token rows of x through the
# dispatch's permutation in the tiled products (gate/up forward, dW1|dW3)
# instead of writing the gathered copy x_perm.  Measured on one MI355X at C2
# (16384 tokens, both variants in one session): dropping the copy saves 11 us
# in the dispatch, but the gate/up forward reading rows through perm takes
# 9-14 us longer and dW1|dW3 18-21 us longer (scattered 128-byte row pieces
# instead of consecutive rows), so the block keeps x_perm.  The entry points
# keep the option (fmoe_gateup_fwd, fmoe_weight_grad): it saves T*k*dim*2
# bytes of HBM.
GATHER_ROWS = False


def gathers_rows(T: int, k: int, has_shared: bool) -> bool:
    """Whether the block reads the routed token rows of x through perm (no
    x_perm): only with GATHER_ROWS, and only for launches of more than
    SMALL_LAUNCH_ROWS rows (the tiled products; the small-group kernels read
    x_perm)."""
    return GATHER_ROWS and T * k >= 8 and T * k + (T if has_shared else 0) > K.SMALL_LAUNCH_ROWS


def _forward_pass(meta, x, gate_w, gate_b, weights, residual=None, counts_host=None):
    """The forward kernels of DeepSeekMoE.forward (models/moe.py:79-87); returns
    the output and every intermediate the backward pass needs.  With a
    residual the output is residual + moe(x) (models/fusionllm.py:52).
    counts_host (pinned int32 [E], optional) receives the expert counts
    asynchronously: written by the routing kernel itself on the
    route_and_dispatch path, by a copy on the others."""
    E, k, inter, rs, has_shared, out_dtype = meta
    T, d = x.shape
    xb, gwb, gbb, *wb = _bf16_operands([x, gate_w, gate_b, *weights])
    G = E + (1 if has_shared else 0)
    w1s, w3s, w2s = wb[0::3][:G], wb[1::3][:G], wb[2::3][:G]
    gather = gathers_rows(T, k, has_shared)

    if 0 < T <= K.TINY_BATCH and T * E <= 64 and d <= 2048:
        # decode-sized: routing and dispatch in one launch (one workgroup)
        idx, idx64, w, v, counts, offsets, perm, pos, x_perm = K.route_dispatch(xb, gwb, gbb, k, rs)
    elif d <= 2048 and T > K.ROUTER_SMALL_T:
        # routing with the dispatch histogram, scan, scatter with the row copies: three launches.
        # Up to ROUTER_SMALL_T tokens the router's one-workgroup-per-token kernel and the
        # one-launch small dispatch below are faster (C3 replay at 32 tokens: 49 against 55 us).
        # The expert counts reach counts_host from the kernel itself.
        idx, idx64, w, v, counts, offsets, perm, pos, x_perm = K.route_and_dispatch(
            xb, gwb, gbb, k, rs, gather=not gather, counts_host=counts_host)
        counts_host = None
    else:
        idx, idx64, w, v = K.router_fwd(xb, gwb, gbb, k, rs)
        counts, offsets, perm, pos, x_perm = K.dispatch(idx, xb, E, gather=not gather)
    if counts_host is not None:
        counts_host.copy_(counts, non_blocking=True)
    rows_r, rows_s = T * k, (T if has_shared else 0)
    # routed rows: token rows of x through perm (gather), or the gathered copy x_perm
    ab, h = K.gateup_fwd(xb if gather else x_perm, xb if has_shared else None, offsets, E, w1s, w3s, inter,
                         gather=perm if gather else None, k=k)
    o = K.down_fwd(h, offsets, E, rows_r, rows_s, w2s, d)
    y = K.combine_fwd(o, idx, w, pos, rows_r, has_shared, out_dtype, residual)
    return xb, gwb, wb, idx, idx64, w, v, counts, offsets, perm, pos, x_perm, ab, h, o, y


def _host_counts(meta):
    """Pinned host buffer for the forward's expert counts (filled
    asynchronously by _forward_pass and read at the end of backward)."""
    return torch.empty(meta[0], dtype=torch.int32, pin_memory=True)


# (event, pinned tensor) pairs: a kernel writes the tensor before the event
# completes, and torch's caching host allocator does not know of that write,
# so the tensor is held here (and not handed out again) until then, also when
# the autograd context that owns it is dropped early (no backward).
_pending_host_writes = collections.deque()


def _hold_until(ev, t):
    while _pending_host_writes and _pending_host_writes[0][0].query():
        _pending_host_writes.popleft()
    _pending_host_writes.append((ev, t))


def _save_forward(ctx, meta, fw, gate_w, gate_b, weights, counts_host):
    """Keep what the backward kernels read; the expert counts travel to the
    host asynchronously (counts_host, given to _forward_pass) and are read at
    the end of backward.  Returns the tensors to save."""
    xb, gwb, wb, idx, idx64, w, v, counts, offsets, perm, pos, x_perm, ab, h, o, y = fw
    # Experts that get no tokens return None gradients (the reference never
    # puts them in the graph, moe.py:66-72).
    ev = torch.cuda.Event()
    ev.record()
    _hold_until(ev, counts_host)
    ctx.meta = meta
    ctx.counts_host = counts_host
    ctx.counts_event = ev
    ctx.param_dtypes = (gate_w.dtype, gate_b.dtype, [t.dtype for t in weights])
    ctx.mark_non_differentiable(idx64, w, counts)
    # The index, weight and count outputs never carry gradients: do not let
    # autograd fill zero tensors for them.
    ctx.set_materialize_grads(False)
    return (xb, gwb, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, *wb)


def _backward_pass(ctx, saved, dy):
    """Backward kernels of the MoE (autograd of models/moe.py:44-87) up to,
    not including, the per-token input-gradient reduction.  Returns
    (dx_rows, d_logits, dgw, dgb, grads_w) with grads_w per weight, None
    for experts that got no tokens when ctx carries the forward's host copy
    of the expert counts (ctx.counts_host / counts_event), zeros otherwise.
    ctx needs .meta and .param_dtypes."""
    E, k, inter, rs, has_shared, out_dtype = ctx.meta
    xb, gwb, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, *wb = saved
    T, d = xb.shape
    G = E + (1 if has_shared else 0)
    w1s, w3s, w2s = wb[0::3][:G], wb[1::3][:G], wb[2::3][:G]
    rows_r, rows_s = T * k, (T if has_shared else 0)
    gw_dtype, gb_dtype, w_dtypes = ctx.param_dtypes

    # Combine backward: routed rows get dy*w (bf16), slots get <dy, o>.
    d_o, d_w = K.combine_bwd(dy, o, w, perm, k)
    dy_sh = _as_bf16(dy).contiguous() if has_shared else None

    # Down projection: dX with the SwiGLU backward fused (reading w2 as it
    # lies), then dW2.
    d_ab = K.down_bwd_dx(d_o, dy_sh, offsets, E, w2s, ab, inter)
    dw2 = [torch.empty(d, inter, dtype=w_dtypes[3 * g + 2], device=xb.device) for g in range(G)]
    K.weight_grad(d_o, dy_sh, h, None, offsets, E, rows_r, rows_s, d, dw2, None,
                  w_dtypes[2], tag="w2")
    # Gate/up projections: dX (one product over [w1; w3]) then dW1, dW3.
    dx_rows = K.gateup_bwd_dx(d_ab, offsets, E, rows_r, rows_s, w1s, w3s, d)
    dw1 = [torch.empty(inter, d, dtype=w_dtypes[3 * g], device=xb.device) for g in range(G)]
    dw3 = [torch.empty(inter, d, dtype=w_dtypes[3 * g + 1], device=xb.device) for g in range(G)]
    gather = x_perm is None or (x_perm.shape[0] == 0 and rows_r > 0)
    K.weight_grad(d_ab, None, xb if gather else x_perm, xb if has_shared else None, offsets, E, rows_r, rows_s,
                  inter, dw1, dw3, w_dtypes[0], b_gather=perm if gather else None, k=k, tag="w13")
    # Router: logits gradient, gate weight/bias gradient.
    d_logits, dgw, dgb = K.router_bwd(d_w, v, perm, offsets, xb, E, rs, gw_dtype)
    if dgb.dtype != gb_dtype:
        dgb = dgb.to(gb_dtype)

    grads_w = [None] * len(wb)
    counts = None
    if getattr(ctx, "counts_host", None) is not None:
        ctx.counts_event.synchronize()
        counts = ctx.counts_host.tolist()
    # Without the host copy of the counts (the graph-capturable operator)
    # every expert gets its gradient: zeros for experts without rows.
    for g in range(G):
        if counts is not None and g < E and counts[g] == 0:
            continue
        grads_w[3 * g], grads_w[3 * g + 1], grads_w[3 * g + 2] = dw1[g], dw3[g], dw2[g]
    return dx_rows, d_logits, dgw, dgb, grads_w


class _MoEBlockFunction(torch.autograd.Function):
    """Forward and backward of DeepSeekMoE.forward (models/moe.py:79-87) on the kernels.

    Inputs: (meta, x[T,d], gate.weight, gate.bias, *weights) where weights
    are, per routed expert, (w1, w3, w2) and then the shared expert's
    (w1, w3, w2) when it exists.  Outputs: y[T,d], indices[T,k] int64,
    weights[T,k] fp32, expert counts[E] int32 (the last three are not
    differentiable).
    """

    @staticmethod
    def forward(ctx, meta, x, gate_w, gate_b, *weights):
        counts_host = _host_counts(meta)
        fw = _forward_pass(meta, x, gate_w, gate_b, weights, counts_host=counts_host)
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(*_save_forward(ctx, meta, fw, gate_w, gate_b, weights, counts_host))
        idx64, w, counts, y = fw[4], fw[5], fw[7], fw[-1]
        return y, idx64, w, counts

    @staticmethod
    def backward(ctx, dy, _d_idx, _d_w, _d_counts):
        if dy is None:  # y did not reach the loss
            return (None,) * (4 + len(ctx.param_dtypes[2]))
        saved = ctx.saved_tensors
        E, k, inter, rs, has_shared, out_dtype = ctx.meta
        xb, gwb, idx, pos = saved[0], saved[1], saved[2], saved[7]
        dx_rows, d_logits, dgw, dgb, grads_w = _backward_pass(ctx, saved, dy.contiguous())
        dx = None
        if ctx.needs_input_grad[1]:
            dx = K.dx_reduce(dx_rows, pos, idx, d_logits, gwb, idx.shape[0] * k, has_shared, ctx.x_dtype)
        return (None, dx, dgw, dgb, *grads_w)


class _NormMoEResidualFunction(torch.autograd.Function):
    """x + DeepSeekMoE(RMSNorm(x)), the FFN half of FusionLLMBlock.forward
    (models/fusionllm.py:48,52), on the kernels: the norm writes the bf16 MoE
    input, the combine adds the residual, and the backward folds the RMSNorm
    backward and the residual's gradient into the per-token reduction.

    Inputs: (meta, eps, x[T,d], norm.weight or None, gate.weight, gate.bias,
    *weights).  Outputs as _MoEBlockFunction.
    """

    @staticmethod
    def forward(ctx, meta, eps, x, norm_w, gate_w, gate_b, *weights):
        xc = x.contiguous()
        nw = None if norm_w is None else norm_w.contiguous()
        xn, rstd = K.rmsnorm_fwd(xc, nw, eps)
        counts_host = _host_counts(meta)
        fw = _forward_pass(meta, xn, gate_w, gate_b, weights, residual=xc, counts_host=counts_host)
        saved = _save_forward(ctx, meta, fw, gate_w, gate_b, weights, counts_host)
        ctx.has_norm_w = nw is not None
        ctx.save_for_backward(xc, rstd, nw, *saved)
        idx64, w, counts, y = fw[4], fw[5], fw[7], fw[-1]
        return y, idx64, w, counts

    @staticmethod
    def backward(ctx, dy, _d_idx, _d_w, _d_counts):
        n_w = len(ctx.param_dtypes[2])
        if dy is None:
            return (None,) * (6 + n_w)
        xc, rstd, nw, *saved = ctx.saved_tensors
        E, k, inter, rs, has_shared, out_dtype = ctx.meta
        gwb, idx, pos = saved[1], saved[2], saved[7]
        dy = dy.contiguous()
        dx_rows, d_logits, dgw, dgb, grads_w = _backward_pass(ctx, saved, dy)
        want_dw = ctx.has_norm_w and ctx.needs_input_grad[3]
        dx, dnw = K.dx_reduce_norm(dx_rows, pos, idx, d_logits, gwb, idx.shape[0] * k, has_shared,
                                   xc, rstd, nw, dy, want_dw)
        if not ctx.needs_input_grad[2]:
            dx = None
        return (None, None, dx, dnw, dgw, dgb, *grads_w)


class DeepSeekMoE(nn.Module):
    """DeepSeekMoE with aux-loss-free biased sigmoid routing (reference: models/moe.py:24-109)."""

    def __init__(self, config: dict):
        super().__init__()
        self.dim = config["dim"]
        self.n_routed_experts = config["n_routed_experts"]
        self.n_shared_experts = config["n_shared_experts"]
        self.n_activated_experts = config["n_activated_experts"]
        self.moe_inter_dim = config["moe_inter_dim"]
        self.route_scale = config.get("route_scale", 1.0)

        self.gate = nn.Linear(self.dim, self.n_routed_experts, bias=True)
        nn.init.zeros_(self.gate.bias)
        nn.init.normal_(self.gate.weight, std=0.006)
        self.experts = nn.ModuleList(
            [SwiGLUExpert(self.dim, self.moe_inter_dim) for _ in range(self.n_routed_experts)])
        # As in the reference, n_shared_experts > 0 means one shared expert.
        self.shared_expert = SwiGLUExpert(self.dim, self.moe_inter_dim) if self.n_shared_experts > 0 else None
        self._last_indices: torch.Tensor | None = None
        # The router's fp32 weights of the last forward (bit-exact with the
        # C oracle) and the dtype the reference's scores have in the same
        # call; _last_weights converts on first access.
        self._route_weights: torch.Tensor | None = None
        self._score_dtype: torch.dtype | None = None
        self._last_weights = None
        # Per-expert slot counts of the last routing, from the dispatch
        # kernel's histogram, and the indices tensor they were counted from.
        self._last_counts: torch.Tensor | None = None
        self._counts_of: torch.Tensor | None = None

    @property
    def _last_weights(self) -> torch.Tensor | None:
        """Routing weights of the last forward, detached (models/moe.py:84), in
        the dtype the reference's scores have in that call: bf16 for a bf16
        module or under bf16 autocast (the gate Linear's output dtype), fp32
        for an fp32 module outside autocast.  The kernels route in fp32; the
        rounding to bf16 happens here, on first access, so the forward pays
        no extra launch."""
        d = self.__dict__
        w = d.get("_lw")
        if w is None:
            rw = d.get("_route_weights")
            if rw is None:
                return None
            dt = d.get("_score_dtype") or rw.dtype
            w = rw if rw.dtype == dt else rw.to(dt)
            d["_lw"] = w
        return w

    @_last_weights.setter
    def _last_weights(self, value: torch.Tensor | None) -> None:
        # an assigned value is taken as it is (the reference's attribute);
        # item assignments, which torch.compile traces (dict.update it does not)
        d = self.__dict__
        d["_lw"] = value
        d["_route_weights"] = None
        d["_score_dtype"] = None

    def _flat_weights(self) -> list[torch.Tensor]:
        # Direct dict access: nn.Module.__getattr__ per weight dominates the
        # host time of a decode-sized call otherwise.
        ws = []
        mods = list(self.experts._modules.values())
        if self.shared_expert is not None:
            mods.append(self.shared_expert)
        for m in mods:
            sub = m._modules
            ws += [sub["w1"]._parameters["weight"], sub["w3"]._parameters["weight"],
                   sub["w2"]._parameters["weight"]]
        return ws

    def _output_dtype(self, x: torch.Tensor, weights: list[torch.Tensor]) -> torch.dtype:
        """dtype of the block's output (models/moe.py:77,87: ``y_routed.to(x.dtype)
        + y_shared``).  Under bf16 autocast the shared output is bf16, so the
        sum takes x's dtype; outside autocast the module and x share one
        dtype (bf16, or fp32: bf16 kernels on bf16 copies, fp32 results)."""
        if torch.is_autocast_enabled("cuda"):
            _autocast_check("fusionllm_amd.DeepSeekMoE", x)
            return x.dtype
        bf = torch.bfloat16
        gate = self._modules["gate"]._parameters
        gw, gb = gate["weight"], gate["bias"]
        if x.dtype == bf and gw.dtype == bf and gb.dtype == bf and all(w.dtype == bf for w in weights):
            return bf  # the common case, without building a set
        return _uniform_dtype("fusionllm_amd.DeepSeekMoE", (x, gw, gb, *weights))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.view(-1, self.dim)
        if not flat.is_cuda:
            raise RuntimeError("fusionllm_amd.DeepSeekMoE runs on a ROCm device only (got a CPU tensor)")
        weights = self._flat_weights()
        out_dtype = self._output_dtype(flat, weights)
        if flat.shape[0] == 0:
            return self._forward_empty(flat, out_dtype).view(shape)
        return self._run(flat, weights, out_dtype).view(shape)

    def forward_norm_residual(self, x: torch.Tensor, norm: nn.RMSNorm) -> torch.Tensor:
        """``x + self(norm(x))`` in one pass: the FFN half of
        FusionLLMBlock.forward (models/fusionllm.py:52) with its
        ``norm2 = nn.RMSNorm(dim, eps=1e-6)`` (models/fusionllm.py:48).

        The norm's parameters stay in ``norm`` (its weight gets its gradient
        as usual).  Same dtype rules as ``forward``, with x standing for the
        norm's output; a bf16 x needs a bf16 norm weight.
        """
        if tuple(norm.normalized_shape) != (self.dim,):
            raise ValueError(f"norm must normalise the last dimension {self.dim} (got {norm.normalized_shape})")
        shape = x.shape
        flat = x.view(-1, self.dim)
        if not flat.is_cuda:
            raise RuntimeError("fusionllm_amd.DeepSeekMoE runs on a ROCm device only (got a CPU tensor)")
        nw = norm.weight
        if nw is not None and flat.dtype == torch.bfloat16 and nw.dtype != torch.bfloat16:
            raise NotImplementedError("a bf16 input needs a bf16 RMSNorm weight")
        if nw is not None and nw.device != flat.device:
            raise RuntimeError("the RMSNorm weight must be on the input's device")
        weights = self._flat_weights()
        out_dtype = self._output_dtype(flat, weights)
        if flat.shape[0] == 0 or torch.compiler.is_compiling():
            # zero tokens (empty tensors only), or traced: the plain expression
            # around the block's operator
            return x + self.forward(norm(x))
        eps = norm.eps if norm.eps is not None else torch.finfo(flat.dtype).eps
        return self._run(flat, weights, out_dtype, norm_w=nw, eps=float(eps), fused_norm=True).view(shape)

    def _run(self, flat, weights, out_dtype, norm_w=None, eps=0.0, fused_norm=False):
        E, k = self.n_routed_experts, self.n_activated_experts
        if torch.compiler.is_compiling():
            # traced (torch.compile): the block as the fusionllm::moe_fwd operator
            y, idx64, w, counts = torch.ops.fusionllm.moe_fwd(
                flat, self.gate.weight, self.gate.bias, weights, k, float(self.route_scale),
                self.shared_expert is not None, out_dtype)[:4]
            score_dtype = torch.bfloat16 if torch.is_autocast_enabled("cuda") else out_dtype
            self._last_indices, self._last_weights = idx64, w.to(score_dtype)
            self._last_counts, self._counts_of = counts, idx64
            return y
        # Direct dict access to the submodules and parameters: nn.Module's
        # __getattr__ / __setattr__ cost host time a decode-sized call notices.
        mods = self._modules
        gate = mods["gate"]._parameters
        gw, gb = gate["weight"], gate["bias"]
        has_shared = mods.get("shared_expert") is not None  # None is a plain attribute, not in _modules
        meta = (E, k, self.moe_inter_dim, float(self.route_scale), has_shared, out_dtype)
        needs_grad = torch.is_grad_enabled() and (
            flat.requires_grad or gw.requires_grad or gb.requires_grad
            or any(t.requires_grad for t in weights) or (norm_w is not None and norm_w.requires_grad))
        # Switch devices only when needed (the context manager costs host time).
        switch = flat.device.index != torch._C._cuda_getDevice()
        with torch.cuda.device(flat.device) if switch else contextlib.nullcontext():
            if needs_grad and fused_norm:
                y, idx64, w, counts = _NormMoEResidualFunction.apply(meta, eps, flat, norm_w, gw, gb, *weights)
            elif needs_grad:
                y, idx64, w, counts = _MoEBlockFunction.apply(meta, flat, gw, gb, *weights)
            else:
                # inference: the same kernels, nothing kept for a backward pass
                x_in, residual = flat, None
                if fused_norm:
                    residual = flat.contiguous()
                    x_in, _ = K.rmsnorm_fwd(residual, None if norm_w is None else norm_w.contiguous(), eps)
                fw = _forward_pass(meta, x_in, gw, gb, weights, residual)
                idx64, w, counts, y = fw[4], fw[5], fw[7], fw[-1]
        # plain attributes (not parameters, buffers or submodules)
        score_dtype = torch.bfloat16 if torch.is_autocast_enabled("cuda") else out_dtype
        self.__dict__.update(_last_indices=idx64, _route_weights=w, _score_dtype=score_dtype, _lw=None,
                             _last_counts=counts, _counts_of=idx64)
        return y

    def _forward_empty(self, flat: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
        # Zero tokens: nothing to compute.  Keep the output connected to the
        # gate and shared-expert parameters so autograd yields zero (not None)
        # gradients for them, as the reference's empty matmuls do.
        k = self.n_activated_experts
        self._last_indices = torch.empty(0, k, dtype=torch.int64, device=flat.device)
        score_dtype = torch.bfloat16 if torch.is_autocast_enabled("cuda") else out_dtype
        self._last_weights = torch.empty(0, k, dtype=score_dtype, device=flat.device)
        self._last_counts = torch.zeros(self.n_routed_experts, dtype=torch.int32, device=flat.device)
        self._counts_of = self._last_indices
        y = flat.new_zeros(0, self.dim, dtype=out_dtype)
        tied = [self.gate.weight, self.gate.bias]
        if self.shared_expert is not None:
            tied += [self.shared_expert.w1.weight, self.shared_expert.w2.weight, self.shared_expert.w3.weight]
        return y + sum(p.sum() * 0 for p in tied).to(out_dtype) + flat.sum().to(out_dtype) * 0

    def _load(self) -> torch.Tensor:
        """Slots per expert of the last routing, as the reference's
        ``bincount(_last_indices, minlength=E).float()`` (models/moe.py:93,105).

        After a forward on the kernels these are the dispatch histogram's
        counts (no extra pass over the indices).  If ``_last_indices`` was
        replaced since, they are counted from it as the reference does.
        """
        if self._last_counts is not None and self._counts_of is self._last_indices:
            return self._last_counts.float()
        return torch.bincount(self._last_indices.flatten(), minlength=self.n_routed_experts).float()

    def update_gate_bias(self, speed: float = 0.001) -> None:
        """Load-balancing bias step from the last routing (reference: models/moe.py:89-98).

        Same rule as the reference: experts above 1.10x the mean load lose
        ``speed`` and experts below 0.90x gain it.  The masked update is
        written as a select, so it needs no device-to-host synchronisation.
        """
        if self._last_indices is None:
            return
        load = self._load()
        mean = load.mean()
        overloaded = load > mean * 1.10
        underloaded = load < mean * 0.90
        with torch.no_grad():
            b = self.gate.bias
            b.copy_(torch.where(overloaded, b - speed, torch.where(underloaded, b + speed, b)))

    def get_load_balance_loss(self) -> torch.Tensor:
        """Diagnostic load-balance loss from the last routing (reference: models/moe.py:100-109).

        ``E * sum_e f_e * P_e`` with ``f`` the slot fraction per expert and
        ``P`` the mean routing weight per expert.  The per-token weight rows
        are scattered into a [T, E] matrix, which equals the reference's
        one-hot product summed over the k slots (the k experts of a token are
        distinct, so each entry is one weight plus zeros), and averaged with
        the same reduction.
        """
        if self._last_indices is None or self._last_weights is None:
            return torch.tensor(0.0, device=self.gate.weight.device)
        T, k = self._last_weights.shape
        E = self.n_routed_experts
        load = self._load()
        frac = load / (load.sum() + 1e-10)
        w = self._last_weights.float()
        prob = torch.zeros(T, E, dtype=w.dtype, device=w.device).scatter_add_(
            1, self._last_indices.reshape(T, k), w.reshape(T, k)).mean(dim=0)
        return (frac * prob).sum() * E


def moe_residual(x: torch.Tensor, norm: nn.Module, moe: nn.Module) -> torch.Tensor:
    """``x + moe(norm(x))``, the FFN half of FusionLLMBlock.forward
    (models/fusionllm.py:52).  A fusionllm_amd ``DeepSeekMoE`` after an
    ``nn.RMSNorm`` runs fused (norm, MoE and residual add in the kernels);
    any other pair runs as the plain expression."""
    if isinstance(moe, DeepSeekMoE) and isinstance(norm, nn.RMSNorm) and x.is_cuda:
        return moe.forward_norm_residual(x, norm)
    return x + moe(norm(x))
