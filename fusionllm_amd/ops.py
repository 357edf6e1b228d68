"""DeepSeekMoE block (and the dense SwiGLU) as torch.library operators, for
torch.compile and graph capture.

``fusionllm::moe_fwd`` and ``fusionllm::moe_bwd`` run the same kernels as
the module's eager path (models/moe.py:44-87 forward, its autograd backward)
but are opaque to the tracer: ``register_fake`` gives their outputs' static
shapes (no data-dependent shape anywhere: rows = T*k routed + T shared), and
``register_autograd`` connects them.  ``DeepSeekMoE.forward`` routes through
them while ``torch.compiler.is_compiling()``, so ``torch.compile(model,
fullgraph=True)`` (training/trainer.py:39 compiles the whole model that way)
traces the block as two nodes.  The one difference from the eager module:
nothing here reads the expert counts on the host, so experts that received
no tokens get zero gradients instead of None.

moe_fwd outputs: y [T,d] (out_dtype), indices [T,k] int64, weights [T,k]
fp32, counts [E] int32, then the tensors the backward reads: idx32 [T,k],
topv [T,k] fp32, offsets [E+1], perm [T*k], pos_of_slot [T*k], x_perm
[T*k,d] bf16 (0 rows when the routed rows are read from x through perm),
ab [rows,2I] bf16, h [rows,I] bf16, o [rows,d] bf16.
moe_bwd returns [dx, d_gate_w, d_gate_b, *d_weights] in the inputs' dtypes.

``fusionllm::swiglu_fwd`` / ``swiglu_bwd`` do the same for the dense SwiGLU
(models/moe.py:11-21 used alone, the DenseFFN of models/fusionllm.py:17-27):
outputs y [T,d] bf16, ab [T,2I] bf16, h [T,I] bf16; gradients [dx, dw1,
dw3, dw2] in the inputs' dtypes.
"""
from __future__ import annotations

import types

import torch
from torch import Tensor

from . import _kernels as K
from .moe import _backward_pass, _bf16_operands, _dense_backward, _dense_offsets, _forward_pass, gathers_rows


def _meta(gate_w: Tensor, weights: list[Tensor], k: int, route_scale: float, has_shared: bool,
          out_dtype: torch.dtype):
    return (gate_w.shape[0], k, weights[0].shape[0], float(route_scale), bool(has_shared), out_dtype)


@torch.library.custom_op("fusionllm::moe_fwd", mutates_args=())
def moe_fwd(x: Tensor, gate_w: Tensor, gate_b: Tensor, weights: list[Tensor], k: int, route_scale: float,
            has_shared: bool, out_dtype: torch.dtype) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                                                Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                                                Tensor]:
    meta = _meta(gate_w, weights, k, route_scale, has_shared, out_dtype)
    fw = _forward_pass(meta, x, gate_w, gate_b, weights)
    xb, gwb, wb, idx, idx64, w, v, counts, offsets, perm, pos, x_perm, ab, h, o, y = fw
    if x_perm is None:  # routed rows read through perm: no gathered copy (0 rows)
        x_perm = xb.new_empty((0, xb.shape[1]))
    return y, idx64, w, counts, idx, v, offsets, perm, pos, x_perm, ab, h, o


@moe_fwd.register_fake
def _(x, gate_w, gate_b, weights, k, route_scale, has_shared, out_dtype):
    T, d = x.shape
    E, inter = gate_w.shape[0], weights[0].shape[0]
    rows = T * k + (T if has_shared else 0)
    i32, f32, bf = torch.int32, torch.float32, torch.bfloat16
    e = lambda *shape, dtype: x.new_empty(shape, dtype=dtype)
    xp_rows = 0 if gathers_rows(T, k, has_shared) else T * k
    return (e(T, d, dtype=out_dtype), e(T, k, dtype=torch.int64), e(T, k, dtype=f32), e(E, dtype=i32),
            e(T, k, dtype=i32), e(T, k, dtype=f32), e(E + 1, dtype=i32), e(T * k, dtype=i32),
            e(T * k, dtype=i32), e(xp_rows, d, dtype=bf), e(rows, 2 * inter, dtype=bf), e(rows, inter, dtype=bf),
            e(rows, d, dtype=bf))


@torch.library.custom_op("fusionllm::moe_bwd", mutates_args=())
def moe_bwd(dy: Tensor, x: Tensor, gate_w: Tensor, gate_b: Tensor, weights: list[Tensor], idx: Tensor,
            w: Tensor, v: Tensor, offsets: Tensor, perm: Tensor, pos: Tensor, x_perm: Tensor, ab: Tensor,
            h: Tensor, o: Tensor, k: int, route_scale: float, has_shared: bool) -> list[Tensor]:
    meta = _meta(gate_w, weights, k, route_scale, has_shared, dy.dtype)
    xb, gwb, *wb = _bf16_operands([x, gate_w, *weights])
    ctx = types.SimpleNamespace(meta=meta, param_dtypes=(gate_w.dtype, gate_b.dtype, [t.dtype for t in weights]))
    saved = (xb, gwb, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, *wb)
    dx_rows, d_logits, dgw, dgb, grads_w = _backward_pass(ctx, saved, dy.contiguous())
    dx = K.dx_reduce(dx_rows, pos, idx, d_logits, gwb, idx.shape[0] * k, has_shared, x.dtype)
    return [dx, dgw, dgb, *grads_w]


@moe_bwd.register_fake
def _(dy, x, gate_w, gate_b, weights, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, k, route_scale,
      has_shared):
    return [torch.empty_like(x), torch.empty_like(gate_w), torch.empty_like(gate_b),
            *[torch.empty_like(t) for t in weights]]


def _setup_context(ctx, inputs, output):
    x, gate_w, gate_b, weights, k, route_scale, has_shared, out_dtype = inputs
    y, idx64, w, counts, idx, v, offsets, perm, pos, x_perm, ab, h, o = output
    ctx.n_w = len(weights)
    ctx.args = (k, route_scale, has_shared)
    ctx.save_for_backward(x, gate_w, gate_b, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, *weights)


def _backward(ctx, dy, *unused):
    x, gate_w, gate_b, idx, w, v, offsets, perm, pos, x_perm, ab, h, o, *weights = ctx.saved_tensors
    if dy is None:
        return None, None, None, [None] * ctx.n_w, None, None, None, None
    k, route_scale, has_shared = ctx.args
    g = torch.ops.fusionllm.moe_bwd(dy, x, gate_w, gate_b, weights, idx, w, v, offsets, perm, pos, x_perm,
                                    ab, h, o, k, route_scale, has_shared)
    return g[0], g[1], g[2], list(g[3:]), None, None, None, None


moe_fwd.register_autograd(_backward, setup_context=_setup_context)


@torch.library.custom_op("fusionllm::swiglu_fwd", mutates_args=())
def swiglu_fwd(x: Tensor, w1: Tensor, w3: Tensor, w2: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    T, d = x.shape
    inter = w1.shape[0]
    xb, w1b, w3b, w2b = _bf16_operands([x, w1, w3, w2])
    off = _dense_offsets(T, x.device)
    ab, h = K.gateup_fwd(xb, None, off, 1, [w1b], [w3b], inter)
    y = K.down_fwd(h, off, 1, T, 0, [w2b], d)
    return y, ab, h


@swiglu_fwd.register_fake
def _(x, w1, w3, w2):
    T, inter = x.shape[0], w1.shape[0]
    bf = torch.bfloat16
    return (x.new_empty((T, w2.shape[0]), dtype=bf), x.new_empty((T, 2 * inter), dtype=bf),
            x.new_empty((T, inter), dtype=bf))


@torch.library.custom_op("fusionllm::swiglu_bwd", mutates_args=())
def swiglu_bwd(dy: Tensor, x: Tensor, w1: Tensor, w3: Tensor, w2: Tensor, ab: Tensor, h: Tensor) -> list[Tensor]:
    xb, w1b, w3b, w2b = _bf16_operands([x, w1, w3, w2])
    off = _dense_offsets(x.shape[0], x.device)
    dx, dw1, dw3, dw2 = _dense_backward(dy, xb, ab, h, w1b, w3b, w2b, off,
                                        (x.dtype, w1.dtype, w3.dtype, w2.dtype), True)
    return [dx, dw1, dw3, dw2]


@swiglu_bwd.register_fake
def _(dy, x, w1, w3, w2, ab, h):
    return [torch.empty_like(x), torch.empty_like(w1), torch.empty_like(w3), torch.empty_like(w2)]


def _swiglu_setup(ctx, inputs, output):
    x, w1, w3, w2 = inputs
    y, ab, h = output
    ctx.save_for_backward(x, w1, w3, w2, ab, h)


def _swiglu_backward(ctx, dy, *unused):
    x, w1, w3, w2, ab, h = ctx.saved_tensors
    if dy is None:
        return None, None, None, None
    dx, dw1, dw3, dw2 = torch.ops.fusionllm.swiglu_bwd(dy, x, w1, w3, w2, ab, h)
    return dx, dw1, dw3, dw2


swiglu_fwd.register_autograd(_swiglu_backward, setup_context=_swiglu_setup)
