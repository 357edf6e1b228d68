"""Python wrappers of the libfusionmoe entry points (one per C function).

Each wrapper checks shapes, dtypes, contiguity and device on the host,
allocates the outputs with torch (device memory and streams are PyTorch's;
the kernels run on the current stream), calls the C ABI and raises on a
nonzero status.  Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
import functools

import torch

from . import _lib
from ._lib import BF16, F32, check, ptr_array

# Optional per-entry-point timing: when a dict is installed with
# set_timer(), every wrapper (or only those named in ``only``) records a pair
# of HIP events around its launches on the current stream (the stream the
# kernels run on) and appends them under its name.  Used by bench.py; off by
# default.
_TIMER: dict | None = None
_TIMER_ONLY: frozenset | None = None


def set_timer(store: dict | None, only=None) -> None:
    global _TIMER, _TIMER_ONLY
    _TIMER = store
    _TIMER_ONLY = None if only is None else frozenset(only)


def _timed(fn):
    name = fn.__name__

    @functools.wraps(fn)
    def wrapper(*args, tag: str | None = None, **kwargs):
        if _TIMER is None:
            return fn(*args, **kwargs)
        key = name if tag is None else f"{name}:{tag}"
        if _TIMER_ONLY is not None and key not in _TIMER_ONLY:
            return fn(*args, **kwargs)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        out = fn(*args, **kwargs)
        end.record()
        _TIMER.setdefault(key, []).append((start, end))
        return out
    return wrapper


def _stream() -> ctypes.c_void_p:
    # The raw current-stream handle of the current device (what
    # torch.cuda.current_stream().cuda_stream returns, without building a
    # Stream object: that costs more than a kernel launch on small batches).
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice()))


def _req(t: torch.Tensor, name: str, dtype: torch.dtype | None = None) -> int:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a ROCm device tensor (got {t.device})")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype} (got {t.dtype})")
    return t.data_ptr()


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float32:
        return F32
    raise RuntimeError(f"unsupported dtype {dt}")


@_timed
def router_fwd(x, gate_w, gate_b, k: int, route_scale: float):
    """fp32-logit biased-sigmoid top-k routing; returns idx32, idx64, weights, topv."""
    lib = _lib.load()
    T, d = x.shape
    E = gate_w.shape[0]
    dev = x.device
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    idx64 = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    v = torch.empty(T, k, dtype=torch.float32, device=dev)
    check(lib.fmoe_router_fwd(_req(x, "x", torch.bfloat16), _req(gate_w, "gate.weight", torch.bfloat16),
                              _req(gate_b, "gate.bias", torch.bfloat16), T, d, E, k, float(route_scale),
                              idx.data_ptr(), idx64.data_ptr(), w.data_ptr(), v.data_ptr(), _stream()),
          "fmoe_router_fwd")
    return idx, idx64, w, v


TINY_BATCH = 16  # fmoe_route_dispatch takes up to this many tokens
ROUTER_SMALL_T = 128  # fmoe_router_fwd runs one workgroup per token up to this many tokens


@_timed
def route_dispatch(x, gate_w, gate_b, k: int, route_scale: float):
    """router_fwd followed by dispatch for T <= TINY_BATCH tokens, one launch;
    returns idx32, idx64, weights, topv, counts, offsets, perm, pos, x_perm."""
    lib = _lib.load()
    T, d = x.shape
    E = gate_w.shape[0]
    dev = x.device
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    idx64 = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    v = torch.empty(T, k, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    pos = torch.empty(T * k, dtype=torch.int32, device=dev)
    x_perm = torch.empty(T * k, d, dtype=torch.bfloat16, device=dev)
    check(lib.fmoe_route_dispatch(_req(x, "x", torch.bfloat16), _req(gate_w, "gate.weight", torch.bfloat16),
                                  _req(gate_b, "gate.bias", torch.bfloat16), T, d, E, k, float(route_scale),
                                  idx.data_ptr(), idx64.data_ptr(), w.data_ptr(), v.data_ptr(),
                                  counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(), pos.data_ptr(),
                                  x_perm.data_ptr(), _stream()),
          "fmoe_route_dispatch")
    return idx, idx64, w, v, counts, offsets, perm, pos, x_perm


def _host_counts(counts_host, E):
    """Address of the host buffer that receives the E expert counts (int32,
    written by a kernel): a contiguous pinned int32 CPU tensor of at least E
    elements, checked in that order (each failure names its reason)."""
    if counts_host is None:
        return None
    if counts_host.device.type != "cpu":
        raise RuntimeError("counts_host must be a CPU tensor")
    if counts_host.dtype != torch.int32:
        raise RuntimeError(f"counts_host must be int32 (got {counts_host.dtype})")
    if counts_host.numel() < E:
        raise RuntimeError(f"counts_host must hold at least n_experts={E} elements (got {counts_host.numel()})")
    if not counts_host.is_contiguous():
        raise RuntimeError("counts_host must be contiguous")
    if not counts_host.is_pinned():
        raise RuntimeError("counts_host must be pinned host memory")
    return counts_host.data_ptr()


@_timed
def route_and_dispatch(x, gate_w, gate_b, k: int, route_scale: float, gather: bool = True,
                       counts_host: torch.Tensor | None = None):
    """router_fwd followed by dispatch for any T, in three launches (the router counts the
    dispatch histogram, the scatter copies the rows); returns idx32, idx64, weights, topv,
    counts, offsets, perm, pos, x_perm.  counts_host: optional pinned int32 [E] tensor that
    also receives the expert counts (readable after the stream has passed this call)."""
    lib = _lib.load()
    T, d = x.shape
    E = gate_w.shape[0]
    dev = x.device
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    idx64 = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    v = torch.empty(T, k, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    pos = torch.empty(T * k, dtype=torch.int32, device=dev)
    x_perm = torch.empty(T * k, d, dtype=torch.bfloat16, device=dev) if gather else None
    ws_bytes = lib.fmoe_route_and_dispatch_workspace_bytes(T, E, k)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    check(lib.fmoe_route_and_dispatch(_req(x, "x", torch.bfloat16), _req(gate_w, "gate.weight", torch.bfloat16),
                                      _req(gate_b, "gate.bias", torch.bfloat16), T, d, E, k, float(route_scale),
                                      idx.data_ptr(), idx64.data_ptr(), w.data_ptr(), v.data_ptr(),
                                      counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(), pos.data_ptr(),
                                      x_perm.data_ptr() if x_perm is not None else None,
                                      _host_counts(counts_host, E), ws.data_ptr(), ws_bytes, _stream()),
          "fmoe_route_and_dispatch")
    return idx, idx64, w, v, counts, offsets, perm, pos, x_perm


@_timed
def dispatch(idx, x, n_experts: int, gather: bool = True, noalloc: bool = False):
    """Histogram + scan + stable scatter (+ row gather); returns counts, offsets, perm, pos, x_perm.
    noalloc: fmoe_dispatch_noalloc, whose scratch is the library's static device array."""
    lib = _lib.load()
    T, k = idx.shape
    d = x.shape[1]
    dev = x.device
    counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    pos = torch.empty(T * k, dtype=torch.int32, device=dev)
    x_perm = torch.empty(T * k, d, dtype=torch.bfloat16, device=dev) if gather else None
    if noalloc:
        check(lib.fmoe_dispatch_noalloc(_req(idx, "idx", torch.int32), _req(x, "x", torch.bfloat16), T, d,
                                        n_experts, k, counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(),
                                        pos.data_ptr(), x_perm.data_ptr() if x_perm is not None else None,
                                        _stream()),
              "fmoe_dispatch_noalloc")
        return counts, offsets, perm, pos, x_perm
    ws_bytes = lib.fmoe_dispatch_workspace_bytes(T, n_experts, k)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    check(lib.fmoe_dispatch(_req(idx, "idx", torch.int32), _req(x, "x", torch.bfloat16), T, d, n_experts, k,
                            counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(), pos.data_ptr(),
                            x_perm.data_ptr() if x_perm is not None else None,
                            ws.data_ptr(), ws_bytes, _stream()),
          "fmoe_dispatch")
    return counts, offsets, perm, pos, x_perm


@_timed
def gateup_fwd(x_rows, x_shared, offsets, n_experts: int, w1s, w3s, inter: int, gather=None, k: int = 1):
    """a|b and h of every routed and shared row.  x_rows: the routed rows [T*k, dim] (x_perm), or,
    with gather (the dispatch's perm, row -> slot t*k + j), the token rows x [T, dim], routed row r
    reading x row gather[r] // k (launches of more than SMALL_LAUNCH_ROWS rows)."""
    lib = _lib.load()
    d = x_rows.shape[1]
    rows_r = gather.numel() if gather is not None else x_rows.shape[0]
    rows_s = x_shared.shape[0] if x_shared is not None else 0
    dev = x_rows.device
    rows = rows_r + rows_s
    ab = torch.empty(rows, 2 * inter, dtype=torch.bfloat16, device=dev)
    h = torch.empty(rows, inter, dtype=torch.bfloat16, device=dev)
    ws, ws_bytes = _split_workspace(dev, rows_r, rows_s, -(-inter // 128), small=True)
    check(lib.fmoe_gateup_fwd(_req(x_rows, "x_rows", torch.bfloat16),
                              _req(gather, "gather", torch.int32) if gather is not None else None, int(k),
                              x_rows.shape[0],
                              _req(x_shared, "x", torch.bfloat16) if x_shared is not None else None,
                              _req(offsets, "offsets", torch.int32), n_experts, rows_r, rows_s, d, inter,
                              ptr_array([w.data_ptr() for w in w1s]), ptr_array([w.data_ptr() for w in w3s]),
                              ab.data_ptr(), h.data_ptr(), _ptr(ws), ws_bytes, _stream()),
          "fmoe_gateup_fwd")
    return ab, h


SMALL_LAUNCH_ROWS = 4096  # launches up to this many rows send groups of <= 128 rows to the small kernel
SPLIT_MAX_ROUNDS = 8      # a row product of this many full rounds of tiles or more is never K-split


@functools.lru_cache(maxsize=None)
def _device_cus(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def _split_workspace(dev, rows_routed: int = 0, rows_shared: int = 0, tile_cols: int = 0, small: bool = False):
    """fp32 workspace for the K-split last round of the row products, or
    (None, 0) when the launch cannot split a tile (the library then runs
    every tile whole): a decode-sized forward launch whose groups all go to
    the small-group kernel (small: the product has one; at most 256 routed
    and 128 shared rows in at most SMALL_LAUNCH_ROWS), or a product of
    SPLIT_MAX_ROUNDS rounds or more (tile_cols: output tiles per 256-row
    block)."""
    if small and rows_routed <= 256 and rows_shared <= 128 and rows_routed + rows_shared <= SMALL_LAUNCH_ROWS:
        return None, 0
    if tile_cols:
        blocks = -(-rows_routed // 256) + -(-rows_shared // 256)
        if blocks * tile_cols >= SPLIT_MAX_ROUNDS * _device_cus(dev.index if dev.index is not None else 0):
            return None, 0
    lib = _lib.load()
    nbytes = lib.fmoe_split_workspace_bytes()
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev), nbytes


def _ptr(t):
    return None if t is None else t.data_ptr()


@_timed
def down_fwd(h, offsets, n_experts: int, rows_routed: int, rows_shared: int, w2s, dim: int):
    lib = _lib.load()
    rows, inter = h.shape
    out = torch.empty(rows, dim, dtype=torch.bfloat16, device=h.device)
    ws, ws_bytes = _split_workspace(h.device, rows_routed, rows_shared, -(-dim // 256), small=True)
    check(lib.fmoe_down_fwd(_req(h, "h", torch.bfloat16), _req(offsets, "offsets", torch.int32), n_experts,
                            rows_routed, rows_shared, dim, inter, ptr_array([w.data_ptr() for w in w2s]),
                            out.data_ptr(), _ptr(ws), ws_bytes, _stream()),
          "fmoe_down_fwd")
    return out


@_timed
def combine_fwd(expert_out, idx, weights, pos, rows_routed: int, has_shared: bool, out_dtype: torch.dtype,
                residual: torch.Tensor | None = None):
    lib = _lib.load()
    T, k = idx.shape
    d = expert_out.shape[1]
    y = torch.empty(T, d, dtype=out_dtype, device=expert_out.device)
    res = 0 if residual is None else _req(residual, "residual", out_dtype)
    check(lib.fmoe_combine_fwd(_req(expert_out, "expert_out", torch.bfloat16), _req(idx, "idx", torch.int32),
                               _req(weights, "weights", torch.float32), _req(pos, "pos_of_slot", torch.int32),
                               T, d, k, rows_routed, int(has_shared), _dtype_code(out_dtype), res,
                               y.data_ptr(), _stream()),
          "fmoe_combine_fwd")
    return y


@_timed
def combine_bwd(dy, expert_out, weights, perm, k: int):
    lib = _lib.load()
    T, d = dy.shape
    d_eo = torch.empty(T * k, d, dtype=torch.bfloat16, device=dy.device)
    d_w = torch.empty(T, k, dtype=torch.float32, device=dy.device)
    check(lib.fmoe_combine_bwd(_req(dy, "dy"), _dtype_code(dy.dtype), _req(expert_out, "expert_out", torch.bfloat16),
                               _req(weights, "weights", torch.float32), _req(perm, "perm", torch.int32),
                               T, d, k, d_eo.data_ptr(), d_w.data_ptr(), _stream()),
          "fmoe_combine_bwd")
    return d_eo, d_w


def _weights(ws, name, shape):
    for w in ws:
        _req(w, name, torch.bfloat16)
        if tuple(w.shape) != shape:
            raise RuntimeError(f"{name} must be {shape} (got {tuple(w.shape)})")
    return ptr_array([w.data_ptr() for w in ws])


@_timed
def down_bwd_dx(d_out_routed, d_out_shared, offsets, n_experts: int, w2s, ab, inter: int):
    """dh = d_out w2 with the SwiGLU backward fused; w2s: per group [dim, inter] as nn.Linear keeps it."""
    lib = _lib.load()
    rows_r, d = d_out_routed.shape
    rows_s = d_out_shared.shape[0] if d_out_shared is not None else 0
    G = n_experts + (1 if rows_s else 0)
    if len(w2s) < G:
        raise RuntimeError(f"down_bwd_dx needs {G} weight matrices (got {len(w2s)})")
    d_ab = torch.empty(rows_r + rows_s, 2 * inter, dtype=torch.bfloat16, device=ab.device)
    ws, ws_bytes = _split_workspace(ab.device, rows_r, rows_s, -(-inter // 256))
    check(lib.fmoe_down_bwd_dx(_req(d_out_routed, "d_out", torch.bfloat16),
                               _req(d_out_shared, "d_out_shared", torch.bfloat16) if d_out_shared is not None else None,
                               _req(offsets, "offsets", torch.int32), n_experts, rows_r, rows_s, d, inter,
                               _weights(w2s[:G], "w2", (d, inter)), _req(ab, "ab", torch.bfloat16),
                               d_ab.data_ptr(), _ptr(ws), ws_bytes, _stream()),
          "fmoe_down_bwd_dx")
    return d_ab


@_timed
def gateup_bwd_dx(d_ab, offsets, n_experts: int, rows_routed: int, rows_shared: int, w1s, w3s, dim: int):
    """dx_rows = da w1 + db w3; w1s, w3s: per group [inter, dim] as nn.Linear keeps them."""
    lib = _lib.load()
    rows, two_i = d_ab.shape
    inter = two_i // 2
    G = n_experts + (1 if rows_shared else 0)
    if len(w1s) < G or len(w3s) < G:
        raise RuntimeError(f"gateup_bwd_dx needs {G} weight matrices of each kind")
    dx_rows = torch.empty(rows, dim, dtype=torch.bfloat16, device=d_ab.device)
    ws, ws_bytes = _split_workspace(d_ab.device, rows_routed, rows_shared, -(-dim // 256))
    check(lib.fmoe_gateup_bwd_dx(_req(d_ab, "d_ab", torch.bfloat16), _req(offsets, "offsets", torch.int32),
                                 n_experts, rows_routed, rows_shared, dim, inter,
                                 _weights(w1s[:G], "w1", (inter, dim)), _weights(w3s[:G], "w3", (inter, dim)),
                                 dx_rows.data_ptr(), _ptr(ws), ws_bytes, _stream()),
          "fmoe_gateup_bwd_dx")
    return dx_rows


@_timed
def weight_grad(a_routed, a_shared, b_routed, b_shared, offsets, n_experts: int, rows_routed: int,
                rows_shared: int, m_split: int, outs_lo, outs_hi, out_dtype: torch.dtype, b_gather=None,
                k: int = 1):
    """G_e = A_e^T B_e for every group, written into outs_lo[e] / outs_hi[e].  With b_gather (the
    dispatch's perm), b_routed is the token rows x [T, n_out] and routed row r of B is x row
    b_gather[r] // k."""
    lib = _lib.load()
    m_out = a_routed.shape[1]
    n_out = b_routed.shape[1]
    ws_bytes = lib.fmoe_weight_grad_workspace_bytes(rows_routed, rows_shared, n_experts, m_out, n_out)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=a_routed.device)
    lo = ptr_array([o.data_ptr() for o in outs_lo])
    hi = ptr_array([o.data_ptr() for o in outs_hi]) if outs_hi is not None else None
    check(lib.fmoe_weight_grad(_req(a_routed, "A", torch.bfloat16),
                               _req(a_shared, "A_shared", torch.bfloat16) if a_shared is not None else None,
                               a_routed.stride(0),
                               _req(b_routed, "B", torch.bfloat16),
                               _req(b_shared, "B_shared", torch.bfloat16) if b_shared is not None else None,
                               b_routed.stride(0),
                               _req(b_gather, "b_gather", torch.int32) if b_gather is not None else None, int(k),
                               b_routed.shape[0],
                               _req(offsets, "offsets", torch.int32), n_experts, rows_routed, rows_shared,
                               m_out, n_out, m_split, lo, hi, _dtype_code(out_dtype),
                               ws.data_ptr(), ws_bytes, _stream()),
          "fmoe_weight_grad")


@_timed
def router_bwd(d_w, topv, perm, offsets, x, n_experts: int, route_scale: float, grad_dtype: torch.dtype):
    """Logit gradients and the gate's weight / bias gradients; x: [T, dim] bf16 token rows (read through perm)."""
    lib = _lib.load()
    T, k = d_w.shape
    d = x.shape[1]
    dev = d_w.device
    d_logits = torch.empty(T, k, dtype=torch.float32, device=dev)
    dgw = torch.empty(n_experts, d, dtype=grad_dtype, device=dev)
    dgb = torch.empty(n_experts, dtype=grad_dtype, device=dev)
    ws_bytes = lib.fmoe_router_bwd_workspace_bytes(T, d, n_experts, k)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    check(lib.fmoe_router_bwd(_req(d_w, "d_weights", torch.float32), _req(topv, "topv", torch.float32),
                              _req(perm, "perm", torch.int32), _req(offsets, "offsets", torch.int32),
                              _req(x, "x", torch.bfloat16), T, d, n_experts, k, float(route_scale),
                              d_logits.data_ptr(), dgw.data_ptr(), dgb.data_ptr(), _dtype_code(grad_dtype),
                              ws.data_ptr(), ws_bytes, _stream()),
          "fmoe_router_bwd")
    return d_logits, dgw, dgb


@_timed
def dx_reduce(dx_rows, pos, idx, d_logits, gate_w, rows_routed: int, has_shared: bool, out_dtype: torch.dtype):
    lib = _lib.load()
    T, k = idx.shape
    d = dx_rows.shape[1]
    dx = torch.empty(T, d, dtype=out_dtype, device=dx_rows.device)
    check(lib.fmoe_dx_reduce(_req(dx_rows, "dx_rows", torch.bfloat16), _req(pos, "pos_of_slot", torch.int32),
                             _req(idx, "idx", torch.int32), _req(d_logits, "d_logits", torch.float32),
                             _req(gate_w, "gate.weight", torch.bfloat16), T, d, k, rows_routed, int(has_shared),
                             _dtype_code(out_dtype), dx.data_ptr(), _stream()),
          "fmoe_dx_reduce")
    return dx


@_timed
def rmsnorm_fwd(x, norm_w, eps: float):
    """RMSNorm of the rows of x into the bf16 MoE input; returns (xn, rstd)."""
    lib = _lib.load()
    T, d = x.shape
    xn = torch.empty(T, d, dtype=torch.bfloat16, device=x.device)
    rstd = torch.empty(T, dtype=torch.float32, device=x.device)
    w_ptr = 0 if norm_w is None else _req(norm_w, "norm weight")
    w_code = F32 if norm_w is None else _dtype_code(norm_w.dtype)
    check(lib.fmoe_rmsnorm_fwd(_req(x, "x"), _dtype_code(x.dtype), w_ptr, w_code, T, d, float(eps),
                               xn.data_ptr(), rstd.data_ptr(), _stream()),
          "fmoe_rmsnorm_fwd")
    return xn, rstd


@_timed
def dx_reduce_norm(dx_rows, pos, idx, d_logits, gate_w, rows_routed: int, has_shared: bool,
                   x, rstd, norm_w, d_out, want_dw: bool):
    """Input gradient of x + moe(rmsnorm(x)) and the norm weight's gradient."""
    lib = _lib.load()
    T, k = idx.shape
    d = dx_rows.shape[1]
    dev = dx_rows.device
    dx = torch.empty(T, d, dtype=x.dtype, device=dev)
    dnw, ws, ws_bytes = None, None, 0
    if want_dw and norm_w is not None:
        dnw = torch.empty(d, dtype=norm_w.dtype, device=dev)
        ws_bytes = lib.fmoe_norm_bwd_workspace_bytes(d)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    w_ptr = 0 if norm_w is None else _req(norm_w, "norm weight")
    w_code = F32 if norm_w is None else _dtype_code(norm_w.dtype)
    check(lib.fmoe_dx_reduce_norm(_req(dx_rows, "dx_rows", torch.bfloat16), _req(pos, "pos_of_slot", torch.int32),
                                  _req(idx, "idx", torch.int32), _req(d_logits, "d_logits", torch.float32),
                                  _req(gate_w, "gate.weight", torch.bfloat16), T, d, k, rows_routed,
                                  int(has_shared), _req(x, "x"), _req(rstd, "rstd", torch.float32), w_ptr,
                                  w_code, _req(d_out, "d_out", x.dtype), _dtype_code(x.dtype), dx.data_ptr(),
                                  0 if dnw is None else dnw.data_ptr(), 0 if ws is None else ws.data_ptr(),
                                  ws_bytes, _stream()),
          "fmoe_dx_reduce_norm")
    return dx, dnw


NORMUON_MAX_TENSORS = 32


@_timed
def normuon_step(params, grads, exp_avgs, exp_avg_sqs, lr: float, beta1: float, beta2: float, eps: float,
                 weight_decay: float, cautious: bool, bias_corr1: float, bias_corr2: float):
    """One fused NorMuon update of up to 32 same-dtype tensors (in place)."""
    lib = _lib.load()
    n = len(params)
    if n > NORMUON_MAX_TENSORS:
        raise RuntimeError(f"at most {NORMUON_MAX_TENSORS} tensors per launch (got {n})")
    dt = params[0].dtype
    rows = (ctypes.c_int64 * n)()
    cols = (ctypes.c_int64 * n)()
    mat = (ctypes.c_int * n)()
    ptrs = [[], [], [], []]
    for i, (p, g, m, v) in enumerate(zip(params, grads, exp_avgs, exp_avg_sqs)):
        for t, name in ((p, "param"), (g, "grad"), (m, "exp_avg"), (v, "exp_avg_sq")):
            _req(t, name, dt)
            if t.shape != p.shape:
                raise RuntimeError(f"{name} shape {tuple(t.shape)} != param shape {tuple(p.shape)}")
        c = p.shape[-1] if p.dim() >= 1 else 1
        rows[i] = p.numel() // c if c else 0
        cols[i] = c
        mat[i] = 1 if p.dim() >= 2 else 0
        for lst, t in zip(ptrs, (p, g, m, v)):
            lst.append(t.data_ptr())
    # ptr_array caches by content: these arrays change every call, build them fresh
    arrs = [(ctypes.c_void_p * n)(*lst) for lst in ptrs]
    check(lib.fmoe_normuon_step(arrs[0], arrs[1], arrs[2], arrs[3], rows, cols, mat, n, _dtype_code(dt),
                                float(lr), float(beta1), float(beta2), float(eps), float(weight_decay),
                                int(bool(cautious)), float(bias_corr1), float(bias_corr2), _stream()),
          "fmoe_normuon_step")


CAST_MAX_TENSORS = 64


def cast_bf16(tensors):
    """bf16 copies of contiguous fp32 device tensors, one launch per 64
    (round to nearest even, bit-identical to .to(torch.bfloat16))."""
    lib = _lib.load()
    outs = []
    for i0 in range(0, len(tensors), CAST_MAX_TENSORS):
        chunk = tensors[i0:i0 + CAST_MAX_TENSORS]
        n = len(chunk)
        dst = [torch.empty(t.shape, dtype=torch.bfloat16, device=t.device) for t in chunk]
        src_p = (ctypes.c_void_p * n)(*[_req(t, "cast source", torch.float32) for t in chunk])
        dst_p = (ctypes.c_void_p * n)(*[d.data_ptr() for d in dst])
        cnt = (ctypes.c_int64 * n)(*[t.numel() for t in chunk])
        check(lib.fmoe_cast_bf16(src_p, dst_p, cnt, n, _stream()), "fmoe_cast_bf16")
        outs += dst
    return outs
