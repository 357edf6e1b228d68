#!/usr/bin/env python3
"""Benchmark of the MI355X DeepSeekMoE block (FusionLLM models/moe.py hot path).

Metric: MoE block tokens/sec, forward + backward, bf16,
8 experts top-2 + shared, d=768 — workload C2: 16384 tokens, inter 2048,
skewed router bias.  One step = forward + backward of the drop-in
``fusionllm_amd.DeepSeekMoE`` over one batch of synthetic, HBM-resident
input (zero_grad(set_to_none) between steps, as the reference trainer does).

The JSON line also carries:
  roofline      the dominant kernel (largest share of the step) against the
                MI355X bf16 dense MFMA peak: algorithmic FLOPs per launch over
                the launch's average duration, timed with HIP events on the
                stream the kernels run on, inside the timed region (only
                that entry point carries events there);
  kernels       the same figures for every entry point of the step: the
                GEMMs from a short untimed pass with events around every
                entry point (it also names the dominant one), the
                HBM-bound routing, dispatch, combine and reduce
                entry points from graphs of 20 back-to-back launches (events
                around such short kernels add their launch gaps);
  cpu_baseline  the reference algorithm (torch-CPU restatement, the oracle)
                timed on this host's cores on a bounded sample of the same
                workload.

Only one GPU is used: --gpus above 1 exits with an explanation.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

PEAK_BF16_FLOPS = 2.5e15   # MI355X dense bf16 MFMA
PEAK_HBM_BYTES = 8.0e12    # MI355X HBM3E
METRIC = "MoE block tokens/sec fwd+bwd (bf16, 8e top-2, d=768); grouped-GEMM % MFMA peak"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="C2-bf16-fwdbwd-skewed",
                   help="workload name from fusionllm_amd.configs, or its prefix C1..C5")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-tokens", type=int, default=4096,
                   help="tokens per CPU-baseline pass (passes repeat for --cpu-seconds)")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU work the baseline sample is sized to (repeated passes, at least 3)")
    p.add_argument("--fwd-only", action="store_true",
                   help="time the forward pass alone (decode-shaped C3 configs); not the headline metric")
    p.add_argument("--autocast", action="store_true",
                   help="fp32 module and input under bf16 autocast (the trainer's setting); single block")
    p.add_argument("--graph", action="store_true",
                   help="with --fwd-only: time HIP-graph replays of the forward (DecodeGraph)")
    p.add_argument("--gather-rows", action="store_true",
                   help="the block reads routed token rows of x through perm (no x_perm copy): "
                        "fusionllm_amd.moe.GATHER_ROWS")
    p.add_argument("--optimizer", action="store_true",
                   help="time the fused NorMuon step on the block's weight matrices (fp32, as the trainer "
                        "keeps them) instead of the block; its own JSON line")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run only a device-to-device copy of COPY_BYTES (3 times): the known-size kernel whose "
                        "FETCH_SIZE / WRITE_SIZE counters scale the GEMM counters to HBM bytes")
    return p.parse_args()


COPY_BYTES = 1 << 30


def copy_calibration():
    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 3}), flush=True)


def kernel_model(cfg, T, active_groups=None):
    """Algorithmic work per launch of each entry point (FLOPs for the GEMMs,
    bytes for the memory-bound kernels) at T tokens.  Decode-sized batches
    (T <= 128, every group <= 128 rows: the weight-streaming kernel) price the
    forward products by HBM bytes: the weights of the active_groups groups
    that received rows (shared expert included), read once, plus the
    activation rows in and out."""
    from fusionllm_amd.moe import gathers_rows
    d, I, E, k = cfg.dim, cfg.inter, cfg.n_experts, cfg.topk
    rows = T * k + (T if cfg.n_shared else 0)
    # the k gathered rows per token (x_perm), unless the block reads token rows through perm
    xp = 0 if gathers_rows(T, k, cfg.n_shared > 0) else k * 2 * d
    if T <= 128 and active_groups is not None:
        return {
            "gateup_fwd": ("hbm", active_groups * 2 * I * d * 2 + rows * (d + 3 * I) * 2),
            "down_fwd": ("hbm", active_groups * d * I * 2 + rows * (I + d) * 2),
            "router_fwd": ("hbm", T * (2 * d + 4 * k + 8 * k + 4 * k + 4 * k) + E * (d + 1) * 2),
            "dispatch": ("hbm", T * (4 * k + 2 * d + k * 2 * d + 8 * k + 4 * k)),
            "route_dispatch": ("hbm", T * (2 * d + 4 * k + 8 * k + 4 * k + 4 * k) + E * (d + 1) * 2
                               + T * (k * 2 * d + 8 * k) + 8 * E),
            "combine_fwd": ("hbm", T * (k * 2 * d + 2 * d + 8 * k + 4 * k + 2 * d)),
        }
    return {
        # MFMA-bound products (FLOPs)
        "gateup_fwd": ("mfma", 2.0 * rows * d * 2 * I),
        "down_fwd": ("mfma", 2.0 * rows * I * d),
        "down_bwd_dx": ("mfma", 2.0 * rows * d * I),
        "gateup_bwd_dx": ("mfma", 2.0 * rows * 2 * I * d),
        "weight_grad:w2": ("mfma", 2.0 * rows * d * I),
        "weight_grad:w13": ("mfma", 2.0 * rows * 2 * I * d),
        # HBM-bound (algorithmic bytes: bf16 activations, int32/fp32 metadata)
        "router_fwd": ("hbm", T * (2 * d + 4 * k + 8 * k + 4 * k + 4 * k)),
        "dispatch": ("hbm", T * (4 * k + (2 * d + xp if xp else 0) + 8 * k + 4 * k)),
        "combine_fwd": ("hbm", T * (k * 2 * d + 2 * d + 8 * k + 4 * k + 2 * d)),
        "combine_bwd": ("hbm", T * k * (2 * d + 2 * d + 2 * d + 4 + 4 + 4)),
        "router_bwd": ("hbm", T * k * (2 * d + 4 * 4)),
        # routing + dispatch in one entry point: x read once; idx, idx64, weights, scores,
        # perm and pos written (and the k rows of x_perm when the block keeps the gathered copy)
        "route_and_dispatch": ("hbm", T * (2 * d + 4 * k + 8 * k + 4 * k + 4 * k + 4 * k + 4 * k
                                           + xp)),
        "dx_reduce": ("hbm", T * (k * 2 * d + 2 * d + 2 * d + 12 * k)),
        # C4 (RMSNorm + MoE + residual): x in, xn and rstd out; the backward
        # reads the k routed + shared rows, x and d_out and writes dx
        "rmsnorm_fwd": ("hbm", T * (2 * d + 2 * d + 4)),
        "dx_reduce_norm": ("hbm", T * (k * 2 * d + 2 * d + 2 * d + 2 * d + 2 * d + 12 * k + 4)),
    }


def graph_entry_times(m, x, reps=20, replays=20):
    """Per-launch time (us) of each forward entry point of the DeepSeekMoE
    block on input x, measured the way a HIP-graph replay runs it: a graph of
    `reps` back-to-back launches of one entry point (same inputs), replayed
    `replays` times between two HIP events on the replaying stream.  Events
    cannot be recorded inside a captured graph, so the per-entry-point figures
    of a graph-replayed forward come from these graphs."""
    from fusionllm_amd import _kernels as K
    from fusionllm_amd.moe import _forward_pass
    E, k = m.n_routed_experts, m.n_activated_experts
    has_shared = m.shared_expert is not None
    meta = (E, k, m.moe_inter_dim, float(m.route_scale), has_shared, x.dtype)
    with torch.no_grad():
        fw = _forward_pass(meta, x, m.gate.weight, m.gate.bias, m._flat_weights())
    xb, gwb, wb, idx, idx64, w, v, counts, offsets, perm, pos, x_perm, ab, h, o, y = fw
    T, d = xb.shape
    G = E + (1 if has_shared else 0)
    w1s, w3s, w2s = wb[0::3][:G], wb[1::3][:G], wb[2::3][:G]
    gbb = m.gate.bias.to(torch.bfloat16).contiguous()
    rows_r, rows_s = T * k, (T if has_shared else 0)
    if T <= K.TINY_BATCH and T * E <= 64:
        calls = {"route_dispatch": lambda: K.route_dispatch(xb, gwb, gbb, k, float(m.route_scale))}
    else:
        calls = {"router_fwd": lambda: K.router_fwd(xb, gwb, gbb, k, float(m.route_scale)),
                 "dispatch": lambda: K.dispatch(idx, xb, E)}
    calls.update({
        "gateup_fwd": lambda: K.gateup_fwd(xb if x_perm is None else x_perm, xb if has_shared else None, offsets,
                                           E, w1s, w3s, m.moe_inter_dim, gather=perm if x_perm is None else None,
                                           k=k),
        "down_fwd": lambda: K.down_fwd(h, offsets, E, rows_r, rows_s, w2s, d),
        "combine_fwd": lambda: K.combine_fwd(o, idx, w, pos, rows_r, has_shared, x.dtype, None),
    })
    return {name: graph_time(fn, reps, replays) for name, fn in calls.items()}


def graph_time(fn, reps=20, replays=20):
    """Per-launch time (us) of fn: a HIP graph of `reps` back-to-back calls,
    replayed `replays` times between two HIP events on the replaying stream
    (no event between the launches, so short kernels are not inflated)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / (reps * replays)
    del g
    return us


def graph_hbm_times(m, x, dy):
    """Per-launch time (us) of the HBM-bound entry points of one forward +
    backward of the DeepSeekMoE block (routing, dispatch, combine and their
    backward), each from a graph of
    back-to-back launches on the workload's own intermediates (graph_time).
    Events around every call of an eager step inflate such short kernels by
    their launch gaps; this is the figure the roofline fractions of these
    kernels use."""
    from fusionllm_amd import _kernels as K
    from fusionllm_amd.moe import _forward_pass
    E, k = m.n_routed_experts, m.n_activated_experts
    has_shared = m.shared_expert is not None
    rs = float(m.route_scale)
    meta = (E, k, m.moe_inter_dim, rs, has_shared, x.dtype)
    with torch.no_grad():
        fw = _forward_pass(meta, x, m.gate.weight, m.gate.bias, m._flat_weights())
        xb, gwb, wb, idx, idx64, w, v, counts, offsets, perm, pos, x_perm, ab, h, o, y = fw
        T, d = xb.shape
        gbb = m.gate.bias.to(torch.bfloat16).contiguous()
        dyb = dy.to(torch.bfloat16).contiguous()
        d_o, d_w = K.combine_bwd(dyb, o, w, perm, k)
        d_logits, _, _ = K.router_bwd(d_w, v, perm, offsets, xb, E, rs, m.gate.weight.dtype)
        dx_rows = torch.empty(o.shape, dtype=torch.bfloat16, device=o.device).normal_()
        calls = {
            "router_fwd": lambda: K.router_fwd(xb, gwb, gbb, k, rs),
            "dispatch": lambda: K.dispatch(idx, xb, E, gather=x_perm is not None),
            "combine_fwd": lambda: K.combine_fwd(o, idx, w, pos, T * k, has_shared, x.dtype, None),
            "combine_bwd": lambda: K.combine_bwd(dyb, o, w, perm, k),
            "router_bwd": lambda: K.router_bwd(d_w, v, perm, offsets, xb, E, rs, m.gate.weight.dtype),
            "route_and_dispatch": lambda: K.route_and_dispatch(xb, gwb, gbb, k, rs, gather=x_perm is not None),
            "dx_reduce": lambda: K.dx_reduce(dx_rows, pos, idx, d_logits, gwb, T * k, has_shared, x.dtype),
        }
        return {name: graph_time(fn) for name, fn in calls.items()}


def hbm_traffic(cfg_name, entry):
    """HBM bytes per launch of an entry point from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE readings (profiles/hbm_counters_c2.json), each
    counter scaled by what it read for a device copy of known size; None when
    no reading covers this workload and entry point."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_counters_c2.json")
    if not cfg_name.startswith("C2") or not os.path.exists(path):
        return None
    with open(path) as f:
        prof = json.load(f)
    cal = prof["calibration"]
    fs = cal["copy_bytes"] / (cal["FETCH_SIZE_KiB"] * 1024.0)
    ws = cal["copy_bytes"] / (cal["WRITE_SIZE_KiB"] * 1024.0)
    names = prof["entry_points"].get(entry.split(":")[0])
    if not names or any(n not in prof["kernels"] for n in names):
        return None
    ks = [prof["kernels"][n] for n in names]
    return round(sum((k["FETCH_SIZE_KiB"] * fs + k["WRITE_SIZE_KiB"] * ws) * 1024.0 for k in ks))


def cpu_info() -> dict:
    """Host CPU model, logical CPUs and the ISA extensions that set torch's
    CPU GEMM rate (AVX-512, its bf16 dot products, AMX tiles)."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    want = ("avx2", "fma", "avx512f", "avx512_bf16", "avx512_vnni", "avx512_fp16", "amx_tile", "amx_bf16")
    return {"cpu_model": model, "nproc": os.cpu_count(), "isa": [f for f in want if f in flags]}


def cpu_c1_forward(runs=3):
    """The headline's CPU baseline: workload C1, the reference forward
    (models/moe.py:79-87, module semantics) in fp32 on the host cores at
    T = 16384 (x [8, 2048, 768] from N(0,1) seed 0, weights N(0, 0.02^2),
    zero bias); one warmup, then the median of `runs` timed forwards."""
    from fusionllm_amd import configs
    from oracle import moe_oracle as mo
    cfg = configs.C1
    data = configs.make_block(cfg, seed=0, with_dy=False)
    sd = data.state_dict()
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(cfg.n_experts)]
    shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    x = data.x.view(*cfg.x_shape)
    times = []
    with torch.no_grad():
        for i in range(runs + 1):
            t0 = time.perf_counter()
            mo.moe_forward(x, sd["gate.weight"], sd["gate.bias"], experts, shared, cfg.topk, cfg.route_scale,
                           mode="module")
            if i > 0:
                times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"workload": cfg.name, "tokens": cfg.tokens, "pass": "forward", "dtype": "f32",
            "value": round(cfg.tokens / med, 1), "unit": "tokens/s", "median_s": round(med, 4),
            "runs_s": [round(t, 4) for t in times], "cores": torch.get_num_threads(),
            "gflops": round(cfg.flops_fwd_bwd() / 3 / med / 1e9, 1)}


def cpu_baseline(cfg, data, n_tokens, seconds=12.0):
    """Reference algorithm on host cores: the oracle's torch-CPU restatement of
    models/moe.py, bf16, forward + backward, on the first n_tokens tokens,
    repeated until about `seconds` of CPU work (at least 3 passes, at most
    2.5x that time); value = n_tokens / the median pass time.  Also runs
    the C1 fp32 forward on the host cores (cpu_c1_forward) and names the host CPU."""
    from oracle import moe_oracle as mo
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    T = min(n_tokens, data.x.shape[0])
    sd = {k: v.bfloat16().clone().requires_grad_(True) for k, v in data.state_dict().items()}
    E = cfg.n_experts
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(E)]
    shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    x0 = data.x[:T].bfloat16()
    dy = data.dy[:T].bfloat16()

    norm_w = torch.ones(cfg.dim, dtype=torch.bfloat16, requires_grad=True)

    def step():
        for t in sd.values():
            t.grad = None
        x = x0.clone().requires_grad_(True)
        if cfg.layers == 1:
            y, _, _ = mo.moe_forward(x, sd["gate.weight"], sd["gate.bias"], experts, shared, cfg.topk,
                                     cfg.route_scale, mode="module")
        else:  # the stack: the same block weights in every layer (time, not values, is measured)
            y = x
            for _ in range(cfg.layers):
                y = y + mo.moe_forward(mo.rms_norm(y, norm_w), sd["gate.weight"], sd["gate.bias"], experts,
                                       shared, cfg.topk, cfg.route_scale, mode="module")[0]
        y.backward(dy)

    step()  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (sum(times) < seconds and time.perf_counter() - t_start < 2.5 * seconds):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    out = {
        "value": round(T / statistics.median(times), 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{cfg.name}: first {T} of {cfg.tokens} tokens"
                   + (f", {cfg.layers} x (RMSNorm + MoE + residual)" if cfg.layers > 1 else "")
                   + f", reference module semantics (bf16 router), bf16 forward+backward in torch CPU, "
                   f"median of {len(times)} passes ({sum(times):.1f} s) after 1 warmup"),
    }
    out.update(cpu_info())
    out["c1_fp32_forward"] = cpu_c1_forward()
    return out


def optimizer_bench(args):
    """NorMuon step (training/optimizer.py:11-58) over the weight matrices of
    the workload's MoE block (what build_optimizers gives NorMuon there: the
    expert and shared-expert matrices and gate.weight), fp32 parameters and
    states as the trainer keeps them, synthetic gradients."""
    from fusionllm_amd import DeepSeekMoE, configs
    from fusionllm_amd.optim import NorMuon
    from fusionllm_amd import _kernels as K
    cfg = configs.ALL.get(args.config) or next(c for n, c in configs.ALL.items() if n.split("-")[0] == args.config)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    m = DeepSeekMoE(cfg.moe_config()).to(dev)
    mats = [p for p in m.parameters() if p.ndim >= 2]
    g = torch.Generator(device=dev).manual_seed(0)
    for p in mats:
        p.grad = torch.randn(p.shape, generator=g, device=dev) * 1e-3
    opt = NorMuon(mats, lr=0.02, betas=(0.95, 0.95))
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    timer = {}
    K.set_timer(timer, only={"normuon_step"})
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        opt.step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    K.set_timer(None)
    elapsed = max(start.elapsed_time(end) / 1e3, wall)
    n_el = sum(p.numel() for p in mats)
    launches = [a.elapsed_time(b) / 1e3 for a, b in timer["normuon_step"]]
    per_launch = sum(launches) / len(launches)
    launches_per_step = len(launches) // args.steps
    bytes_per_el = 7 * 4  # read p, grad, exp_avg, exp_avg_sq; write p, exp_avg, exp_avg_sq (fp32)
    work = n_el * bytes_per_el / launches_per_step
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import moe_oracle as mo
        torch.set_num_threads(os.cpu_count() or 1)
        sample = [p.detach().cpu().clone() for p in mats[:3]]
        grads = [p.grad.cpu() for p in mats[:3]]
        states = [{} for _ in sample]
        for q, gq, st in zip(sample, grads, states):  # warmup (state allocation)
            mo.normuon_step(q, gq, st, lr=0.02, betas=(0.95, 0.95))
        times = []
        for _ in range(3):
            c0 = time.perf_counter()
            for q, gq, st in zip(sample, grads, states):
                mo.normuon_step(q, gq, st, lr=0.02, betas=(0.95, 0.95))
            times.append(time.perf_counter() - c0)
        n_s = sum(q.numel() for q in sample)
        cpu = {"value": round(n_s / statistics.median(times), 1), "unit": "elements/s",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"3 of the {len(mats)} matrices ({n_s} elements), the reference's step op by op in torch "
                         f"CPU, fp32, median of 3 after 1 warmup"}
    line = {
        "metric": "NorMuon step elements/sec (fp32 weight matrices of the MoE block)",
        "value": round(n_el * args.steps / elapsed, 1),
        "unit": "elements/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (N(0, 1e-3^2) gradients; module init weights)",
        "config": {"workload": f"NorMuon on {cfg.name} block matrices", "tensors": len(mats), "elements": n_el},
        "roofline": {"kernel": "normuon_step", "bound": "hbm", "achieved": round(work / per_launch / 1e9, 1),
                     "peak": PEAK_HBM_BYTES / 1e9, "unit": "GB/s",
                     "frac": round(work / per_launch / PEAK_HBM_BYTES, 4), "traffic": None,
                     "work_per_launch": work, "launches_timed": len(launches)},
        "cpu_baseline": cpu,
    }
    c1 = (cpu or {}).get("c1_fp32_forward")
    if c1 and c1.get("value") and not args.fwd_only:
        line["vs_c1_fp32_forward"] = round(tok_s / c1["value"], 1)
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.optimizer:
        optimizer_bench(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (one MI355X per box); "
                                   "run without --gpus or with --gpus 1"}))
        sys.exit(2)
    from fusionllm_amd import DeepSeekMoE, configs, moe_residual
    from fusionllm_amd import _kernels as K
    from fusionllm_amd import moe as moe_mod
    if args.gather_rows:
        moe_mod.GATHER_ROWS = True

    cfg = configs.ALL.get(args.config) or next(
        (c for n, c in configs.ALL.items() if n.split("-")[0] == args.config), None)
    if cfg is None:
        raise SystemExit(f"unknown --config {args.config!r}: one of {sorted(configs.ALL)} or C1..C5")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    data = configs.make_block(cfg, seed=0)

    # --autocast: the trainer's setting (training/trainer.py:158), fp32
    # parameters and activations under bf16 autocast; default: a bf16 module.
    pdt = torch.float32 if args.autocast else torch.bfloat16

    def module(d):
        m = DeepSeekMoE(cfg.moe_config())
        m.load_state_dict({k: v.to(pdt) for k, v in d.state_dict().items()})
        return m.to(device=dev, dtype=pdt)

    # C4: a stack of cfg.layers blocks x + MoE(RMSNorm(x)) (models/fusionllm.py:48,52),
    # independent seeded weights per layer, norm weights ones (their init).
    mods = [module(data)] + [module(configs.make_block(cfg, seed=l, with_dy=False))
                             for l in range(1, cfg.layers)]
    norms = [torch.nn.RMSNorm(cfg.dim, eps=1e-6).to(device=dev, dtype=torch.bfloat16)
             for _ in range(cfg.layers)] if cfg.layers > 1 else []
    x = data.x.to(dev, pdt).requires_grad_(True)
    dy = data.dy.to(dev, pdt)
    if args.autocast and norms:
        raise SystemExit("--autocast times the single block (C1..C3, C5)")
    T = x.shape[0]

    def forward():
        if args.autocast:
            with torch.autocast("cuda", dtype=torch.bfloat16):
                return mods[0](x)
        if not norms:
            return mods[0](x)
        h = x
        for m, n in zip(mods, norms):
            h = moe_residual(h, n, m)
        return h

    def step():
        if args.fwd_only:
            with torch.no_grad():
                forward()
            return
        for m in mods:
            m.zero_grad(set_to_none=True)
        for n in norms:
            n.weight.grad = None
        x.grad = None
        forward().backward(dy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # groups that received rows in this workload's routing (decode pricing)
    active = None
    if not norms and mods[0]._last_counts is not None:
        active = int((mods[0]._last_counts > 0).sum()) + (1 if cfg.n_shared else 0)
    model = kernel_model(cfg, T, active)

    def table_of(timer, n_steps, span_s):
        """Per-entry-point figures from HIP-event pairs."""
        out = {}
        for name, evs in timer.items():
            ms = [a.elapsed_time(b) for a, b in evs]
            avg_s = sum(ms) / len(ms) / 1e3
            bound, work = model.get(name, (None, None))
            entry = {"avg_us": round(avg_s * 1e6, 2), "calls": len(ms), "steps": n_steps,
                     "share": round(sum(ms) / 1e3 / span_s, 4)}
            if bound == "mfma":
                entry.update(bound="mfma", achieved_tflops=round(work / avg_s / 1e12, 1),
                             frac=round(work / avg_s / PEAK_BF16_FLOPS, 4))
            elif bound == "hbm":
                entry.update(bound="hbm", achieved_gbs=round(work / avg_s / 1e9, 1),
                             frac=round(work / avg_s / PEAK_HBM_BYTES, 4))
            out[name] = entry
        return out

    # Per-entry-point table: a few untimed steps with HIP events around every
    # entry point (on the stream the kernels run on).  Events between
    # back-to-back launches add gaps, so this pass is kept out of the timed
    # region; it also names the dominant entry point.
    table_steps = max(2, min(args.steps, 5))
    full = {}
    K.set_timer(full)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(table_steps):
        step()
    s1.record()
    torch.cuda.synchronize()
    K.set_timer(None)
    kernels = table_of(full, table_steps, s0.elapsed_time(s1) / 1e3)
    dom = max(kernels, key=lambda n: kernels[n]["share"])

    # Timed region: K steps between two synchronisations.  The dominant entry
    # point's launches are bracketed by HIP events on the stream they run on
    # (the roofline figures).  A forward-only (decode-sized) run is host-bound,
    # where even those events add host time: it is timed bare, and its
    # roofline comes from the table pass.
    if args.graph:
        # Decode as a serving loop runs it: the forward captured once into a
        # HIP graph, each step copies the tokens in and replays it.
        if not args.fwd_only or norms:
            raise SystemExit("--graph times the single-block forward: use it with --fwd-only on C1..C3/C5")
        from fusionllm_amd import DecodeGraph
        graph = DecodeGraph(mods[0], x.detach())
        xin = x.detach()

        def step():
            graph(xin)
        for _ in range(args.warmup):
            step()
    timer = {}
    K.set_timer(None if args.fwd_only else timer, only={dom})
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    K.set_timer(None)
    gpu_s = start.elapsed_time(end) / 1e3
    elapsed = max(gpu_s, wall)
    tok_s = T * args.steps / elapsed
    if args.graph:
        # Per-entry-point figures of the replayed forward: graphs of
        # back-to-back launches of each entry point (the eager table pass
        # above measures host-bound launches).
        step_us = elapsed / args.steps * 1e6
        kernels = {}
        for name, us in graph_entry_times(mods[0], x.detach()).items():
            bound, work = model.get(name, (None, None))
            e = {"avg_us": round(us, 2), "calls": "graph", "share": round(us / step_us, 4)}
            if bound == "hbm":
                e.update(bound="hbm", achieved_gbs=round(work / (us / 1e6) / 1e9, 1),
                         frac=round(work / (us / 1e6) / PEAK_HBM_BYTES, 4))
            elif bound == "mfma":
                e.update(bound="mfma", achieved_tflops=round(work / (us / 1e6) / 1e12, 1),
                         frac=round(work / (us / 1e6) / PEAK_BF16_FLOPS, 4))
            kernels[name] = e
        dom = max(kernels, key=lambda n: kernels[n]["share"])
        timer = {}
    dk = (table_of(timer, args.steps, elapsed) if timer else kernels)[dom]
    if not args.graph and not args.fwd_only:
        # GEMM pass: as many steps as the table pass, with HIP events around
        # the grouped GEMMs only (each 150 us or longer at C2, so the gaps the
        # events leave are small beside them).  The GEMM rows of the table and
        # the grouped-GEMM fraction come from it: the table pass brackets every
        # entry point, and its gaps between the short kernels (the GPU idles,
        # clocks drop) make the GEMMs measure 10-15 % slower than in a step.
        gtimer = {}
        K.set_timer(gtimer, only={n for n, (b, _) in model.items() if b == "mfma"})
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        for _ in range(table_steps):
            step()
        g1.record()
        torch.cuda.synchronize()
        K.set_timer(None)
        kernels.update(table_of(gtimer, table_steps, g0.elapsed_time(g1) / 1e3))
    if not args.fwd_only and not norms and not args.autocast:
        # the HBM-bound entry points from graphs of back-to-back launches
        step_us = elapsed / args.steps * 1e6
        for name, us in graph_hbm_times(mods[0], x.detach(), dy).items():
            bound, work = model[name]
            kernels[name] = {"avg_us": round(us, 2), "calls": "graph x20", "share": round(us / step_us, 4),
                             "bound": "hbm", "achieved_gbs": round(work / (us / 1e6) / 1e9, 1),
                             "frac": round(work / (us / 1e6) / PEAK_HBM_BYTES, 4)}

    bound, work = model[dom]
    avg_s = dk["avg_us"] / 1e6
    traffic = hbm_traffic(cfg.name, dom)
    if bound == "mfma":
        roofline = {"kernel": dom, "bound": "mfma", "achieved": round(work / avg_s / 1e12, 2),
                    "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s", "frac": round(work / avg_s / PEAK_BF16_FLOPS, 4),
                    "traffic": traffic, "work_per_launch": work, "launches_timed": dk["calls"]}
    else:
        roofline = {"kernel": dom, "bound": "hbm", "achieved": round(work / avg_s / 1e9, 1),
                    "peak": PEAK_HBM_BYTES / 1e9, "unit": "GB/s", "frac": round(work / avg_s / PEAK_HBM_BYTES, 4),
                    "traffic": traffic, "work_per_launch": work, "launches_timed": dk["calls"]}
    gemm_names = ("gateup_fwd", "down_fwd", "down_bwd_dx", "gateup_bwd_dx", "weight_grad:w2", "weight_grad:w13")
    gemm_s = sum(kernels[n]["avg_us"] * (1 if args.graph else kernels[n]["calls"] / table_steps)
                 for n in kernels if n in gemm_names) / 1e6
    gemm_flops = cfg.flops_fwd_bwd() / (3.0 if args.fwd_only else 1.0)

    cpu = None
    if not args.no_cpu_baseline and not args.fwd_only:
        cpu = cpu_baseline(cfg, data, args.cpu_tokens, args.cpu_seconds)

    line = {
        "metric": (METRIC if cfg.layers == 1 else
                   f"MoE FFN stack ({cfg.layers} x RMSNorm+MoE+residual) tokens/sec fwd+bwd (bf16)")
        if not args.fwd_only else "MoE block forward tokens/sec (bf16)",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        # the same-run CPU baseline of this metric (BASELINE.md publishes no
        # number): the reference's module semantics on the box's host cores
        "vs_baseline": (round(tok_s / cpu["value"], 1) if cpu and cpu.get("value") else None),
        "vs_baseline_of": ("cpu_baseline.value: " + cpu["sample"]) if cpu and cpu.get("value") else None,
        "dtype": "bf16",
        "data": f"synthetic (seeded N(0,1) input, N(0,0.02^2) weights, router bias {cfg.bias})",
        "config": {"workload": cfg.name, "tokens": T, "dim": cfg.dim, "inter": cfg.inter,
                   "experts": cfg.n_experts, "topk": cfg.topk, "shared": int(cfg.n_shared > 0),
                   "bias": cfg.bias, "layers": cfg.layers,
                   "pass": "forward" if args.fwd_only else "forward+backward",
                   "launch": "hip-graph replay" if args.graph else "eager",
                   "routed_rows": "read through perm" if args.gather_rows else "x_perm copy",
                   "params": "fp32 under bf16 autocast" if args.autocast else "bf16"},
        # (null when the step runs no separate GEMM entry point: the fused decode forward)
        "grouped_gemm_mfma_frac": round(gemm_flops / gemm_s / PEAK_BF16_FLOPS, 4) if gemm_s > 0 else None,
        "step_mfma_frac": round(gemm_flops / (elapsed / args.steps) / PEAK_BF16_FLOPS, 4),
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    c1 = (cpu or {}).get("c1_fp32_forward")
    if c1 and c1.get("value") and not args.fwd_only:
        line["vs_c1_fp32_forward"] = round(tok_s / c1["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
