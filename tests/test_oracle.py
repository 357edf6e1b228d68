"""Pins the CPU oracle (oracle/) against what the mathematics and torch fix.

Every check is independent of the oracle's own formula: fp64 closed forms
with error bounds, torch's own ops (the reference's third-party dependency),
brute force on tiny inputs, invariants, and planted mistakes that must fail.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as mo
from fusionllm_amd import configs


def ulp_diff_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


# ---- exp / sigmoid -------------------------------------------------------------

def test_expf_against_fp64():
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001), np.linspace(-1, 1, 2001)]).astype(np.float32)
    got = np.array([mo.expf_c(v) for v in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)  # correctly rounded to fp32 (almost always)
    assert ulp_diff_f32(got, want).max() <= 1


def test_expf_special_values():
    assert math.isnan(mo.expf_c(float("nan")))
    assert mo.expf_c(float("inf")) == float("inf")
    assert mo.expf_c(float("-inf")) == 0.0
    assert mo.expf_c(89.0) == float("inf")
    assert mo.expf_c(-104.0) == 0.0
    assert mo.expf_c(0.0) == 1.0
    # denormal results are formed by one final rounding
    for v in (-90.0, -95.5, -100.0, -103.0):
        want = np.float32(math.exp(v))
        assert mo.expf_c(v) == pytest.approx(float(want), rel=2 ** -20, abs=2 ** -149)


def test_sigmoid_against_torch_and_fp64():
    xs = np.linspace(-30, 30, 60001).astype(np.float32)
    got = mo.sigmoid_c_vec(xs)
    ref_t = torch.sigmoid(torch.from_numpy(xs)).numpy()
    ref_64 = (1.0 / (1.0 + np.exp(-xs.astype(np.float64)))).astype(np.float32)
    # both are within 2 ulp of the fp64 value rounded to fp32, so they agree
    # to within 4 ulp of each other
    assert ulp_diff_f32(got, ref_64).max() <= 2
    assert ulp_diff_f32(ref_t, ref_64).max() <= 2
    assert ulp_diff_f32(got, ref_t).max() <= 4


# ---- router ---------------------------------------------------------------------

def _bf16_block(T=512, d=768, E=8, seed=0, bias="skew"):
    cfg = configs.BlockConfig("t", T, dim=d, n_experts=E, bias=bias)
    b = configs.make_block(cfg, seed=seed, experts=False, with_dy=False)
    return b.x.bfloat16(), b.gate_w.bfloat16(), b.gate_b.bfloat16()


@pytest.mark.parametrize("d,E,k", [(768, 8, 2), (2048, 64, 6), (64, 16, 4)])
def test_router_logits_within_fp64_bound(d, E, k):
    x, gw, gb = _bf16_block(T=256, d=d, E=E)
    idx, w, v, logits, scores = mo.router_c(x, gw, gb, k, want_scores=True)
    x64, w64, b64 = x.double(), gw.double(), gb.double()
    exact = x64 @ w64.T + b64
    mag = (x64.abs() @ w64.abs().T) + b64.abs()
    n = d // 16 + 4 + 1  # longest chain: per-lane partial, 4 butterfly adds, bias add
    bound = 1.01 * n * 2.0 ** -24 * mag
    assert ((logits.double() - exact).abs() <= bound).all()


@pytest.mark.parametrize("d,E,k", [(768, 8, 2), (2048, 64, 6)])
def test_router_topk_matches_torch_topk_when_tie_free(d, E, k):
    x, gw, gb = _bf16_block(T=512, d=d, E=E, seed=3)
    idx, w, v, logits, scores = mo.router_c(x, gw, gb, k, want_scores=True)
    # no exact ties among each row's scores at this size
    srt = torch.sort(scores, dim=-1, descending=True).values
    assert (srt[:, :-1] != srt[:, 1:]).all()
    tv, ti = torch.topk(scores, k, dim=-1)
    assert torch.equal(idx.long(), ti)
    assert torch.equal(v, tv)


def test_router_matches_torch_route_except_near_ties():
    # The torch restatement (MKL summation order) agrees with the C router
    # on every token whose k-th / (k+1)-th logit gap exceeds the rounding bound.
    x, gw, gb = _bf16_block(T=2048, d=768, E=8, seed=5)
    k = 2
    idx, w, v, logits, _ = mo.router_c(x, gw, gb, k, want_scores=True)
    tw, ti = mo.route(x, gw, gb, k, 1.0, mode="fp32")
    srt = torch.sort(logits, dim=-1, descending=True).values
    gap = (srt[:, k - 1] - srt[:, k]).abs()
    safe = gap > 1e-4
    assert torch.equal(idx.long()[safe], ti[safe])
    assert (~safe).sum() < 20
    close = torch.equal(idx.long(), ti)
    assert torch.allclose(w[safe], tw[safe], rtol=4e-7, atol=0) or close


@pytest.mark.parametrize("cfg", [configs.C2, configs.C5], ids=["C2", "C5"])
def test_router_differs_from_bf16_module_router_only_at_bf16_near_ties(cfg):
    # Decision D4: the build routes on fp32 logits of the bf16 operands; the
    # reference's bf16 module (and bf16 autocast) rounds logits and scores to
    # bf16 and lets torch.topk order the resulting ties (models/moe.py:46-48).
    # The two choose different expert sets only where the fp64 scores of the
    # k-th and (k+1)-th expert lie within bf16 rounding of each other: score
    # s in (0, 1) is rounded to 2^-9 relative, its logit l (|l| < 8 here) to
    # 2^-9 |l| before the sigmoid, whose slope is at most 1/4.
    T = 4096 if cfg.n_experts == 64 else cfg.tokens
    data = configs.make_block(cfg, seed=0, tokens=T, experts=False, with_dy=False)
    x, gw, gb = data.x.bfloat16(), data.gate_w.bfloat16(), data.gate_b.bfloat16()
    idx, _, _ = mo.router_c(x, gw, gb, cfg.topk, cfg.route_scale)
    _, im = mo.route(x, gw, gb, cfg.topk, cfg.route_scale, mode="module")
    logits = F.linear(x.double(), gw.double(), gb.double())
    s = torch.sigmoid(logits)
    srt = torch.sort(s, dim=-1, descending=True).values
    k = cfg.topk
    gap = srt[:, k - 1] - srt[:, k]
    bound = 2.0 * (2.0 ** -9 * srt[:, k - 1] + 0.25 * 2.0 ** -9 * logits.abs().max(-1).values)
    differ = (torch.sort(idx.long(), -1).values != torch.sort(im, -1).values).any(-1)
    assert differ.any()  # the bf16 module does route differently (seed 0, full size: C2 0.59 %, C5 6.3 % of tokens)
    assert bool((gap[differ] <= bound[differ]).all()), "a set difference that bf16 rounding does not explain"
    # and against fp64 logits on the same operands the build's router agrees everywhere but exact ties
    _, i64 = mo.route(x.double(), gw.double(), gb.double(), k, cfg.route_scale, mode="fp32")
    assert torch.equal(torch.sort(i64, -1).values, torch.sort(idx.long(), -1).values)


@pytest.mark.parametrize("cfg", [configs.C2, configs.C5], ids=lambda c: c.name)
def test_fp32_module_routing_differs_only_within_bf16_operand_rounding(cfg):
    # Decision D19: an fp32 module outside autocast computes on bf16 copies of
    # its operands (fmoe_cast_bf16), so it routes on fp32 logits of the
    # bf16-rounded x, gate weight and bias (the C router, which the GPU
    # matches bit for bit), while the reference's fp32 module routes on the
    # fp32 operands themselves (models/moe.py:46-48).  The expert sets differ
    # only where the fp64 scores of the k-th and (k+1)-th expert lie within
    # what rounding the operands moves them: each product x_i W_ei changes by
    # at most 2^-8 |x_i W_ei|, the bias by 2^-9 |b_e|, a score by at most 1/4
    # of its logit's change (measured at full size, seed 0: C2 24 of 16384
    # tokens (0.15 %) get a different set, 70 a different order; C5 452 of
    # 32768 (1.4 %), 1670).
    T = 4096 if cfg.n_experts == 64 else cfg.tokens
    data = configs.make_block(cfg, seed=0, tokens=T, experts=False, with_dy=False)
    x, gw, gb = data.x.float(), data.gate_w.float(), data.gate_b.float()
    idx, _, _ = mo.router_c(x.bfloat16(), gw.bfloat16(), gb.bfloat16(), cfg.topk, cfg.route_scale)
    _, im = mo.route(x, gw, gb, cfg.topk, cfg.route_scale, mode="module")
    k = cfg.topk
    logits = F.linear(x.double(), gw.double(), gb.double())
    srt = torch.sort(torch.sigmoid(logits), dim=-1, descending=True).values
    gap = srt[:, k - 1] - srt[:, k]
    delta = 2.0 ** -8 * (x.double().abs() @ gw.double().abs().T) + 2.0 ** -9 * gb.double().abs()
    bound = 2 * 0.25 * delta.max(-1).values * 1.01
    differ = (torch.sort(idx.long(), -1).values != torch.sort(im, -1).values).any(-1)
    assert differ.any()
    assert float(differ.double().mean()) < 0.02
    assert bool((gap[differ] <= bound[differ]).all()), "a set difference that operand rounding does not explain"
    # a planted mistake fails: the bound with the bias term alone is too small
    assert not bool((gap[differ] <= (0.5 * 2.0 ** -9 * gb.double().abs().max())).all())


def test_router_normalisation_closed_form():
    x, gw, gb = _bf16_block(T=256, d=768, E=8)
    for rs in (1.0, 2.5):
        idx, w, v = mo.router_c(x, gw, gb, 2, route_scale=rs)
        v64 = v.double()
        want = v64 / (v64.sum(-1, keepdim=True) + 1e-10) * rs
        assert torch.allclose(w.double(), want, rtol=3e-7, atol=0)
        assert torch.allclose(w.double().sum(-1), torch.full((256,), rs, dtype=torch.float64), rtol=1e-6)


def test_router_ties_lowest_index():
    # muP init zeroes the gate (models/fusionllm.py:67-73): every score is 0.5.
    T, d, E, k = 16, 768, 8, 2
    x = torch.randn(T, d).bfloat16()
    gw = torch.zeros(E, d).bfloat16()
    gb = torch.zeros(E).bfloat16()
    idx, w, v = mo.router_c(x, gw, gb, k)
    assert (idx == torch.tensor([0, 1], dtype=torch.int32)).all()
    assert torch.equal(w, torch.full((T, k), 0.5))
    # Duplicate gate rows: experts 5 and 2 tie for first -> 2 wins, then 5.
    gw = torch.randn(E, d).bfloat16() * 0.01
    gw[5] = gw[2] = torch.ones(d).bfloat16() * 0.05
    x = torch.ones(T, d).bfloat16()
    idx, _, _ = mo.router_c(x, gw, gb, k)
    assert (idx == torch.tensor([2, 5], dtype=torch.int32)).all()
    # brute force on random tiny ties
    g = torch.Generator().manual_seed(1)
    for _ in range(50):
        s = torch.randint(0, 3, (6,), generator=g).float()
        _, ti = mo.topk_lowest_index(s[None], 3)
        bf = sorted(range(6), key=lambda e: (-s[e].item(), e))[:3]
        assert ti[0].tolist() == bf


def test_router_nan_ranks_first_and_propagates():
    T, d, E, k = 4, 64, 8, 2
    x = torch.randn(T, d).bfloat16()
    x[1, 3] = float("nan")
    gw = torch.randn(E, d).bfloat16()
    gb = torch.zeros(E).bfloat16()
    idx, w, v = mo.router_c(x, gw, gb, k)
    assert idx[1].tolist() == [0, 1]          # all logits NaN: lowest indices
    assert torch.isnan(w[1]).all()
    assert not torch.isnan(w[0]).any()


def test_planted_router_mistake_is_caught():
    # A transposed operand or a dropped bias must fail the fp64 bound check.
    x, gw, gb = _bf16_block(T=64, d=768, E=8)
    _, _, _, logits, _ = mo.router_c(x, gw, gb, 2, want_scores=True)
    exact = x.double() @ gw.double().T + gb.double()
    dropped_bias = exact - gb.double()
    assert not torch.allclose(logits.double(), dropped_bias, atol=1e-6)


@pytest.mark.parametrize("k,rs", [(1, 1.0), (2, 1.0), (6, 2.5), (8, 1.0)])
def test_router_dlogits_against_fp64_autograd(k, rs):
    # The fp32 restatement of the router backward against torch's fp64 autograd of the
    # reference's normalisation (moe.py:49) and sigmoid (moe.py:47) on the same scores:
    # w = v / (sum v + 1e-10) * rs, dlogit = dv * v * (1 - v).
    g = torch.Generator().manual_seed(7 + k)
    T = 4096
    v = torch.rand(T, k, generator=g, dtype=torch.float64) * 0.98 + 0.01
    v = v.float()
    d_w = torch.randn(T, k, generator=g).float()
    got = mo.router_dlogits(d_w.numpy(), v.numpy(), rs)
    v64 = v.double().requires_grad_(True)
    w = v64 / (v64.sum(-1, keepdim=True) + 1e-10) * rs
    w.backward(d_w.double())
    ref = v64.grad * v64.detach() * (1 - v64.detach())
    err = np.abs(got.astype(np.float64) - ref.numpy())
    scale = np.abs(d_w.numpy()).max() * rs
    assert err.max() <= 1e-5 * scale, err.max()
    if k >= 2:  # (k = 1: w = v / (v + 1e-10) is flat, the gradient is ~0)
        # planted mistakes the bound catches: a dropped normalisation term, a sign flip
        dropped = v64.detach() * (1 - v64.detach()) * d_w.double() * rs / v64.detach().sum(-1, keepdim=True)
        assert np.abs(dropped.numpy() - ref.numpy()).max() > 1e-3 * scale
        assert np.abs(-got - ref.numpy()).max() > 1e-3 * scale


# ---- dispatch -------------------------------------------------------------------

@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (37, 8, 2), (4096, 8, 2), (1000, 64, 6)])
def test_dispatch_matches_stable_argsort(T, E, k):
    g = torch.Generator().manual_seed(T)
    # distinct experts per token (as top-k produces)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    counts, offsets, perm, pos = mo.dispatch_c(idx, E)
    flat = idx.flatten().long()
    assert torch.equal(perm.long(), torch.argsort(flat, stable=True))
    assert torch.equal(counts.long(), torch.bincount(flat, minlength=E))
    assert offsets[0] == 0 and torch.equal(offsets[1:].long(), torch.cumsum(counts.long(), 0))
    assert torch.equal(pos.long()[perm.long()], torch.arange(T * k))
    # segments are contiguous and token-ascending
    tok = perm.long() // k
    for e in range(E):
        seg = flat[perm.long()][offsets[e]:offsets[e + 1]]
        assert (seg == e).all()
        st = tok[offsets[e]:offsets[e + 1]]
        assert (st[1:] > st[:-1]).all()


# ---- expert FFN, combine, backward ------------------------------------------------

def _tiny(T=24, d=16, I=32, E=4, k=2, shared=True, dtype=torch.float64, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: (torch.randn(*s, generator=g, dtype=torch.float64) * 0.3).to(dtype)
    x = r(T, d) * 3
    gw, gb = r(E, d), r(E)
    experts = [(r(I, d), r(I, d), r(d, I)) for _ in range(E)]
    sh = (r(I, d), r(I, d), r(d, I)) if shared else None
    return x, gw, gb, experts, sh


def test_swiglu_closed_form():
    x, _, _, ex, _ = _tiny()
    w1, w3, w2 = ex[0]
    a, b = x @ w1.T, x @ w3.T
    want = ((a / (1 + torch.exp(-a))) * b) @ w2.T
    assert torch.allclose(mo.swiglu(x, w1, w3, w2), want, rtol=1e-12, atol=1e-12)


def test_combine_equals_dense_brute_force():
    x, gw, gb, ex, sh = _tiny(E=5, k=3)
    y, w, idx = mo.moe_forward(x, gw, gb, ex, sh, 3, 1.0, mode="fp32")
    want = torch.zeros_like(x)
    for t in range(x.shape[0]):
        for j in range(3):
            e = int(idx[t, j])
            want[t] += w[t, j].double() * mo.swiglu(x[t:t + 1], *ex[e])[0]
        want[t] += mo.swiglu(x[t:t + 1], *sh)[0]
    # the reference accumulates the routed sum in fp32 (moe.py:65) even for
    # fp64 inputs, so agreement is to fp32 precision
    assert torch.allclose(y, want, rtol=2e-6, atol=1e-6)
    # planted mistakes: dropping the shared term or a routing weight must fail
    assert not torch.allclose(y, want - mo.swiglu(x, *sh), atol=1e-6)


def test_gradcheck_fp64():
    x, gw, gb, ex, sh = _tiny(T=6, d=8, I=8, E=4, k=2)
    leaves = [x, gw, gb] + [w for e in ex for w in e] + list(sh)
    for t in leaves:
        t.requires_grad_(True)

    def f(x, gw, gb, *ws):
        exs = [tuple(ws[3 * e:3 * e + 3]) for e in range(4)]
        return mo.moe_forward(x, gw, gb, exs, tuple(ws[12:15]), 2, 1.0, mode="module",
                              acc_dtype=torch.float64)[0]

    assert torch.autograd.gradcheck(f, tuple(leaves), eps=1e-6, atol=1e-5)


def test_block_forward_residual_and_norm():
    x, gw, gb, ex, sh = _tiny()
    nw = torch.ones(x.shape[1], dtype=torch.float64)
    out = mo.block_forward(x, nw, dict(gate_w=gw, gate_b=gb, experts=ex, shared=sh, k=2))
    xn = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)
    y, _, _ = mo.moe_forward(xn, gw, gb, ex, sh, 2)
    assert torch.allclose(out, x + y, rtol=1e-12, atol=1e-12)


def test_rms_norm_is_torch_rms_norm_and_planted_mistakes_fail():
    # oracle.rms_norm is nn.RMSNorm(dim, eps=1e-6) of models/fusionllm.py:48
    # (F.rms_norm); fp64 closed form x / sqrt(mean(x^2) + eps) * w, and the
    # 1-ulp bf16 check used against the kernel rejects a norm without its
    # weight or without eps.
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 768, generator=g, dtype=torch.float64)
    w = 1.0 + 0.1 * torch.randn(768, generator=g, dtype=torch.float64)
    want = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    assert torch.allclose(mo.rms_norm(x, w), want, rtol=1e-13, atol=0)

    def ulps(a, b):
        def key(t):
            i = t.contiguous().view(torch.int16).to(torch.int32)
            return torch.where(i < 0, -(i & 0x7FFF), i)
        return int((key(a) - key(b)).abs().max())

    xb, wb = x.bfloat16(), w.bfloat16()
    ref = mo.rms_norm(xb, wb, 1e-6)
    x64, w64 = xb.double(), wb.double()
    want = x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + 1e-6) * w64
    assert ulps(ref, want.bfloat16()) <= 1
    assert ulps(mo.rms_norm(xb, None, 1e-6), ref) > 1
    xb[0] = 1e-4
    ref = mo.rms_norm(xb, wb, 1e-6)
    assert ulps(mo.rms_norm(xb, wb, 0.0)[0], ref[0]) > 1


def test_normuon_oracle_closed_forms():
    # training/optimizer.py:18-58.  Constant gradient g from zero state: the
    # bias-corrected moments are g and g^2 at every step, so the update is
    # u = g / (|g| + eps) (then each matrix row divided by its RMS + eps), and
    # with wd = 0 the parameter moves by -lr * u per step.
    g64 = torch.Generator().manual_seed(1)
    p0 = torch.randn(6, 8, generator=g64, dtype=torch.float64)
    g = torch.randn(6, 8, generator=g64, dtype=torch.float64)
    p, st = p0.clone(), {}
    for t in range(1, 4):
        mo.normuon_step(p, g, st, lr=0.01, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)
        u = g / (g.abs() + 1e-8)
        rms = u.norm(dim=-1, keepdim=True) / (8 ** 0.5 + 1e-8)
        u = u / (rms + 1e-8)
        assert torch.allclose(p, p0 - 0.01 * t * u, rtol=0, atol=1e-12)
        assert st["step"] == t
        assert torch.allclose(st["exp_avg"], (1 - 0.9 ** t) * g, rtol=1e-12, atol=0)
    # a vector: no row normalisation, plain (not cautious) decay
    v0 = torch.randn(8, generator=g64, dtype=torch.float64)
    gv = torch.randn(8, generator=g64, dtype=torch.float64)
    v, st = v0.clone(), {}
    mo.normuon_step(v, gv, st, lr=0.01, eps=1e-8, weight_decay=0.1)
    assert torch.allclose(v, v0 * (1 - 0.001) - 0.01 * gv / (gv.abs() + 1e-8), rtol=0, atol=1e-12)
    # cautious decay: only where grad * param > 0
    q0 = torch.tensor([[1.0, -1.0, 2.0, -2.0]], dtype=torch.float64)
    gq = torch.tensor([[1.0, 1.0, -1.0, -1.0]], dtype=torch.float64)
    q, st = q0.clone(), {}
    mo.normuon_step(q, gq, st, lr=0.01, eps=0.0, weight_decay=0.5)
    decayed = q0 * torch.tensor([[1 - 0.005, 1.0, 1.0, 1 - 0.005]], dtype=torch.float64)
    assert torch.allclose(q, decayed - 0.01 * gq.sign(), rtol=0, atol=1e-12)


def test_normuon_oracle_bf16_matches_fp32_reference():
    # The bf16 path (GPU scalar semantics, per-operation rounding) stays
    # within bf16 rounding of the reference's fp32 operations on the same
    # bf16-valued inputs (a dropped bias correction or a wrong scalar would not).
    g = torch.Generator().manual_seed(2)
    p16 = (torch.randn(16, 64, generator=g) * 0.02).bfloat16()
    g16 = (torch.randn(16, 64, generator=g) * 1e-3).bfloat16()
    p32, s16, s32 = p16.float(), {}, {}
    mo.normuon_step(p16, g16, s16, lr=0.02, weight_decay=0.1)
    mo.normuon_step(p32, g16.float(), s32, lr=0.02, weight_decay=0.1)
    assert torch.allclose(s16["exp_avg"].float(), s32["exp_avg"], rtol=2 ** -7, atol=0)
    assert torch.allclose(s16["exp_avg_sq"].float(), s32["exp_avg_sq"], rtol=2 ** -7, atol=0)
    assert torch.allclose(p16.float(), p32, rtol=2 ** -7, atol=0.02 * 2 ** -6)
