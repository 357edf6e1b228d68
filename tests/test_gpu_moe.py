"""Module-level parity of the drop-in DeepSeekMoE on the GPU.

Reference: the torch-CPU restatement of models/moe.py in bf16 (oracle), run
on the routing the GPU chose (the routing itself is checked bit-exact against
the C router oracle), with autograd for the gradients.

Tolerances (stated here, applied below):
  output y          elementwise rtol 2e-2, atol 2e-3 against the bf16
                    reference composition                  (north star)
  dx                against the fp64 ground truth t (same bf16 operands, same
                    routing, fp64 arithmetic), r = the bf16 reference's dx:
                      rel_L2(dx_gpu, t) <= 1e-2  and  <= 1.5 rel_L2(r, t) + 1e-4
                      |dx_gpu - t| <= |r - t| + (k+2) * 2.5e-3 + 2e-2 |t|
                    Each dx element is a sum of k+2 contributions (k routed
                    experts, the shared expert, the router), each O(1) and
                    rounded to bf16 before the sum on both paths (half an ulp
                    is up to 2e-3 at magnitude 0.5-1); where they cancel, the
                    error of either path is a few 1e-3 on a small result.
  weight gradients  relative L2 <= 1e-2 per tensor (expert, shared and gate)
"""
import numpy as np
import pytest
import torch

from fusionllm_amd import configs
from oracle import moe_oracle as mo
from tests.gpu_util import build_module, close, f32_bits, rel_l2

pytestmark = pytest.mark.gpu

Y_TOL = dict(rtol=2e-2, atol=2e-3)
DX_ATOL_PER_TERM = 2.5e-3
DX_RTOL = 2e-2
W_REL_L2 = 1e-2


def _gpu_run(cfg, data, dev, backward=True):
    m = build_module(cfg, data, dev)
    x = data.x.to(dev, torch.bfloat16).requires_grad_(backward)
    y = m(x)
    # "w": the router's fp32 weights (bit-exact with the C oracle); the
    # reference-facing _last_weights is their bf16 rounding for a bf16 module
    assert m._last_weights.dtype == torch.bfloat16
    out = {"y": y.detach().cpu(), "idx": m._last_indices.cpu(), "w": m._route_weights.cpu(), "module": m}
    if backward:
        y.backward(data.dy.to(dev, torch.bfloat16))
        out["dx"] = x.grad.cpu()
        out["grads"] = {n: (p.grad.cpu() if p.grad is not None else None) for n, p in m.named_parameters()}
    return out


def _oracle_run(cfg, data, idx_gpu, backward=True, dtype=torch.bfloat16):
    """The reference composition on the CPU, on the routing the GPU chose.

    dtype bf16: the reference's bf16 path; dtype fp64: ground truth on the
    same bf16-valued operands (fp64 arithmetic and accumulator).
    """
    sd = {k: v.bfloat16().to(dtype).clone().requires_grad_(backward) for k, v in data.state_dict().items()}
    x = data.x.bfloat16().to(dtype).clone().requires_grad_(backward)
    E, k = cfg.n_experts, cfg.topk
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(E)]
    shared = None
    if cfg.n_shared:
        shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    w, idx = mo.route(x, sd["gate.weight"], sd["gate.bias"], k, cfg.route_scale, mode="fp32", indices=idx_gpu)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    y, _, _ = mo.moe_forward(x, sd["gate.weight"], sd["gate.bias"], experts, shared, k, cfg.route_scale,
                             routing=(w, idx), acc_dtype=acc)
    out = {"y": y.detach(), "w": w.detach()}
    if backward:
        y.backward(data.dy.bfloat16().to(dtype))
        out["dx"] = x.grad
        out["grads"] = {n: t.grad for n, t in sd.items()}
    return out


def _check_dx(dx_gpu, dx_ref, truth, k):
    a, r, t = dx_gpu.double().cpu(), dx_ref.double().cpu(), truth.double().cpu()
    err = (a - t).abs()
    bad = err > (r - t).abs() + (k + 2) * DX_ATOL_PER_TERM + DX_RTOL * t.abs()
    assert not bad.any(), (f"dx: {int(bad.sum())}/{bad.numel()} elements beyond tolerance; "
                           f"max abs err {float(err.max()):.3e}")
    e_gpu, e_ref = rel_l2(a, t), rel_l2(r, t)
    assert e_gpu <= 1e-2, f"dx relative L2 to fp64 truth {e_gpu:.3e}"
    assert e_gpu <= 1.5 * e_ref + 1e-4, f"dx rel L2 {e_gpu:.3e} vs the bf16 reference's {e_ref:.3e}"


def _compare(cfg, data, g, o, backward=True):
    close(g["y"], o["y"], **Y_TOL)
    if not backward:
        return
    truth = _oracle_run(cfg, data, g["idx"], dtype=torch.float64)
    _check_dx(g["dx"], o["dx"], truth["dx"], cfg.topk)
    for name, ref in o["grads"].items():
        got = g["grads"][name]
        if ref is None:
            assert got is None, f"{name}: expected None gradient (expert got no tokens)"
            continue
        assert got is not None, f"{name}: missing gradient"
        assert got.dtype == torch.bfloat16
        err = rel_l2(got, ref)
        assert err <= W_REL_L2, f"{name}: relative L2 error {err:.3e}"


def _routing_exact(data, g, cfg):
    ridx, rw, rv = mo.router_c(data.x.bfloat16(), data.gate_w.bfloat16(), data.gate_b.bfloat16(), cfg.topk,
                               cfg.route_scale)
    assert torch.equal(g["idx"], ridx.long())
    assert torch.equal(f32_bits(g["w"]), f32_bits(rw))


@pytest.mark.parametrize("T", [2048, 777])
def test_c2_block_forward_backward(gpu_device, T):
    cfg = configs.C2
    data = configs.make_block(cfg, seed=0, tokens=T)
    g = _gpu_run(cfg, data, gpu_device)
    _routing_exact(data, g, cfg)
    o = _oracle_run(cfg, data, g["idx"])
    assert torch.equal(f32_bits(g["w"]), f32_bits(o["w"].float())) or torch.allclose(g["w"], o["w"], rtol=4e-7)
    _compare(cfg, data, g, o)


def test_c1_weights_zero_bias(gpu_device):
    cfg = configs.C1
    data = configs.make_block(cfg, seed=0, tokens=1024)
    g = _gpu_run(cfg, data, gpu_device)
    _routing_exact(data, g, cfg)
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"]))


def test_c5_shape_forward_backward(gpu_device):
    cfg = configs.C5
    data = configs.make_block(cfg, seed=0, tokens=384)
    g = _gpu_run(cfg, data, gpu_device)
    _routing_exact(data, g, cfg)
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"]))


@pytest.mark.parametrize("cfg", configs.C3, ids=lambda c: c.name)
def test_c3_decode_forward(gpu_device, cfg):
    data = configs.make_block(cfg, seed=0)
    g = _gpu_run(cfg, data, gpu_device, backward=False)
    _routing_exact(data, g, cfg)
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"], backward=False), backward=False)


@pytest.mark.parametrize("cfg", configs.C3, ids=lambda c: c.name)
def test_c3_inference_forward(gpu_device, cfg):
    # the module's inference branch (no autograd: nothing kept for a backward)
    data = configs.make_block(cfg, seed=0)
    m = build_module(cfg, data, gpu_device)
    with torch.no_grad():
        y = m(data.x.to(gpu_device, torch.bfloat16))
    g = {"y": y.cpu(), "idx": m._last_indices.cpu(), "w": m._route_weights.cpu()}
    _routing_exact(data, g, cfg)
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"], backward=False), backward=False)


def test_empty_experts_get_none_grads(gpu_device):
    cfg = configs.BlockConfig("skew-all", 300, dim=256, inter=512, n_experts=8, topk=2)
    data = configs.make_block(cfg, seed=4)
    data.gate_b[:] = -20.0
    data.gate_b[:2] = 20.0  # every token picks experts 0 and 1
    g = _gpu_run(cfg, data, gpu_device)
    assert g["idx"].unique().tolist() == [0, 1]
    for e in range(2, 8):
        for w in ("w1", "w2", "w3"):
            assert g["grads"][f"experts.{e}.{w}.weight"] is None
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"]))


def test_deterministic_full_c2(gpu_device):
    cfg = configs.C2
    data = configs.make_block(cfg, seed=0)
    a = _gpu_run(cfg, data, gpu_device)
    b = _gpu_run(cfg, data, gpu_device)
    assert torch.equal(a["y"].view(torch.int16), b["y"].view(torch.int16))
    assert torch.equal(a["dx"].view(torch.int16), b["dx"].view(torch.int16))
    for n, t in a["grads"].items():
        assert torch.equal(t.view(torch.int16), b["grads"][n].view(torch.int16)), n


def test_full_c2_routing_exact_and_sampled_rows(gpu_device):
    # Full-size C2: routing bit-exact for all 16384 tokens; the output of 256
    # sampled tokens against the oracle run on just those tokens (the block is
    # token-local).
    cfg = configs.C2
    data = configs.make_block(cfg, seed=0)
    g = _gpu_run(cfg, data, gpu_device, backward=False)
    _routing_exact(data, g, cfg)
    counts = torch.bincount(g["idx"].flatten(), minlength=8)
    assert counts[:2].sum() > 0.6 * counts.sum()  # skewed routing as configured
    sel = torch.from_numpy(np.random.default_rng(0).choice(cfg.tokens, 256, replace=False))
    sub = configs.BlockData(data.x[sel], data.gate_w, data.gate_b, data.experts, data.shared, None)
    o = _oracle_run(cfg, sub, g["idx"][sel], backward=False)
    close(g["y"][sel], o["y"], **Y_TOL)


def test_autocast_fp32_module(gpu_device):
    cfg = configs.BlockConfig("autocast", 512, dim=256, inter=512, n_experts=8, topk=2, bias="skew")
    data = configs.make_block(cfg, seed=6)
    m = build_module(cfg, data, gpu_device, dtype=torch.float32)
    x = data.x.to(gpu_device).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = m(x)
    assert y.dtype == torch.float32
    y.backward(data.dy.to(gpu_device))
    assert x.grad.dtype == torch.float32
    assert all(p.grad is None or p.grad.dtype == torch.float32 for p in m.parameters())
    # oracle under CPU autocast: fp32 x and params, bf16 linears (trainer.py:158)
    sd = {k: v.clone().requires_grad_(True) for k, v in data.state_dict().items()}
    xo = data.x.clone().requires_grad_(True)
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(8)]
    shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    idx = m._last_indices.cpu()
    # the build's router: fp32 logits from the bf16-cast operands (outside autocast)
    w, _ = mo.route(xo.bfloat16(), sd["gate.weight"].bfloat16(), sd["gate.bias"].bfloat16(), 2, 1.0,
                    mode="fp32", indices=idx)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        yo, _, _ = mo.moe_forward(xo, None, None, experts, shared, 2, 1.0, routing=(w, idx))
    assert yo.dtype == torch.float32
    close(y.detach().cpu(), yo.detach(), **Y_TOL)
    yo.backward(data.dy)
    # autocast rounds dy to bf16 at the Linears' backward, so the fp64 truth
    # (bf16-valued operands and dy) applies unchanged
    truth = _oracle_run(cfg, data, idx, dtype=torch.float64)
    _check_dx(x.grad, xo.grad, truth["dx"], cfg.topk)
    for n, p in m.named_parameters():
        ref = sd[n].grad
        assert (p.grad is None) == (ref is None), n
        if ref is not None:
            assert rel_l2(p.grad.cpu(), ref) <= W_REL_L2, n


def test_checkpoint_recompute_matches(gpu_device):
    cfg = configs.BlockConfig("ckpt", 1024, dim=256, inter=512, bias="skew")
    data = configs.make_block(cfg, seed=8)
    m = build_module(cfg, data, gpu_device)
    dy = data.dy.to(gpu_device, torch.bfloat16)
    res = []
    for use_ckpt in (False, True):
        m.zero_grad(set_to_none=True)
        x = data.x.to(gpu_device, torch.bfloat16).requires_grad_(True)
        y = torch.utils.checkpoint.checkpoint(m, x, use_reentrant=False) if use_ckpt else m(x)
        y.backward(dy)
        res.append((y.detach().clone(), x.grad.clone(),
                    [None if p.grad is None else p.grad.clone() for p in m.parameters()]))
    assert torch.equal(res[0][0].view(torch.int16), res[1][0].view(torch.int16))
    assert torch.equal(res[0][1].view(torch.int16), res[1][1].view(torch.int16))
    for a, b in zip(res[0][2], res[1][2]):
        assert (a is None) == (b is None)  # experts without tokens: None on both paths
        if a is not None:
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("cfg,tokens", [(configs.C2, 4096), (configs.C5, 2048)], ids=["C2", "C5"])
@pytest.mark.parametrize("train", [False, True], ids=["inference", "training"])
def test_bias_update_and_aux_loss_on_gpu(gpu_device, cfg, tokens, train):
    # The dispatch histogram stands in for bincount (models/moe.py:93,105):
    # the counts, the bias step and the loss equal the reference formulas.
    data = configs.make_block(cfg, seed=0, tokens=tokens)
    m = build_module(cfg, data, gpu_device)
    x = data.x.to(gpu_device, torch.bfloat16)
    with torch.set_grad_enabled(train):
        y = m(x.requires_grad_(train))
    if train:
        y.float().sum().backward()
    E = cfg.n_experts
    idx, w = m._last_indices, m._last_weights
    assert m._counts_of is idx
    assert torch.equal(m._last_counts.long(), torch.bincount(idx.flatten(), minlength=E))
    want_loss = mo.load_balance_loss(idx, w, E)
    loss = m.get_load_balance_loss()
    assert loss.requires_grad is False and torch.equal(loss, want_loss)
    want_bias = mo.gate_bias_step(m.gate.bias, idx, E, 0.001)
    m.update_gate_bias(0.001)
    assert torch.equal(m.gate.bias.detach(), want_bias)


@pytest.mark.parametrize("T,dim,inter,E,k,shared,rs", [
    (1, 64, 64, 1, 1, 0, 1.0),        # one expert, one token
    (5, 128, 192, 4, 4, 1, 2.5),      # every expert chosen (k = E)
    (300, 256, 320, 16, 3, 0, 1.0),   # no shared expert, odd inter / 64
    (7, 768, 2048, 8, 2, 1, 1.0),     # a decode-sized training step (one-launch routing and dispatch)
    (33, 2048, 1408, 64, 6, 1, 1.0),  # C5 shapes, few tokens
], ids=["E1", "k_eq_E", "no_shared", "tiny_train", "c5_small"])
def test_block_edge_shapes(gpu_device, T, dim, inter, E, k, shared, rs):
    cfg = configs.BlockConfig("edge", T, dim=dim, inter=inter, n_experts=E, topk=k, n_shared=shared,
                              route_scale=rs, bias="uniform:0.1")
    data = configs.make_block(cfg, seed=T + E)
    g = _gpu_run(cfg, data, gpu_device)
    _routing_exact(data, g, cfg)
    _compare(cfg, data, g, _oracle_run(cfg, data, g["idx"]))


def test_zero_tokens_forward_backward(gpu_device):
    # An empty batch (the reference's ops on empty tensors): empty output,
    # zero gradients for the gate and the shared expert, None for the experts.
    cfg = configs.BlockConfig("empty", 4, dim=128, inter=128, n_experts=4, topk=2)
    m = build_module(cfg, configs.make_block(cfg, seed=1), gpu_device)
    x = torch.zeros(2, 0, 128, device=gpu_device, dtype=torch.bfloat16, requires_grad=True)
    y = m(x)
    assert y.shape == (2, 0, 128) and m._last_indices.shape == (0, 2)
    y.sum().backward()
    assert x.grad.shape == x.shape
    assert not m.gate.weight.grad.any() and not m.gate.bias.grad.any()
    assert not m.shared_expert.w1.weight.grad.any()
    assert all(e.w1.weight.grad is None for e in m.experts)
    # the reference's formula divides by T*k and averages over no tokens: NaN
    ref = mo.load_balance_loss(torch.empty(0, 2, dtype=torch.int64), torch.empty(0, 2), 4)
    assert torch.isnan(ref) and torch.isnan(m.get_load_balance_loss().cpu())
