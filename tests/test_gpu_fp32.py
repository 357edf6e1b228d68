"""fp32 modules outside autocast on the GPU: the reference trainer's
``dtype: fp32`` mode (training/trainer.py:31,158: fp32 parameters, autocast
disabled) and its evaluation (trainer.py:332 -> training/validation.py:34-56:
``model.eval()``, ``torch.no_grad()``, no autocast).

The drop-in runs the same bf16 kernels there as under bf16 autocast: the fp32
operands are cast to bf16 (round to nearest even, one launch), the output is
fp32 and every gradient comes back in fp32.  What pins it:
  * bit-equality with the same module called under
    ``torch.autocast("cuda", dtype=torch.bfloat16)`` (the path
    tests/test_gpu_moe.py::test_autocast_fp32_module checks against the
    reference's autocast composition within the north star's rtol 2e-2 /
    atol 2e-3): output, input gradient and every parameter gradient;
  * the reference's own fp32 computation (oracle, fp32 module, no autocast)
    on the GPU's routing: relative L2 <= 2e-2 for the output, dx and every
    weight gradient.  The bf16 rounding of the operands is the whole
    difference: the reference's own bf16 path sits 0.6 % (output, dx) and up
    to 1.2 % (weight gradients) from its fp32 path at the C2 and C5 shapes.
"""
import pytest
import torch
import torch.nn as nn

from fusionllm_amd import DenseFFN, configs, dense_swiglu, moe_residual
from oracle import moe_oracle as mo
from tests.gpu_util import build_module, rel_l2

pytestmark = pytest.mark.gpu

FP32_REL_L2 = 2e-2


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view(torch.int32)


def _oracle_fp32(cfg, data, idx, backward):
    """The reference composition with fp32 parameters and input, no autocast,
    on the given routing (models/moe.py:79-87 in fp32)."""
    sd = {k: v.clone().requires_grad_(backward) for k, v in data.state_dict().items()}
    x = data.x.clone().requires_grad_(backward)
    E, k = cfg.n_experts, cfg.topk
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(E)]
    shared = None
    if cfg.n_shared:
        shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    w, idx = mo.route(x, sd["gate.weight"], sd["gate.bias"], k, cfg.route_scale, mode="fp32", indices=idx)
    y, _, _ = mo.moe_forward(x, None, None, experts, shared, k, cfg.route_scale, routing=(w, idx))
    out = {"y": y.detach()}
    if backward:
        y.backward(data.dy)
        out["dx"] = x.grad
        out["grads"] = {n: t.grad for n, t in sd.items()}
    return out


@pytest.mark.parametrize("cfg,tokens", [(configs.C2, 4096), (configs.C5, 512)], ids=["C2", "C5"])
def test_fp32_module_eval_outside_autocast(gpu_device, cfg, tokens):
    # compute_validation_loss (training/validation.py:34-56) calls the fp32
    # model this way
    data = configs.make_block(cfg, seed=3, tokens=tokens)
    m = build_module(cfg, data, gpu_device, dtype=torch.float32)
    m.eval()
    x = data.x.to(gpu_device)
    assert not torch.is_autocast_enabled("cuda")
    with torch.no_grad():
        y = m(x)
    assert y.dtype == torch.float32 and y.shape == x.shape
    assert m._last_weights.dtype == torch.float32  # an fp32 gate gives fp32 scores
    idx = m._last_indices.clone()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y_ac = m(x)
    assert m._last_weights.dtype == torch.bfloat16  # the gate's output dtype under autocast
    assert torch.equal(idx, m._last_indices)
    assert torch.equal(_bits(y), _bits(y_ac))
    ref = _oracle_fp32(cfg, data, idx.cpu(), backward=False)
    err = rel_l2(y.cpu(), ref["y"])
    assert err <= FP32_REL_L2, f"output relative L2 to the fp32 reference {err:.3e}"


def test_fp32_training_step_outside_autocast(gpu_device):
    # training/trainer.py with dtype fp32: autocast disabled (trainer.py:158)
    cfg = configs.C2
    data = configs.make_block(cfg, seed=4, tokens=2048)
    runs = []
    for autocast in (False, True):
        m = build_module(cfg, data, gpu_device, dtype=torch.float32)
        x = data.x.to(gpu_device).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y = m(x)
        assert y.dtype == torch.float32
        y.backward(data.dy.to(gpu_device))
        assert x.grad.dtype == torch.float32
        assert all(p.grad is None or p.grad.dtype == torch.float32 for p in m.parameters())
        runs.append((y.detach(), x.grad, {n: p.grad for n, p in m.named_parameters()}, m._last_indices.cpu()))
    (y, dx, grads, idx), (y_ac, dx_ac, grads_ac, idx_ac) = runs
    assert torch.equal(idx, idx_ac)
    assert torch.equal(_bits(y), _bits(y_ac)) and torch.equal(_bits(dx), _bits(dx_ac))
    for n, g in grads.items():
        ga = grads_ac[n]
        assert (g is None) == (ga is None), n
        if g is not None:
            assert torch.equal(_bits(g), _bits(ga)), n
    ref = _oracle_fp32(cfg, data, idx, backward=True)
    assert rel_l2(y.cpu(), ref["y"]) <= FP32_REL_L2
    assert rel_l2(dx.cpu(), ref["dx"]) <= FP32_REL_L2
    for n, r in ref["grads"].items():
        g = grads[n]
        assert (g is None) == (r is None), n
        if r is not None:
            err = rel_l2(g.cpu(), r)
            assert err <= FP32_REL_L2, f"{n}: relative L2 to the fp32 reference {err:.3e}"


def test_fp32_dense_swiglu_outside_autocast(gpu_device):
    # DenseFFN / SwiGLUExpert used alone (models/fusionllm.py:17-27, models/mtp.py:28)
    g = torch.Generator().manual_seed(11)
    d, inter, T = 768, 2048, 1000
    ffn = DenseFFN(d, inter)
    with torch.no_grad():
        for p in ffn.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    ffn = ffn.to(gpu_device)
    x0 = torch.randn(T, d, generator=g)
    dy = torch.randn(T, d, generator=g)
    runs = []
    for autocast in (False, True):
        ffn.zero_grad(set_to_none=True)
        x = x0.to(gpu_device).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y = ffn(x)
        # outside autocast the fp32 Linears give fp32; under autocast bf16
        assert y.dtype == (torch.bfloat16 if autocast else torch.float32)
        y.backward(dy.to(gpu_device, y.dtype))
        runs.append((y.detach().float(), x.grad.clone(), [p.grad.clone() for p in ffn.parameters()]))
    (y, dx, gs), (y_ac, dx_ac, gs_ac) = runs
    assert torch.equal(_bits(y), _bits(y_ac)) and torch.equal(_bits(dx), _bits(dx_ac))
    for a, b in zip(gs, gs_ac):
        assert a.dtype == torch.float32 and torch.equal(_bits(a), _bits(b))
    # the reference's fp32 forward and backward
    xr = x0.clone().requires_grad_(True)
    w1, w3, w2 = (ffn.w1.weight.detach().cpu().clone().requires_grad_(True),
                  ffn.w3.weight.detach().cpu().clone().requires_grad_(True),
                  ffn.w2.weight.detach().cpu().clone().requires_grad_(True))
    yr = mo.swiglu(xr, w1, w3, w2)
    yr.backward(dy)
    assert rel_l2(y.cpu(), yr.detach()) <= FP32_REL_L2
    assert rel_l2(dx.cpu(), xr.grad) <= FP32_REL_L2
    for got, want in zip(gs, (w1.grad, w2.grad, w3.grad)):  # parameters() order: w1, w2, w3
        assert rel_l2(got.cpu(), want) <= FP32_REL_L2
    # mixed dtypes outside autocast raise, as nn.Linear does
    with pytest.raises(RuntimeError):
        dense_swiglu(x0.to(gpu_device, torch.bfloat16), ffn.w1.weight, ffn.w3.weight, ffn.w2.weight)


def test_fp32_norm_residual_outside_autocast(gpu_device):
    # x + MoE(RMSNorm(x)) (models/fusionllm.py:52) with an fp32 block
    cfg = configs.BlockConfig("fp32-block", 1024, bias="uniform:0.05")
    data = configs.make_block(cfg, seed=9)
    runs = []
    for autocast in (False, True):
        m = build_module(cfg, data, gpu_device, dtype=torch.float32)
        norm = nn.RMSNorm(cfg.dim, eps=1e-6).to(gpu_device)
        x = data.x.to(gpu_device).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            out = moe_residual(x, norm, m)
        assert out.dtype == torch.float32
        out.backward(data.dy.to(gpu_device))
        runs.append((out.detach(), x.grad, norm.weight.grad, m.gate.weight.grad, m._last_indices.cpu()))
    a, b = runs
    assert torch.equal(a[4], b[4])
    for u, v in zip(a[:4], b[:4]):
        assert u.dtype == torch.float32 and torch.equal(_bits(u), _bits(v))
    # against the reference block in fp32 on the same routing
    xr = data.x.clone().requires_grad_(True)
    sd = {k: v.clone() for k, v in data.state_dict().items()}
    experts = [(sd[f"experts.{e}.w1.weight"], sd[f"experts.{e}.w3.weight"], sd[f"experts.{e}.w2.weight"])
               for e in range(cfg.n_experts)]
    shared = (sd["shared_expert.w1.weight"], sd["shared_expert.w3.weight"], sd["shared_expert.w2.weight"])
    xn = mo.rms_norm(xr, torch.ones(cfg.dim), 1e-6)
    w, idx = mo.route(xn, sd["gate.weight"], sd["gate.bias"], cfg.topk, 1.0, mode="fp32", indices=a[4])
    y, _, _ = mo.moe_forward(xn, None, None, experts, shared, cfg.topk, 1.0, routing=(w, idx))
    outr = xr + y
    outr.backward(data.dy)
    assert rel_l2(a[0].cpu(), outr.detach()) <= FP32_REL_L2
    assert rel_l2(a[1].cpu(), xr.grad) <= FP32_REL_L2
