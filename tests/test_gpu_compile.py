"""The block under torch.compile(fullgraph=True): the reference's trainer
compiles the whole model that way (training/trainer.py:39).  Traced, the
block is the fusionllm::moe_fwd / moe_bwd operators (fusionllm_amd.ops); they
run the eager path's kernels in the same order, so outputs and gradients are
bit-equal to the eager module's, except that experts without tokens get zero
gradients instead of None.  Backends: aot_eager (the traced graph run op by
op) and cudagraphs (the same graph captured and replayed as a HIP graph).
"""
import pytest
import torch

from fusionllm_amd import configs, moe_residual
from tests.gpu_util import build_module

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


def _run(m, x, dy, fn):
    m.zero_grad(set_to_none=True)
    xx = x.clone().requires_grad_(True)
    y = fn(xx)
    y.backward(dy)
    return y.detach(), xx.grad, {n: p.grad for n, p in m.named_parameters()}


@pytest.mark.parametrize("backend", ["aot_eager", "cudagraphs"])
def test_compiled_block_matches_eager(gpu_device, backend):
    torch._dynamo.reset()
    cfg = configs.BlockConfig("compile", 512, bias="skew")
    data = configs.make_block(cfg, seed=3)
    m = build_module(cfg, data, gpu_device)
    x = data.x.to(gpu_device, torch.bfloat16)
    dy = data.dy.to(gpu_device, torch.bfloat16)
    y0, dx0, g0 = _run(m, x, dy, m)
    idx0 = m._last_indices.clone()
    cm = torch.compile(m, fullgraph=True, backend=backend)
    for rep in range(3):  # cudagraphs: recorded, then replayed
        y1, dx1, g1 = _run(m, x, dy, cm)
        assert torch.equal(_bits(y1), _bits(y0)), rep
        assert torch.equal(_bits(dx1), _bits(dx0)), rep
        assert torch.equal(m._last_indices, idx0)
        for n, t in g0.items():
            if t is None:  # an expert without tokens: zeros when traced
                assert not g1[n].any(), n
            else:
                assert torch.equal(_bits(g1[n]), _bits(t)), (rep, n)


def test_compiled_block_under_autocast_and_empty_experts(gpu_device):
    # The trainer's setting: fp32 module and input, bf16 autocast
    # (training/trainer.py:158); experts 2..7 receive no tokens.
    torch._dynamo.reset()
    cfg = configs.BlockConfig("compile-ac", 300, dim=256, inter=512, n_experts=8, topk=2)
    data = configs.make_block(cfg, seed=4)
    data.gate_b[:] = -20.0
    data.gate_b[:2] = 20.0
    m = build_module(cfg, data, gpu_device, dtype=torch.float32)
    x = data.x.to(gpu_device)
    dy = data.dy.to(gpu_device)

    def fwd(mod):
        def f(xx):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                return mod(xx)
        return f
    y0, dx0, g0 = _run(m, x, dy, fwd(m))
    y1, dx1, g1 = _run(m, x, dy, torch.compile(fwd(m), fullgraph=True, backend="aot_eager"))
    assert y1.dtype == torch.float32 and torch.equal(_bits(y1), _bits(y0))
    assert torch.equal(_bits(dx1), _bits(dx0))
    for n, t in g0.items():
        if t is None:
            assert n.startswith("experts.") and int(n.split(".")[1]) >= 2 and not g1[n].any(), n
        else:
            assert torch.equal(_bits(g1[n]), _bits(t)), n


def test_compiled_norm_residual_stack(gpu_device):
    # FusionLLMBlock's FFN half, x + moe(norm2(x)), two layers, traced: the
    # RMSNorm and the residual stay torch ops around the block's operator.
    torch._dynamo.reset()
    cfg = configs.BlockConfig("compile-c4", 256, bias="uniform:0.05")
    mods = [build_module(cfg, configs.make_block(cfg, seed=s), gpu_device) for s in (5, 6)]
    norms = [torch.nn.RMSNorm(cfg.dim, eps=1e-6).to(gpu_device, torch.bfloat16) for _ in mods]
    x = configs.make_block(cfg, seed=5).x.to(gpu_device, torch.bfloat16)

    def stack(h):
        for m, n in zip(mods, norms):
            h = moe_residual(h, n, m)
        return h
    with torch.no_grad():
        want = x
        for m, n in zip(mods, norms):
            want = want + m(n(want))
        got = torch.compile(stack, fullgraph=True, backend="aot_eager")(x)
    assert torch.equal(_bits(got), _bits(want))


def test_operator_opcheck(gpu_device):
    cfg = configs.BlockConfig("opcheck", 64, dim=128, inter=256, n_experts=4, topk=2)
    data = configs.make_block(cfg, seed=7)
    m = build_module(cfg, data, gpu_device)
    x = data.x.to(gpu_device, torch.bfloat16).requires_grad_(True)
    args = (x, m.gate.weight, m.gate.bias, m._flat_weights(), 2, 1.0, True, torch.bfloat16)
    torch.library.opcheck(torch.ops.fusionllm.moe_fwd.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


def test_compiled_dense_ffn_matches_eager(gpu_device):
    # DenseFFN (models/fusionllm.py:17-27) traced: the fusionllm::swiglu_fwd /
    # swiglu_bwd operators, bit-equal to the eager module.
    from fusionllm_amd import DenseFFN
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(8)
    f = DenseFFN(256, 512)
    with torch.no_grad():
        for p in f.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    f = f.to(gpu_device, torch.bfloat16)
    x = torch.randn(3, 70, 256, generator=g).to(gpu_device, torch.bfloat16)
    dy = torch.randn(3, 70, 256, generator=g).to(gpu_device, torch.bfloat16)

    def run(fn):
        f.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        y = fn(xx)
        y.backward(dy)
        return y.detach(), xx.grad, [p.grad for p in f.parameters()]
    y0, dx0, g0 = run(f)
    y1, dx1, g1 = run(torch.compile(f, fullgraph=True, backend="aot_eager"))
    assert torch.equal(_bits(y1), _bits(y0)) and torch.equal(_bits(dx1), _bits(dx0))
    for a, b in zip(g1, g0):
        assert torch.equal(_bits(a), _bits(b))
