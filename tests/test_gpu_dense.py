"""Parity of the dense SwiGLU on the one-group kernels (DenseFFN,
models/fusionllm.py:17-27; SwiGLUExpert used on its own, models/mtp.py:28).

Reference: oracle.moe_oracle.swiglu (F.linear / F.silu, models/moe.py:20-21)
on the CPU in bf16 (the reference composition) and in fp64 on the same bf16
operands (ground truth).

Tolerances (stated here, applied below):
  y                 elementwise rtol 2e-2, atol 2e-3 against the bf16
                    reference (north star)
  dx                rel-L2 to the fp64 truth <= 1e-2 and <= 1.5x the bf16
                    reference's own (+1e-4); elementwise
                    |dx - t| <= |dx_ref - t| + 3 * 2.5e-3 + 2e-2 |t|:
                    the reference rounds da.w1 and db.w3 to bf16 and then
                    their sum (3 roundings of O(1) terms), the kernel one
                    K = 2I product (1 rounding); where the terms cancel, the
                    reference's rounding shows as absolute error (a CPU
                    emulation of the one-product path at T=1000, d=2048,
                    I=1408 exceeds the one-rounding bound by up to 3.8e-3)
  dW1, dW3, dW2     rel-L2 <= 1e-2 against the bf16 reference
"""
import pytest
import torch

from fusionllm_amd import DenseFFN, SwiGLUExpert
from oracle import moe_oracle as mo
from tests.gpu_util import close, rel_l2

pytestmark = pytest.mark.gpu

Y_TOL = dict(rtol=2e-2, atol=2e-3)


def _data(T, d, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g)
    ws = (torch.randn(I, d, generator=g) * 0.02, torch.randn(I, d, generator=g) * 0.02,
          torch.randn(d, I, generator=g) * 0.02)
    dy = torch.randn(T, d, generator=g)
    return x, ws, dy


def _oracle(x, ws, dy, dtype):
    xs = x.bfloat16().to(dtype).requires_grad_(True)
    w1, w3, w2 = (w.bfloat16().to(dtype).requires_grad_(True) for w in ws)
    y = mo.swiglu(xs, w1, w3, w2)
    y.backward(dy.bfloat16().to(dtype))
    return y.detach(), xs.grad, (w1.grad, w3.grad, w2.grad)


def _module(cls, ws, dev, dtype=torch.bfloat16):
    I, d = ws[0].shape
    m = cls(d, I)
    with torch.no_grad():
        m.w1.weight.copy_(ws[0])
        m.w3.weight.copy_(ws[1])
        m.w2.weight.copy_(ws[2])
    return m.to(device=dev, dtype=dtype)


@pytest.mark.parametrize("T,d,I", [(1, 768, 2048), (77, 768, 2048), (4096, 768, 2048), (1000, 2048, 1408)])
def test_dense_ffn_forward_backward(gpu_device, T, d, I):
    x, ws, dy = _data(T, d, I, seed=T + d)
    m = _module(DenseFFN, ws, gpu_device)
    xg = x.to(gpu_device, torch.bfloat16).requires_grad_(True)
    y = m(xg)
    assert y.dtype == torch.bfloat16 and y.shape == (T, d)
    y.backward(dy.to(gpu_device, torch.bfloat16))
    y_ref, dx_ref, g_ref = _oracle(x, ws, dy, torch.bfloat16)
    _, dx_t, _ = _oracle(x, ws, dy, torch.float64)
    close(y.detach(), y_ref, **Y_TOL)
    a, r, t = xg.grad.double().cpu(), dx_ref.double(), dx_t
    bad = (a - t).abs() > (r - t).abs() + 3 * 2.5e-3 + 2e-2 * t.abs()
    assert not bad.any(), f"dx: {int(bad.sum())} elements beyond tolerance"
    e_gpu, e_ref = rel_l2(a, t), rel_l2(r, t)
    assert e_gpu <= 1e-2 and e_gpu <= 1.5 * e_ref + 1e-4, (e_gpu, e_ref)
    for p, ref, name in ((m.w1.weight, g_ref[0], "w1"), (m.w3.weight, g_ref[1], "w3"), (m.w2.weight, g_ref[2], "w2")):
        assert p.grad.dtype == torch.bfloat16
        assert rel_l2(p.grad.cpu(), ref) <= 1e-2, name


def test_swiglu_expert_alone_equals_dense_ffn(gpu_device):
    # The MTP module's SwiGLUExpert (models/mtp.py:28) takes the same path.
    x, ws, dy = _data(300, 768, 2048, seed=5)
    outs = []
    for cls in (SwiGLUExpert, DenseFFN):
        m = _module(cls, ws, gpu_device)
        xg = x.to(gpu_device, torch.bfloat16).requires_grad_(True)
        y = m(xg.view(3, 100, 768))
        assert y.shape == (3, 100, 768)
        y.backward(dy.to(gpu_device, torch.bfloat16).view(3, 100, 768))
        outs.append((y.detach(), xg.grad, m.w1.weight.grad, m.w2.weight.grad))
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_dense_ffn_autocast_fp32(gpu_device):
    # training/trainer.py:158: fp32 module and input under bf16 autocast; the
    # Linears give a bf16 output, the gradients come back in fp32.
    x, ws, dy = _data(512, 768, 2048, seed=9)
    m = _module(DenseFFN, ws, gpu_device, dtype=torch.float32)
    xg = x.to(gpu_device).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = m(xg)
    assert y.dtype == torch.bfloat16
    y.backward(dy.to(gpu_device, torch.bfloat16))
    assert xg.grad.dtype == torch.float32 and m.w1.weight.grad.dtype == torch.float32
    y_t, dx_t, g_t = _oracle(x, ws, dy, torch.float64)
    assert rel_l2(y.detach().cpu(), y_t) <= 1e-2
    assert rel_l2(xg.grad.cpu(), dx_t) <= 1e-2
    for p, t in zip((m.w1.weight, m.w3.weight, m.w2.weight), g_t):
        assert rel_l2(p.grad.cpu(), t) <= 1e-2
