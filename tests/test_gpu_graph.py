"""HIP-graph replay of the decode-sized forward (workload C3) on the GPU.

Every replay, with eager work and synchronisations between replays, is
checked bit for bit against the eager forward of the same input (the
captured launches are the eager ones), including the routing outputs.
"""
import pytest
import torch

from fusionllm_amd import DecodeGraph, configs
from tests.gpu_util import build_module

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", configs.C3, ids=lambda c: c.name)
def test_decode_graph_replays_match_eager(gpu_device, cfg):
    data = configs.make_block(cfg, seed=1)
    m = build_module(cfg, data, gpu_device)
    x0 = data.x.to(gpu_device, torch.bfloat16)
    g = DecodeGraph(m, x0)
    gen = torch.Generator().manual_seed(5)
    for rep in range(4):
        x = (torch.randn(x0.shape, generator=gen) * (1 + rep)).to(gpu_device, torch.bfloat16)
        y = g(x).clone()
        idx, w, wl = m._last_indices.clone(), m._route_weights.clone(), m._last_weights.clone()
        torch.cuda.synchronize()
        with torch.no_grad():
            want = m(x)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"replay {rep}"
        assert torch.equal(idx, m._last_indices) and torch.equal(w.view(torch.int32), m._route_weights.view(torch.int32))
        assert wl.dtype == torch.bfloat16 and torch.equal(wl.view(torch.int16), m._last_weights.view(torch.int16))
        z = torch.full((1024,), float(rep), device=gpu_device).sum()  # unrelated eager kernels
        assert float(z) == 1024.0 * rep


def test_decode_graph_replay_in_place(gpu_device):
    cfg = configs.C3[1]
    data = configs.make_block(cfg, seed=2)
    m = build_module(cfg, data, gpu_device)
    g = DecodeGraph(m, data.x.to(gpu_device, torch.bfloat16))
    x = (torch.randn(data.x.shape, generator=torch.Generator().manual_seed(9)) * 3).to(gpu_device, torch.bfloat16)
    g.x.copy_(x)  # the caller writes the tokens into the captured input
    y = g.replay().clone()
    with torch.no_grad():
        want = m(x)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
