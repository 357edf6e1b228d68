"""The allocation-free dispatch (fmoe_dispatch_noalloc) against fmoe_dispatch,
through the C ABI, on two calls in a row (the second smaller, so stale
scratch from the first would show), bit for bit: counts, offsets, perm,
pos_of_slot and the gathered rows are integer / byte results.  Also the host
rejection of a workload beyond the static scratch, and the C oracle."""
import pytest
import torch

from fusionllm_amd import _kernels as K
from fusionllm_amd._lib import FusionMoEError
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


def _inputs(T, d, E, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g).bfloat16()
    gw = (torch.randn(E, d, generator=g) * 0.02).bfloat16()
    gb = (torch.rand(E, generator=g) * 0.2 - 0.1).bfloat16()
    return x, gw, gb


def test_dispatch_noalloc_matches_dispatch_on_two_calls(gpu_device):
    # first a C5-like workload (64 experts, top-6, 469 slot blocks), then a
    # smaller C2-like one (8 experts, top-2)
    for T, d, E, k, seed in ((20000, 2048, 64, 6, 1), (4096, 768, 8, 2, 2)):
        x, gw, gb = _inputs(T, d, E, seed)
        xd = x.to(gpu_device)
        idx, _, _, _ = K.router_fwd(xd, gw.to(gpu_device), gb.to(gpu_device), k, 1.0)
        want = K.dispatch(idx, xd, E)
        got = K.dispatch(idx, xd, E, noalloc=True)
        torch.cuda.synchronize()
        for name, a, b in zip(("counts", "offsets", "perm", "pos", "x_perm"), got, want):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b), (T, name)
        rc, ro, rp, rpos = mo.dispatch_c(idx.cpu(), E)
        assert torch.equal(got[0].cpu(), rc) and torch.equal(got[2].cpu(), rp)


def test_dispatch_noalloc_rejects_workloads_beyond_its_scratch(gpu_device):
    T, d, E, k = 87382, 64, 64, 6  # 2 * ceil(T*k/256) * E int32 = 1 MiB + 512 B
    idx = torch.zeros(T, k, dtype=torch.int32, device=gpu_device)
    x = torch.zeros(T, d, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(FusionMoEError, match="static scratch"):
        K.dispatch(idx, x, E, gather=False, noalloc=True)


def test_dispatch_noalloc_under_hip_graph_capture(gpu_device):
    # The caller it is for: code under HIP-graph capture, which may not
    # allocate.  The dispatch is captured once and replayed on new routings
    # (written into the captured index tensor), with eager work and
    # synchronisations between the replays; every replay equals the eager
    # fmoe_dispatch of the same routing, bit for bit.
    T, d, E, k = 2048, 768, 8, 2
    x, gw, gb = _inputs(T, d, E, 3)
    xd, gwd = x.to(gpu_device), gw.to(gpu_device)
    idx0, _, _, _ = K.router_fwd(xd, gwd, gb.to(gpu_device), k, 1.0)
    K.dispatch(idx0, xd, E, noalloc=True)  # resolves the device's scratch outside the capture
    torch.cuda.synchronize()
    idx_in = idx0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = K.dispatch(idx_in, xd, E, noalloc=True)
    gen = torch.Generator().manual_seed(11)
    for rep in range(4):
        gb_r = (torch.rand(E, generator=gen) * 0.4 - 0.2).bfloat16().to(gpu_device)
        idx_r, _, _, _ = K.router_fwd(xd, gwd, gb_r, k, 1.0)
        idx_in.copy_(idx_r)
        g.replay()
        got = [t.clone() for t in out]
        torch.cuda.synchronize()
        want = K.dispatch(idx_r, xd, E)  # eager work between replays
        torch.cuda.synchronize()
        for name, a, b in zip(("counts", "offsets", "perm", "pos", "x_perm"), got, want):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b), (rep, name)
        z = torch.full((1024,), float(rep), device=gpu_device).sum()  # unrelated eager kernels
        assert float(z) == 1024.0 * rep
