"""Kernel-level parity on the GPU, called through the C ABI.

Router and dispatch (integer / index work and the fp32 router) must be bit
exact against the C oracle; the grouped GEMMs are compared with a plain
PyTorch fp32 product of the same bf16 operands (tolerances stated per test).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fusionllm_amd import _kernels as K
from fusionllm_amd import configs
from oracle import moe_oracle as mo
from tests.gpu_util import close, f32_bits, rel_l2

pytestmark = pytest.mark.gpu


def _routing_inputs(T, d, E, seed, bias="skew"):
    cfg = configs.BlockConfig("t", T, dim=d, n_experts=E, bias=bias)
    b = configs.make_block(cfg, seed=seed, experts=False, with_dy=False)
    return b.x.bfloat16(), b.gate_w.bfloat16(), b.gate_b.bfloat16()


def _check_router(x, gw, gb, k, rs, dev):
    idx, idx64, w, v = K.router_fwd(x.to(dev), gw.to(dev), gb.to(dev), k, rs)
    ridx, rw, rv = mo.router_c(x, gw, gb, k, rs)
    assert torch.equal(idx.cpu(), ridx)
    assert torch.equal(idx64.cpu(), ridx.long())
    wc, vc = w.cpu(), v.cpu()
    assert torch.equal(torch.isnan(wc), torch.isnan(rw))
    ok = ~torch.isnan(rw)
    assert torch.equal(f32_bits(wc)[ok], f32_bits(rw)[ok])
    assert torch.equal(f32_bits(vc)[ok], f32_bits(rv)[ok])
    return idx


@pytest.mark.parametrize("T,d,E,k,rs", [(2048, 768, 8, 2, 1.0), (1, 768, 8, 2, 1.0), (333, 768, 8, 2, 2.5),
                                        (512, 2048, 64, 6, 1.0), (200, 256, 16, 4, 1.0), (64, 64, 3, 3, 1.0),
                                        # decode-sized batches (one workgroup per token) and the boundary
                                        (128, 2048, 64, 6, 1.0), (129, 768, 8, 2, 1.0), (5, 768, 8, 2, 2.5),
                                        (17, 256, 33, 8, 1.0),
                                        # more than 16 experts above 128 tokens (8-token x S-expert
                                        # blocks per 16-lane group): dim not a multiple of 128, E not a
                                        # multiple of 8, a partial last workgroup
                                        (300, 192, 40, 5, 1.0), (257, 64, 64, 8, 1.0), (1000, 1344, 48, 6, 2.5),
                                        (4097, 2048, 64, 6, 1.0), (200, 768, 17, 3, 1.0)])
def test_router_bit_exact(gpu_device, T, d, E, k, rs):
    x, gw, gb = _routing_inputs(T, d, E, seed=T + E)
    _check_router(x, gw, gb, k, rs, gpu_device)


def test_router_ties_and_nan(gpu_device):
    T, d, E, k = 64, 768, 8, 2
    x = torch.randn(T, d).bfloat16()
    x[7, 5] = float("nan")
    gw = torch.zeros(E, d).bfloat16()  # muP-style zero gate: all scores 0.5
    gb = torch.zeros(E).bfloat16()
    idx = _check_router(x, gw, gb, k, 1.0, gpu_device)
    assert (idx.cpu()[torch.arange(T) != 7] == torch.tensor([0, 1], dtype=torch.int32)).all()
    gw = (torch.randn(E, d) * 0.02).bfloat16()
    gw[6] = gw[3]  # duplicate experts: exact ties broken toward 3
    _check_router(x, gw, gb, k, 1.0, gpu_device)


@pytest.mark.parametrize("T,d,E,k", [(16384, 768, 8, 2), (1, 768, 8, 2), (129, 768, 8, 2), (3000, 2048, 64, 6),
                                     # single-launch path for <= 256 slots, and its boundary
                                     (128, 768, 8, 2), (3, 2048, 64, 6), (40, 256, 64, 6), (37, 64, 3, 3)])
def test_dispatch_bit_exact(gpu_device, T, d, E, k):
    x, gw, gb = _routing_inputs(T, d, E, seed=7)
    xd = x.to(gpu_device)
    idx, _, _, _ = K.router_fwd(xd, gw.to(gpu_device), gb.to(gpu_device), k, 1.0)
    counts, offsets, perm, pos, x_perm = K.dispatch(idx, xd, E)
    rc, ro, rp, rpos = mo.dispatch_c(idx.cpu(), E)
    assert torch.equal(counts.cpu(), rc)
    assert torch.equal(offsets.cpu(), ro)
    assert torch.equal(perm.cpu(), rp)
    assert torch.equal(pos.cpu(), rpos)
    assert torch.equal(perm.cpu().long(), torch.argsort(idx.cpu().flatten().long(), stable=True))
    assert torch.equal(x_perm.cpu().view(torch.int16), x[rp.long() // k].view(torch.int16))


@pytest.mark.parametrize("T,d,E,k", [(5, 4096, 8, 2), (100, 2048, 8, 2), (100, 2112, 8, 2)])
def test_dispatch_given_indices(gpu_device, T, d, E, k):
    # indices chosen here (no router: it takes dim <= 2048), around the row
    # width up to which tiny batches use the one-launch dispatch
    g = torch.Generator().manual_seed(T + d)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    x = torch.randn(T, d, generator=g).bfloat16()
    counts, offsets, perm, pos, x_perm = K.dispatch(idx.to(gpu_device), x.to(gpu_device), E)
    rc, ro, rp, rpos = mo.dispatch_c(idx, E)
    assert torch.equal(counts.cpu(), rc) and torch.equal(offsets.cpu(), ro)
    assert torch.equal(perm.cpu(), rp) and torch.equal(pos.cpu(), rpos)
    assert torch.equal(x_perm.cpu().view(torch.int16), x[rp.long() // k].view(torch.int16))


@pytest.mark.parametrize("T", [5000, 200])
def test_dispatch_all_on_one_expert(gpu_device, T):
    d, E, k = 64, 8, 1
    idx = torch.full((T, k), 5, dtype=torch.int32)
    x = torch.randn(T, d).bfloat16()
    counts, offsets, perm, pos, x_perm = K.dispatch(idx.to(gpu_device), x.to(gpu_device), E)
    assert counts.cpu().tolist() == [0, 0, 0, 0, 0, T, 0, 0]
    assert torch.equal(perm.cpu(), torch.arange(T, dtype=torch.int32))
    assert torch.equal(pos.cpu(), torch.arange(T, dtype=torch.int32))
    assert torch.equal(x_perm.cpu().view(torch.int16), x.view(torch.int16))


@pytest.mark.parametrize("T,d,E,k,rs", [(16384, 768, 8, 2, 1.0), (777, 768, 8, 2, 2.5), (1, 768, 8, 2, 1.0),
                                        (31, 512, 16, 4, 1.0), (32, 768, 8, 2, 1.0), (33, 2048, 64, 6, 1.0),
                                        (4096, 2048, 64, 6, 1.0), (129, 1024, 32, 8, 1.0), (200, 64, 3, 3, 1.0),
                                        # many scan blocks: 2048 (and 1024 in fmoe_dispatch) with 64 experts;
                                        # 1250 (313) with 5 experts, which do not divide 64
                                        (65536, 256, 64, 4, 1.0), (40000, 128, 5, 2, 1.0)])
def test_route_and_dispatch_equals_router_then_dispatch(gpu_device, T, d, E, k, rs):
    # fmoe_route_and_dispatch (router with the dispatch histogram, scan, scatter with the row
    # copies) against fmoe_router_fwd + fmoe_dispatch and the C oracle: every output bit-equal
    x, gw, gb = _routing_inputs(T, d, E, seed=T + 3 * E)
    xd, gwd, gbd = x.to(gpu_device), gw.to(gpu_device), gb.to(gpu_device)
    counts_host = torch.full((E,), -1, dtype=torch.int32).pin_memory()
    got = K.route_and_dispatch(xd, gwd, gbd, k, rs, counts_host=counts_host)
    torch.cuda.synchronize()
    assert torch.equal(counts_host, got[4].cpu())  # the host copy written by the kernel
    idx, idx64, w, v = K.router_fwd(xd, gwd, gbd, k, rs)
    ref = (idx, idx64, w, v) + tuple(K.dispatch(idx, xd, E))
    names = ("idx", "idx64", "weights", "topv", "counts", "offsets", "perm", "pos", "x_perm")
    for n, a, b in zip(names, got, ref):
        if a.dtype == torch.float32:
            a, b = f32_bits(a.cpu()), f32_bits(b.cpu())
        elif a.dtype == torch.bfloat16:
            a, b = a.cpu().view(torch.int16), b.cpu().view(torch.int16)
        assert torch.equal(a.cpu(), b.cpu()), n
    ridx, _, _ = mo.router_c(x, gw, gb, k, rs)
    rc, ro, rp, rpos = mo.dispatch_c(ridx, E)
    assert torch.equal(got[0].cpu(), ridx) and torch.equal(got[6].cpu(), rp) and torch.equal(got[4].cpu(), rc)
    # without the gather: the same index outputs
    nog = K.route_and_dispatch(xd, gwd, gbd, k, rs, gather=False)
    assert nog[8] is None and torch.equal(nog[6].cpu(), rp) and torch.equal(nog[7].cpu(), rpos)


@pytest.mark.parametrize("case", ["all_tied", "one_expert"])
def test_route_and_dispatch_degenerate_routing(gpu_device, case):
    # all_tied: zero gate and bias, so every score is 0.5 and each token takes experts 0..k-1
    # (lowest index first), two full groups and six empty ones; one_expert: a bias that puts
    # every first choice on expert 5.  Against router + dispatch and the C oracle.
    T, d, E, k = 5000, 768, 8, 2
    x, gw, gb = _routing_inputs(T, d, E, seed=11)
    if case == "all_tied":
        gw = torch.zeros_like(gw)
        gb = torch.zeros_like(gb)
    else:
        gb = torch.full_like(gb, -20.0)
        gb[5] = 20.0
    xd, gwd, gbd = x.to(gpu_device), gw.to(gpu_device), gb.to(gpu_device)
    counts_host = torch.full((E,), -1, dtype=torch.int32).pin_memory()
    got = K.route_and_dispatch(xd, gwd, gbd, k, 1.0, counts_host=counts_host)
    torch.cuda.synchronize()
    assert torch.equal(counts_host, got[4].cpu())
    idx, idx64, w, v = K.router_fwd(xd, gwd, gbd, k, 1.0)
    ref = (idx, idx64, w, v) + tuple(K.dispatch(idx, xd, E))
    for a, b in zip(got, ref):
        if a.dtype == torch.float32:
            a, b = f32_bits(a.cpu()), f32_bits(b.cpu())
        elif a.dtype == torch.bfloat16:
            a, b = a.cpu().view(torch.int16), b.cpu().view(torch.int16)
        assert torch.equal(a.cpu(), b.cpu())
    ridx, _, _ = mo.router_c(x, gw, gb, k, 1.0)
    rc, ro, rp, rpos = mo.dispatch_c(ridx, E)
    assert torch.equal(got[0].cpu(), ridx) and torch.equal(got[6].cpu(), rp)
    counts = got[4].cpu().tolist()
    if case == "all_tied":
        assert counts == [T, T] + [0] * (E - 2)
        assert torch.equal(got[0].cpu(), torch.tensor([[0, 1]] * T, dtype=torch.int32))
    else:
        assert counts[5] == T and sum(counts) == T * k


def test_route_and_dispatch_empty_batch(gpu_device):
    d, E, k = 768, 8, 2
    x = torch.empty(0, d, dtype=torch.bfloat16, device=gpu_device)
    gw = torch.randn(E, d, device=gpu_device).bfloat16()
    gb = torch.zeros(E, device=gpu_device).bfloat16()
    counts_host = torch.full((E,), -1, dtype=torch.int32).pin_memory()
    out = K.route_and_dispatch(x, gw, gb, k, 1.0, counts_host=counts_host)
    torch.cuda.synchronize()
    assert counts_host.tolist() == [0] * E
    assert out[4].cpu().tolist() == [0] * E and out[5].cpu().tolist() == [0] * (E + 1)
    assert out[6].numel() == 0 and out[8].shape == (0, d)


@pytest.mark.parametrize("T,d,E,k,gdt,empty", [(16384, 768, 8, 2, torch.bfloat16, None),
                                              (777, 512, 8, 2, torch.float32, 3),
                                              (2000, 2048, 64, 6, torch.bfloat16, None),
                                              (129, 256, 6, 3, torch.float32, None),
                                              (1, 64, 4, 2, torch.float32, None)])
def test_router_bwd(gpu_device, T, d, E, k, gdt, empty):
    # fmoe_router_bwd (logit gradients formed inside the gate partial kernel, chunk partials
    # added in chunk order): d_logits bit-equal to the oracle's fp32 restatement of the
    # autograd of moe.py:46-49; the gate weight and bias gradients against their fp64
    # closed forms sum_{slots of e} dlogit * x_token and sum_{slots of e} dlogit, an expert
    # without slots exactly zero.  Shapes cover chunk tails (experts of non-multiples of 32
    # rows), 64 experts at top-6 and a single token.
    rs = 1.5
    x, gw, gb = _routing_inputs(T, d, E, seed=T + E)
    if empty is not None:
        gb = gb.clone()
        gb[empty] = -30.0  # never selected
    xd, gwd, gbd = x.to(gpu_device), gw.to(gpu_device), gb.to(gpu_device)
    idx, _, _, v = K.router_fwd(xd, gwd, gbd, k, rs)
    counts, offsets, perm, pos, x_perm = K.dispatch(idx, xd, E)
    g = torch.Generator().manual_seed(5)
    d_w = torch.randn(T, k, generator=g).float()
    d_logits, dgw, dgb = K.router_bwd(d_w.to(gpu_device), v, perm, offsets, xd, E, rs, gdt)
    ref_dl = mo.router_dlogits(d_w.numpy(), v.cpu().numpy(), rs)
    assert torch.equal(f32_bits(d_logits.cpu()), f32_bits(torch.from_numpy(ref_dl)))
    dl64 = torch.from_numpy(ref_dl).double().reshape(-1)
    e_of = idx.cpu().long().reshape(-1)
    tok = torch.arange(T).repeat_interleave(k)
    W = torch.zeros(E, d, dtype=torch.float64).index_add_(0, e_of, dl64[:, None] * x.double()[tok])
    B = torch.zeros(E, dtype=torch.float64).index_add_(0, e_of, dl64)
    tol = 2e-5 if gdt == torch.float32 else 4e-3
    for got, ref in ((dgw.cpu().double(), W), (dgb.cpu().double(), B)):
        assert got.dtype == torch.float64 and torch.isfinite(got).all()
        err = (got - ref).norm() / max(ref.norm().item(), 1e-30)
        assert err <= tol, err
    if empty is not None:
        assert counts.cpu()[empty].item() == 0
        assert not dgw.cpu()[empty].any() and dgb.cpu()[empty].item() == 0


def _combine_inputs(T, d, E, k, dev, seed):
    x, gw, gb = _routing_inputs(T, d, E, seed=seed)
    idx, _, w, _ = K.router_fwd(x.to(dev), gw.to(dev), gb.to(dev), k, 1.0)
    counts, offsets, perm, pos, _ = K.dispatch(idx, x.to(dev), E, gather=False)
    g = torch.Generator().manual_seed(seed + 1)
    o = torch.randn(T * k + T, d, generator=g).bfloat16()  # routed rows, then the shared rows
    return x, gw, idx, w, perm, pos, o


@pytest.mark.parametrize("T,d,E,k", [(4096, 768, 8, 2), (333, 512, 64, 6), (1, 64, 4, 2)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shared", [True, False])
def test_combine_fwd_is_index_add_in_expert_order(gpu_device, T, d, E, k, out_dtype, shared):
    # fmoe_combine_fwd against torch's own ops in the reference's order (moe.py:65-77,87):
    # y = zeros fp32; per expert ascending, y[tok] += (out * w).to(fp32); y.to(x.dtype); + shared.
    # Bit-exact: every product and add is one IEEE fp32 operation in that order.
    x, gw, idx, w, perm, pos, o = _combine_inputs(T, d, E, k, gpu_device, seed=17 + T)
    rows_r = T * k
    y = K.combine_fwd(o.to(gpu_device), idx, w, pos, rows_r, shared, out_dtype, None)
    idx_c, w_c, pos_c = idx.cpu().long(), w.cpu(), pos.cpu().long().reshape(T, k)
    order = torch.argsort(idx_c, dim=1, stable=True)  # a token's choices by ascending expert
    acc = torch.zeros(T, d, dtype=torch.float32)
    for jj in range(k):
        sel = order[:, jj:jj + 1]
        rows = pos_c.gather(1, sel)[:, 0]
        acc = acc + o.float()[rows] * w_c.gather(1, sel)
    ref = acc.to(out_dtype)
    if shared:
        ref = ref + o[rows_r:].to(out_dtype)
    got = y.cpu()
    if out_dtype == torch.bfloat16:
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    else:
        assert torch.equal(f32_bits(got), f32_bits(ref))


@pytest.mark.parametrize("T,d,E,k", [(4096, 768, 8, 2), (333, 512, 64, 6)])
def test_combine_bwd(gpu_device, T, d, E, k):
    # d_o[r] = bf16(dy[t] * w_slot) bit-exact (moe.py:76 backward of out * w); d_w[slot] =
    # <dy[t], o[r]> against its fp64 closed form.
    x, gw, idx, w, perm, pos, o = _combine_inputs(T, d, E, k, gpu_device, seed=31 + T)
    g = torch.Generator().manual_seed(3)
    dy = torch.randn(T, d, generator=g).bfloat16()
    rows_r = T * k
    o_r = o[:rows_r]
    d_o, d_w = K.combine_bwd(dy.to(gpu_device), o_r.to(gpu_device), w, perm, k)
    perm_c = perm.cpu().long()
    tok, slot = perm_c // k, perm_c
    ref_do = (dy.float()[tok] * w.cpu().reshape(-1)[slot][:, None]).bfloat16()
    assert torch.equal(d_o.cpu().view(torch.int16), ref_do.view(torch.int16))
    ref_dw = torch.zeros(T * k, dtype=torch.float64)
    ref_dw[slot] = (dy.double()[tok] * o_r.double()).sum(1)
    got = d_w.cpu().reshape(-1).double()
    l1 = torch.zeros(T * k, dtype=torch.float64)
    l1[slot] = (dy.double()[tok] * o_r.double()).abs().sum(1)  # fp32 sum of d terms: error <= ~d ulps of this
    assert ((got - ref_dw).abs() <= 2e-5 * l1).all()


@pytest.mark.parametrize("T,d,E,k", [(4096, 768, 8, 2), (333, 512, 64, 6)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_dx_reduce(gpu_device, T, d, E, k, out_dtype):
    # dx[t] = sum of the token's routed rows (ascending expert) + its shared row + the router
    # term sum_j dlogit_j * Wg[e_j] (the gate Linear's input gradient), against fp64.
    x, gw, idx, w, perm, pos, o = _combine_inputs(T, d, E, k, gpu_device, seed=47 + T)
    g = torch.Generator().manual_seed(9)
    dl = torch.randn(T, k, generator=g).float() * 0.1
    rows_r = T * k
    dx = K.dx_reduce(o.to(gpu_device), pos, idx, dl.to(gpu_device), gw.to(gpu_device), rows_r, True, out_dtype)
    pos_c, idx_c = pos.cpu().long().reshape(T, k), idx.cpu().long()
    ref = o.double()[rows_r:].clone()
    l1 = ref.abs()  # sum of the terms' magnitudes: the fp32 sums' error scales with it
    for j in range(k):
        a, b = o.double()[pos_c[:, j]], dl.double()[:, j:j + 1] * gw.double()[idx_c[:, j]]
        ref += a + b
        l1 += a.abs() + b.abs()
    got = dx.cpu().double()
    bound = 1e-6 * l1 + (2.0 ** -8 * ref.abs() if out_dtype == torch.bfloat16 else 0.0)
    assert ((got - ref).abs() <= bound).all()


# ---- grouped GEMMs -----------------------------------------------------------------

def _groups(counts, dev):
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return torch.from_numpy(off).to(dev), int(off[-1])


def _bf(*shape, scale=1.0, g=None):
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


@pytest.mark.parametrize("counts,shared,d,I", [
    ([0, 300, 517], 400, 192, 320), ([1, 2, 700], 0, 768, 2048), ([256, 256], 256, 256, 128),
    # decode-sized launches (groups of <= 128 rows go to the small-group kernel,
    # built for 1, 2, 4 or 8 blocks of 16 rows from a bound on the group sizes;
    # with at most 256 routed rows, every group, a larger one as 128-row slabs)
    ([0, 1], 1, 256, 128), ([1, 0, 0, 1, 0, 0, 0, 0], 1, 768, 2048), ([1, 5, 16, 17], 32, 768, 2048),
    ([33, 64, 100, 128, 7], 128, 192, 320), ([129, 3, 0], 2, 256, 512), ([2], 0, 2048, 1408),
    ([200, 40, 16], 128, 768, 2048), ([0, 256], 0, 192, 320),
    # the shared group as 64-row slabs (also with fewer routed rows than experts)
    ([3, 90], 100, 256, 512), ([1, 0, 0, 0, 0, 0, 0, 0], 100, 256, 512)])
def test_gateup_and_down_fwd(gpu_device, counts, shared, d, I):
    g = torch.Generator().manual_seed(1)
    E = len(counts)
    offsets, rows_r = _groups(counts, gpu_device)
    G = E + (1 if shared else 0)
    x_r = _bf(rows_r, d, g=g)
    x_s = _bf(shared, d, g=g) if shared else None
    w1 = [_bf(I, d, scale=0.05, g=g) for _ in range(G)]
    w3 = [_bf(I, d, scale=0.05, g=g) for _ in range(G)]
    w2 = [_bf(d, I, scale=0.05, g=g) for _ in range(G)]
    dv = lambda ts: [t.to(gpu_device) for t in ts]
    ab, h = K.gateup_fwd(x_r.to(gpu_device), x_s.to(gpu_device) if shared else None, offsets, E,
                         dv(w1), dv(w3), I)
    o = K.down_fwd(h, offsets, E, rows_r, shared, dv(w2), d)
    ab, h, o = ab.cpu(), h.cpu(), o.cpu()
    off = offsets.cpu().tolist() + ([rows_r + shared] if shared else [])
    xs = torch.cat([x_r] + ([x_s] if shared else []))
    for grp in range(G):
        r0, r1 = off[grp], off[grp + 1]
        if r1 == r0:
            continue
        xg = xs[r0:r1].float()
        a_ref = xg @ w1[grp].float().T
        b_ref = xg @ w3[grp].float().T
        # bf16 outputs of fp32 accumulations: within one bf16 rounding of the fp32 product
        close(ab[r0:r1, :I], a_ref, rtol=8e-3, atol=1e-3)
        close(ab[r0:r1, I:], b_ref, rtol=8e-3, atol=1e-3)
        a, b = ab[r0:r1, :I].float(), ab[r0:r1, I:].float()
        h_ref = (F.silu(a).bfloat16().float() * b)
        close(h[r0:r1], h_ref, rtol=8e-3, atol=1e-4)
        o_ref = h[r0:r1].float() @ w2[grp].float().T
        close(o[r0:r1], o_ref, rtol=8e-3, atol=1e-3)


@pytest.mark.parametrize("counts,shared,d,I", [([0, 300, 517], 400, 192, 320), ([100, 1, 2000], 700, 768, 2048),
                                               ([40, 300, 700], 200, 320, 1408)])
def test_backward_products(gpu_device, counts, shared, d, I):
    # The dX products read the nn.Linear weights as they lie (w2 [d, I],
    # w1 / w3 [I, d]) through transposing LDS reads; partial n tiles
    # (I = 320, 1408; d = 192, 320) and a single 64-deep K stage per tile are
    # covered.
    g = torch.Generator().manual_seed(2)
    E = len(counts)
    offsets, rows_r = _groups(counts, gpu_device)
    rows = rows_r + shared
    G = E + (1 if shared else 0)
    do_r = _bf(rows_r, d, g=g)
    do_s = _bf(shared, d, g=g) if shared else None
    ab = _bf(rows, 2 * I, g=g)
    x_r = _bf(rows_r, d, g=g)
    x_s = _bf(shared, d, g=g) if shared else None
    h = _bf(rows, I, scale=0.3, g=g)
    w1 = [_bf(I, d, scale=0.05, g=g) for _ in range(G)]
    w3 = [_bf(I, d, scale=0.05, g=g) for _ in range(G)]
    w2 = [_bf(d, I, scale=0.05, g=g) for _ in range(G)]
    D = gpu_device
    dv = lambda ts: [t.to(D) for t in ts]
    d_ab = K.down_bwd_dx(do_r.to(D), do_s.to(D) if shared else None, offsets, E, dv(w2), ab.to(D), I)
    dx_rows = K.gateup_bwd_dx(d_ab, offsets, E, rows_r, shared, dv(w1), dv(w3), d)
    dw2 = [torch.empty(d, I, dtype=torch.bfloat16, device=D) for _ in range(G)]
    K.weight_grad(do_r.to(D), do_s.to(D) if shared else None, h.to(D), None, offsets, E, rows_r, shared,
                  d, dw2, None, torch.bfloat16)
    dw1 = [torch.empty(I, d, dtype=torch.float32, device=D) for _ in range(G)]
    dw3 = [torch.empty(I, d, dtype=torch.float32, device=D) for _ in range(G)]
    K.weight_grad(d_ab, None, x_r.to(D), x_s.to(D) if shared else None, offsets, E, rows_r, shared,
                  I, dw1, dw3, torch.float32)
    d_ab, dx_rows = d_ab.cpu(), dx_rows.cpu()
    off = offsets.cpu().tolist() + ([rows] if shared else [])
    dos = torch.cat([do_r] + ([do_s] if shared else []))
    xs = torch.cat([x_r] + ([x_s] if shared else []))
    for grp in range(G):
        r0, r1 = off[grp], off[grp + 1]
        if r1 == r0:
            continue
        dh = (dos[r0:r1].float() @ w2[grp].float()).bfloat16().float()
        a, b = ab[r0:r1, :I].float(), ab[r0:r1, I:].float()
        sg = torch.sigmoid(a)
        s = (a * sg).bfloat16().float()
        ds = (dh * b).bfloat16().float()
        da_ref = ds * (sg * (1 + a * (1 - sg)))
        db_ref = dh * s
        # dh itself may differ by one bf16 rounding (accumulation order), which
        # propagates into da/db; compare in relative L2 and elementwise loosely.
        assert rel_l2(d_ab[r0:r1, :I], da_ref) < 6e-3
        assert rel_l2(d_ab[r0:r1, I:], db_ref) < 6e-3
        dag, dbg = d_ab[r0:r1, :I].float(), d_ab[r0:r1, I:].float()
        dx_ref = dag @ w1[grp].float() + dbg @ w3[grp].float()
        close(dx_rows[r0:r1], dx_ref, rtol=1e-2, atol=2e-3)
        dw2_ref = dos[r0:r1].float().T @ h[r0:r1].float()
        close(dw2[grp].cpu(), dw2_ref, rtol=1e-2, atol=2e-2)
        dw1_ref = dag.T @ xs[r0:r1].float()
        dw3_ref = dbg.T @ xs[r0:r1].float()
        assert rel_l2(dw1[grp].cpu(), dw1_ref) < 1e-5
        assert rel_l2(dw3[grp].cpu(), dw3_ref) < 1e-5


@pytest.mark.parametrize("T,d,I,E,k,bias", [(3000, 768, 2048, 8, 2, "skew"), (2400, 256, 320, 16, 3, "spread"),
                                              (4500, 192, 128, 4, 1, "tiny_last")])
def test_gathered_rows_match_the_gathered_copy(gpu_device, T, d, I, E, k, bias):
    # Launches of more than 4096 rows can read the routed token rows of x
    # through the dispatch's permutation (routed row r = x row perm[r] // k)
    # instead of a gathered copy x_perm: gate/up forward and the w1 / w3 weight
    # gradient bit-identical to the same products over x_perm (the same values reach
    # the same MFMAs), for skewed groups, partial tiles and a last expert with
    # fewer than 8 rows (the index windows' clamp at the end of perm).
    D = gpu_device
    g = torch.Generator().manual_seed(T + E)
    x = _bf(T, d, g=g).to(D)
    gw = _bf(E, d, scale=0.05, g=g).to(D)
    gb = torch.zeros(E)
    if bias == "skew":
        gb[:2] = 1.5
    elif bias == "tiny_last":
        gb[E - 1] = -2.5  # the last expert gets only a few tokens
    idx, _, _, _ = K.router_fwd(x, gw, gb.bfloat16().to(D), k, 1.0)
    counts, offsets, perm, pos, x_perm = K.dispatch(idx, x, E)
    if bias == "tiny_last":
        assert 0 < int(counts[E - 1]) < 8
    G = E + 1
    w1 = [_bf(I, d, scale=0.05, g=g).to(D) for _ in range(G)]
    w3 = [_bf(I, d, scale=0.05, g=g).to(D) for _ in range(G)]
    rows_r = T * k
    ab0, h0 = K.gateup_fwd(x_perm, x, offsets, E, w1, w3, I)
    ab1, h1 = K.gateup_fwd(x, x, offsets, E, w1, w3, I, gather=perm, k=k)
    assert torch.equal(ab0.view(torch.int16), ab1.view(torch.int16))
    assert torch.equal(h0.view(torch.int16), h1.view(torch.int16))
    d_ab = _bf(rows_r + T, 2 * I, scale=0.05, g=g).to(D)
    outs = []
    for gathered in (False, True):
        dw1 = [torch.empty(I, d, dtype=torch.bfloat16, device=D) for _ in range(G)]
        dw3 = [torch.empty(I, d, dtype=torch.bfloat16, device=D) for _ in range(G)]
        K.weight_grad(d_ab, None, x if gathered else x_perm, x, offsets, E, rows_r, T, I, dw1, dw3,
                      torch.bfloat16, b_gather=perm if gathered else None, k=k)
        outs.append(dw1 + dw3)
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # and one expert's w1 gradient against fp32 arithmetic on the gathered rows
    e = int(torch.argmax(counts))
    r0, r1 = int(offsets[e]), int(offsets[e + 1])
    xs = x.cpu().float()[perm[r0:r1].cpu().long() // k]
    ref = d_ab[r0:r1, :I].cpu().float().T @ xs
    assert rel_l2(outs[1][e].cpu(), ref) < 5e-3


def _row_products(D, x_r, x_s, do_r, do_s, offsets, E, w1, w3, w2, ab_in, h_in, dab_in, split,
                  short_ws=False):
    """The four row products through the C ABI, with the split workspace or
    without it (short_ws: a workspace one byte smaller than the query asks
    for, which the products must treat as none); each product reads fixed
    inputs (not the previous product's output), so only its own summation
    order differs between the two runs."""
    from fusionllm_amd import _lib
    lib = _lib.load()
    rows_r, d = x_r.shape
    rows_s = x_s.shape[0]
    I = w1[0].shape[0]
    rows = rows_r + rows_s
    ws_bytes = lib.fmoe_split_workspace_bytes() if split else 0
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=D)
    wsp = ws.data_ptr() if split else None
    if short_ws:
        ws_bytes -= 1
    pa = lambda ts: _lib.ptr_array([t.data_ptr() for t in ts])
    st = K._stream()
    ab = torch.empty(rows, 2 * I, dtype=torch.bfloat16, device=D)
    h = torch.empty(rows, I, dtype=torch.bfloat16, device=D)
    _lib.check(lib.fmoe_gateup_fwd(x_r.data_ptr(), None, 0, 0, x_s.data_ptr(), offsets.data_ptr(), E, rows_r, rows_s, d, I,
                                   pa(w1), pa(w3), ab.data_ptr(), h.data_ptr(), wsp, ws_bytes, st), "gateup_fwd")
    o = torch.empty(rows, d, dtype=torch.bfloat16, device=D)
    _lib.check(lib.fmoe_down_fwd(h_in.data_ptr(), offsets.data_ptr(), E, rows_r, rows_s, d, I, pa(w2),
                                 o.data_ptr(), wsp, ws_bytes, st), "down_fwd")
    d_ab = torch.empty(rows, 2 * I, dtype=torch.bfloat16, device=D)
    _lib.check(lib.fmoe_down_bwd_dx(do_r.data_ptr(), do_s.data_ptr(), offsets.data_ptr(), E, rows_r, rows_s, d, I,
                                    pa(w2), ab_in.data_ptr(), d_ab.data_ptr(), wsp, ws_bytes, st),
               "down_bwd_dx")
    dx = torch.empty(rows, d, dtype=torch.bfloat16, device=D)
    _lib.check(lib.fmoe_gateup_bwd_dx(dab_in.data_ptr(), offsets.data_ptr(), E, rows_r, rows_s, d, I,
                                      pa(w1), pa(w3), dx.data_ptr(), wsp, ws_bytes, st), "gateup_bwd_dx")
    return [t.cpu() for t in (ab, h, o, d_ab, dx)]


def test_split_tail_matches_whole_tiles(gpu_device):
    """The last, partial round of the persistent grid split along K (summed in
    range order, then the product's own epilogue) against the same tiles run
    whole.  26000 rows of d=768, I=2048 put every product's tile count above
    the 256-CU grid with a remainder: gate/up 1664 tiles, down 312, down
    backward 832, gate/up backward 312.  Only the fp32 summation order of the
    split tiles differs: an output agrees with the whole-tile one to a few
    bf16 roundings (one on the sum, up to three more through the SwiGLU
    epilogues, each at most 2^-7 relative), and every row of the first group
    (tiles of the first rounds) is bit-identical."""
    D = gpu_device
    g = torch.Generator().manual_seed(7)
    counts, shared, d, I = [6000, 6000, 6000, 6000], 2000, 768, 2048
    E = len(counts)
    offsets, rows_r = _groups(counts, D)
    G = E + 1
    x_r, x_s = _bf(rows_r, d, g=g).to(D), _bf(shared, d, g=g).to(D)
    do_r, do_s = _bf(rows_r, d, g=g).to(D), _bf(shared, d, g=g).to(D)
    ab_in = _bf(rows_r + shared, 2 * I, g=g).to(D)
    h_in = _bf(rows_r + shared, I, scale=0.3, g=g).to(D)
    dab_in = _bf(rows_r + shared, 2 * I, scale=0.05, g=g).to(D)
    w1 = [_bf(I, d, scale=0.05, g=g).to(D) for _ in range(G)]
    w3 = [_bf(I, d, scale=0.05, g=g).to(D) for _ in range(G)]
    w2 = [_bf(d, I, scale=0.05, g=g).to(D) for _ in range(G)]
    args = (D, x_r, x_s, do_r, do_s, offsets, E, w1, w3, w2, ab_in, h_in, dab_in)
    split = _row_products(*args, split=True)
    whole = _row_products(*args, split=False)
    # a workspace smaller than the query runs every tile whole
    short = _row_products(*args, split=True, short_ws=True)
    for name, a, b in zip(("ab", "h", "out", "d_ab", "dx_rows"), short, whole):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
    names = ("ab", "h", "out", "d_ab", "dx_rows")
    for name, a, b in zip(names, split, whole):
        assert torch.equal(a[:counts[0]], b[:counts[0]]), name
        close(a, b, rtol=3.2e-2, atol=2e-3)
        assert rel_l2(a, b.float()) < 2e-3, name
    # and the split outputs against fp32 products of the shared group's rows
    # (the last tiles in tile order, where the split round lands)
    xs = x_s.cpu().float()
    a_ref = xs @ w1[E].cpu().float().T
    close(split[0][rows_r:, :I], a_ref, rtol=8e-3, atol=1e-3)
    o_ref = h_in[rows_r:].cpu().float() @ w2[E].cpu().float().T
    close(split[2][rows_r:], o_ref, rtol=8e-3, atol=1e-3)
    dag, dbg = dab_in[rows_r:, :I].cpu().float(), dab_in[rows_r:, I:].cpu().float()
    dx_ref = dag @ w1[E].cpu().float() + dbg @ w3[E].cpu().float()
    close(split[4][rows_r:], dx_ref, rtol=1e-2, atol=2e-3)


def test_cast_bf16_bit_exact(gpu_device):
    # One-launch fp32 -> bf16 copies (the autocast casts of the block's
    # operands): bit-identical to torch's .to(torch.bfloat16), round to
    # nearest even, tails shorter than 8 values, more tensors than one launch
    # takes, special values.
    g = torch.Generator().manual_seed(0)
    sizes = [0, 1, 7, 8, 9, 2047, 2048, 2049, 100003] + [64] * 60
    ts = [torch.randn(n, generator=g) * 10 for n in sizes]
    ts.append(torch.tensor([float("inf"), -float("inf"), 0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38,
                            1.00390625, 1.01171875, -1.00390625, 2.0 ** -126, 2.0 ** -133, 65504.0,
                            3.3895313892515355e38, float("nan")]))
    ts.append(torch.randn(3, 5, generator=g))  # 2-D, 15 values
    out = K.cast_bf16([t.to(gpu_device) for t in ts])
    assert len(out) == len(ts)
    for t, o in zip(ts, out):
        want = t.to(torch.bfloat16)
        got = o.cpu()
        assert got.shape == want.shape and got.dtype == torch.bfloat16
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan)
        assert torch.equal(got[~nan].view(torch.int16), want[~nan].view(torch.int16))


@pytest.mark.parametrize("T,d,E,k,rs", [(1, 768, 8, 2, 1.0), (8, 768, 8, 2, 1.0), (16, 2048, 64, 6, 2.5),
                                        (3, 64, 3, 3, 1.0), (5, 256, 33, 8, 1.0), (16, 768, 8, 1, 1.0)])
def test_route_dispatch_matches_two_launches(gpu_device, T, d, E, k, rs):
    # The one-launch tiny-batch path gives the outputs of fmoe_router_fwd
    # followed by fmoe_dispatch, bit for bit (and so the C oracle's).
    x, gw, gb = _routing_inputs(T, d, E, seed=T * 31 + E)
    xd, gwd, gbd = x.to(gpu_device), gw.to(gpu_device), gb.to(gpu_device)
    one = K.route_dispatch(xd, gwd, gbd, k, rs)
    idx, idx64, w, v = K.router_fwd(xd, gwd, gbd, k, rs)
    two = (idx, idx64, w, v) + K.dispatch(idx, xd, E)
    for a, b in zip(one, two):
        assert torch.equal(a.cpu().view(torch.int32) if a.dtype == torch.float32 else a.cpu(),
                           b.cpu().view(torch.int32) if b.dtype == torch.float32 else b.cpu())
    ridx, rw, rv = mo.router_c(x, gw, gb, k, rs)
    assert torch.equal(one[0].cpu(), ridx)
    rc, ro, rp, rpos = mo.dispatch_c(one[0].cpu(), E)
    assert torch.equal(one[4].cpu(), rc) and torch.equal(one[6].cpu(), rp)


def test_block_with_gathered_rows_matches_the_default(gpu_device, monkeypatch):
    # The block's gathered-rows option (moe.GATHER_ROWS: no x_perm; the gate/up
    # forward and dW1|dW3 read token rows through perm) gives the bits of the
    # default path, forward and backward.
    from fusionllm_amd import configs, moe as moe_mod
    from tests.gpu_util import build_module
    cfg = configs.C2
    data = configs.make_block(cfg, seed=3, tokens=2048)
    outs = []
    for flag in (False, True):
        monkeypatch.setattr(moe_mod, "GATHER_ROWS", flag)
        assert moe_mod.gathers_rows(2048, 2, True) == flag
        m = build_module(cfg, data, gpu_device)
        x = data.x.to(gpu_device, torch.bfloat16).requires_grad_(True)
        y = m(x)
        y.backward(data.dy.to(gpu_device, torch.bfloat16))
        outs.append([y.detach(), x.grad] + [p.grad for p in m.parameters()])
    for a, b in zip(*outs):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
