"""CPU tests of the host side: the C-ABI library loads and exports every
declared symbol, argument checks return errors without touching a GPU, and
the drop-in module keeps the reference's interface (models/moe.py:24-109)."""
import re
from pathlib import Path

import pytest
import torch

from fusionllm_amd import DeepSeekMoE, SwiGLUExpert, configs
from fusionllm_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "fusionmoe.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fmoe_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = declared_symbols()
    assert len(syms) == 26
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_lib.SIGNATURES), "ctypes binding and header disagree"
    assert lib.fmoe_abi_version() == _lib.ABI_VERSION


def test_status_strings():
    lib = _lib.load()
    assert lib.fmoe_status_string(0) == b"ok"
    for code in range(1, 9):
        assert lib.fmoe_status_string(code) != b"unknown status"
    assert lib.fmoe_status_string(99) == b"unknown status"


def test_argument_errors_without_gpu():
    import ctypes
    lib = _lib.load()
    # rejected on the host before any HIP call
    assert lib.fmoe_router_fwd(None, None, None, 4, 100, 8, 2, 1.0, None, None, None, None, None) == 2  # dim % 64
    assert lib.fmoe_router_fwd(None, None, None, 4, 768, 65, 2, 1.0, None, None, None, None, None) == 7
    assert lib.fmoe_router_fwd(None, None, None, 4, 768, 8, 9, 1.0, None, None, None, None, None) == 2
    assert lib.fmoe_router_fwd(None, None, None, -1, 768, 8, 2, 1.0, None, None, None, None, None) == 1
    assert lib.fmoe_router_fwd(None, None, None, 4, 768, 8, 2, 1.0, None, None, None, None, None) == 1
    # the allocation-free dispatch: shape errors as fmoe_dispatch, and a
    # workload beyond its 1 MiB static scratch (2 * ceil(T*k/256) * E int32)
    assert lib.fmoe_dispatch_noalloc(None, None, 4, 768, 65, 2, None, None, None, None, None, None) == 7
    assert lib.fmoe_dispatch_noalloc(None, None, 4, 100, 8, 2, None, None, None, None, None, None) == 2
    assert lib.fmoe_dispatch_workspace_bytes(87381, 64, 6) <= 1 << 20
    assert lib.fmoe_dispatch_workspace_bytes(87382, 64, 6) > 1 << 20
    assert lib.fmoe_dispatch_noalloc(None, None, 87382, 2048, 64, 6, None, None, None, None, None, None) == 8
    assert b"1 MiB" in lib.fmoe_status_string(8)
    pp = _lib.ptr_array([0])
    assert lib.fmoe_gateup_fwd(None, None, 0, 0, None, None, 1, 10, 0, 96, 128, pp, pp, None, None, None, 0,
                               None) == 2
    assert lib.fmoe_gateup_fwd(None, None, 0, 0, None, None, 1, 10, 0, 128, 128, pp, pp, None, None, None, 0,
                               None) == 1
    # the row products' 32-bit copy offsets: rows below 2^22 elements, a weight below 2^31
    assert lib.fmoe_gateup_fwd(None, None, 0, 0, None, None, 1, 10, 0, 1 << 16, 1 << 15, pp, pp, None, None, None,
                               0, None) == 2
    assert lib.fmoe_gateup_fwd(None, None, 0, 0, None, None, 1, 10, 0, 1 << 22, 64, pp, pp, None, None, None, 0,
                               None) == 2
    assert lib.fmoe_gateup_fwd(None, None, 0, 0, None, None, 1, 10, 0, (1 << 22) - 64, 64, pp, pp, None, None,
                               None, 0, None) == 1  # admitted (then the null pointers)
    assert lib.fmoe_down_fwd(None, None, 1, 10, 0, 64, 1 << 22, pp, None, None, 0, None) == 2
    assert lib.fmoe_down_bwd_dx(None, None, None, 1, 10, 0, 1 << 16, 1 << 15, pp, None, None, None, 0, None) == 2
    assert lib.fmoe_gateup_bwd_dx(None, None, 1, 10, 0, 1 << 15, 1 << 16, pp, pp, None, None, 0, None) == 2
    assert lib.fmoe_combine_fwd(None, None, None, None, 4, 768, 2, 8, 1, 5, None, None, None) == 4
    # RMSNorm around the block
    assert lib.fmoe_rmsnorm_fwd(None, 0, None, 0, 4, 100, 1e-6, None, None, None) == 2
    assert lib.fmoe_rmsnorm_fwd(None, 0, None, 0, 4, 8192, 1e-6, None, None, None) == 2
    assert lib.fmoe_rmsnorm_fwd(None, 5, None, 0, 4, 768, 1e-6, None, None, None) == 4
    assert lib.fmoe_rmsnorm_fwd(None, 0, None, 0, 4, 768, 1e-6, None, None, None) == 1
    assert lib.fmoe_rmsnorm_fwd(None, 0, None, 0, 0, 768, 1e-6, None, None, None) == 0
    fake = 1 << 20  # a non-null address that is never dereferenced (rejected first)
    assert lib.fmoe_dx_reduce_norm(None, None, None, None, None, 4, 768, 2, 8, 1, None, None, None, 0,
                                   None, 0, None, fake, fake, 1 << 30, None) == 1  # d_norm_w without norm_w
    assert lib.fmoe_dx_reduce_norm(None, None, None, None, None, 4, 768, 2, 8, 1, None, None, fake, 0,
                                   None, 0, None, fake, fake, 100, None) == 6  # workspace too small
    assert lib.fmoe_dx_reduce_norm(None, None, None, None, None, 4, 768, 2, 8, 1, None, None, None, 0,
                                   None, 0, None, None, None, 0, None) == 1  # null inputs
    assert lib.fmoe_weight_grad(None, None, 8, None, None, 8, None, 0, 0, None, 1, 10, 0, 128, 128, 0, pp, None,
                                0, None, 0, None) == 2
    # weight gradients: every output 16-byte aligned (the chunk reduction writes 8 outputs per store),
    # checked before anything is launched
    ws = lib.fmoe_weight_grad_workspace_bytes(64, 0, 1, 128, 128)
    odd, even = _lib.ptr_array([fake + 8]), _lib.ptr_array([fake])
    assert lib.fmoe_weight_grad(fake, None, 128, fake, None, 128, None, 0, 0, fake, 1, 64, 0, 128, 128, 128, odd,
                                None, 0, fake, ws, None) == 3
    assert lib.fmoe_weight_grad(fake, None, 128, fake, None, 128, None, 0, 0, fake, 1, 64, 0, 128, 128, 64, even,
                                odd, 0, fake, ws, None) == 3
    # leading dimensions: at least the row length, below 2^24 (32-bit copy offsets)
    assert lib.fmoe_weight_grad(fake, None, 64, fake, None, 128, None, 0, 0, fake, 1, 64, 0, 128, 128, 128, even,
                                None, 0, fake, ws, None) == 2
    assert lib.fmoe_weight_grad(fake, None, 128, fake, None, 1 << 24, None, 0, 0, fake, 1, 64, 0, 128, 128, 128,
                                even, None, 0, fake, ws, None) == 2
    # one-launch bf16 casts: count and sizes checked before any pointer is used
    n1 = (ctypes.c_int64 * 1)(-1)
    assert lib.fmoe_cast_bf16(pp, pp, n1, 1, None) == 1
    assert lib.fmoe_cast_bf16(pp, pp, n1, 65, None) == 1
    assert lib.fmoe_cast_bf16(None, None, None, 0, None) == 0
    assert lib.fmoe_cast_bf16(_lib.ptr_array([fake + 4]), _lib.ptr_array([fake]), (ctypes.c_int64 * 1)(8), 1,
                              None) == 3
    # tiny-batch routing + dispatch: more than 16 tokens is the two-launch path
    assert lib.fmoe_route_dispatch(None, None, None, 17, 768, 8, 2, 1.0, None, None, None, None, None, None,
                                   None, None, None, None) == 2
    assert lib.fmoe_route_dispatch(None, None, None, 4, 768, 8, 2, 1.0, None, None, None, None, None, None,
                                   None, None, None, None) == 1
    # routing + dispatch of any batch: shape checks before any pointer is used, workspace size
    assert lib.fmoe_route_and_dispatch(None, None, None, 4, 4096, 8, 2, 1.0, None, None, None, None, None, None,
                                       None, None, None, None, None, 0, None) == 2  # dim > 2048
    assert lib.fmoe_route_and_dispatch(None, None, None, 4, 768, 65, 2, 1.0, None, None, None, None, None, None,
                                       None, None, None, None, None, 0, None) == 7
    assert lib.fmoe_route_and_dispatch(None, None, None, 4, 768, 8, 2, 1.0, None, None, None, None, None, None,
                                       None, None, None, None, None, 0, None) == 1  # null outputs
    assert lib.fmoe_route_and_dispatch_workspace_bytes(16384, 8, 2) == 2 * 512 * 8 * 4
    assert lib.fmoe_route_and_dispatch_workspace_bytes(33, 64, 6) == 2 * 2 * 64 * 4
    # size queries
    assert lib.fmoe_dispatch_workspace_bytes(16384, 8, 2) == 2 * 128 * 8 * 4
    assert lib.fmoe_weight_grad_workspace_bytes(32768, 16384, 8, 768, 2048) > 0
    assert lib.fmoe_router_bwd_workspace_bytes(16384, 768, 8, 2) == (16384 * 2 // 32 + 8) * 769 * 4
    assert lib.fmoe_norm_bwd_workspace_bytes(768) == 4160 * 768 * 4
    # fused NorMuon step: limits checked before any pointer is used
    import ctypes
    pp1 = _lib.ptr_array([1 << 20])
    r1, c1, m1 = (ctypes.c_int64 * 1)(4), (ctypes.c_int64 * 1)(6), (ctypes.c_int * 1)(1)
    assert lib.fmoe_normuon_step(pp1, pp1, pp1, pp1, r1, c1, m1, 33, 0, .02, .9, .95, 1e-8, .1, 1, .1, .05,
                                 None) == 1  # more than 32 tensors
    assert lib.fmoe_normuon_step(pp1, pp1, pp1, pp1, r1, c1, m1, 1, 7, .02, .9, .95, 1e-8, .1, 1, .1, .05,
                                 None) == 4  # dtype
    assert lib.fmoe_normuon_step(pp1, pp1, pp1, pp1, r1, c1, m1, 1, 0, .02, .9, .95, 1e-8, .1, 1, .1, .05,
                                 None) == 2  # cols not a multiple of 4


def test_gathered_rows_argument_checks():
    from fusionllm_amd import _lib
    lib = _lib.load()
    pp = _lib.ptr_array([1 << 20])
    fake = 1 << 20
    # decode-sized launches (<= 4096 rows) keep x_perm; gather_k must be positive
    assert lib.fmoe_gateup_fwd(fake, fake, 2, 100, None, fake, 1, 200, 0, 256, 256, pp, pp, fake, fake, None, 0,
                               None) == 2
    assert lib.fmoe_gateup_fwd(fake, fake, 0, 3000, None, fake, 1, 6000, 0, 256, 256, pp, pp, fake, fake, None, 0,
                               None) == 2
    assert lib.fmoe_weight_grad(fake, None, 256, fake, None, 256, fake, 0, 100, fake, 1, 10, 0, 256, 256, 256,
                                pp, None, 0, fake, 1 << 30, None) == 2


def test_slot_division_by_multiplication():
    # The kernels find a routed slot's token as floor(n / k) = high half of
    # n * m, m = ceil(2^32 / k) (fmoe_common.h: slot_token), exact for
    # n < 2^29.  Checked at both ends of that range, at every multiple of k
    # and its neighbours near the top, and on a stride through it.
    import numpy as np
    for k in range(1, 9):
        m = ((1 << 32) + k - 1) // k
        lo, hi = m & 0xFFFFFFFF, m >> 32
        top = 1 << 29
        n = np.concatenate([np.arange(0, 1 << 16), np.arange(top - (1 << 16), top),
                            np.arange(0, top, 997), (np.arange(top // k - 4096, top // k) * k)[:, None].repeat(3, 1).ravel()
                            + np.tile([-1, 0, 1], 4096)]).astype(np.uint64)
        n = n[n < top]
        got = ((n * np.uint64(lo)) >> np.uint64(32)) + n * np.uint64(hi)
        assert np.array_equal(got, n // np.uint64(k)), k


def test_host_counts_buffer_checks():
    # the routing entry point writes the expert counts into host memory only
    # through a contiguous pinned int32 buffer of at least E entries
    from fusionllm_amd import _kernels as K
    # (the kernel writes E int32 there: a smaller or differently typed buffer
    # would be a host-memory overrun)
    assert K._host_counts(None, 8) is None
    with pytest.raises(RuntimeError, match="pinned"):
        K._host_counts(torch.zeros(8, dtype=torch.int32), 8)  # pageable
    with pytest.raises(RuntimeError, match="int32"):
        K._host_counts(torch.zeros(8, dtype=torch.int64), 8)  # wrong dtype
    with pytest.raises(RuntimeError, match="at least n_experts=8"):
        K._host_counts(torch.zeros(7, dtype=torch.int32), 8)  # too small
    with pytest.raises(RuntimeError, match="contiguous"):
        K._host_counts(torch.zeros(16, dtype=torch.int32)[::2], 8)  # strided view
    with pytest.raises(RuntimeError, match="CPU tensor"):
        K._host_counts(torch.zeros(8, dtype=torch.int32, device="meta"), 8)


def _synthetic(lines):
    """A kernel from (op, operands) pairs at consecutive addresses; "jmp N"
    branches back to instruction N."""
    from tests import isa_check as ic
    k = ic.Kernel("synthetic")
    for i, (op, opnds) in enumerate(lines):
        ins = ic.Insn(0x1000 + 4 * i, op, opnds)
        if op.startswith("s_cbranch"):
            ins.target = 0x1000 + 4 * int(opnds)
        k.insns.append(ins)
    return k


def test_isa_checker_finds_planted_hazards():
    # The checker itself: each planted mistake is reported, its fixed form is not.
    from tests import isa_check as ic
    read = ("ds_read_b128", "v[40:43], v5 offset:2048")
    mfma = ("v_mfma_f32_16x16x32_bf16", "v[0:3], v[40:43], v[60:63], v[0:3]")
    assert ic.check_kernel(_synthetic([read, mfma, ("s_endpgm", "")]))  # no wait
    assert not ic.check_kernel(_synthetic([read, ("s_waitcnt", "lgkmcnt(0)"), mfma, ("s_endpgm", "")]))
    # a younger read may stay in flight; the consumed one may not
    younger = ("ds_read_b128", "v[44:47], v6")
    assert not ic.check_kernel(_synthetic([read, younger, ("s_waitcnt", "lgkmcnt(1)"), mfma, ("s_endpgm", "")]))
    assert ic.check_kernel(_synthetic([younger, read, ("s_waitcnt", "lgkmcnt(1)"), mfma, ("s_endpgm", "")]))
    # a register copy of an in-flight destination (the compiler moving it)
    assert ic.check_kernel(_synthetic([read, ("v_mov_b32", "v7, v41"), ("s_waitcnt", "lgkmcnt(0)"),
                                       ("s_endpgm", "")]))
    # a dead destination handed to another value while the load is in flight
    assert ic.check_kernel(_synthetic([read, ("v_add_u32", "v42, v1, v2"), ("s_waitcnt", "lgkmcnt(0)"),
                                       ("s_endpgm", "")]))
    # carried around a loop: read at the end of the body, used at its top
    loop = [("s_nop", "0"), mfma, ("s_waitcnt", "lgkmcnt(0)"), read, ("s_cbranch_scc1", "1"), ("s_endpgm", "")]
    assert ic.check_kernel(_synthetic(loop))
    loop[2], loop[3] = loop[3], loop[2]
    assert not ic.check_kernel(_synthetic(loop))
    # vector memory loads and vmcnt
    gload = ("global_load_dwordx4", "v[40:43], v1, s[2:3]")
    assert ic.check_kernel(_synthetic([gload, mfma, ("s_endpgm", "")]))
    assert not ic.check_kernel(_synthetic([gload, ("s_waitcnt", "vmcnt(0)"), mfma, ("s_endpgm", "")]))


def test_gemm_code_reads_no_register_a_load_is_still_filling():
    # The GEMM kernels issue their LDS fragment reads and operand copies from
    # inline assembly with explicit waits, which the compiler does not see:
    # check the built gfx950 code of every kernel in gemm.o (and the other
    # kernel sources) for an access to a register whose load may be in flight.
    from tests import isa_check as ic
    objs = sorted((ROOT / "fusionllm_amd" / "_build").glob("*.o"))
    if not (ic.ROCM_LLVM / "llvm-objdump").exists() or not objs:
        pytest.skip("no built objects or no llvm-objdump")
    checked = 0
    for o in objs:
        if o.name not in ("gemm.o", "dispatch.o", "combine.o", "cast.o", "optim.o"):
            continue  # router.o / norm.o: compiler-scheduled code only (and slow to scan)
        n, hazards = ic.check_object(o)
        assert not hazards, "\n".join(hazards[:10])
        checked += n
    assert checked >= 16


def test_parameter_names_shapes_and_count():
    cfg = configs.C2.moe_config()
    m = DeepSeekMoE(cfg)
    sd = m.state_dict()
    want = {"gate.weight": (8, 768), "gate.bias": (8,)}
    for e in range(8):
        want[f"experts.{e}.w1.weight"] = (2048, 768)
        want[f"experts.{e}.w3.weight"] = (2048, 768)
        want[f"experts.{e}.w2.weight"] = (768, 2048)
    for n in ("w1", "w3"):
        want[f"shared_expert.{n}.weight"] = (2048, 768)
    want["shared_expert.w2.weight"] = (768, 2048)
    assert {k: tuple(v.shape) for k, v in sd.items()} == want
    # documentation/moe.md:20 of the reference: 42,473,480 parameters per MoE layer
    assert sum(p.numel() for p in m.parameters()) == 42_473_480
    assert torch.equal(m.gate.bias, torch.zeros(8))
    assert 0.004 < m.gate.weight.std().item() < 0.008
    assert m._last_indices is None and m._last_weights is None
    assert isinstance(m.experts[0], SwiGLUExpert)


def test_n_shared_experts_is_a_flag():
    cfg = dict(configs.C5.moe_config())
    m = DeepSeekMoE(cfg)
    assert cfg["n_shared_experts"] == 2 and m.shared_expert is not None
    assert m.shared_expert.w1.weight.shape == (1408, 2048)
    cfg["n_shared_experts"] = 0
    assert DeepSeekMoE(cfg).shared_expert is None


def test_forward_on_cpu_raises():
    m = DeepSeekMoE(configs.C2.moe_config()).bfloat16()
    with pytest.raises(RuntimeError, match="ROCm device"):
        m(torch.randn(2, 768).bfloat16())


def test_non_viewable_input_raises_like_reference():
    m = DeepSeekMoE(configs.C2.moe_config())
    x = torch.randn(4, 768 * 2)[:, ::2]
    with pytest.raises(RuntimeError):
        m(x)


def test_update_gate_bias_and_aux_loss_semantics():
    # models/moe.py:89-109 semantics on a synthetic routing
    m = DeepSeekMoE(configs.C2.moe_config())
    assert m.get_load_balance_loss().item() == 0.0
    m.update_gate_bias()  # no routing yet: no-op
    assert torch.equal(m.gate.bias, torch.zeros(8))
    idx = torch.tensor([[0, 1], [0, 2], [0, 1], [3, 0]])
    w = torch.tensor([[0.6, 0.4], [0.5, 0.5], [0.7, 0.3], [0.2, 0.8]])
    m._last_indices, m._last_weights = idx, w
    m.update_gate_bias(0.01)
    counts = torch.bincount(idx.flatten(), minlength=8).float()  # [4,2,1,1,0,0,0,0], mean 1
    expect = torch.zeros(8)
    expect[counts > 1.1] -= 0.01
    expect[counts < 0.9] += 0.01
    assert torch.allclose(m.gate.bias.detach(), expect)
    f = counts / counts.sum()
    P = torch.zeros(8)
    for t in range(4):
        for j in range(2):
            P[idx[t, j]] += w[t, j] / 4
    assert torch.allclose(m.get_load_balance_loss(), (f * P).sum() * 8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_aux_outputs_match_reference_formulas_bitwise(dtype):
    # Both count sources (dispatch counts recorded at forward, or bincount of
    # a replaced _last_indices) against models/moe.py:89-109 as written.
    from oracle import moe_oracle as mo
    g = torch.Generator().manual_seed(3)
    for E, k, T in ((8, 2, 257), (64, 6, 300)):
        cfg = dict(configs.C2.moe_config(), n_routed_experts=E, n_activated_experts=k)
        m = DeepSeekMoE(cfg).to(dtype)
        with torch.no_grad():
            m.gate.bias.uniform_(-0.1, 0.1, generator=g)
        idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
        for t in range(T // 2):  # skew: half the tokens pick expert 0 first
            r = idx[t].tolist()
            r.remove(0) if 0 in r else r.pop()
            idx[t] = torch.tensor([0] + r)
        w = torch.rand(T, k, generator=g)
        w = w / w.sum(-1, keepdim=True)
        for recorded in (False, True):
            m._last_indices, m._last_weights = idx, w
            if recorded:
                m._last_counts = torch.bincount(idx.flatten(), minlength=E).int()
                m._counts_of = idx
            want = mo.gate_bias_step(m.gate.bias, idx, E, 0.003)
            loss = m.get_load_balance_loss()
            assert torch.equal(loss, mo.load_balance_loss(idx, w, E))
            m.update_gate_bias(0.003)
            assert torch.equal(m.gate.bias.detach(), want)


def test_swiglu_and_dense_ffn_interface():
    # models/moe.py:11-21 and models/fusionllm.py:17-27: bias-free w1, w2, w3;
    # the forward runs on the kernels only (a CPU tensor raises, no fallback).
    from fusionllm_amd import DenseFFN
    for cls in (SwiGLUExpert, DenseFFN):
        e = cls(64, 128)
        assert {n: tuple(p.shape) for n, p in e.named_parameters()} == {
            "w1.weight": (128, 64), "w2.weight": (64, 128), "w3.weight": (128, 64)}
        with pytest.raises(RuntimeError):
            e(torch.randn(5, 64))


def test_checkpoint_round_trip_keeps_reference_layout(tmp_path):
    # training/checkpoint.py:27-28,45-50: the model state goes to safetensors
    # as {name: bf16 contiguous tensor}; the drop-in's keys and shapes are the
    # reference's, so a checkpoint written from one loads into the other.
    from safetensors.torch import load_file, save_file
    torch.manual_seed(0)
    a = DeepSeekMoE(configs.C2.moe_config())
    state = {k: v.contiguous().to(torch.bfloat16) for k, v in a.state_dict().items()}
    save_file(state, str(tmp_path / "model.safetensors"))
    b = DeepSeekMoE(configs.C2.moe_config())
    missing, unexpected = b.load_state_dict(load_file(str(tmp_path / "model.safetensors")), strict=True)
    assert not missing and not unexpected
    for k, v in b.state_dict().items():
        assert torch.equal(v, state[k].float()), k
    assert sorted(state) == sorted(dict(a.named_parameters()))


def test_operator_fake_shapes():
    # The fusionllm::moe_fwd / moe_bwd operators under fake tensors (what
    # torch.compile traces with): static output shapes and dtypes, no kernel
    # call, no GPU needed.
    import fusionllm_amd  # noqa: F401  (registers the operators)
    from torch._subclasses.fake_tensor import FakeTensorMode
    T, d, E, k, inter = 5, 64, 4, 2, 128
    with FakeTensorMode():
        bf = dict(device="cuda", dtype=torch.bfloat16)
        x = torch.empty(T, d, device="cuda", dtype=torch.float32)
        gw, gb = torch.empty(E, d, **bf), torch.empty(E, **bf)
        ws = []
        for _ in range(E + 1):
            ws += [torch.empty(inter, d, **bf), torch.empty(inter, d, **bf), torch.empty(d, inter, **bf)]
        out = torch.ops.fusionllm.moe_fwd(x, gw, gb, ws, k, 1.0, True, torch.float32)
        rows = T * k + T
        assert [tuple(o.shape) for o in out] == [
            (T, d), (T, k), (T, k), (E,), (T, k), (T, k), (E + 1,), (T * k,), (T * k,), (T * k, d),
            (rows, 2 * inter), (rows, inter), (rows, d)]
        assert [o.dtype for o in out[:4]] == [torch.float32, torch.int64, torch.float32, torch.int32]
        y, idx64, w, counts, idx, v, offsets, perm, pos, x_perm, ab, h, o = out
        g = torch.ops.fusionllm.moe_bwd(y, x, gw, gb, ws, idx, w, v, offsets, perm, pos, x_perm, ab, h, o,
                                        k, 1.0, True)
        assert len(g) == 3 + len(ws)
        assert (tuple(g[0].shape), g[0].dtype) == ((T, d), torch.float32)
        assert all(tuple(a.shape) == tuple(b.shape) for a, b in zip(g[3:], ws))
