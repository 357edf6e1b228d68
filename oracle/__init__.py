"""CPU oracle for FusionLLM's DeepSeekMoE hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the
timed CPU baseline).  The product (``fusionllm_amd``) never imports it.

* ``moe_oracle`` — torch-CPU restatement of models/moe.py:11-109 (op order,
  dtypes, fp32 index_add_ accumulator, ascending-expert combine) with a
  router switch: the reference's own module-dtype router, or the build's
  fp32-logit router.
* ``router_ref.c`` (``c_oracle()``) — bit-exact C restatement of the gfx950
  router (fp32 logits in the kernel's order, same exp) and of the dispatch
  counting sort.

Pinning (what checks each function; see tests/test_oracle.py):
* fp32 router: logits against an fp64 closed form (error bound), sigmoid
  against torch.sigmoid and fp64 (ulps), top-k against torch.topk on tie-free
  scores and against brute force with constructed ties, normalisation
  against its closed form.
* dispatch: torch.argsort(stable=True), torch.bincount, bijection.
* expert FFN / combine / backward: fp64 closed forms, brute-force dense
  combine, torch.autograd.gradcheck in fp64, and the golden vectors written
  by tests/golden/make_golden.py from the reference module itself.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
C_LIB = ORACLE_DIR / "_build" / "liboracle.so"

_c = None


def build_c() -> Path:
    """Compile router_ref.c with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return C_LIB


def c_oracle() -> ctypes.CDLL:
    global _c
    if _c is None:
        if not C_LIB.exists():
            build_c()
        lib = ctypes.CDLL(str(C_LIB))
        P = ctypes.c_void_p
        lib.oracle_expf.restype = ctypes.c_float
        lib.oracle_expf.argtypes = [ctypes.c_float]
        lib.oracle_sigmoid.restype = ctypes.c_float
        lib.oracle_sigmoid.argtypes = [ctypes.c_float]
        lib.oracle_router_fwd.restype = ctypes.c_int
        lib.oracle_router_fwd.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_float, P, P, P, P, P]
        lib.oracle_dispatch.restype = ctypes.c_int
        lib.oracle_dispatch.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P, P, P, P]
        _c = lib
    return _c
