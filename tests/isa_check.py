"""Check the gfx950 machine code of this build for accesses to registers that a
memory load has not filled yet (not collected: no test_ prefix).

The GEMM kernels issue their LDS fragment reads from inline assembly and
wait for them with explicit s_waitcnt instructions, which the compiler does
not see.  If the compiler ever moved, copied or reused a register that such a
read is still filling (between the read and the s_waitcnt that covers it),
the kernel would compute with stale values, or a late read would overwrite a
live one.  This module disassembles the code objects built here (llvm-objdump
from ROCm) and runs a dataflow pass over each kernel's control-flow graph:

* every LDS instruction (ds_*) and scalar memory load (s_load*, s_buffer_load*)
  takes a slot in the LGKM counter, every vector memory instruction (global_*,
  buffer_*, scratch_*) one in the VM counter; flat_* one in both.  A slot
  records the registers that instruction writes;
* `s_waitcnt lgkmcnt(N)` / `vmcnt(N)` leaves only the N youngest slots of that
  counter pending (both counters complete in issue order for the loads this
  check cares about; the compiler waits for its scalar loads with
  lgkmcnt(0));
* any instruction that reads or writes a register of a pending slot is a
  hazard, except a later load of the same counter writing it again (the two
  complete in order);
* at a control-flow join the pending lists of the predecessors are merged
  youngest-first (register sets united position by position), which over-
  approximates every path.

Only the AMD assembly of code built in this repository is read.
"""
from __future__ import annotations

import re
import shutil
import subprocess
import tempfile
from dataclasses import dataclass, field
from pathlib import Path

ROCM_LLVM = Path("/opt/rocm/llvm/bin")
_REG = re.compile(r"\b([vas])\[(\d+):(\d+)\]|\b([vas])(\d+)\b")
_ADDR = re.compile(r"//\s*([0-9A-Fa-f]{8,16}):")
_TARGET = re.compile(r"<([^>+]+)\+0x([0-9a-fA-F]+)>")
_FUNC = re.compile(r"^[0-9a-fA-F]+ <([^>]+)>:$")


def _regs(text: str) -> set[tuple[str, int]]:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            kind, lo, hi = m.group(1), int(m.group(2)), int(m.group(3))
        else:
            kind, lo = m.group(4), int(m.group(5))
            hi = lo
        for r in range(lo, hi + 1):
            out.add((kind, r))
    return out


@dataclass
class Insn:
    addr: int
    op: str
    operands: str
    target: int | None = None  # branch target address


@dataclass
class Kernel:
    name: str
    insns: list[Insn] = field(default_factory=list)


def disassemble(obj: Path) -> list[Kernel]:
    """Kernels of the gfx950 code object inside a hipcc -c object file."""
    objdump = ROCM_LLVM / "llvm-objdump"
    with tempfile.TemporaryDirectory() as td:
        local = Path(td) / obj.name
        shutil.copy(obj, local)
        subprocess.run([str(objdump), "--offloading", str(local)], check=True, capture_output=True, cwd=td)
        dev = [p for p in Path(td).iterdir() if "gfx950" in p.name]
        if not dev:
            return []  # host-only object
        res = subprocess.run([str(objdump), "-d", "--no-show-raw-insn", str(dev[0])], check=True,
                             capture_output=True, text=True)
    kernels: list[Kernel] = []
    cur = None
    for line in res.stdout.splitlines():
        m = _FUNC.match(line.strip())
        if m:
            cur = Kernel(m.group(1))
            kernels.append(cur)
            continue
        if cur is None or not line.startswith("\t"):
            continue
        am = _ADDR.search(line)
        if not am:
            continue
        body = line.split("//")[0].strip()
        if not body:
            continue
        parts = body.split(None, 1)
        ins = Insn(int(am.group(1), 16), parts[0], parts[1] if len(parts) > 1 else "")
        tm = _TARGET.search(line)
        if tm and parts[0].startswith(("s_branch", "s_cbranch")):
            base = cur.insns[0].addr if cur.insns else ins.addr
            ins.target = base + int(tm.group(2), 16)
        cur.insns.append(ins)
    return kernels


def _classify(ins: Insn):
    """(counters it takes a slot in, registers it writes as a load, registers it reads or writes otherwise)."""
    op, text = ins.op, ins.operands
    regs = _regs(text)
    first = text.split(",")[0] if text else ""
    if op.startswith("ds_"):
        loads = op.startswith(("ds_read", "ds_load", "ds_bpermute", "ds_permute", "ds_swizzle")) or "_rtn" in op
        dst = _regs(first) if loads else set()
        return ("lgkm",), dst, regs - dst
    if op.startswith(("s_load", "s_buffer_load")):
        dst = _regs(first)
        return ("lgkm",), dst, regs - dst
    if op.startswith(("global_", "buffer_", "scratch_", "flat_")):
        counters = ("vm", "lgkm") if op.startswith("flat_") else ("vm",)
        writes = ("load" in op and "_lds" not in op and not op.endswith("lds")) or ("atomic" in op and "_rtn" in op)
        dst = _regs(first) if writes else set()
        return counters, dst, regs - dst
    return (), set(), regs


def _waits(ins: Insn) -> dict[str, int]:
    if ins.op != "s_waitcnt":
        return {}
    out = {}
    for name, key in (("vmcnt", "vm"), ("lgkmcnt", "lgkm")):
        m = re.search(name + r"\((\d+)\)", ins.operands)
        if m:
            out[key] = int(m.group(1))
    return out


State = dict  # counter -> tuple of frozensets (oldest first)
# A wave stops issuing when a counter would exceed its maximum, so at most this
# many operations of each counter are ever in flight (gfx9: 6-bit vmcnt, 4-bit
# lgkmcnt); older slots have completed.
LIMIT = {"vm": 63, "lgkm": 15}


def _merge(a: State, b: State) -> State:
    out = {}
    for c in ("vm", "lgkm"):
        x, y = list(a.get(c, ())), list(b.get(c, ()))
        n = min(max(len(x), len(y)), LIMIT[c])
        x, y = x[len(x) - min(len(x), n):], y[len(y) - min(len(y), n):]
        x = [frozenset()] * (n - len(x)) + x
        y = [frozenset()] * (n - len(y)) + y
        out[c] = tuple(p | q for p, q in zip(x, y))
    return out


def check_kernel(k: Kernel) -> list[str]:
    """Hazards of one kernel, as readable strings (empty list: none found)."""
    insns = k.insns
    index = {ins.addr: i for i, ins in enumerate(insns)}
    # basic-block leaders
    leaders = {0}
    for i, ins in enumerate(insns):
        if ins.target is not None:
            if ins.target in index:
                leaders.add(index[ins.target])
            leaders.add(i + 1)
        elif ins.op in ("s_endpgm", "s_setpc_b64"):
            leaders.add(i + 1)
    starts = sorted(s for s in leaders if s < len(insns))
    block_of = {}
    blocks = []
    for j, s in enumerate(starts):
        e = starts[j + 1] if j + 1 < len(starts) else len(insns)
        blocks.append((s, e))
        block_of[s] = j
    succ = []
    for s, e in blocks:
        last = insns[e - 1]
        nxt = []
        if last.target is not None and last.target in index:
            nxt.append(block_of[index[last.target]])
        if last.op not in ("s_branch", "s_endpgm", "s_setpc_b64") and e < len(insns):
            nxt.append(block_of[e])
        succ.append(nxt)

    entry: dict[int, State] = {0: {"vm": (), "lgkm": ()}}
    hazards: dict[int, str] = {}
    work = [0]
    visits = 0
    while work:
        visits += 1
        if visits > 200000:
            raise RuntimeError(f"{k.name}: dataflow did not converge")
        b = work.pop()
        state = {c: list(v) for c, v in entry[b].items()}
        s, e = blocks[b]
        for ins in insns[s:e]:
            w = _waits(ins)
            for c, n in w.items():
                state[c] = state[c][len(state[c]) - n:] if n < len(state[c]) else state[c]
            counters, dst, used = _classify(ins)
            for c in ("vm", "lgkm"):
                pend = set().union(*state[c]) if state[c] else set()
                # rewriting a pending destination with a load of the same counter is ordered
                touched = used | (dst if c not in counters else set())
                bad = touched & pend
                if bad and ins.addr not in hazards:
                    regs = ", ".join(f"{kd}{r}" for kd, r in sorted(bad))
                    hazards[ins.addr] = (f"{k.name} @0x{ins.addr:x}: {ins.op} {ins.operands} touches {regs} "
                                         f"while a {c} load into it may be in flight")
            for c in counters:
                state[c].append(frozenset(dst))
                if len(state[c]) > LIMIT[c]:
                    del state[c][0]
        out = {c: tuple(v) for c, v in state.items()}
        for nb in succ[b]:
            old = entry.get(nb)
            new = out if old is None else _merge(old, out)
            if new != old:
                entry[nb] = new
                work.append(nb)
    return list(hazards.values())


def check_object(obj: Path, kernel_filter=None) -> tuple[int, list[str]]:
    """(kernels checked, hazards) for the gfx950 code of one object file."""
    kernels = disassemble(obj)
    if kernel_filter is not None:
        kernels = [k for k in kernels if kernel_filter(k.name)]
    hazards = []
    for k in kernels:
        hazards += check_kernel(k)
    return len(kernels), hazards
