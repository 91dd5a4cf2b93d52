"""Static check of matrix-core result hazards in the library's own gfx950 ISA.

A v_mfma writes its destination over several passes, and the hardware does
not interlock a later instruction that touches those registers: the code
must put enough independent instructions (or s_nop) in between. On gfx950
the required distance for a read or write by a VALU, LDS, VMEM or
accumulator-move instruction, and for a SrcA/SrcB read by another MFMA, is
passes + 4 wait states (8 for v_mfma_f32_16x16x32_bf16, 4 passes; 12 for
v_mfma_f32_32x32x16_bf16, 8 passes). An MFMA whose SrcC is exactly the
earlier MFMA's destination (full overlap: the chained accumulation, whatever
its own destination) is the one access that needs none; a partial overlap
of SrcC, or any overlap of SrcA/SrcB, is checked like the rest.

This module compiles HIP sources to assembly (hipcc --cuda-device-only -S),
splits the kernels into instructions and basic blocks, and walks every path
forward from each MFMA (through conditional and unconditional branches,
including loop back edges) until the required number of wait states has
passed, reporting any instruction on the way that touches the destination.
It checks what the compiler emitted, so it covers accesses after a branch
join (the shape that a uniform branch around an MFMA creates).
"""

from __future__ import annotations

import os
import re
import subprocess
from dataclasses import dataclass, field

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# passes of the MFMA opcodes the kernels use (gfx950)
PASSES = {
    "v_mfma_f32_16x16x32_bf16": 4,
    "v_mfma_f32_32x32x16_bf16": 8,
}
EXTRA_WAIT = 4  # required wait states = passes + EXTRA_WAIT (gfx950)

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")
_LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")


@dataclass
class Insn:
    text: str
    mnem: str
    ops: list
    label: str | None = None  # branch target
    waits: int = 1


@dataclass
class Kernel:
    name: str
    insns: list = field(default_factory=list)
    labels: dict = field(default_factory=dict)  # label -> index of the next instruction


def _regs(op: str) -> set:
    out = set()
    for m in _REG.finditer(op):
        kind = m.group(1)
        if m.group(4) is not None:
            lo = hi = int(m.group(4))
        else:
            lo, hi = int(m.group(2)), int(m.group(3))
        out.update((kind, r) for r in range(lo, hi + 1))
    return out


def _split_ops(rest: str) -> list:
    ops, depth, cur = [], 0, ""
    for ch in rest:
        if ch == "[":
            depth += 1
        elif ch == "]":
            depth -= 1
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return ops


def parse_asm(text: str) -> list:
    """Kernels of an AMDGPU assembly listing, as instruction lists with labels."""
    kernels, cur = [], None
    for raw in text.splitlines():
        line = raw.split(";")[0].rstrip()
        if not line.strip():
            continue
        m = _LABEL.match(line.strip())
        if m and not line.startswith("\t") and not line.startswith(" "):
            name = m.group(1)
            if not name.startswith("."):
                cur = Kernel(name)
                kernels.append(cur)
            elif cur is not None:
                cur.labels[name] = len(cur.insns)
            continue
        if cur is None:
            continue
        s = line.strip()
        if s.startswith("."):
            if s.startswith(".Lfunc_end"):
                cur = None
            continue
        parts = s.split(None, 1)
        mnem = parts[0]
        ops = _split_ops(parts[1]) if len(parts) > 1 else []
        ins = Insn(s, mnem, ops)
        if mnem == "s_nop":
            ins.waits = int(ops[0], 0) + 1
        if mnem.startswith("s_cbranch") or mnem == "s_branch":
            ins.label = ops[0] if ops else None
        cur.insns.append(ins)
    return kernels


def _defs_uses(ins: Insn):
    """(registers written, registers read) of one instruction, v and a only."""
    m = ins.mnem
    if m.startswith("s_"):
        return set(), set()
    regs = [_regs(o) for o in ins.ops]
    if not regs:
        return set(), set()
    stores = ("ds_write", "ds_store", "buffer_store", "global_store", "flat_store", "scratch_store")
    if m.startswith(stores) or m.startswith("exp"):
        return set(), set().union(*regs)
    if m.startswith("ds_") and not m.startswith(("ds_read", "ds_load")) and len(regs) > 1:
        # LDS atomics with return: first operand written, the rest read
        return regs[0], set().union(*regs[1:])
    return regs[0], set().union(*regs[1:]) if len(regs) > 1 else set()


@dataclass
class Violation:
    kernel: str
    mfma_index: int
    mfma: str
    index: int
    insn: str
    distance: int
    required: int


def check_kernel(k: Kernel) -> tuple:
    """(violations, number of MFMAs checked) for one kernel."""
    n = len(k.insns)
    succ = []
    for i, ins in enumerate(k.insns):
        s = []
        if ins.mnem == "s_endpgm":
            pass
        elif ins.mnem == "s_branch":
            if ins.label in k.labels:
                s.append(k.labels[ins.label])
        else:
            if i + 1 < n:
                s.append(i + 1)
            if ins.label in k.labels:
                s.append(k.labels[ins.label])
        succ.append(s)
    du = [_defs_uses(ins) for ins in k.insns]
    out, count = [], 0
    for i, ins in enumerate(k.insns):
        if not ins.mnem.startswith("v_mfma"):
            continue
        passes = PASSES.get(ins.mnem.split("_e64")[0])
        if passes is None:
            raise ValueError(f"unknown MFMA opcode {ins.mnem} in {k.name}")
        count += 1
        need = passes + EXTRA_WAIT
        dst = _regs(ins.ops[0])
        # (instruction index, wait states elapsed before it); DFS over paths
        stack = [(j, 0) for j in succ[i]]
        seen = {}
        while stack:
            j, dist = stack.pop()
            if dist >= need:
                continue
            if seen.get(j, -1) >= need - dist:
                continue
            seen[j] = need - dist
            nxt = k.insns[j]
            d, u = du[j]
            touched = (d | u) & dst
            if touched:
                ok = False
                if nxt.mnem.startswith("v_mfma"):
                    # chained accumulation: SrcC exactly the earlier vDst, which
                    # the new vDst may overwrite in place or not at all
                    src_ab = _regs(nxt.ops[1]) | _regs(nxt.ops[2])
                    new_dst = _regs(nxt.ops[0])
                    ok = (not (src_ab & dst) and _regs(nxt.ops[3]) == dst
                          and (new_dst == dst or not (new_dst & dst)))
                if not ok:
                    out.append(Violation(k.name, i, ins.text, j, nxt.text, dist, need))
                continue  # stop on this path at the first access
            for s in succ[j]:
                stack.append((s, dist + nxt.waits))
    return out, count


def _successors(k: Kernel) -> list:
    n = len(k.insns)
    succ = []
    for i, ins in enumerate(k.insns):
        s = []
        if ins.mnem == "s_branch":
            if ins.label in k.labels:
                s.append(k.labels[ins.label])
        elif ins.mnem != "s_endpgm":
            if i + 1 < n:
                s.append(i + 1)
            if ins.label in k.labels:
                s.append(k.labels[ins.label])
        succ.append(s)
    return succ


def _writes_exec(ins: Insn) -> bool:
    return ("saveexec" in ins.mnem or ins.mnem.startswith("v_cmpx")
            or (ins.mnem.startswith("s_") and bool(ins.ops) and ins.ops[0] == "exec"))


DPP_AFTER_VALU = 2  # wait states between a VALU write of a VGPR and a DPP read of it
DPP_AFTER_EXEC = 5  # wait states between a write of EXEC and a DPP instruction


def check_dpp(k: Kernel) -> tuple:
    """(violations, number of DPP instructions checked): on every path into a
    DPP instruction (…_dpp), no VALU instruction writes its DPP source (the
    first source operand) within DPP_AFTER_VALU wait states and nothing
    writes EXEC within DPP_AFTER_EXEC. The compiler keeps these distances
    for the DPP instructions it creates, but not for ones written in inline
    asm."""
    succ = _successors(k)
    pred = [[] for _ in k.insns]
    for i, s in enumerate(succ):
        for j in s:
            pred[j].append(i)
    out, count = [], 0
    for i, ins in enumerate(k.insns):
        if not ins.mnem.endswith("_dpp"):
            continue
        count += 1
        src = _regs(ins.ops[1]) if len(ins.ops) > 1 else set()
        stack = [(p, 0) for p in pred[i]]
        seen = {}
        while stack:
            j, dist = stack.pop()
            if dist >= DPP_AFTER_EXEC or seen.get(j, DPP_AFTER_EXEC + 1) <= dist:
                continue
            seen[j] = dist
            prev = k.insns[j]
            if _writes_exec(prev):
                out.append(Violation(k.name, i, ins.text, j, prev.text, dist, DPP_AFTER_EXEC))
                continue
            if (dist < DPP_AFTER_VALU and prev.mnem.startswith("v_") and not prev.mnem.startswith("v_mfma")
                    and prev.ops and _regs(prev.ops[0]) & src):
                out.append(Violation(k.name, i, ins.text, j, prev.text, dist, DPP_AFTER_VALU))
                continue
            for p in pred[j]:
                stack.append((p, dist + prev.waits))
    return out, count


_VMCNT = re.compile(r"\bvmcnt\((\d+)\)")


def _lds_copy(ins: Insn) -> bool:
    return ins.mnem.startswith("buffer_load") and ins.text.endswith(" lds")


def main_loop(k: Kernel):
    """(first, last) instruction indices of the kernel's pipelined loop: of
    the loops (a label and a later branch back to it) that copy global
    memory into LDS (buffer_load ... lds), the one with the most MFMAs.
    None without one."""
    best, most = None, -1
    for i, ins in enumerate(k.insns):
        if ins.label is None or ins.label not in k.labels or k.labels[ins.label] > i:
            continue
        lo = k.labels[ins.label]
        if not any(_lds_copy(k.insns[j]) for j in range(lo, i + 1)):
            continue
        n = sum(1 for j in range(lo, i + 1) if k.insns[j].mnem.startswith("v_mfma"))
        if n > most:
            best, most = (lo, i), n
    return best


def stage_waits(k: Kernel) -> list:
    """A pipelined loop of the shape `s_waitcnt vmcnt(W); s_barrier; <this
    step's loads>; <matrix-core work>` per step: for each s_barrier of the
    main loop, (W of the last vmcnt wait before it, buffer loads from it to
    the next barrier or the loop's end). W is None if no wait precedes the
    barrier inside the loop."""
    loop = main_loop(k)
    if loop is None:
        return []
    lo, hi = loop
    bars = [j for j in range(lo, hi + 1) if k.insns[j].mnem == "s_barrier"]
    out = []
    for n, j in enumerate(bars):
        w = None
        for p in range(j - 1, lo - 1, -1):
            if k.insns[p].mnem == "s_barrier":
                break
            m = _VMCNT.search(k.insns[p].text) if k.insns[p].mnem == "s_waitcnt" else None
            if m:
                w = int(m.group(1))
                break
        end = bars[n + 1] if n + 1 < len(bars) else hi + 1
        loads = sum(1 for q in range(j + 1, end) if k.insns[q].mnem.startswith("buffer_load"))
        out.append((w, loads))
    return out


def compile_asm(src: str, include: str, out_dir: str) -> str:
    """Device assembly of one HIP source for gfx950, with the library's flags."""
    out = os.path.join(out_dir, os.path.splitext(os.path.basename(src))[0] + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-I", include, src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stderr}")
    with open(out) as f:
        return f.read()
