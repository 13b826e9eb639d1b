"""Wait-state checks for the inline-asm loads of the prefill kernel.

The prefill kernel's direct-to-LDS buffer loads are inline asm, and the
compiler's hazard recognizer does not look inside inline asm, so it cannot
insert the wait states those loads need.  This scans gfx950 assembly for the
two rules of gfx9-family parts that apply to them:

* a scalar write of M0 needs one wait state before an LDS-DMA load (the asm
  itself starts with s_nop);
* a vector instruction writing an SGPR (v_readfirstlane, or v_readlane when
  the compiler reloads a spilled SGPR) needs five wait states before a buffer
  load reads that SGPR as its scalar offset or resource descriptor, unless a
  scalar instruction rewrote it in between.  A descriptor read too early makes
  the load address memory through a stale base, which faults the GPU.

`build.py` runs the scan on every build and refuses a library that breaks
either rule; tests/test_kernel_asm.py checks the scan itself.
"""
from __future__ import annotations

import re


def _sgprs(tok: str) -> set:
    tok = tok.strip().rstrip(",")
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _instructions(asm: str):
    """(opcode, operands, line) of every instruction; None marks a label or a
    function start (where the scan conservatively forgets its history)."""
    for line in asm.split("\n"):
        t = line.strip()
        if re.match(r"^_Z\S*:", line) or (t.endswith(":") and not t.startswith(";")):
            yield None
            continue
        if not t or t.startswith(";") or t.startswith("."):
            continue
        op = t.split()[0]
        ops = [x for x in re.split(r"[ ,]+", t[len(op):].strip()) if x]
        yield op, ops, t


def lds_dma_violations(asm: str) -> list:
    """LDS-DMA buffer loads not directly preceded by an s_nop."""
    bad, prev = [], None
    for ins in _instructions(asm):
        if ins is None:
            prev = None
            continue
        op, ops, t = ins
        if op.startswith("buffer_load") and t.endswith(" lds") and (prev is None or prev != "s_nop"):
            bad.append(t)
        prev = op
    return bad


def valu_sgpr_vmem_violations(asm: str) -> list:
    """Buffer / global / flat accesses reading an SGPR that a vector
    instruction wrote fewer than five wait states before."""
    bad, hist = [], []
    for ins in _instructions(asm):
        if ins is None:
            hist = []
            continue
        op, ops, t = ins
        if op.startswith(("buffer_", "global_", "flat_")):
            live = set()
            for x in ops[1:]:
                live |= _sgprs(x)
            waits = 0
            for op2, w2, n2 in reversed(hist):
                if waits >= 5 or not live:
                    break
                if op2.startswith("v_") and w2 & live:
                    bad.append(f"{op2} -> {t}")
                    break
                if op2.startswith("s_"):
                    live -= w2
                waits += n2
        writes = set()
        if ops and op.startswith(("v_", "s_")) and not op.startswith(
                ("s_cmp", "s_waitcnt", "s_nop", "s_barrier", "s_branch", "s_cbranch")):
            writes = _sgprs(ops[0])
        n = int(ops[0], 0) + 1 if op == "s_nop" and ops else 1
        hist = (hist + [(op, writes, n)])[-12:]
    return bad


def check(asm: str) -> list:
    """Every violation of both rules (empty: the assembly is safe to run)."""
    return [f"M0 wait state: {x}" for x in lds_dma_violations(asm)] + \
        [f"VALU-written SGPR: {x}" for x in valu_sgpr_vmem_violations(asm)]
