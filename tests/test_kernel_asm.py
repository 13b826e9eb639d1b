"""Wait states the compiler cannot insert: the prefill kernel's direct-to-LDS
buffer loads are inline asm, so its hazard recognizer does not see them.  This
compiles prefill_attention.hip to gfx950 assembly (with the library's own
flags) and checks two rules of gfx9-family parts on every such load:

* a scalar write of M0 needs one wait state before an LDS-DMA load (the asm
  starts with s_nop);
* a vector instruction writing an SGPR (v_readfirstlane) needs five wait
  states before a buffer load reads that SGPR (as its scalar offset or its
  resource descriptor), unless a scalar instruction rewrote it in between.

CPU only (hipcc cross-compiles); skipped where hipcc is absent.
"""
import os
import re
import shutil
import subprocess

import pytest

from mycustomcudaengine_amd import build

SRC = os.path.join(build.CSRC, "prefill_attention.hip")


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


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    cc = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc")
                                   else None)
    if cc is None:
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "prefill.s")
    flags = [f for f in build.compile_flags() if f not in ("-fPIC",)]
    res = subprocess.run([build.hipcc(), *flags, "--cuda-device-only", "-S", SRC, "-o", out],
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    with open(out) as f:
        return f.read()


def test_every_lds_dma_load_follows_a_wait_state(prefill_asm):
    n = sum(1 for line in prefill_asm.split("\n")
            if "buffer_load_dwordx4" in line and line.strip().endswith(" lds"))
    assert n > 100  # the staging of every instantiation
    assert lds_dma_violations(prefill_asm) == []


def test_no_vector_written_sgpr_read_by_a_buffer_load_too_soon(prefill_asm):
    assert valu_sgpr_vmem_violations(prefill_asm) == []


def test_the_scans_catch_planted_hazards():
    """The checks themselves: each rule flags a sequence that breaks it."""
    m0 = "\ts_mov_b32 m0, s4\n\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n"
    assert len(lds_dma_violations(m0)) == 1
    ok = "\ts_mov_b32 m0, s4\n\ts_nop 0\n\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n"
    assert lds_dma_violations(ok) == []
    rfl = "\tv_readfirstlane_b32 s3, v1\n\ts_nop 0\n\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n"
    assert len(valu_sgpr_vmem_violations(rfl)) == 1
    fixed = "\tv_readfirstlane_b32 s3, v1\n\ts_nop 4\n\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n"
    assert valu_sgpr_vmem_violations(fixed) == []
    rewritten = ("\tv_readfirstlane_b32 s3, v1\n\ts_lshl_b32 s3, s3, 1\n"
                 "\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n")
    assert valu_sgpr_vmem_violations(rewritten) == []
    rsrc = "\tv_readfirstlane_b32 s9, v1\n\tbuffer_load_dwordx4 v2, s[8:11], s3 offen lds\n"
    assert len(valu_sgpr_vmem_violations(rsrc)) == 1
