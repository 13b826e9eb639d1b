"""Wait states the compiler cannot insert: the prefill kernel's direct-to-LDS
buffer loads are inline asm, so its hazard recognizer does not see them.  This
compiles prefill_attention.hip to gfx950 assembly (with the library's own
flags) and checks, with the scan build.py also runs, two rules of gfx9-family
parts on every such load:

* a scalar write of M0 needs one wait state before an LDS-DMA load (the asm
  starts with s_nop);
* a vector instruction writing an SGPR (v_readfirstlane) needs five wait
  states before a buffer load reads that SGPR (as its scalar offset or its
  resource descriptor), unless a scalar instruction rewrote it in between.

CPU only (hipcc cross-compiles); skipped where hipcc is absent.
"""
import os
import shutil
import subprocess

import pytest

from mycustomcudaengine_amd import build
from mycustomcudaengine_amd.asm_check import check, lds_dma_violations, valu_sgpr_vmem_violations

SRC = os.path.join(build.CSRC, "prefill_attention.hip")


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    cc = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc")
                                   else None)
    if cc is None:
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "prefill.s")
    res = subprocess.run([build.hipcc(), *build.compile_flags(), "--cuda-device-only", "-S", SRC,
                          "-o", out],
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
    # a spilled descriptor reloaded from a VGPR lane right before the load
    spill = ("\tv_readlane_b32 s6, v247, 2\n\tv_readlane_b32 s7, v247, 3\n\ts_nop 0\n"
             "\tbuffer_load_dwordx4 v1, s[4:7], s35 offen lds\n")
    assert len(valu_sgpr_vmem_violations(spill)) == 1
    assert len(check(spill)) == 1 and check(ok) == []
