"""Builds libmce.so (the C-ABI kernel library) in-tree with hipcc for gfx950.

Replaces the reference's nvcc CUDAExtension build (setup.py:22-42).  There is
no torch dependency at build time: the library exports only the `extern "C"`
entry points declared in include/mce_abi.h.

Usage:  python -m mycustomcudaengine_amd.build [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

if __package__:
    from . import asm_check
else:  # run as a script
    import asm_check

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libmce.so")
SOURCES = [
    "mce_runtime.hip",
    "elementwise.hip",
    "decode_attention.hip",
    "prefill_attention.hip",
    "decode_gemm.hip",
    "decode_loop.hip",
]
# sources whose inline-asm buffer loads are scanned for missing wait states
ASM_CHECKED = ["prefill_attention.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fvisibility=hidden",
        # 16-bit storage is read and written through wider vector types.
        "-fno-strict-aliasing",
        "-Wall",
        "-Wno-unused-function",
        # Packed fp32 VALU ops are kept out of every kernel.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{os.path.join(REPO_DIR, 'include')}",
    ]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature,
    # and a device-only -S compile that --hip-link goes unused.
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops" not in l and "'--hip-link'" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compiles every source and links libmce.so; returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    cc = hipcc()
    flags = compile_flags()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *flags, "-c", os.path.join(CSRC, src), "-o", obj])
    # gfx950 assembly of the sources with inline-asm loads, for the wait-state
    # scan below
    asm_files = []
    for src in ASM_CHECKED:
        out = os.path.join(BUILD_DIR, src.replace(".hip", ".s"))
        asm_files.append(out)
        cmds.append([cc, *flags, "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", out])
    jobs = jobs or min(len(cmds), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    # The compiler inserts no wait states for instructions inside inline asm;
    # a library whose inline-asm loads could read a stale SGPR is refused
    # (such a load can fault the GPU).
    for path in asm_files:
        with open(path) as f:
            bad = asm_check.check(f.read())
        if bad:
            raise RuntimeError(f"{os.path.basename(path)}: {len(bad)} inline-asm wait-state "
                               "violation(s):\n  " + "\n  ".join(bad[:20]))
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
