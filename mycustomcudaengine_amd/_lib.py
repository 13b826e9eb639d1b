"""ctypes binding of libmce.so (declarations: include/mce_abi.h).

The library is loaded after torch, so its `libamdhip64.so.7` dependency binds
to the HIP runtime torch already mapped: device pointers and stream handles
from torch are valid in the library.  `load()` verifies that only one HIP
runtime is mapped into the process.

There is no fallback: if libmce.so is missing, `load()` raises.
"""
from __future__ import annotations

import ctypes
import os
import re
import threading

import torch  # noqa: F401  (maps torch's HIP runtime first)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmce.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "mce_abi.h")

MCE_OK = 0
MCE_ERR_INVALID = 1
MCE_ERR_UNSUPPORTED = 2
MCE_ERR_LAUNCH = 3
MCE_ERR_WORKSPACE = 4
MCE_F16 = 0
MCE_BF16 = 1
MCE_DECODE_NOALLOC_SCRATCH_BYTES = 16 << 20
# MCE_ABI_VERSION of include/mce_abi.h: the argument lists in SIGNATURES
# below are those of this version, so load() refuses a library of another.
MCE_ABI_VERSION = 101

_c_int, _c_i64, _c_f, _c_sz, _vp = (
    ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p)

# name -> (restype, argtypes); mirrors include/mce_abi.h.
SIGNATURES = {
    "mce_last_error": (ctypes.c_char_p, []),
    "mce_abi_version": (_c_int, []),
    "mce_rmsnorm": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f, _vp]),
    "mce_swiglu": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
    "mce_paged_kv_store": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_int, _c_int,
                                    _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
    "mce_paged_attention_decode_workspace_size": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "mce_paged_attention_decode": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                            _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                            _c_f, _vp, _c_sz, _vp]),
    "mce_paged_attention_decode_noalloc": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                                    _c_int, _c_int, _c_int, _c_int, _c_int,
                                                    _c_i64, _c_f, _vp]),
    "mce_rope_inplace": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                  _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                  _c_i64, _c_i64, _vp]),
    "mce_prefill_attention": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _c_f, _vp]),
    "mce_decode_gemm": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_i64, _c_i64,
                                 _c_int, _vp]),
    "mce_rmsnorm_decode_gemm": (_c_int, [_c_int, _vp, _vp, _c_f, _vp, _vp, _c_int, _c_int, _c_int,
                                         _c_i64, _c_i64, _c_int, _vp]),
    "mce_argmax_rows_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "mce_argmax_rows": (_c_int, [_c_int, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_sz, _vp]),
    "mce_prefill_attention_paged_workspace_size": (_c_sz, [_c_int, _c_int, _c_int, _c_int]),
    "mce_prefill_attention_paged": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                             _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                             _c_i64, _c_f, _vp, _c_sz, _vp]),
    "mce_decode_advance": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                    _c_int, _vp]),
    "mce_paged_attention_decode_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                                 _c_int, _c_int, _c_int, _c_int, _c_i64,
                                                 _c_i64, _c_i64, _c_i64, _c_f, _vp]),
    "mce_rope_kv_store": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _c_i64, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_i64,
                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
}

_lib = None
_lock = threading.Lock()


class MCEError(RuntimeError):
    """A libmce entry point returned a nonzero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of the entry points the C header declares (MCE_API ... name()."""
    text = open(path).read()
    return re.findall(r"MCE_API\s+[\w\s\*]*?\b(mce_\w+)\s*\(", text)


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    paths.add(os.path.realpath(line.split()[-1]))
    except OSError:
        pass
    return paths


def load() -> ctypes.CDLL:
    """Loads libmce.so once and returns it; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m mycustomcudaengine_amd.build` "
                "(no CPU fallback exists for these ops)")
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.mce_abi_version()
        if version != MCE_ABI_VERSION:
            raise ImportError(
                f"{LIB_PATH} has ABI version {version}, this binding expects "
                f"{MCE_ABI_VERSION}; rebuild with `python -m mycustomcudaengine_amd.build`")
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise ImportError(
                "two HIP runtimes are mapped into this process "
                f"({sorted(runtimes)}); libmce.so must share torch's")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Calls entry point `name`; raises MCEError on a nonzero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != MCE_OK:
        msg = lib.mce_last_error().decode(errors="replace")
        raise MCEError(name, status, msg)
