"""CPU: the C-ABI library loads, exports every entry point include/mce_abi.h
declares, and rejects bad arguments on the host before any device work.

No test here launches a kernel: every call below fails validation (or is a
pure size query), so it runs on a machine without a GPU.
"""
import ctypes
import os
import re

import pytest
import torch

from mycustomcudaengine_amd import _lib

HEADER_ENTRY_POINTS = {
    "mce_last_error", "mce_abi_version", "mce_rmsnorm", "mce_swiglu",
    "mce_paged_kv_store", "mce_paged_attention_decode_workspace_size",
    "mce_paged_attention_decode", "mce_rope_inplace", "mce_prefill_attention",
    "mce_rope_kv_store", "mce_decode_gemm", "mce_paged_attention_decode_rope",
    "mce_rmsnorm_decode_gemm", "mce_argmax_rows", "mce_argmax_rows_workspace_size",
    "mce_decode_advance",
    "mce_prefill_attention_paged", "mce_prefill_attention_paged_workspace_size",
    "mce_paged_attention_decode_noalloc",
}


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_the_six_ops_engine_ops_and_helpers():
    assert set(_lib.header_symbols()) == HEADER_ENTRY_POINTS


def test_library_exports_every_header_symbol(lib):
    for name in _lib.header_symbols():
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == HEADER_ENTRY_POINTS


def test_single_hip_runtime_mapped(lib):
    assert len(_lib._hip_runtimes_mapped()) <= 1


def test_version(lib):
    # exact: the ctypes signatures in _lib are those of this version
    assert lib.mce_abi_version() == _lib.MCE_ABI_VERSION == 101
    hdr = open(_lib.HEADER_PATH).read()
    assert re.search(r"#define MCE_ABI_VERSION 101\b", hdr)


def _err(lib):
    return lib.mce_last_error().decode()


def test_rmsnorm_validation(lib):
    assert lib.mce_rmsnorm(7, None, None, None, 1, 8, 8, 8, 1e-5, None) == _lib.MCE_ERR_INVALID
    assert "dtype" in _err(lib)
    assert lib.mce_rmsnorm(0, None, None, None, 1, 0, 0, 0, 1e-5, None) == _lib.MCE_ERR_INVALID
    assert lib.mce_rmsnorm(0, None, None, None, 2, 8, 4, 8, 1e-5, None) == _lib.MCE_ERR_INVALID
    assert lib.mce_rmsnorm(0, None, None, None, 2, 8, 8, 8, 1e-5, None) == _lib.MCE_ERR_INVALID
    assert "null" in _err(lib)
    assert lib.mce_rmsnorm(0, None, None, None, 0, 8, 8, 8, 1e-5, None) == _lib.MCE_OK


def test_swiglu_validation(lib):
    assert lib.mce_swiglu(0, None, None, 2, 8, 15, 8, None) == _lib.MCE_ERR_INVALID
    assert lib.mce_swiglu(0, None, None, 0, 8, 16, 8, None) == _lib.MCE_OK


def test_kv_store_validation(lib):
    assert lib.mce_paged_kv_store(0, None, None, None, None, None, 4, 8, 128, 16, 10,
                                  1024, 128, 1024, 128, None) == _lib.MCE_ERR_INVALID
    assert lib.mce_paged_kv_store(0, None, None, None, None, None, 0, 8, 128, 16, 10,
                                  1024, 128, 1024, 128, None) == _lib.MCE_OK


def _decode(lib, **kw):
    args = dict(dtype=0, q=1 << 12, kc=1 << 12, vc=1 << 12, bt=1 << 12, cl=1 << 12,
                out=1 << 12, B=2, Hq=24, Hkv=8, D=128, maxb=128, bs=16, nb=10, scale=0.088,
                ws=None, ws_bytes=0, stream=None)
    args.update(kw)
    a = args
    return lib.mce_paged_attention_decode(
        a["dtype"], a["q"], a["kc"], a["vc"], a["bt"], a["cl"], a["out"], a["B"], a["Hq"],
        a["Hkv"], a["D"], a["maxb"], a["bs"], a["nb"], a["scale"], a["ws"], a["ws_bytes"],
        a["stream"])


def test_decode_validation(lib):
    assert _decode(lib, D=64) == _lib.MCE_ERR_INVALID and "head_dim" in _err(lib)
    assert _decode(lib, Hq=20) == _lib.MCE_ERR_INVALID
    assert _decode(lib, bs=12) == _lib.MCE_ERR_INVALID and "block_size" in _err(lib)
    assert _decode(lib, bs=4) == _lib.MCE_ERR_INVALID
    assert _decode(lib, Hq=80) == _lib.MCE_ERR_UNSUPPORTED  # GQA group 10
    assert _decode(lib, dtype=1) == _lib.MCE_ERR_WORKSPACE  # bf16 is supported
    assert _decode(lib, q=None) == _lib.MCE_ERR_INVALID
    assert _decode(lib, nb=0) == _lib.MCE_ERR_INVALID
    # the pool is addressed by 32-bit token slots
    assert _decode(lib, nb=(1 << 28) + 1) == _lib.MCE_ERR_INVALID and "2^32" in _err(lib)
    assert _decode(lib, nb=1 << 28) == _lib.MCE_ERR_WORKSPACE  # 2^32 slots: accepted
    assert _decode(lib) == _lib.MCE_ERR_WORKSPACE  # no workspace given
    assert _decode(lib, B=0) == _lib.MCE_OK


def test_decode_workspace_size(lib):
    f = lib.mce_paged_attention_decode_workspace_size
    assert f(0, 24, 8, 128, 16) == 0
    assert f(32, 24, 8, 64, 16) == 0  # <= 1024 tokens of capacity: per-sequence mode
    small, big = f(1, 24, 8, 128, 16), f(32, 24, 8, 256, 16)
    assert 0 < small < big
    assert big % 256 == 0

    # J + B compact part slots per query head: (m, l) and 128 partial dims in
    # fp32, then (first slot, part count) per sequence; J = one workgroup per CU
    # for one group of 8 kv heads (the library assumes 256 CUs without a GPU)
    cus = torch.cuda.get_device_properties(0).multi_processor_count \
        if torch.cuda.is_available() else 256

    def expect(b, hq, groups=1):
        up = lambda x: (x + 255) // 256 * 256
        rows = hq * (min(512, max(1, cus // groups)) + b)
        return up(rows * 2 * 4) + up(rows * 128 * 4) + up(b * 8)
    assert big == expect(32, 24)                                # cfg2
    assert f(8, 24, 8, 2048, 16) == expect(8, 24)               # cfg4
    assert f(32, 24, 8, 100, 16) == expect(32, 24)              # independent of the width
    assert f(16, 32, 32, 128, 16) == expect(16, 32, groups=4)   # 32 kv heads: 4 groups
    if cus == 256:
        assert big < 4 * 2 ** 20                                # 3.6 MB at cfg2


def test_decode_noalloc_rejects_shapes_beyond_its_scratch(lib):
    """The allocation-free decode refuses, before any device work, shapes whose
    split-K partials would not fit its static scratch (16 MiB)."""
    f = lib.mce_paged_attention_decode_workspace_size
    assert _lib.MCE_DECODE_NOALLOC_SCRATCH_BYTES == 16 << 20
    assert f(2000, 64, 8, 256, 16) > _lib.MCE_DECODE_NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(16)
    rc = lib.mce_paged_attention_decode_noalloc(0, p, p, p, p, p, p, 2000, 64, 8, 128, 256, 16,
                                                 1000, 0.1, None)
    assert rc == _lib.MCE_ERR_UNSUPPORTED
    assert b"static" in lib.mce_last_error()


def test_rope_and_prefill_validation(lib):
    assert lib.mce_rope_inplace(0, None, None, None, None, None, 1, 1, 2, 1, 7, 16,
                                0, 0, 0, 0, 0, 0, None) == _lib.MCE_ERR_INVALID
    assert lib.mce_rope_inplace(0, None, None, None, None, None, 0, 1, 2, 1, 8, 16,
                                0, 0, 0, 0, 0, 0, None) == _lib.MCE_OK
    assert lib.mce_prefill_attention(0, None, None, None, None, 1, 8, 24, 8, 64, 0.1,
                                     None) == _lib.MCE_ERR_INVALID
    assert lib.mce_prefill_attention(0, None, None, None, None, 1, 8, 24, 7, 128, 0.1,
                                     None) == _lib.MCE_ERR_INVALID
    assert lib.mce_prefill_attention(0, None, None, None, None, 0, 8, 24, 8, 128, 0.1,
                                     None) == _lib.MCE_OK


def test_rope_kv_store_validation(lib):
    f = lib.mce_rope_kv_store
    args = [0] + [None] * 10 + [4, 24, 8, 128, 4096, 16, 10, 0, 0, 0, 0, 0, 0, None]
    assert f(*args) == _lib.MCE_ERR_INVALID and "null" in _err(lib)
    bad = list(args); bad[0] = 5
    assert f(*bad) == _lib.MCE_ERR_INVALID and "dtype" in _err(lib)
    odd = list(args); odd[14] = 127
    assert f(*odd) == _lib.MCE_ERR_INVALID
    empty = list(args); empty[11] = 0
    assert f(*empty) == _lib.MCE_OK


def test_decode_gemm_validation(lib):
    f = lib.mce_decode_gemm
    assert f(0, None, None, None, 8, 64, 2048, 2048, 64, 0, None) == _lib.MCE_ERR_INVALID
    assert "null" in _err(lib)
    assert f(0, None, None, None, 8, 64, 2048, 2048, 64, 7, None) == _lib.MCE_ERR_INVALID
    assert f(0, None, None, None, 17, 64, 2048, 2048, 64, 0, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 8, 60, 2048, 2048, 64, 0, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 8, 64, 512, 512, 64, 0, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 8, 64, 2560, 2560, 64, 0, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 8, 64, 8192, 8192, 64, 2, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 9, 64, 8192, 8192, 64, 1, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(1, None, None, None, 8, 64, 2048, 2048, 64, 0, None) == _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, None, None, 0, 64, 2048, 2048, 64, 0, None) == _lib.MCE_OK
    # out overlapping x (a residual add into the input itself) is refused
    p = ctypes.c_void_p(1 << 20)
    assert f(0, p, p, p, 8, 2048, 2048, 2048, 2048, 1, None) == _lib.MCE_ERR_INVALID
    assert "overlap" in _err(lib)


def test_rmsnorm_decode_gemm_validation(lib):
    f = lib.mce_rmsnorm_decode_gemm
    one = ctypes.c_void_p(16)  # non-null, never dereferenced: validation fails first
    assert f(0, None, None, 1e-5, None, None, 8, 64, 3072, 3072, 64, 0, None) == \
        _lib.MCE_ERR_INVALID
    assert "norm weight" in _err(lib)
    assert f(0, None, one, -1.0, None, None, 8, 64, 3072, 3072, 64, 0, None) == \
        _lib.MCE_ERR_INVALID
    # k = 8192 is only taken without the fused RMSNorm
    assert f(0, None, one, 1e-5, None, None, 8, 64, 8192, 8192, 64, 1, None) == \
        _lib.MCE_ERR_UNSUPPORTED
    assert f(0, None, one, 1e-5, None, None, 8, 64, 3072, 3072, 64, 2, None) == \
        _lib.MCE_ERR_INVALID
    assert "null" in _err(lib)


def test_python_ops_reject_cpu_tensors():
    import my_cuda_engine_cpp as ops
    x = torch.zeros(2, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        ops.rmsnorm(x, torch.ones(8, dtype=torch.float16), 1e-5)
    with pytest.raises(RuntimeError):
        ops.swiglu(x)
    q = torch.zeros(1, 24, 128, dtype=torch.float16)
    kc = torch.zeros(4, 16, 8, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        ops.paged_attention_decode(q, kc, kc, torch.zeros(1, 4, dtype=torch.int32),
                                   torch.ones(1, dtype=torch.int32), 4, 16, 0.088)
    with pytest.raises(RuntimeError):
        ops.prefill_attention(torch.zeros(1, 4, 24, 128, dtype=torch.float16),
                              torch.zeros(1, 4, 8, 128, dtype=torch.float16),
                              torch.zeros(1, 4, 8, 128, dtype=torch.float16), 0.088)


def test_error_exception_carries_status(lib):
    with pytest.raises(_lib.MCEError) as ei:
        _lib.call("mce_rmsnorm", 9, None, None, None, 1, 8, 8, 8, 1e-5, None)
    assert ei.value.code == _lib.MCE_ERR_INVALID and isinstance(ei.value, RuntimeError)


def test_decode_loop_entry_points_validate(lib):
    f = lib.mce_argmax_rows
    assert f(0, None, 8, 100, 100, None, None, 0, None) == _lib.MCE_ERR_INVALID
    assert "null" in _err(lib)
    assert f(0, None, 8, 100, 50, None, None, 0, None) == _lib.MCE_ERR_INVALID   # stride < cols
    assert f(2, None, 8, 100, 100, None, None, 0, None) == _lib.MCE_ERR_INVALID  # dtype
    assert f(0, None, 0, 100, 100, None, None, 0, None) == _lib.MCE_OK
    one = ctypes.c_void_p(16)  # non-null, never dereferenced: validation fails first
    ws = lib.mce_argmax_rows_workspace_size
    assert ws(8, 128256) == 8 * 32 * 8 and ws(3, 7) == 3 * 8 and ws(0, 9) == 0
    # aligned rows are split: the workspace is required
    assert f(0, one, 8, 128256, 128256, one, None, 0, None) == _lib.MCE_ERR_WORKSPACE
    assert f(0, one, 8, 128256, 128256, one, one, 8, None) == _lib.MCE_ERR_WORKSPACE
    # the split (rows on grid.y) takes at most 65535 rows; the one-workgroup-per-row
    # path (unaligned rows: rows on grid.x) is not limited to that
    assert f(0, one, 70000, 128, 128, one, one, 1 << 30, None) == _lib.MCE_ERR_INVALID
    assert "65535" in _err(lib)
    odd = ctypes.c_void_p(18)  # 2-byte aligned only: the unsplit path
    assert f(0, odd, 1 << 31, 128, 129, one, None, 0, None) == _lib.MCE_ERR_INVALID
    assert "too many rows" in _err(lib)
    g = lib.mce_decode_advance
    assert g(None, None, None, None, None, None, None, 4, 8, 16, 0, None) == _lib.MCE_ERR_INVALID
    one = ctypes.c_void_p(16)  # non-null, never dereferenced: validation fails first
    assert g(one, one, one, one, None, one, None, 4, 8, 16, 4, None) == _lib.MCE_ERR_INVALID
    assert "token log" in _err(lib)
    assert g(one, one, one, one, None, None, None, 4, 8, 0, 0, None) == _lib.MCE_ERR_INVALID
    assert g(None, None, None, None, None, None, None, 0, 8, 16, 0, None) == _lib.MCE_OK


def test_prefill_paged_validation(lib):
    f = lib.mce_prefill_attention_paged
    one = ctypes.c_void_p(16)  # non-null, never dereferenced: validation fails first
    args = [0, one, one, one, one, one, one, 2, 64, 24, 8, 128, 8, 16, 64, 0.1, None, 0, None]
    # (args itself is valid and would launch: only invalid variants are called)
    bad = list(args); bad[11] = 64
    assert f(*bad) == _lib.MCE_ERR_INVALID and "head_dim" in _err(lib)
    bad = list(args); bad[13] = 12
    assert f(*bad) == _lib.MCE_ERR_INVALID and "power of two" in _err(lib)
    bad = list(args); bad[12] = 3   # 3 blocks x 16 tokens < 64 query positions
    assert f(*bad) == _lib.MCE_ERR_INVALID and "fewer than" in _err(lib)
    bad = list(args); bad[12] = 9000
    assert f(*bad) == _lib.MCE_ERR_INVALID and "8192" in _err(lib)
    bad = list(args); bad[1] = None
    assert f(*bad) == _lib.MCE_ERR_INVALID and "null" in _err(lib)
    bad = list(args); bad[14] = 1 << 20   # pool of 4 GiB
    assert f(*bad) == _lib.MCE_ERR_INVALID and "2 GiB" in _err(lib)
    empty = list(args); empty[8] = 0
    assert f(*empty) == _lib.MCE_OK
    # one sequence, a 64-query chunk: 2 items x 8 kv heads = 16 workgroups, so
    # a workspace given for the key split must be large enough and aligned
    # (no GPU: 256 CUs assumed)
    ws = lib.mce_prefill_attention_paged_workspace_size
    need = ws(1, 64, 24, 8)
    assert need >= 8 * 64 * 24 * 130 * 4
    split = list(args); split[7] = 1
    split[17] = need - 1; split[16] = ctypes.c_void_p(1 << 20)
    assert f(*split) == _lib.MCE_ERR_WORKSPACE and "workspace" in _err(lib)
    split[17] = need; split[16] = ctypes.c_void_p((1 << 20) + 16)   # misaligned
    assert f(*split) == _lib.MCE_ERR_WORKSPACE
    # grids of at least half the CUs need none
    assert ws(8, 512, 24, 8) == 0 and ws(0, 64, 24, 8) == 0 and ws(1, 2048, 24, 8) == 0


def test_header_compiles_as_c_and_cpp(tmp_path):
    """include/mce_abi.h is usable from plain C (cgo / JNI / FFI hosts) and C++."""
    import shutil
    import subprocess
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    for comp, std, ext in (("gcc", "-std=c99", "c"), ("g++", "-std=c++17", "cpp")):
        if shutil.which(comp) is None:
            pytest.skip(f"{comp} not available")
        src = tmp_path / f"use.{ext}"
        src.write_text('#include "mce_abi.h"\nint main(void) { return mce_abi_version() > 0 ? 0 : 1; }\n')
        r = subprocess.run([comp, std, "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-I", inc,
                            str(src)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
