"""The `my_cuda_engine_cpp` op surface on PyTorch-ROCm tensors.

Same six names, positional arguments and return conventions as the
reference's pybind module (csrc/bindings.cpp:4-19,22-29):

    rmsnorm(input, weight, eps) -> Tensor
    swiglu(gate_up) -> Tensor
    paged_kv_store(key, value, key_cache, value_cache, slot_mapping) -> None
    paged_attention_decode(query, key_cache, value_cache, block_tables,
                           context_lens, max_blocks_per_seq, block_size,
                           scale) -> Tensor
    rope_inplace(query, key, cos_table, sin_table, positions) -> None
    prefill_attention(query, key, value, scale) -> Tensor

Each op validates dtype, device, shape and layout on the host and raises
RuntimeError (the exception type TORCH_CHECK raises in the reference), then
calls libmce.so on torch's current HIP stream.  Outputs and the decode
workspace are allocated with torch, so every op can be recorded by
torch.cuda.graph (hipGraph).  No op synchronises or reads device memory on the
host.  There is no CPU path: CPU tensors are rejected.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = [
    "rmsnorm",
    "swiglu",
    "paged_kv_store",
    "paged_attention_decode",
    "rope_inplace",
    "prefill_attention",
]

_DTYPES = {torch.float16: _lib.MCE_F16, torch.bfloat16: _lib.MCE_BF16}


def _check(cond: bool, msg) -> None:
    """Raises RuntimeError(msg) when cond is false; msg may be a callable that
    builds the message (formatted only on failure: these checks run on every
    op call)."""
    if not cond:
        raise RuntimeError(msg() if callable(msg) else msg)


def _dtype_code(t: torch.Tensor, name: str) -> int:
    code = _DTYPES.get(t.dtype)
    _check(code is not None,
           lambda: f"{name() if callable(name) else name} must be float16 or bfloat16 "
                   f"(got {t.dtype})")
    return code


def _on_gpu(name: str, *ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        _check(isinstance(t, torch.Tensor), lambda: f"{name}: expected tensors")
        _check(t.is_cuda, lambda: f"{name}: tensors must be on a GPU (got {t.device})")
        _check(t.device == dev, lambda: f"{name}: tensors are on different devices")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


class _on_device:
    """Makes `dev` current for the duration of a call (a device guard)."""

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.dev.index:
            self.prev = cur
            torch.cuda.set_device(self.dev)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def rmsnorm(input: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Fused RMSNorm over the last dim (reference: csrc/kernels/rmsnorm.cu:110-130)."""
    dev = _on_gpu("rmsnorm", input, weight)
    code = _dtype_code(input, "rmsnorm input")
    _check(weight.dtype == input.dtype, "rmsnorm: weight dtype must match input")
    _check(input.dim() >= 1, "rmsnorm: input must have at least one dim")
    hidden = input.size(-1)
    _check(weight.dim() == 1 and weight.size(0) == hidden and weight.is_contiguous(),
           lambda: f"rmsnorm: weight must be contiguous [{hidden}]")
    x = input if input.is_contiguous() else input.contiguous()
    out = torch.empty_like(x)
    rows = x.numel() // hidden if hidden else 0
    with _on_device(dev):
        _lib.call("mce_rmsnorm", code, x.data_ptr(), weight.data_ptr(), out.data_ptr(),
                  rows, hidden, hidden, hidden, float(eps), _stream(dev))
    return out


def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(first half) * second half of the last dim (reference: swiglu.cu:29-52)."""
    dev = _on_gpu("swiglu", gate_up)
    code = _dtype_code(gate_up, "swiglu gate_up")
    _check(gate_up.dim() >= 1, "swiglu: input must have at least one dim")
    two_i = gate_up.size(-1)
    _check(two_i % 2 == 0, lambda: f"swiglu: last dim must be even (got {two_i})")
    x = gate_up if gate_up.is_contiguous() else gate_up.contiguous()
    inter = two_i // 2
    shape = list(x.shape)
    shape[-1] = inter
    out = torch.empty(shape, dtype=x.dtype, device=x.device)
    rows = x.numel() // two_i if two_i else 0
    with _on_device(dev):
        _lib.call("mce_swiglu", code, x.data_ptr(), out.data_ptr(), rows, inter, two_i,
                  inter, _stream(dev))
    return out


def paged_kv_store(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter per-token K/V rows into the paged pools (reference: paged_kv.cu:45-69).

    key/value: [N, Hkv, D] (any token/head strides, contiguous last dim);
    caches: contiguous [num_blocks, block_size, Hkv, D]; slot_mapping int32 [N].
    """
    dev = _on_gpu("paged_kv_store", key, value, key_cache, value_cache, slot_mapping)
    code = _dtype_code(key, "paged_kv_store key")
    for t, n in ((value, "value"), (key_cache, "key_cache"), (value_cache, "value_cache")):
        _check(t.dtype == key.dtype, lambda: f"paged_kv_store: {n} dtype must match key")
    _check(key.dim() == 3 and value.shape == key.shape,
           lambda: f"paged_kv_store: key/value must be [N, Hkv, D] (got {tuple(key.shape)}, "
           f"{tuple(value.shape)})")
    n_tok, hkv, d = key.shape
    _check(key_cache.dim() == 4 and key_cache.shape == value_cache.shape,
           "paged_kv_store: caches must be [num_blocks, block_size, Hkv, D]")
    nb, bs, chkv, cd = key_cache.shape
    _check(chkv == hkv and cd == d,
           lambda: f"paged_kv_store: cache head shape {(chkv, cd)} != key head shape {(hkv, d)}")
    _check(key_cache.is_contiguous() and value_cache.is_contiguous(),
           "paged_kv_store: caches must be contiguous")
    _check(key.stride(-1) == 1 and value.stride(-1) == 1,
           "paged_kv_store: key/value last dim must be contiguous")
    _check(slot_mapping.dtype == torch.int32 and slot_mapping.dim() == 1 and
           slot_mapping.size(0) == n_tok and slot_mapping.is_contiguous(),
           lambda: f"paged_kv_store: slot_mapping must be contiguous int32 [{n_tok}]")
    with _on_device(dev):
        _lib.call("mce_paged_kv_store", code, key.data_ptr(), value.data_ptr(),
                  key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(),
                  n_tok, hkv, d, bs, nb, key.stride(0), key.stride(1),
                  value.stride(0), value.stride(1), _stream(dev))


_DECODE_WS = {}  # (device, batch, heads, kv heads, table width, block size) -> bytes


def _decode_workspace_bytes(device: int, b: int, hq: int, hkv: int, mb: int, bs: int) -> int:
    """mce_paged_attention_decode_workspace_size for the current device, cached
    per shape (the size depends on the device's CU count and the shape only)."""
    key = (device, b, hq, hkv, mb, bs)
    size = _DECODE_WS.get(key)
    if size is None:
        size = _DECODE_WS[key] = _lib.load().mce_paged_attention_decode_workspace_size(
            b, hq, hkv, mb, bs)
    return size


def paged_attention_decode(query: torch.Tensor, key_cache: torch.Tensor,
                           value_cache: torch.Tensor, block_tables: torch.Tensor,
                           context_lens: torch.Tensor, max_blocks_per_seq: int,
                           block_size: int, scale: float) -> torch.Tensor:
    """One-token paged attention with GQA (reference: flash_attn_paged.cu:144-168).

    query [B, Hq, D]; caches [num_blocks, block_size, Hkv, D];
    block_tables int32 [B, max_blocks_per_seq]; context_lens int32 [B].
    Returns a new [B, Hq, D] tensor.  Rows with context_len 0 are zeros.
    """
    dev = _on_gpu("paged_attention_decode", query, key_cache, value_cache,
                  block_tables, context_lens)
    code = _dtype_code(query, "paged_attention_decode query")
    _check(key_cache.dtype == query.dtype and value_cache.dtype == query.dtype,
           "paged_attention_decode: cache dtype must match query")
    _check(query.dim() == 3, "paged_attention_decode: query must be [B, Hq, D]")
    b, hq, d = query.shape
    _check(key_cache.dim() == 4 and key_cache.shape == value_cache.shape,
           "paged_attention_decode: caches must be [num_blocks, block_size, Hkv, D]")
    nb, bs, hkv, cd = key_cache.shape
    _check(cd == d, lambda: f"paged_attention_decode: cache head_dim {cd} != query head_dim {d}")
    _check(int(block_size) == bs,
           lambda: f"paged_attention_decode: block_size {block_size} != cache block size {bs}")
    _check(key_cache.is_contiguous() and value_cache.is_contiguous(),
           "paged_attention_decode: caches must be contiguous")
    mb = int(max_blocks_per_seq)
    _check(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and
           block_tables.size(0) == b and block_tables.size(1) == mb and
           block_tables.is_contiguous(),
           lambda: f"paged_attention_decode: block_tables must be contiguous int32 [{b}, {mb}] "
           f"(got {block_tables.dtype} {tuple(block_tables.shape)})")
    _check(context_lens.dtype == torch.int32 and context_lens.dim() == 1 and
           context_lens.size(0) == b and context_lens.is_contiguous(),
           lambda: f"paged_attention_decode: context_lens must be contiguous int32 [{b}]")
    q = query if query.is_contiguous() else query.contiguous()
    out = torch.empty_like(q)
    with _on_device(dev):
        ws_bytes = _decode_workspace_bytes(dev.index, b, hq, hkv, mb, bs) if b else 0
        ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=dev) if ws_bytes else None
        ws_ptr = (ws.data_ptr() + 255) & ~255 if ws is not None else None
        _lib.call("mce_paged_attention_decode", code, q.data_ptr(), key_cache.data_ptr(),
                  value_cache.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                  out.data_ptr(), b, hq, hkv, d, mb, bs, nb, float(scale), ws_ptr, ws_bytes,
                  _stream(dev))
    return out


def rope_inplace(query: torch.Tensor, key, cos_table: torch.Tensor,
                 sin_table: torch.Tensor, positions: torch.Tensor) -> None:
    """Rotate Q (and K) in place, half-split form (reference: rope.cu:64-99).

    query [B, S, Hq, D], key [B, S, Hkv, D] or None (any strides with a
    contiguous last dim); cos/sin fp32 [P, D/2]; positions int32 [B, S].
    """
    tensors = [query, cos_table, sin_table, positions] + ([key] if key is not None else [])
    dev = _on_gpu("rope_inplace", *tensors)
    code = _dtype_code(query, "rope_inplace query")
    _check(query.dim() == 4, "rope_inplace: query must be [B, S, Hq, D]")
    b, s, hq, d = query.shape
    _check(d % 2 == 0, lambda: f"rope_inplace: head_dim must be even (got {d})")
    _check(query.stride(-1) == 1, "rope_inplace: query last dim must be contiguous")
    hkv = 0
    if key is not None:
        _check(key.dtype == query.dtype, "rope_inplace: key dtype must match query")
        _check(key.dim() == 4 and key.size(0) == b and key.size(1) == s and key.size(3) == d,
               lambda: f"rope_inplace: key must be [{b}, {s}, Hkv, {d}] (got {tuple(key.shape)})")
        _check(key.stride(-1) == 1, "rope_inplace: key last dim must be contiguous")
        hkv = key.size(2)
    for t, n in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _check(t.dtype == torch.float32 and t.dim() == 2 and t.size(1) == d // 2 and
               t.is_contiguous(), lambda: f"rope_inplace: {n} must be contiguous fp32 [P, {d // 2}]")
    _check(cos_table.size(0) == sin_table.size(0), "rope_inplace: table lengths differ")
    _check(positions.dtype == torch.int32 and positions.numel() == b * s and
           positions.is_contiguous(),
           lambda: f"rope_inplace: positions must be contiguous int32 with {b * s} elements")
    ks = key.stride() if key is not None else (0, 0, 0, 0)
    with _on_device(dev):
        _lib.call("mce_rope_inplace", code, query.data_ptr(),
                  key.data_ptr() if key is not None else None, cos_table.data_ptr(),
                  sin_table.data_ptr(), positions.data_ptr(), b, s, hq, hkv, d,
                  cos_table.size(0), query.stride(0), query.stride(1), query.stride(2),
                  ks[0], ks[1], ks[2], _stream(dev))


def rope_kv_store(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  key_cache: torch.Tensor, value_cache: torch.Tensor,
                  cos_table: torch.Tensor, sin_table: torch.Tensor, positions: torch.Tensor,
                  slot_mapping: torch.Tensor, query_out: torch.Tensor = None) -> None:
    """rope_inplace(query, key) then paged_kv_store(key, value) in one launch.

    Engine-side fusion of the two calls the reference decode step makes back
    to back (engine/models/llama.py:117-127); identical results.  query
    [N, Hq, D], key/value [N, Hkv, D] (any token/head strides, contiguous last
    dim); caches contiguous [num_blocks, block_size, Hkv, D]; cos/sin fp32
    [P, D/2]; positions and slot_mapping contiguous int32 [N].  With
    query_out (contiguous [N, Hq, D]) the rotated query is written there and
    query is left as it was.
    """
    dev = _on_gpu("rope_kv_store", query, key, value, key_cache, value_cache, cos_table,
                  sin_table, positions, slot_mapping)
    code = _dtype_code(query, "rope_kv_store query")
    for t, n in ((key, "key"), (value, "value"), (key_cache, "key_cache"),
                 (value_cache, "value_cache")):
        _check(t.dtype == query.dtype, lambda: f"rope_kv_store: {n} dtype must match query")
    _check(query.dim() == 3 and key.dim() == 3 and value.shape == key.shape and
           key.size(0) == query.size(0) and key.size(2) == query.size(2),
           "rope_kv_store: query [N, Hq, D], key/value [N, Hkv, D] expected")
    n_tok, hq, d = query.shape
    hkv = key.size(1)
    _check(d % 2 == 0, lambda: f"rope_kv_store: head_dim must be even (got {d})")
    for t, n in ((query, "query"), (key, "key"), (value, "value")):
        _check(t.stride(-1) == 1, lambda: f"rope_kv_store: {n} last dim must be contiguous")
    _check(key_cache.dim() == 4 and key_cache.shape == value_cache.shape and
           key_cache.size(2) == hkv and key_cache.size(3) == d and
           key_cache.is_contiguous() and value_cache.is_contiguous(),
           "rope_kv_store: caches must be contiguous [num_blocks, block_size, Hkv, D]")
    nb, bs = key_cache.shape[:2]
    for t, n in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _check(t.dtype == torch.float32 and t.dim() == 2 and t.size(1) == d // 2 and
               t.is_contiguous(), lambda: f"rope_kv_store: {n} must be contiguous fp32 [P, {d // 2}]")
    _check(cos_table.size(0) == sin_table.size(0), "rope_kv_store: table lengths differ")
    for t, n in ((positions, "positions"), (slot_mapping, "slot_mapping")):
        _check(t.dtype == torch.int32 and t.numel() == n_tok and t.is_contiguous(),
               lambda: f"rope_kv_store: {n} must be contiguous int32 with {n_tok} elements")
    if query_out is not None:
        _check(query_out.dtype == query.dtype and query_out.shape == query.shape and
               query_out.is_contiguous() and query_out.device == query.device,
               "rope_kv_store: query_out must be a contiguous tensor like query")
    with _on_device(dev):
        _lib.call("mce_rope_kv_store", code, query.data_ptr(),
                  query_out.data_ptr() if query_out is not None else None, key.data_ptr(),
                  value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                  cos_table.data_ptr(), sin_table.data_ptr(), positions.data_ptr(),
                  slot_mapping.data_ptr(), n_tok, hq, hkv, d, cos_table.size(0), bs, nb,
                  query.stride(0), query.stride(1), key.stride(0), key.stride(1),
                  value.stride(0), value.stride(1), _stream(dev))


PER_SEQ_MAX_TOKENS = 1024  # table capacity up to which decode runs one workgroup per sequence


def decode_rope_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                          key_cache: torch.Tensor, value_cache: torch.Tensor,
                          cos_table: torch.Tensor, sin_table: torch.Tensor,
                          positions: torch.Tensor, slot_mapping: torch.Tensor,
                          block_tables: torch.Tensor, context_lens: torch.Tensor,
                          max_blocks_per_seq: int, scale: float) -> torch.Tensor:
    """rope_inplace + paged_kv_store of the new token + paged_attention_decode
    in one launch (engine/models/llama.py:117-134 makes the three calls);
    outputs and caches bit-identical to rope_kv_store(query_out=...) followed
    by paged_attention_decode.  query [B, Hq, D], key/value [B, Hkv, D] with
    batch strides (views into a fused projection, head rows contiguous);
    query and key are not modified.  Only for table capacities
    (max_blocks_per_seq * block_size) up to PER_SEQ_MAX_TOKENS.
    """
    dev = _on_gpu("decode_rope_attention", query, key, value, key_cache, value_cache,
                  cos_table, sin_table, positions, slot_mapping, block_tables, context_lens)
    code = _dtype_code(query, "decode_rope_attention query")
    for t, n in ((key, "key"), (value, "value"), (key_cache, "key_cache"),
                 (value_cache, "value_cache")):
        _check(t.dtype == query.dtype, lambda: f"decode_rope_attention: {n} dtype must match query")
    _check(query.dim() == 3 and key.dim() == 3 and value.shape == key.shape and
           key.size(0) == query.size(0) and key.size(2) == query.size(2),
           "decode_rope_attention: query [B, Hq, D], key/value [B, Hkv, D] expected")
    b, hq, d = query.shape
    hkv = key.size(1)
    for t, n in ((query, "query"), (key, "key"), (value, "value")):
        _check(t.stride(2) == 1 and t.stride(1) == d,
               lambda: f"decode_rope_attention: {n} heads must be contiguous rows of head_dim")
    _check(key.stride(0) == value.stride(0),
           "decode_rope_attention: key and value need the same batch stride")
    _check(key_cache.dim() == 4 and key_cache.shape == value_cache.shape and
           key_cache.size(2) == hkv and key_cache.size(3) == d and
           key_cache.is_contiguous() and value_cache.is_contiguous(),
           "decode_rope_attention: caches must be contiguous [num_blocks, block_size, Hkv, D]")
    nb, bs = key_cache.shape[:2]
    mb = int(max_blocks_per_seq)
    _check(mb * bs <= PER_SEQ_MAX_TOKENS,
           lambda: f"decode_rope_attention: table capacity {mb * bs} > {PER_SEQ_MAX_TOKENS}; use "
           "rope_kv_store + paged_attention_decode")
    for t, n in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _check(t.dtype == torch.float32 and t.dim() == 2 and t.size(1) == d // 2 and
               t.is_contiguous(), lambda: f"decode_rope_attention: {n} must be contiguous fp32 "
               f"[P, {d // 2}]")
    _check(cos_table.size(0) == sin_table.size(0), "decode_rope_attention: table lengths differ")
    for t, n in ((positions, "positions"), (slot_mapping, "slot_mapping"),
                 (context_lens, "context_lens")):
        _check(t.dtype == torch.int32 and t.numel() == b and t.is_contiguous(),
               lambda: f"decode_rope_attention: {n} must be contiguous int32 with {b} elements")
    _check(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and
           block_tables.size(0) == b and block_tables.size(1) == mb and
           block_tables.is_contiguous(),
           lambda: f"decode_rope_attention: block_tables must be contiguous int32 [{b}, {mb}]")
    out = torch.empty(b, hq, d, dtype=query.dtype, device=query.device)
    with _on_device(dev):
        _lib.call("mce_paged_attention_decode_rope", code, query.data_ptr(), key.data_ptr(),
                  value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                  cos_table.data_ptr(), sin_table.data_ptr(), positions.data_ptr(),
                  slot_mapping.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                  out.data_ptr(), b, hq, hkv, d, mb, bs, nb, cos_table.size(0),
                  query.stride(0), key.stride(0), float(scale), _stream(dev))
    return out


_EPILOGUES = {"store": 0, "add": 1, "swiglu": 2}


def _projection(name: str, x: torch.Tensor, weight: torch.Tensor, out, epilogue: str):
    """Shared argument checks of the decode-sized projections; returns
    (device, dtype code, m, n, k, out)."""
    dev = _on_gpu(name, x, weight)
    code = _dtype_code(x, lambda: f"{name} x")
    _check(weight.dtype == x.dtype, lambda: f"{name}: weight dtype must match x")
    _check(x.dim() == 2 and weight.dim() == 2 and x.size(1) == weight.size(1),
           lambda: f"{name}: x [M, K] and weight [N, K] expected (got {tuple(x.shape)}, "
           f"{tuple(weight.shape)})")
    _check(epilogue in _EPILOGUES, lambda: f"{name}: unknown epilogue {epilogue!r}")
    _check(x.stride(1) == 1 and weight.is_contiguous(),
           lambda: f"{name}: x last dim and weight must be contiguous")
    m, k = x.shape
    n = weight.size(0) // 2 if epilogue == "swiglu" else weight.size(0)
    _check(epilogue != "swiglu" or weight.size(0) % 2 == 0,
           lambda: f"{name}: swiglu weight needs an even number of rows")
    if out is None:
        _check(epilogue != "add", lambda: f"{name}: epilogue 'add' needs out")
        out = torch.empty(m, n, dtype=x.dtype, device=x.device)
    _check(out.dtype == x.dtype and out.dim() == 2 and tuple(out.shape) == (m, n) and
           out.stride(1) == 1 and out.device == x.device,
           lambda: f"{name}: out must be [{m}, {n}] with a contiguous last dim")
    return dev, code, m, n, k, out


def decode_gemm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor = None,
                epilogue: str = "store") -> torch.Tensor:
    """Decode-sized projection out (op)= x . weight^T for at most 16 rows.

    x [M, K] (rows may be strided, contiguous last dim), weight contiguous
    [N, K] ([2N, K] gate rows then up rows for "swiglu").  epilogue "store"
    writes a new (or the given) [M, N] tensor; "add" accumulates into `out`
    in place (residual stream); "swiglu" returns silu(x W_gate^T) * x W_up^T.
    Raises MCEError with code MCE_ERR_UNSUPPORTED for inputs the kernel does
    not take (other than fp16, M > 16, N % 16, K outside {2048, 3072, 4096},
    K = 8192 needs M <= 8 and no SwiGLU); the engine then uses torch.matmul.  Engine-side op:
    the reference runs these projections through torch.matmul
    (engine/models/llama.py:94-174).
    """
    dev, code, m, n, k, out = _projection("decode_gemm", x, weight, out, epilogue)
    with _on_device(dev):
        _lib.call("mce_decode_gemm", code, x.data_ptr(), weight.data_ptr(), out.data_ptr(),
                  m, n, k, x.stride(0), out.stride(0), _EPILOGUES[epilogue], _stream(dev))
    return out


def rmsnorm_decode_gemm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                        weight: torch.Tensor, out: torch.Tensor = None,
                        epilogue: str = "store") -> torch.Tensor:
    """decode_gemm(rmsnorm(x, norm_weight, eps), weight, out, epilogue) in one
    launch; the normalised rows are bit-identical to rmsnorm()'s and are not
    written out.  K in {2048, 3072, 4096}.  Replaces the RMSNorm + projection
    pairs of engine/models/llama.py:82-108, :147-159 and :169-174."""
    dev, code, m, n, k, out = _projection("rmsnorm_decode_gemm", x, weight, out, epilogue)
    _check(norm_weight.device == x.device and norm_weight.dtype == x.dtype and
           norm_weight.dim() == 1 and norm_weight.numel() == k and norm_weight.is_contiguous(),
           lambda: f"rmsnorm_decode_gemm: norm_weight must be a contiguous [{k}] tensor like x")
    with _on_device(dev):
        _lib.call("mce_rmsnorm_decode_gemm", code, x.data_ptr(), norm_weight.data_ptr(),
                  float(eps), weight.data_ptr(), out.data_ptr(), m, n, k, x.stride(0),
                  out.stride(0), _EPILOGUES[epilogue], _stream(dev))
    return out


def argmax_rows(logits: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """Greedy token of each row of logits [R, C] (fp16 / bf16, contiguous last
    dim): int64 [R], torch.argmax's rule (the first of equal maxima, NaN above
    every number).  `out` may be any contiguous int64 tensor of R elements
    (e.g. the [R, 1] input ids of the next step).  Replaces the torch.argmax
    between replays of benchmarks/benchmark_engine.py:255-265."""
    dev = _on_gpu("argmax_rows", logits)
    code = _dtype_code(logits, "argmax_rows logits")
    _check(logits.dim() == 2 and logits.stride(1) == 1 and logits.size(1) >= 1,
           "argmax_rows: logits must be [R, C] with a contiguous last dim")
    r = logits.size(0)
    if out is None:
        out = torch.empty(r, dtype=torch.int64, device=logits.device)
    _check(out.dtype == torch.int64 and out.numel() == r and out.is_contiguous() and
           out.device == logits.device, lambda: f"argmax_rows: out must be {r} contiguous int64 values")
    with _on_device(dev):
        # partial maxima of each row's slices (graph-safe: from torch's allocator)
        ws_bytes = _lib.load().mce_argmax_rows_workspace_size(r, logits.size(1)) if r else 0
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        _lib.call("mce_argmax_rows", code, logits.data_ptr(), r, logits.size(1), logits.stride(0),
                  out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes,
                  _stream(dev))
    return out


def decode_advance(block_tables: torch.Tensor, positions: torch.Tensor,
                   context_lens: torch.Tensor, slot_mapping: torch.Tensor, block_size: int,
                   input_ids: torch.Tensor = None, token_log: torch.Tensor = None,
                   step_counter: torch.Tensor = None) -> None:
    """Prepares the next decode step on the device, in place: positions and
    context_lens move one on, slot_mapping gets the new positions' slots from
    block_tables ([B, W] int32, zero-padded, blocks of block_size tokens; -1
    past W).  With token_log
    ([steps, B] int64) input_ids ([B] or [B, 1] int64) is first written to row
    step_counter[0] (int32, incremented).  Replaces the host-side
    preparation of every replay in engine/runner.py:39-60,153-178."""
    dev = _on_gpu("decode_advance", block_tables, positions, context_lens, slot_mapping)
    _check(block_size >= 1, "decode_advance: block_size must be >= 1")
    _check(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and
           block_tables.is_contiguous(), "decode_advance: block_tables must be contiguous int32 [B, W]")
    b, w = block_tables.shape
    for name, t in (("positions", positions), ("context_lens", context_lens),
                    ("slot_mapping", slot_mapping)):
        _check(t.dtype == torch.int32 and t.numel() == b and t.is_contiguous() and t.device == dev,
               lambda: f"decode_advance: {name} must be {b} contiguous int32 values")
    log_ptr = ids_ptr = ctr_ptr = 0
    cap = 0
    if token_log is not None:
        _check(input_ids is not None and step_counter is not None,
               "decode_advance: token_log needs input_ids and step_counter")
        _check(token_log.dtype == torch.int64 and token_log.dim() == 2 and token_log.size(1) == b
               and token_log.is_contiguous() and token_log.device == dev,
               lambda: f"decode_advance: token_log must be contiguous int64 [steps, {b}]")
        _check(input_ids.dtype == torch.int64 and input_ids.numel() == b and
               input_ids.is_contiguous() and input_ids.device == dev,
               lambda: f"decode_advance: input_ids must be {b} contiguous int64 values")
        _check(step_counter.dtype == torch.int32 and step_counter.numel() >= 1 and
               step_counter.device == dev, "decode_advance: step_counter must be int32")
        log_ptr, ids_ptr, ctr_ptr = token_log.data_ptr(), input_ids.data_ptr(), step_counter.data_ptr()
        cap = token_log.size(0)
    with _on_device(dev):
        _lib.call("mce_decode_advance", block_tables.data_ptr(), positions.data_ptr(),
                  context_lens.data_ptr(), slot_mapping.data_ptr(), ids_ptr, log_ptr, ctr_ptr, b, w,
                  int(block_size), cap, _stream(dev))


def prefill_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      scale: float) -> torch.Tensor:
    """Causal GQA attention on contiguous Q/K/V (reference: prefill_attention.cu:271-309).

    query [B, S, Hq, D]; key/value [B, S, Hkv, D].  Returns [B, S, Hq, D].
    """
    dev = _on_gpu("prefill_attention", query, key, value)
    code = _dtype_code(query, "prefill_attention query")
    _check(key.dtype == query.dtype and value.dtype == query.dtype,
           "prefill_attention: key/value dtype must match query")
    _check(query.dim() == 4 and key.dim() == 4 and value.shape == key.shape,
           "prefill_attention: expected query [B, S, Hq, D], key/value [B, S, Hkv, D]")
    b, s, hq, d = query.shape
    _check(key.size(0) == b and key.size(1) == s and key.size(3) == d,
           lambda: f"prefill_attention: key shape {tuple(key.shape)} does not match query "
           f"{tuple(query.shape)}")
    hkv = key.size(2)
    q = query if query.is_contiguous() else query.contiguous()
    k = key if key.is_contiguous() else key.contiguous()
    v = value if value.is_contiguous() else value.contiguous()
    out = torch.empty_like(q)
    with _on_device(dev):
        _lib.call("mce_prefill_attention", code, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                  out.data_ptr(), b, s, hq, hkv, d, float(scale), _stream(dev))
    return out


def prefill_attention_paged(query: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, block_tables: torch.Tensor,
                            context_lens: torch.Tensor, scale: float,
                            split_keys: bool = True) -> torch.Tensor:
    """Chunked causal prefill attention reading K/V from the page pool.

    query [B, S, Hq, D] holds the last S positions of each sequence; sequence
    b has context_lens[b] (>= S) tokens whose K/V are already in the caches
    ([num_blocks, block_size, Hkv, D], e.g. written by rope_kv_store) at the
    slots block_tables[b] ([B, W] int32) gives.  Query i of sequence b sits at
    position context_lens[b] - S + i and attends to keys 0 .. that position.
    Returns [B, S, Hq, D].  Widens the reference's prefill
    (benchmarks/benchmark_engine.py:64-89, contiguous K/V of the whole prompt)
    to prompts processed in chunks against the cached prefix.

    split_keys: on small grids (few sequences, short chunks) let query blocks
    with long key ranges (a cached prefix of about 1024 tokens or more) split
    their keys over several workgroups, merged by a second launch that costs a
    few microseconds even when nothing is split; pass False when the prefixes
    are known to be short."""
    dev = _on_gpu("prefill_attention_paged", query, key_cache, value_cache, block_tables,
                  context_lens)
    code = _dtype_code(query, "prefill_attention_paged query")
    _check(key_cache.dtype == query.dtype and value_cache.dtype == query.dtype,
           "prefill_attention_paged: cache dtype must match query")
    _check(query.dim() == 4 and key_cache.dim() == 4 and value_cache.shape == key_cache.shape
           and key_cache.is_contiguous() and value_cache.is_contiguous(),
           "prefill_attention_paged: expected query [B, S, Hq, D] and contiguous caches "
           "[num_blocks, block_size, Hkv, D]")
    b, s, hq, d = query.shape
    nb, bs, hkv, dk = key_cache.shape
    _check(dk == d, "prefill_attention_paged: head_dim of query and caches differ")
    _check(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and
           block_tables.size(0) == b and block_tables.is_contiguous(),
           lambda: f"prefill_attention_paged: block_tables must be contiguous int32 [{b}, W]")
    _check(context_lens.dtype == torch.int32 and context_lens.numel() == b and
           context_lens.is_contiguous(),
           lambda: f"prefill_attention_paged: context_lens must be {b} contiguous int32 values")
    q = query if query.is_contiguous() else query.contiguous()
    out = torch.empty_like(q)
    with _on_device(dev):
        lib = _lib.load()
        # small grids split each query block's keys over workgroups (partials
        # in a workspace, merged by a second launch)
        ws_bytes = (lib.mce_prefill_attention_paged_workspace_size(b, s, hq, hkv)
                    if split_keys and b and s else 0)
        ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=dev) if ws_bytes else None
        ws_ptr = (ws.data_ptr() + 255) & ~255 if ws is not None else None
        _lib.call("mce_prefill_attention_paged", code, q.data_ptr(), key_cache.data_ptr(),
                  value_cache.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                  out.data_ptr(), b, s, hq, hkv, d, block_tables.size(1), bs, nb, float(scale),
                  ws_ptr, ws_bytes, _stream(dev))
    return out
