"""GPU: the allocation-free decode entry point (mce_paged_attention_decode_noalloc,
split-K partials in the library's static scratch) against the workspace entry
point (mce_paged_attention_decode), both called through the C ABI.

Both run the same kernels with the same partition, so the outputs must be
equal bit for bit: first on a cfg2-sized batch (32 sequences, contexts
U[128, 4096]), then on a smaller one (8 sequences) that reuses the scratch
with the first call's partials still in it, then on short tables (the
per-sequence mode, which uses no scratch).  The first output is also within
the north star's max-abs 1e-2 of the fp32 oracle.
"""
import pytest
import torch

from mycustomcudaengine_amd import _lib
from oracle.inputs import cfg2_context_lens, cfg2_decode, make_decode_case
from oracle.ops_ref import decode_attention_ref

pytestmark = pytest.mark.gpu


def _call(name, case, dev):
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    b, hq, d = q.shape
    nb, bs, hkv, _ = kc.shape
    out = torch.full_like(q, float("nan"))
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = [_lib.MCE_F16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
            cl.data_ptr(), out.data_ptr(), b, hq, hkv, d, case.max_blocks, bs, nb, case.scale]
    if name == "mce_paged_attention_decode":
        lib = _lib.load()
        size = lib.mce_paged_attention_decode_workspace_size(b, hq, hkv, case.max_blocks, bs)
        buf = torch.empty(size + 256, dtype=torch.uint8, device=dev)
        args += [(buf.data_ptr() + 255) & ~255 if size else None, size]
    _lib.call(name, *args, stream)
    torch.cuda.synchronize(dev)
    return out.cpu()


def test_noalloc_decode_equals_workspace_decode_twice(dev):
    big = cfg2_decode(nan_pool=True)
    small = make_decode_case(44, 8, cfg2_context_lens(44, 8, 1100, 3000), max_blocks=200)
    short = make_decode_case(45, 5, [1, 700, 1024, 33, 0], max_blocks=64)
    for case in (big, small, short):
        want = _call("mce_paged_attention_decode", case, dev)
        got = _call("mce_paged_attention_decode_noalloc", case, dev)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    ref = decode_attention_ref(big.query, big.key_cache, big.value_cache, big.block_tables,
                               big.context_lens, big.scale)
    got = _call("mce_paged_attention_decode_noalloc", big, dev)
    assert (got.float() - ref).abs().max().item() <= 1e-2


def test_noalloc_decode_graph_replays(dev):
    """The use the header names: code under HIP graph capture.  After a first,
    uncaptured call (which looks up the scratch address), the entry point is
    recorded in a torch.cuda graph and replayed three times; before each
    replay an eager call of another shape overwrites the shared scratch, and
    every replay equals the eager result bit for bit."""
    case = cfg2_decode()
    other = make_decode_case(46, 6, cfg2_context_lens(46, 6, 1500, 4000), max_blocks=256)
    want = _call("mce_paged_attention_decode_noalloc", case, dev)
    q = case.query.to(dev)
    kc, vc = case.key_cache.to(dev), case.value_cache.to(dev)
    bt, cl = case.block_tables.to(dev), case.context_lens.to(dev)
    b, hq, d = q.shape
    nb, bs, hkv, _ = kc.shape
    out = torch.full_like(q, float("nan"))
    args = [_lib.MCE_F16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
            cl.data_ptr(), out.data_ptr(), b, hq, hkv, d, case.max_blocks, bs, nb, case.scale]
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up on the capture stream, outside capture
        _lib.call("mce_paged_attention_decode_noalloc", *args,
                  torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.call("mce_paged_attention_decode_noalloc", *args,
                  torch.cuda.current_stream(dev).cuda_stream)
    for _ in range(3):
        _call("mce_paged_attention_decode_noalloc", other, dev)  # clobbers the scratch
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))
