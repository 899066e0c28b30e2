"""nvk_paged_decode_noalloc (the decode entry point that allocates nothing:
its workspace is a static device array inside the library) called through
the C ABI, against nvk_paged_decode with a torch-allocated workspace: the
same kernels, so the outputs must be bit-identical, on calls in a row whose
sizes shrink (the scratch keeps the previous call's contents) and against
the oracle within 2e-2 abs / 1e-2 rel, and captured in a graph and
replayed.  The rejection of sizes beyond the scratch is checked with fake
pointers on a host without a GPU (tests/test_host.py): on a GPU a regression
of that check would launch kernels that write past the scratch.  The GPU
cases here only make calls whose sizes fit it."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_decode, say
from nanovllm_amd import _lib, paged_decode
from nanovllm_amd.workloads import decode_case

pytestmark = pytest.mark.gpu


def _noalloc(lib, c, scale, out):
    q, kc, bt = c.q, c.k_cache, c.block_tables
    nb, bs, hkv, d = kc.shape
    return lib.nvk_paged_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), c.v_cache.data_ptr(),
        bt.data_ptr(), bt.stride(0), c.context_lens.data_ptr(), q.shape[0], q.shape[1], hkv, d,
        bs, bt.shape[1], nb, scale, out.data_ptr(), out.stride(0), out.stride(1),
        _lib.NVK_DTYPE_BF16, torch.cuda.current_stream().cuda_stream)


def test_noalloc_decode_equals_workspace_decode_on_shrinking_calls():
    lib = _lib.load()
    cases = [
        ("batch 64, contexts U{100..2048}", decode_case(seed=70, pool_blocks=600)),
        ("batch 5 with empty contexts", decode_case(seed=71, ctx=[0, 3000, 17, 0, 900],
                                                    pool_blocks=20)),
        ("batch 2, G=4", decode_case(seed=72, hq=16, hkv=4, ctx=[1, 4097], pool_blocks=20)),
    ]
    for what, case in cases:
        c = case.to("cuda")
        say(f"no-alloc decode: {what}")
        ref_ws = paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens, c.block_tables,
                              case.scale)
        out = torch.full_like(ref_ws, float("nan"))
        rc = _noalloc(lib, c, case.scale, out)
        assert rc == 0, lib.nvk_strerror(rc)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_ws), f"{what}: differs from the workspace entry point"
        ref = oracle_decode(case.q, case.k_cache, case.v_cache, case.block_tables,
                            case.context_lens, case.block_size, case.scale)
        assert_attn_close(out, ref, what)


def test_noalloc_decode_replays_under_graph_capture():
    """Captured after nvk_paged_decode_noalloc_init (so only kernel launches
    happen under capture), the no-allocation decode replays bit for bit like
    nvk_paged_decode, replay after replay, with eager decodes of other sizes
    (which reuse the same static scratch) run between the replays."""
    lib = _lib.load()
    assert lib.nvk_paged_decode_noalloc_init() == 0
    case = decode_case(seed=74, pool_blocks=600)
    c = case.to("cuda")
    other = decode_case(seed=75, ctx=[4000, 9, 2048], pool_blocks=40).to("cuda")
    say("no-alloc decode under capture: reference")
    ref = paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens, c.block_tables, case.scale)
    out = torch.zeros_like(ref)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                    # warm-up off the capture
        assert _noalloc(lib, c, case.scale, out) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc(lib, c, case.scale, out)
    assert rc == 0, lib.nvk_strerror(rc)
    other_out = torch.empty_like(other.q)
    for i in range(4):
        say(f"no-alloc decode under capture: replay {i}")
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i} differs from the workspace entry point"
        # eager work between replays, on the same scratch
        assert _noalloc(lib, other, case.scale, other_out) == 0
        torch.cuda.synchronize()
