"""nvk_paged_decode_noalloc (the decode entry point that allocates nothing:
its workspace is a static device array inside the library) called through
the C ABI, against nvk_paged_decode with a torch-allocated workspace: the
same kernels, so the outputs must be bit-identical, on calls in a row whose
sizes shrink (the scratch keeps the previous call's contents) and against
the oracle within 2e-2 abs / 1e-2 rel.  Sizes beyond the scratch are
rejected before anything is launched."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_decode, say
from nanovllm_amd import _lib, paged_decode
from nanovllm_amd.workloads import decode_case

pytestmark = pytest.mark.gpu

NVK_ESCRATCH = -5


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


def test_noalloc_decode_rejects_sizes_beyond_its_scratch():
    lib = _lib.load()
    c = decode_case(seed=73, ctx=[5], pool_blocks=2).to("cuda")
    out = torch.zeros(1, 16, 128, dtype=torch.bfloat16, device="cuda")
    # 2048 sequences x 1024 kv heads x group 8: ~34 MB of workspace
    rc = lib.nvk_paged_decode_noalloc(
        c.q.data_ptr(), 128, 128, c.k_cache.data_ptr(), c.v_cache.data_ptr(),
        c.block_tables.data_ptr(), 1, c.context_lens.data_ptr(), 2048, 8192, 1024, 128, 256, 1, 2,
        0.088, out.data_ptr(), 128, 128, _lib.NVK_DTYPE_BF16,
        torch.cuda.current_stream().cuda_stream)
    assert rc == NVK_ESCRATCH
    assert b"scratch" in lib.nvk_strerror(rc)
    need = lib.nvk_paged_decode_workspace_size(2048, 8192, 1024, 128, 256, 1)
    assert need > (20 << 20)
    torch.cuda.synchronize()
    assert out.eq(0).all(), "a rejected call must launch nothing"
