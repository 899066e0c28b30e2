"""Output layouts of the varlen prefill.  A 16-byte aligned output whose token
and head strides are multiples of 8 elements gets its rows written through
LDS, four whole rows per store; any other accepted layout (8-byte aligned,
strides multiples of 4) is written lane by lane.  Both must give the same
bits, touch nothing outside the output rows, and match the oracle
(2e-2 abs / 1e-2 rel)."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_prefill_paged, say
from nanovllm_amd import _lib
from test_gpu_prefill_split import _paged_case

pytestmark = pytest.mark.gpu


def _prefill_into(out, q, kc, vc, bt, cu_q, cu_k, max_q, max_k, hkv=8):
    lib = _lib.load()
    tq, hq, d = q.shape
    batch = cu_q.numel() - 1
    nb, bs = kc.shape[0], kc.shape[1]
    rc = lib.nvk_varlen_prefill(q.data_ptr(), q.stride(0), q.stride(1), tq, kc.data_ptr(),
                                vc.data_ptr(), 0, 0, 0, nb * bs, cu_q.data_ptr(), cu_k.data_ptr(),
                                batch, max_q, max_k, bt.data_ptr(), bt.stride(0), bt.shape[1], bs,
                                nb, hq, hkv, d, 128 ** -0.5, out.data_ptr(), out.stride(0),
                                out.stride(1), None, 0, _lib.dtype_code(q),
                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.nvk_strerror(rc)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_whole_row_and_per_lane_stores_agree(dtype):
    rng = np.random.default_rng(95)
    lens_q = [int(x) for x in rng.integers(1, 300, 10)] + [0, 1, 64, 65]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 400, len(lens_q)))]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(96, lens_q, lens_k)
    tq, hq, d = q.shape
    dq, dkc, dvc = (x.to(dtype).cuda() for x in (q, kc, vc))
    args = (dq, dkc, dvc, bt.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k))
    nan = float("nan")
    # 16-byte aligned, contiguous: whole-row stores
    aligned = torch.full((tq, hq, d), nan, dtype=dtype, device="cuda")
    say("prefill output: aligned rows")
    _prefill_into(aligned, *args)
    # 8-byte aligned (4 elements into a buffer): per-lane stores
    buf = torch.full((tq * hq * d + 8,), nan, dtype=dtype, device="cuda")
    shifted = buf[4:4 + tq * hq * d].view(tq, hq, d)
    assert shifted.data_ptr() % 16 == 8
    say("prefill output: shifted by 8 bytes")
    _prefill_into(shifted, *args)
    # head stride 132 (a multiple of 4, not of 8): per-lane stores
    wide = torch.full((tq, hq, 132), nan, dtype=dtype, device="cuda")
    padded = wide[:, :, :d]
    say("prefill output: head stride 132")
    _prefill_into(padded, *args)
    torch.cuda.synchronize()
    bits = lambda t: t.contiguous().view(torch.int16)
    assert torch.equal(bits(aligned), bits(shifted))
    assert torch.equal(bits(aligned), bits(padded))
    # nothing written outside the output rows
    assert torch.isnan(buf[:4].float()).all() and torch.isnan(buf[4 + tq * hq * d:].float()).all()
    assert torch.isnan(wide[:, :, d:].float()).all()
    if dtype == torch.bfloat16:  # (fp16 prefill parity: test_gpu_fp16.py)
        ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
        assert_attn_close(aligned, ref, "prefill, aligned output rows")
