"""GPU parity of the short-query kernels (<= 16 rows of query tokens x query
heads per kv head over paged keys, e.g. speculative-decode verification)
against the oracle, through nvk_varlen_prefill with its workspace.  Cases:
every row count from 1 to 16 rows, key counts around the 64-key chunk, rows
that see no key, sequences without queries, G = 1, 2, 4, 8, several page
sizes and graph replay."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_prefill_paged, say
from nanovllm_amd import _lib
from tests.test_gpu_prefill_split import _call, _paged_case

pytestmark = pytest.mark.gpu


def _check(seed, lens_q, lens_k, bs=256, hq=16, hkv=8, max_k=None, what=""):
    q, kc, vc, bt, cu_q, cu_k = _paged_case(seed, lens_q, lens_k, bs, hq, hkv)
    scale = 128 ** -0.5
    mk = max_k if max_k is not None else max(lens_k)
    say(f"short query {what}")
    out, ws = _call(q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(max(lens_q), 1),
                    mk, scale, bt=bt.cuda())
    assert ws > 0
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, bs, scale)
    assert_attn_close(out, ref, what)


@pytest.mark.parametrize("nq", [1, 2, 3, 6, 8])
def test_short_query_rows_and_chunk_edges(nq):
    # key counts on and around the 64-key chunk and the 256-key page
    lens_k = [nq, 63, 64, 65, 255, 256, 257, 1000, 4097]
    _check(40 + nq, [nq] * len(lens_k), [max(k, nq) for k in lens_k], what=f"{nq} queries")


def test_short_query_group_sizes_and_pages():
    _check(51, [16, 3, 9], [700, 2000, 64], hq=16, hkv=16, what="G=1, 16 rows")
    _check(52, [4, 1, 2], [3000, 10, 129], hq=16, hkv=4, what="G=4")
    _check(53, [2, 1], [5000, 777], hq=16, hkv=2, what="G=8")
    _check(54, [6, 6, 5], [900, 1300, 64], bs=64, what="64-key pages")
    _check(55, [6, 4], [3000, 2000], bs=512, what="512-key pages")


def test_short_query_rows_without_keys_and_empty_sequences():
    # more queries than keys: the first rows see nothing (zeros); a sequence
    # without queries; a sequence with one key
    _check(56, [5, 0, 3, 1], [3, 800, 2500, 1], what="rows without keys")


def test_short_query_spec_verify_shape_and_underreported_max_k():
    _check(57, [6] * 32, list(np.random.default_rng(0).integers(1024, 8193, 32)), what="spec 32x6")
    _check(58, [6, 6], [3000, 2900], max_k=1024, what="max_seqlen_k too small")


def test_short_query_graph_replays():
    say("short query graph replay")
    q, kc, vc, bt, cu_q, cu_k = _paged_case(59, [6] * 8, [1500, 3000, 64, 999, 4000, 2222, 70, 512])
    dq, dk, dv, dbt, dcq, dck = (t.cuda() for t in (q, kc, vc, bt, cu_q, cu_k))
    lib = _lib.load()
    ws_bytes = lib.nvk_varlen_prefill_workspace_size(8, 6, 4000, 16, 8, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(dq)

    def call():
        rc = lib.nvk_varlen_prefill(dq.data_ptr(), dq.stride(0), dq.stride(1), dq.shape[0],
                                    dk.data_ptr(), dv.data_ptr(), 0, 0, 0, dk.shape[0] * 256,
                                    dcq.data_ptr(), dck.data_ptr(), 8, 6, 4000, dbt.data_ptr(),
                                    dbt.stride(0), dbt.shape[1], 256, dk.shape[0], 16, 8, 128,
                                    128 ** -0.5, out.data_ptr(), out.stride(0), out.stride(1),
                                    ws.data_ptr(), ws_bytes, 0,
                                    torch.cuda.current_stream().cuda_stream)
        assert rc == 0

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
    assert_attn_close(out, ref, "graph replay")
