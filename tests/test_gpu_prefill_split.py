"""Split-K varlen prefill on the GPU: short query ranges over long contexts are
split across workgroups (partials in the workspace, then a merge kernel).  Each
case runs through the C ABI with the workspace (split) and without it (one
workgroup per query tile) and both are checked against the oracle within
2e-2 abs / 1e-2 rel; the two GPU results must agree to the same tolerance."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_prefill_dense, oracle_prefill_paged, say
from nanovllm_amd import _lib

pytestmark = pytest.mark.gpu


def _call(q, k, v, cu_q, cu_k, max_q, max_k, scale, bt=None, use_ws=True):
    lib = _lib.load()
    tq, hq, d = q.shape
    batch = cu_q.numel() - 1
    if bt is not None:
        nb, bs, hkv, _ = k.shape
        k_st = v_st = kv_sh = 0
        total_k, max_blocks, bt_stride = nb * bs, bt.shape[1], bt.stride(0)
    else:
        total_k, hkv, _ = k.shape
        k_st, v_st, kv_sh = k.stride(0), v.stride(0), k.stride(1)
        nb = bs = max_blocks = bt_stride = 0
    ws_bytes = lib.nvk_varlen_prefill_workspace_size(batch, max_q, max_k, hq, hkv, d)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if (use_ws and ws_bytes) else None
    out = torch.full_like(q, float("nan"))
    rc = lib.nvk_varlen_prefill(q.data_ptr(), q.stride(0), q.stride(1), tq, k.data_ptr(),
                                v.data_ptr(), k_st, v_st, kv_sh, total_k, cu_q.data_ptr(),
                                cu_k.data_ptr(), batch, max_q, max_k, _lib.ptr(bt), bt_stride,
                                max_blocks, bs, nb, hq, hkv, d, scale, out.data_ptr(),
                                out.stride(0), out.stride(1), _lib.ptr(ws),
                                ws_bytes if ws is not None else 0, 0,
                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.load().nvk_strerror(rc)
    torch.cuda.synchronize()
    return out, ws_bytes


def _paged_case(seed, lens_q, lens_k, bs=256, hq=16, hkv=8):
    gen = torch.Generator().manual_seed(seed)
    tables, nxt = [], 0
    pages = [(lk + bs - 1) // bs for lk in lens_k]
    perm = torch.randperm(sum(pages) + 3, generator=gen).tolist()
    for p in pages:
        tables.append(perm[nxt:nxt + p])
        nxt += p
    nb = len(perm)
    w = max(pages)
    bt = torch.full((len(lens_k), w), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    kc = torch.randn(nb, bs, hkv, 128, generator=gen).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(sum(lens_q), hq, 128, generator=gen).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(lens_q).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lens_k).tolist(), dtype=torch.int32)
    return q, kc, vc, bt, cu_q, cu_k


def _check_paged(seed, lens_q, lens_k, bs=256, hq=16, hkv=8, max_k=None, what="",
                 expect_split=True):
    q, kc, vc, bt, cu_q, cu_k = _paged_case(seed, lens_q, lens_k, bs, hq, hkv)
    scale = 128 ** -0.5
    mk = max_k if max_k is not None else max(lens_k)
    args = (q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(max(lens_q), 1), mk,
            scale)
    say(f"split prefill {what}: split")
    split, ws_bytes = _call(*args, bt=bt.cuda())
    assert (ws_bytes > 0) == expect_split, f"split path expected: {expect_split}"
    say(f"split prefill {what}: unsplit")
    whole, _ = _call(*args, bt=bt.cuda(), use_ws=False)
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, bs, scale)
    assert_attn_close(split, ref, what + " split")
    assert_attn_close(whole, ref, what + " unsplit")
    assert_attn_close(split, whole.float().cpu().numpy(), what + " split vs unsplit")


def test_spec_verify_shape_split():
    # 6 queries per sequence over 1000..7000 keys: 8 kv heads x 6 seqs = 48 workgroups
    _check_paged(31, [6] * 6, [1000, 2500, 4097, 5000, 6001, 7000], what="spec 6x6")


def test_long_query_ranges_are_not_split():
    # 300 queries (5 tiles of 64 tokens at G=2) over 5000 keys: the query tiles carry
    # the parallelism; partial records of full tiles would cost more than they save
    _check_paged(32, [300], [5000], what="5 query tiles", expect_split=False)


def test_split_small_pages_and_group_sizes():
    _check_paged(33, [7, 1, 12], [1500, 900, 2100], bs=16, what="block_size 16")
    _check_paged(34, [5, 9], [3000, 2000], hq=16, hkv=16, what="G=1")
    _check_paged(35, [5, 7], [3000, 2000], hq=16, hkv=2, what="G=8")


def test_split_underreported_max_seqlen_k_still_attends_every_key():
    # the split plan is made for 1024 keys; the last split runs to the real end
    _check_paged(36, [4, 4], [3000, 2900], max_k=1024, what="max_seqlen_k too small")


def test_split_dense_keys_and_empty_query_ranges():
    gen = torch.Generator().manual_seed(37)
    lens_q, lens_k = [3, 0, 8], [2000, 1500, 2600]     # the second sequence has no query
    q = torch.randn(sum(lens_q), 16, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(sum(lens_k), 8, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(sum(lens_k), 8, 128, generator=gen).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(lens_q).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lens_k).tolist(), dtype=torch.int32)
    args = (q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), 8, 2600, 0.09)
    say("split prefill dense: split")
    split, ws_bytes = _call(*args)
    assert ws_bytes > 0
    say("split prefill dense: unsplit")
    whole, _ = _call(*args, use_ws=False)
    ref = oracle_prefill_dense(q, k, v, cu_q, cu_k, 0.09)
    assert_attn_close(split, ref, "dense split")
    assert_attn_close(whole, ref, "dense unsplit")


def test_split_where_some_rows_of_a_wave_see_no_key_of_the_split():
    # 32 queries over 2072 keys, planned for 4096 keys: 8 splits of 8 tiles, the
    # fifth holding keys 2048..2071.  Query token t sees keys <= t + 2040, so in the
    # wave of tokens 0..15 tokens 0..7 see no key of that split while 8..15 do; the
    # empty rows' partial must stay (m=-inf, l=0, O=0) (regression: their
    # lazy-rescale factor was exp2(-inf - -inf) = NaN)
    _check_paged(38, [32], [2072], max_k=4096, what="rows without keys in a split")
