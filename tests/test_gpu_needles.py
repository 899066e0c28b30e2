"""Closed-form needle checks of the attention kernels on the GPU.

A tolerance against random data cannot see one dropped key at long context
(one key moves an output of magnitude ~0.03 by less than the 2e-2 bound).
Here the softmax is made one-hot (tests/needles.py): each query row must
return exactly the V row of the dominant key it can see, so a key lost at a
tile, chunk, page or wave-split edge, a shifted causal diagonal, or a read
past the last key (the poison) is an O(1) error.  Over the calls of a
schedule the needle of every (sequence, kv head) group visits both sides of
every 32-key chunk edge (decode), every 64-key tile / chunk edge (prefill,
short queries) and every page edge of its context, so every point where the
stream-K plan can cut a context is covered whatever the plan.

Reference calls: attention.py:67-70 (varlen prefill, paged and dense) and
attention.py:72-74 (decode).
"""
import numpy as np
import pytest
import torch

from needles import NeedleCase, run_schedule
from nanovllm_amd import flash_attn_with_kvcache, paged_decode, varlen_prefill

pytestmark = pytest.mark.gpu


def _lens(seed, n, lo, hi):
    return [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, n)]


def _decode(case):
    lens = case.cu_k[1:] - case.cu_k[:-1]
    return paged_decode(case.q, case.k, case.v, lens, case.block_tables, case.scale)


def _prefill(case):
    return varlen_prefill(case.q, case.k, case.v, case.cu_q, case.cu_k, max(case.lens_q),
                          case.scale, block_table=case.block_tables,
                          max_seqlen_k=max(case.lens_k))


@pytest.mark.parametrize("name,lens,bs,hq,hkv", [
    ("batch 64, contexts U{100..2048}", _lens(1, 64, 100, 2048), 256, 16, 8),
    ("batch 4, contexts cut into many parts", [1976, 1362, 1686, 1273], 256, 16, 8),
    ("batch 512, contexts U{256..4096}", _lens(2, 512, 256, 4096), 256, 16, 8),
    ("batch 1, context 16384", [16384], 256, 16, 8),
    ("16-key pages", _lens(3, 24, 2, 700), 16, 16, 8),
    ("64-key pages, G=4", _lens(4, 24, 2, 900), 64, 16, 4),
    ("512-key pages, G=8", _lens(5, 16, 2, 1500), 512, 16, 2),
    ("G=1", _lens(6, 32, 2, 1100), 256, 16, 16),
])
def test_decode_needles(name, lens, bs, hq, hkv):
    case = NeedleCase(10, [1] * len(lens), lens, block_size=bs, hq=hq, hkv=hkv)
    run_schedule(case, _decode, 32, f"decode {name}")


@pytest.mark.parametrize("name,lens_q,lens_k,bs,hq,hkv", [
    # 32 sequences, 512 cached + U{100..1024} new tokens
    ("32 seqs after a 512-token prefix",
     *(lambda n: (n, [512 + x for x in n]))(_lens(7, 32, 100, 1024)), 256, 16, 8),
    # chunked prefill: 8 chunks of 512 after U{0..1536} cached (mid-page starts)
    ("8 chunks of 512 after U{0..1536}",
     *(lambda c: ([512] * 8, [512 + x for x in c]))(_lens(8, 8, 0, 1536)), 256, 16, 8),
    ("no prefix, ragged", [2, 63, 64, 65, 129, 300, 777], [2, 63, 64, 65, 129, 300, 777],
     256, 16, 8),
    ("G=1 and 64-key pages", [5, 70, 200], [300, 700, 460], 64, 16, 16),
    ("G=4, 16-key pages", [33, 100, 7], [100, 400, 900], 16, 16, 4),
    ("G=8, 512-key pages", [90, 300], [1400, 600], 512, 16, 2),
    # few short query ranges over long keys: the split-K tile path
    ("2 x 40 queries over 6000 keys", [40, 40], [6000, 5000], 256, 16, 8),
])
def test_paged_prefill_needles(name, lens_q, lens_k, bs, hq, hkv):
    case = NeedleCase(11, lens_q, lens_k, block_size=bs, hq=hq, hkv=hkv)
    run_schedule(case, _prefill, 64, f"prefill {name}")


@pytest.mark.parametrize("lens,hq,hkv", [
    ([2, 63, 64, 65, 128, 129, 700, 1500], 16, 8),
    ([5, 300, 1000], 16, 2),
])
def test_dense_prefill_needles(lens, hq, hkv):
    case = NeedleCase(12, lens, lens, block_size=0, hq=hq, hkv=hkv)
    run_schedule(case, _prefill, 64, f"dense prefill G={hq // hkv}")


@pytest.mark.parametrize("name,nq,lens,hq,hkv", [
    ("spec-verify 32 x 6 over U{1024..8192}", 6, _lens(13, 32, 1024, 8192), 16, 8),
    ("1 query over U{64..3000}", 1, _lens(14, 24, 64, 3000), 16, 8),
    ("2 queries, G=8", 2, _lens(15, 12, 64, 5000), 16, 2),
    ("16 queries, G=1", 16, _lens(16, 6, 64, 3000), 16, 16),
    ("batch 4, long contexts cut into many parts", 6, [8192, 7000, 6100, 4321], 16, 8),
    # the sliced combine: one sequence's groups cut into ~128 parts; three
    # query rows of G=1, so a workgroup's second row is past the last one
    ("1 sequence over 16384 keys", 6, [16384], 16, 8),
    ("3 queries over 2 long sequences, G=1", 3, [9000, 12000], 16, 16),
])
def test_short_query_needles(name, nq, lens, hq, hkv):
    case = NeedleCase(13, [nq] * len(lens), lens, block_size=256, hq=hq, hkv=hkv)
    run_schedule(case, _prefill, 64, f"short query {name}")


def test_spec_verify_needles_through_flash_api():
    lens = _lens(17, 16, 1024, 8192)
    case = NeedleCase(14, [6] * 16, lens, block_size=256)

    def call(c):
        lens_t = c.cu_k[1:] - c.cu_k[:-1]
        out = flash_attn_with_kvcache(c.q.view(16, 6, 16, 128), c.k, c.v, cache_seqlens=lens_t,
                                      block_table=c.block_tables, softmax_scale=c.scale,
                                      causal=True)
        return out.view(-1, 16, 128)

    run_schedule(case, call, 64, "flash_attn_with_kvcache, 6 queries")
