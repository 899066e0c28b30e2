"""Longest-first query-tile order of the varlen prefill.  With a workspace
(multi-sequence prefills) a small kernel ranks the (sequence, query tile)
pairs by their key count and the attention kernel takes its tile from that
order; without one the grid order is used.  The order only changes when a
tile runs, so both calls must give the same bits, and the ordered one is also
checked against the oracle (2e-2 abs / 1e-2 rel).  Cases: paged with cached
prefixes (GQA groups 2, 4, 8; an empty sequence; one-token sequences; pages of
16, 64, 128, 256 and 512 tokens), dense self-attention, and 300 short
sequences (ties, empty sequences)."""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_prefill_dense, oracle_prefill_paged, say
from test_gpu_prefill_split import _call, _paged_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 4), (8, 1)])
def test_ordered_equals_grid_order_paged(hq, hkv):
    rng = np.random.default_rng(60 + hkv)
    lens_q = [int(x) for x in rng.integers(1, 700, 24)] + [0, 1, 1] + [699]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 600, len(lens_q)))]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(61 + hkv, lens_q, lens_k, hq=hq, hkv=hkv)
    args = (q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k),
            128 ** -0.5)
    say(f"prefill order paged G={hq // hkv}: ordered")
    ordered, ws = _call(*args, bt=bt.cuda(), use_ws=True)
    tq = 128 * hkv // hq                      # query tokens per tile
    pairs = len(lens_q) * ((max(lens_q) + tq - 1) // tq)
    assert pairs * hkv > 1024 and ws >= 4 * pairs   # the order is used
    say(f"prefill order paged G={hq // hkv}: grid order")
    grid, _ = _call(*args, bt=bt.cuda(), use_ws=False)
    assert torch.equal(ordered, grid)
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
    assert_attn_close(ordered, ref, f"ordered paged prefill G={hq // hkv}")


@pytest.mark.parametrize("bs", [16, 64, 128, 512])
def test_ordered_equals_grid_order_block_sizes(bs):
    """Pages of 64 / 128 / 512 tokens (the kernel's first page ids come from
    shifts of another width) and of 16 tokens (tiles span pages: per-row
    page lookups), each with the longest-first order in use."""
    rng = np.random.default_rng(90 + bs)
    lens_q = [int(x) for x in rng.integers(1, 700, 16)] + [0, 699]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 800, len(lens_q)))]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(91 + bs, lens_q, lens_k, bs=bs)
    args = (q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k),
            128 ** -0.5)
    say(f"prefill order, {bs}-token pages: ordered")
    ordered, ws = _call(*args, bt=bt.cuda(), use_ws=True)
    pairs = len(lens_q) * ((max(lens_q) + 63) // 64)
    assert pairs * 8 > 1024 and ws >= 4 * pairs   # the order is used
    say(f"prefill order, {bs}-token pages: grid order")
    grid, _ = _call(*args, bt=bt.cuda(), use_ws=False)
    assert torch.equal(ordered, grid)
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, bs, 128 ** -0.5)
    assert_attn_close(ordered, ref, f"ordered paged prefill, {bs}-token pages")


def test_ordered_equals_grid_order_dense():
    rng = np.random.default_rng(70)
    lens = [int(x) for x in rng.integers(1, 500, 20)] + [499]   # 21 x 8 tiles x 8 heads
    gen = torch.Generator().manual_seed(71)
    t = sum(lens)
    q = torch.randn(t, 16, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(t, 8, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(t, 8, 128, generator=gen).to(torch.bfloat16)
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    args = (q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), max(lens), max(lens), 128 ** -0.5)
    say("prefill order dense: ordered")
    ordered, _ = _call(*args, use_ws=True)
    say("prefill order dense: grid order")
    grid, _ = _call(*args, use_ws=False)
    assert torch.equal(ordered, grid)
    assert_attn_close(ordered, oracle_prefill_dense(q, k, v, cu, cu, 128 ** -0.5),
                      "ordered dense prefill")


def test_ordered_many_short_sequences_with_empty_ones():
    """300 sequences of 0-40 tokens (one query tile each, many ties and empty
    sequences) over paged prefixes of 0-300 keys."""
    rng = np.random.default_rng(80)
    lens_q = [int(x) for x in rng.integers(0, 41, 300)]
    lens_q[:3] = [0, 40, 1]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 301, 300))]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(81, lens_q, lens_k)
    args = (q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k),
            128 ** -0.5)
    say("prefill order, 300 short sequences: ordered")
    ordered, ws = _call(*args, bt=bt.cuda(), use_ws=True)
    assert ws >= 4 * 300
    say("prefill order, 300 short sequences: grid order")
    grid, _ = _call(*args, bt=bt.cuda(), use_ws=False)
    assert torch.equal(ordered, grid)
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
    assert_attn_close(ordered, ref, "ordered prefill, 300 short sequences")


def test_order_ranked_once_serves_every_layer():
    """nvk_prefill_tile_order once, then three layers' prefills (their own
    caches, the same metadata) through nvk_varlen_prefill_ordered: each equals
    nvk_varlen_prefill, which ranks the tiles itself, bit for bit; the order
    is a permutation of the (sequence, query tile) pairs."""
    from nanovllm_amd import _lib, varlen_prefill
    from nanovllm_amd.flash_api import prefill_tile_order
    rng = np.random.default_rng(75)
    lens_q = [int(x) for x in rng.integers(1, 600, 40)]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 900, len(lens_q)))]
    base = _paged_case(76, lens_q, lens_k)
    q, kc, vc, bt, cu_q, cu_k = base
    gen = torch.Generator().manual_seed(77)
    layers = [base] + [(q, torch.randn(kc.shape, generator=gen).to(torch.bfloat16),
                        torch.randn(vc.shape, generator=gen).to(torch.bfloat16), bt, cu_q, cu_k)
                       for _ in range(2)]
    dcu_q, dcu_k, dbt = cu_q.cuda(), cu_k.cuda(), bt.cuda()
    say("prefill order once per step: rank")
    order = prefill_tile_order(dcu_q, dcu_k, max(lens_q), kc.cuda(), 16, block_table=dbt,
                               max_seqlen_k=max(lens_k))
    assert order is not None
    n_qtiles = (max(lens_q) + 63) // 64
    pairs = len(lens_q) * n_qtiles
    assert sorted(order[:pairs].cpu().tolist()) == list(range(pairs))
    # the tag after the pairs names the batch and the tile count
    assert int(order[pairs]) == np.int32(np.uint32(0xA0000000 | (len(lens_q) << 16) | n_qtiles))
    for i, (q, kc, vc, bt_i, _, _) in enumerate(layers):
        assert torch.equal(bt_i, bt)
        dq, dkc, dvc = q.cuda(), kc.cuda(), vc.cuda()
        say(f"prefill order once per step: layer {i}")
        a = varlen_prefill(dq, dkc, dvc, dcu_q, dcu_k, max(lens_q), 128 ** -0.5, block_table=dbt,
                           max_seqlen_k=max(lens_k), order=order)
        b = varlen_prefill(dq, dkc, dvc, dcu_q, dcu_k, max(lens_q), 128 ** -0.5, block_table=dbt,
                           max_seqlen_k=max(lens_k))
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"layer {i}"
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
    assert_attn_close(a, ref, "ordered prefill, last layer")
    # a launch that runs in grid order needs no order
    assert _lib.load().nvk_prefill_tile_order_size(3, 100, 1536, 16, 8, 256) == 0


def test_order_of_other_sizes_is_rejected_or_ignored():
    """An order buffer too small for the call is rejected before any launch;
    an order ranked for another batch (its tag differs) is ignored and the
    tiles run in grid order, with the output of an unordered call."""
    from nanovllm_amd import _lib, varlen_prefill
    from nanovllm_amd.flash_api import prefill_tile_order
    rng = np.random.default_rng(78)
    lens_q = [int(x) for x in rng.integers(64, 700, 48)]
    lens_k = [q + int(c) for q, c in zip(lens_q, rng.integers(0, 900, len(lens_q)))]
    q, kc, vc, bt, cu_q, cu_k = (x.cuda() for x in _paged_case(79, lens_q, lens_k))
    args = (q, kc, vc, cu_q, cu_k, max(lens_q), 128 ** -0.5)
    kw = dict(block_table=bt, max_seqlen_k=max(lens_k))
    say("prefill order: a smaller batch's order")
    small = prefill_tile_order(cu_q[:41], cu_k[:41], max(lens_q), kc, 16, block_table=bt[:40],
                               max_seqlen_k=max(lens_k))
    assert small is not None
    with pytest.raises(_lib.NvkError, match="order holds"):
        varlen_prefill(*args, order=small, **kw)
    # a buffer large enough whose tag names another batch: ignored
    big = torch.zeros(small.numel() + 4096, dtype=torch.int32, device="cuda")
    big[:small.numel()] = small
    ref = varlen_prefill(*args, **kw)
    got = varlen_prefill(*args, order=big, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
