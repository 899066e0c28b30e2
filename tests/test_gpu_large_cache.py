"""Layer caches larger than 4 GiB.

The reference allocates one KV cache for all layers with torch.empty
(model_runner.py:100-118); with 288 GB of HBM one layer's K (or V) cache of a
small model passes 4 GiB.  Here each cache is 8224 pages of 256 x 8 x 128
bf16 (4.31 GB), and a case uses 44 pages placed either at the top of the
cache (pages 8180..8223, across page 8192, which starts at byte 2^32) or at
the bottom (pages 0..43) with the same contents.  Every kernel that addresses
the cache -- the store, the fused prologue's store, decode, paged prefill and
the short-query path -- must give bit-identical results for both placements,
and the low placement is checked against the oracle.  Unused cache slots hold
NaN (as uninitialised memory may), so a kernel that read past a context would
turn its output non-finite.
"""
import numpy as np
import pytest
import torch

from nanovllm_amd import (paged_decode, qk_norm_rope_store, rope_cos_sin_cache, store_kvcache,
                          varlen_prefill)
from tests.gpu_utils import assert_attn_close, bits, oracle_decode, oracle_prefill_paged, say

pytestmark = pytest.mark.gpu

NB, BS, HKV, HQ, D = 8224, 256, 8, 16, 128
P = 44                      # pages one case uses
HIGH0 = NB - P              # first high page: 8180
ROW_BYTES = HKV * D * 2
SCALE = D ** -0.5
NAN_BITS = 0x7FC0


@pytest.fixture(scope="module")
def caches():
    assert HIGH0 * BS * ROW_BYTES < 2 ** 32 < NB * BS * ROW_BYTES
    say(f"large cache: 2 x {NB * BS * ROW_BYTES / 1e9:.2f} GB")
    kc = torch.empty((NB, BS, HKV, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    yield kc, vc
    del kc, vc
    torch.cuda.empty_cache()


def _fill_nan(kc, vc):
    kc.fill_(float("nan"))
    vc.fill_(float("nan"))


def _tables(gen, ctx):
    """Block tables of the contexts over page offsets 0..P-1 (shuffled), padded
    with -1; returns (low, high) tables as int32 CPU tensors."""
    pages = [(c + BS - 1) // BS for c in ctx]
    assert sum(pages) <= P
    perm = torch.randperm(P, generator=gen)[:sum(pages)].tolist()
    w = max(pages)
    low = torch.full((len(ctx), w), -1, dtype=torch.int32)
    nxt = 0
    for i, p in enumerate(pages):
        low[i, :p] = torch.tensor(perm[nxt:nxt + p], dtype=torch.int32)
        nxt += p
    high = torch.where(low >= 0, low + HIGH0, low)
    return low, high


def _slots(table, ctx):
    """Flat cache rows of the first ctx[i] tokens of every sequence."""
    out = []
    for i, c in enumerate(ctx):
        t = torch.arange(c)
        out.append(table[i, t // BS].long() * BS + t % BS)
    return torch.cat(out)


def _fill_contexts(gen, kc, vc, ctx, low, high):
    n = sum(ctx)
    k = torch.randn(n, HKV, D, generator=gen).to(torch.bfloat16).cuda()
    v = torch.randn(n, HKV, D, generator=gen).to(torch.bfloat16).cuda()
    for table in (low, high):
        rows = _slots(table, ctx).cuda()
        kc.view(-1, HKV, D)[rows] = k
        vc.view(-1, HKV, D)[rows] = v


def _low_copy(kc, vc):
    return kc[:P].cpu(), vc[:P].cpu()


def test_store_rows_past_4gib(caches):
    kc, vc = caches
    _fill_nan(kc, vc)
    gen = torch.Generator().manual_seed(71)
    t = 3000
    slots = (HIGH0 * BS + torch.randperm(P * BS, generator=gen)[:t]).to(torch.int32)
    slots[torch.randperm(t, generator=gen)[:150]] = -1
    assert int(slots.max()) * ROW_BYTES >= 2 ** 32
    key = torch.randn(t, HKV, D, generator=gen).to(torch.bfloat16)
    value = torch.randn(t, HKV, D, generator=gen).to(torch.bfloat16)
    say("large cache: store")
    store_kvcache(key.cuda(), value.cuda(), kc, vc, slots.cuda())
    torch.cuda.synchronize()
    ok = slots >= 0
    rows = slots[ok].long().cuda()
    assert torch.equal(kc.view(-1, HKV, D)[rows].cpu(), key[ok])
    assert torch.equal(vc.view(-1, HKV, D)[rows].cpu(), value[ok])
    # rows of the high pages that no token names keep their NaN bytes
    untouched = torch.ones(P * BS, dtype=torch.bool)
    untouched[(slots[ok].long() - HIGH0 * BS)] = False
    spare = (HIGH0 * BS + torch.nonzero(untouched).flatten()[:64]).cuda()
    assert (bits(kc.view(-1, HKV, D)[spare]) == NAN_BITS).all()
    assert (bits(vc.view(-1, HKV, D)[spare]) == NAN_BITS).all()


def test_decode_prefill_short_query_past_4gib(caches):
    kc, vc = caches
    _fill_nan(kc, vc)
    gen = torch.Generator().manual_seed(72)
    ctx = [300, 1000, 2000, 513, 64, 1500, 1, 3000]
    low, high = _tables(gen, ctx)
    assert int(high.max()) >= 2 ** 32 // (BS * ROW_BYTES)
    _fill_contexts(gen, kc, vc, ctx, low, high)
    kl, vl = _low_copy(kc, vc)
    lens = torch.tensor(ctx, dtype=torch.int32)

    # decode: one query per sequence
    q = torch.randn(len(ctx), HQ, D, generator=gen).to(torch.bfloat16)
    outs = []
    for name, table in (("low", low), ("high", high)):
        say(f"large cache: decode {name}")
        outs.append(paged_decode(q.cuda(), kc, vc, lens.cuda(), table.cuda(), SCALE))
    torch.cuda.synchronize()
    assert torch.isfinite(outs[1].float()).all()
    assert torch.equal(outs[0], outs[1])
    assert_attn_close(outs[0], oracle_decode(q, kl, vl, low, lens, BS, SCALE), "decode low")

    # prefill (the last lens_q of each context are queries) and short queries
    for what, lens_q in (("prefill", [100, 64, 700, 13, 64, 1, 1, 256]),
                         ("short query", [min(6, c) for c in ctx])):
        cu_q = torch.tensor([0] + np.cumsum(lens_q).tolist(), dtype=torch.int32)
        cu_k = torch.tensor([0] + np.cumsum(ctx).tolist(), dtype=torch.int32)
        qp = torch.randn(int(cu_q[-1]), HQ, D, generator=gen).to(torch.bfloat16)
        outs = []
        for name, table in (("low", low), ("high", high)):
            say(f"large cache: {what} {name}")
            outs.append(varlen_prefill(qp.cuda(), kc, vc, cu_q.cuda(), cu_k.cuda(), max(lens_q),
                                       SCALE, block_table=table.cuda(), max_seqlen_k=max(ctx)))
        torch.cuda.synchronize()
        assert torch.isfinite(outs[1].float()).all(), what
        assert torch.equal(outs[0], outs[1]), what
        ref = oracle_prefill_paged(qp, kl, vl, low, cu_q, cu_k, BS, SCALE)
        assert_attn_close(outs[0], ref, what + " low")


def test_prologue_store_past_4gib(caches):
    kc, vc = caches
    _fill_nan(kc, vc)
    gen = torch.Generator().manual_seed(73)
    t, max_pos = 1000, 40960
    qkv = (torch.randn(t, (HQ + 2 * HKV) * D, generator=gen) * 2.0).to(torch.bfloat16).cuda()
    qw = (1.0 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).cuda()
    kw = (1.0 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).cuda()
    pos = torch.randint(0, max_pos, (t,), generator=gen, dtype=torch.int64).cuda()
    cos_sin = rope_cos_sin_cache(D, max_pos, 1_000_000.0, device="cuda")
    off = torch.randperm(P * BS, generator=gen)[:t].to(torch.int32)
    off[torch.randperm(t, generator=gen)[:50]] = -1
    res = []
    for name, base in (("low", 0), ("high", HIGH0 * BS)):
        slots = torch.where(off >= 0, off + base, off).cuda()
        say(f"large cache: prologue {name}")
        q, k, _ = qk_norm_rope_store(pos, qkv, HQ, HKV, D, qw, kw, 1e-6, cos_sin, kc, vc, slots)
        torch.cuda.synchronize()
        rows = slots[slots >= 0].long()
        res.append((q, k, kc.view(-1, HKV, D)[rows].clone(), vc.view(-1, HKV, D)[rows].clone()))
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)
    ok = (off >= 0).cuda()
    assert torch.equal(res[1][2], res[1][1][ok])                        # cached k = returned k
    v_in = qkv[:, (HQ + HKV) * D:].reshape(t, HKV, D)
    assert torch.equal(res[1][3], v_in[ok])                             # raw v rows
