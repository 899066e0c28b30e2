"""Seeded random sweep over the shapes the kernels accept, against the oracle.

Every case draws its own GQA group (1, 2, 4, 8), page size (16, 64, 256,
512), batch, ragged lengths (zeros included), a shuffled page pool and bf16
N(0, 1) data from one seed, then runs the store, decode and prefill (paged
with a cached prefix, dense without) through the production wrappers:
store bit for bit, attention within 2e-2 abs / 1e-2 rel.  Sizes stay small
so the numpy oracle finishes in seconds.
"""
import numpy as np
import pytest
import torch

from gpu_utils import (assert_attn_close, bits, oracle_decode, oracle_prefill_dense,
                       oracle_prefill_paged, oracle_store, say)
from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill

pytestmark = pytest.mark.gpu

HD = 128
SEEDS = list(range(100, 112))


def _draw(seed):
    rng = np.random.default_rng(seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8]))
    bs = int(rng.choice([16, 64, 256, 512]))
    batch = int(rng.integers(1, 9))
    lens_k = [int(x) for x in rng.integers(0, 1500, batch)]
    lens_k[int(rng.integers(0, batch))] = int(rng.choice([0, 1, bs, bs + 1]))
    return rng, hkv, g * hkv, bs, batch, lens_k


def _pool(rng, lens_k, bs, hkv, spare=3):
    pages = [(n + bs - 1) // bs for n in lens_k]
    nb = sum(pages) + spare
    perm = rng.permutation(nb)
    w = max(max(pages), 1)
    bt = np.full((len(lens_k), w), -1, np.int32)
    nxt = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[nxt:nxt + p]
        nxt += p
    gen = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    kc = torch.randn(nb, bs, hkv, HD, generator=gen).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, HD, generator=gen).to(torch.bfloat16)
    return torch.from_numpy(bt), kc, vc, gen


@pytest.mark.parametrize("seed", SEEDS)
def test_random_store_decode_prefill(seed):
    rng, hkv, hq, bs, batch, lens_k = _draw(seed)
    what = f"seed {seed}: Hq/Hkv {hq}/{hkv}, page {bs}, lens {lens_k}"
    bt, kc, vc, gen = _pool(rng, lens_k, bs, hkv)
    scale = HD ** -0.5

    # store: the last min(len, 40) tokens of every context, 5 % of slots -1
    news = [min(n, int(rng.integers(1, 41))) for n in lens_k]
    slots = []
    for i, (n, m) in enumerate(zip(lens_k, news)):
        pos = np.arange(n - m, n)
        slots += (bt[i, pos // bs].long() * bs + torch.from_numpy(pos % bs)).tolist()
    slots = torch.tensor(slots, dtype=torch.int32)
    t = slots.numel()
    if t:
        slots[torch.from_numpy(rng.choice(t, size=max(0, t // 20), replace=False))] = -1
    key = torch.randn(t, hkv, HD, generator=gen).to(torch.bfloat16)
    value = torch.randn(t, hkv, HD, generator=gen).to(torch.bfloat16)
    ek, ev = oracle_store(key, value, kc, vc, slots)
    dk, dv = kc.cuda(), vc.cuda()
    say(f"sweep store {what}")
    store_kvcache(key.cuda(), value.cuda(), dk, dv, slots.cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(dk), ek, err_msg=what)
    np.testing.assert_array_equal(bits(dv), ev, err_msg=what)
    kc = dk.cpu()
    vc = dv.cpu()

    # decode: one query per context
    lens = torch.tensor(lens_k, dtype=torch.int32)
    q = torch.randn(batch, hq, HD, generator=gen).to(torch.bfloat16)
    say(f"sweep decode {what}")
    out = paged_decode(q.cuda(), dk, dv, lens.cuda(), bt.cuda(), scale)
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_decode(q, kc, vc, bt, lens, bs, scale), "decode " + what)

    # paged prefill: the last lens_q of every context are queries
    lens_q = [min(n, int(rng.integers(0, 300))) for n in lens_k]
    cu_q = torch.tensor([0] + np.cumsum(lens_q).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lens_k).tolist(), dtype=torch.int32)
    qp = torch.randn(int(cu_q[-1]), hq, HD, generator=gen).to(torch.bfloat16)
    if int(cu_q[-1]):
        say(f"sweep paged prefill {what}, lens_q {lens_q}")
        out = varlen_prefill(qp.cuda(), dk, dv, cu_q.cuda(), cu_k.cuda(), max(lens_q), scale,
                             block_table=bt.cuda(), max_seqlen_k=max(lens_k))
        torch.cuda.synchronize()
        ref = oracle_prefill_paged(qp, kc, vc, bt, cu_q, cu_k, bs, scale)
        assert_attn_close(out, ref, "paged prefill " + what)

    # dense prefill (no prefix): Lq == Lk per sequence, k/v the step's own rows
    lens_d = [min(n, 400) for n in lens_k]
    cu_d = torch.tensor([0] + np.cumsum(lens_d).tolist(), dtype=torch.int32)
    td = int(cu_d[-1])
    if td:
        qd = torch.randn(td, hq, HD, generator=gen).to(torch.bfloat16)
        kd = torch.randn(td, hkv, HD, generator=gen).to(torch.bfloat16)
        vd = torch.randn(td, hkv, HD, generator=gen).to(torch.bfloat16)
        say(f"sweep dense prefill {what}, lens {lens_d}")
        out = varlen_prefill(qd.cuda(), kd.cuda(), vd.cuda(), cu_d.cuda(), cu_d.cuda(),
                             max(lens_d), scale)
        torch.cuda.synchronize()
        assert_attn_close(out, oracle_prefill_dense(qd, kd, vd, cu_d, cu_d, scale),
                          "dense prefill " + what)
