"""The needle construction (tests/needles.py) on the CPU: the pinned oracle
returns exactly the closed-form expectation for every needle position, and
each planted oracle mistake that moves a key across the causal edge or reads
the wrong kv head fails it.  This is what makes the GPU needle checks sharp.
"""
import numpy as np
import pytest
import torch

from needles import NeedleCase, interesting_positions, mismatches
from oracle import kv_oracle as orc


def _oracle(case, mutation=None):
    f = lambda t: t.float().numpy()
    lens_k = np.asarray(case.lens_k)
    if case.block_tables is not None:
        out = orc.paged_attention(f(case.q), f(case.k), f(case.v), case.cu_q.numpy(), lens_k,
                                  case.scale, block_tables=case.block_tables.numpy(),
                                  block_size=case.bs, _mutation=mutation)
    else:
        out = orc.paged_attention(f(case.q), f(case.k), f(case.v), case.cu_q.numpy(), lens_k,
                                  case.scale, cu_seqlens_k=case.cu_k.numpy(), _mutation=mutation)
    return torch.from_numpy(out)


def _cases():
    return [
        NeedleCase(1, [1, 1, 1], [40, 257, 100], block_size=16, hq=4, hkv=2, d=32, device="cpu"),
        NeedleCase(2, [3, 20, 7], [70, 20, 300], block_size=64, hq=4, hkv=2, d=32,
                   device="cpu"),
        NeedleCase(3, [5, 33], [5, 33], block_size=0, hq=2, hkv=1, d=32, device="cpu"),
    ]


@pytest.mark.parametrize("ci", range(3))
def test_oracle_returns_the_closed_form_for_every_needle(ci):
    case = _cases()[ci]
    calls = case.position_schedule(16)
    assert len(calls) >= 5
    for pos in calls:
        planted = case.plant(pos)
        bad = mismatches(_oracle(case).to(torch.bfloat16), case.expected(pos))
        case.restore(planted)
        assert not bool(bad.any()), f"needles at {pos.tolist()}"


@pytest.mark.parametrize("mutation", ["strict", "top_left", "gqa_mod"])
def test_planted_oracle_mistakes_fail_the_needles(mutation):
    # (a top-left mask equals the bottom-right one when Lq == Lk, so the
    # dense case cannot catch it; the paged cases with a prefix do)
    caught = []
    for case in _cases():
        hit = False
        for pos in case.position_schedule(16):
            planted = case.plant(pos)
            bad = mismatches(_oracle(case, mutation).to(torch.bfloat16), case.expected(pos))
            case.restore(planted)
            hit |= bool(bad.any())
        caught.append(hit)
    assert caught[0] and caught[1], f"{mutation} not caught: {caught}"


def test_needle_scores_dominate_and_poison_sits_past_the_end():
    case = NeedleCase(4, [1], [300], block_size=64, hq=2, hkv=1, d=128, device="cpu")
    q = case.q[0, 0].float()
    kf = case.k.view(-1, 1, 128)[:, 0].float()
    sl = case.slots(torch.arange(301).view(1, -1))[0]           # keys 0 .. 300 of sequence 0
    scores = (kf[sl] @ q) * case.scale
    assert 40 < float(scores[0]) < 50                            # floor needle ~45 nats
    assert float(scores[300]) > 170                              # the poison, one past key 299
    assert float(scores[1:300].max()) < 15                       # random keys stay far below


def test_positions_cover_every_edge():
    p = interesting_positions(1000, 64, 256, lq=300)
    for e in range(64, 1000, 64):
        assert e - 1 in p and e in p
    for e in (255, 256, 257, 511, 512, 513, 699, 700, 701, 998, 999):
        assert e in p
    assert min(p) == 1 and max(p) == 999
