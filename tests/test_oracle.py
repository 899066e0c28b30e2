"""Pins the CPU oracle (oracle/kv_oracle.py) before anything is compared with it.

Each oracle function is checked against data it did not produce: the study
guide's worked answers, scalar brute force (tests/golden), torch's CPU
scaled_dot_product_attention where the conventions coincide, and closed
forms.  The last group plants known mistakes in the oracle (its `_mutation`
knob) and shows each one fails at least one of the checks.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def known():
    with open(os.path.join(GOLDEN, "guide_known_answers.json")) as f:
        return json.load(f)


# ---------------------------------------------------------------------------
# KV store
# ---------------------------------------------------------------------------
def test_slot_formula_known_answer():
    ex = known()["slot_example"]
    assert orc.slots_for(ex["block_table"], ex["positions"], ex["block_size"]) == ex["slots"]


def test_slot_formula_independent_of_block_size():
    # The guide's follow-up: change block_size to 3; the formula still matches a
    # page-by-page enumeration of the logical positions.
    table = [3, 0, 5]
    for bs in (3, 4, 7):
        flat = [page * bs + off for page in table for off in range(bs)]
        assert orc.slots_for(table, range(len(table) * bs), bs) == flat


def test_store_tiny_known_answer():
    ex = known()["store_tiny"]
    kc = np.full((ex["num_blocks"], ex["block_size"], ex["Hkv"], ex["D"]), ex["fill"], np.float32)
    vc = kc.copy()
    key = np.array(ex["key"], np.float32).reshape(ex["N"], ex["Hkv"], ex["D"])
    before = kc.copy()
    orc.kv_store(key, key + 100, kc, vc, np.array(ex["slots"], np.int32))
    changed = np.argwhere(kc != before)
    assert len(changed) == len(ex["changed"])
    for blk, off, h, d, val in ex["changed"]:
        assert kc[blk, off, h, d] == val
        assert vc[blk, off, h, d] == val + 100


def test_store_matrix_matches_brute_force_fixture():
    data = np.load(os.path.join(GOLDEN, "store_small.npz"))
    for ci in range(3):
        key, value = data[f"c{ci}_key"], data[f"c{ci}_value"]
        kc, vc = data[f"c{ci}_k_cache"].copy(), data[f"c{ci}_v_cache"].copy()
        key0, value0 = key.copy(), value.copy()
        slots = data[f"c{ci}_slots"]
        orc.kv_store(key, value, kc, vc, slots)
        np.testing.assert_array_equal(kc, data[f"c{ci}_expect_k"])
        np.testing.assert_array_equal(vc, data[f"c{ci}_expect_v"])
        # inputs unmodified, K and V not swapped, untouched cells keep the fill
        np.testing.assert_array_equal(key, key0)
        np.testing.assert_array_equal(value, value0)
        written = np.zeros(kc.shape[:2], bool)
        for s in slots[slots >= 0]:
            written[s // 256, s % 256] = True
        assert np.all(kc[~written] == 0x7F7F) and np.all(vc[~written] == 0x3F3F)


def test_store_matrix_shapes_cover_the_guide():
    m = known()["store_matrix"]
    data = np.load(os.path.join(GOLDEN, "store_small.npz"))
    for ci, (slots, n, (hkv, d)) in enumerate(zip(m["slots"], m["N"], m["hkv_d"])):
        s = data[f"c{ci}_slots"]
        assert list(s[:len(slots)]) == slots
        assert data[f"c{ci}_key"].shape == (max(n, len(slots)), hkv, d)


def test_store_gather_round_trip_with_shared_prefix():
    # logical sequences -> slots via tables -> store into a shuffled pool -> gather
    rng = np.random.default_rng(0)
    bs = 4
    pool = rng.permutation(12)
    shared = [int(pool[0])]
    tables = [shared + [int(pool[1]), int(pool[2])], shared + [int(pool[3])]]
    lens = [9, 5]
    prefix = rng.standard_normal((bs, 2, 8)).astype(np.float32)
    seqs = []
    for n in lens:
        x = rng.standard_normal((n, 2, 8)).astype(np.float32)
        x[:bs] = prefix                    # identical shared-prefix K/V
        seqs.append(x)
    kc = np.zeros((12, bs, 2, 8), np.float32)
    vc = np.zeros_like(kc)
    for x, t, n in zip(seqs, tables, lens):
        orc.kv_store(x, -x, kc, vc, np.array(orc.slots_for(t, range(n), bs), np.int32))
    for x, t, n in zip(seqs, tables, lens):
        np.testing.assert_array_equal(orc.gather_rows(kc, t, n, bs), x)
        np.testing.assert_array_equal(orc.gather_rows(vc, t, n, bs), -x)


def test_store_rejects_out_of_range_slot():
    kc = np.zeros((1, 4, 1, 2), np.float32)
    with pytest.raises(ValueError):
        orc.kv_store(np.ones((1, 1, 2)), np.ones((1, 1, 2)), kc, kc.copy(), np.array([4]))


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def _golden_attn(name):
    data = np.load(os.path.join(GOLDEN, "attn_small.npz"))
    hq, hkv, d, bs = [int(x) for x in data[f"{name}_meta"]]
    lens_q = data[f"{name}_lens_q"]
    cu_q = np.concatenate([[0], np.cumsum(lens_q)])
    return dict(q=orc.bf16_to_f32(data[f"{name}_q"]), k=orc.bf16_to_f32(data[f"{name}_k_cache"]),
                v=orc.bf16_to_f32(data[f"{name}_v_cache"]), bt=data[f"{name}_block_tables"],
                cu_q=cu_q, lens_k=data[f"{name}_lens_k"], bs=bs, d=d,
                expect=data[f"{name}_expect"])


GOLDEN_ATTN = ["decode_minimal", "decode_shared", "decode_gqa", "prefill_prefix", "prefill_page"]


def _run_golden(name, mutation=None):
    c = _golden_attn(name)
    return c, orc.paged_attention(c["q"], c["k"], c["v"], c["cu_q"], c["lens_k"], c["d"] ** -0.5,
                                  block_tables=c["bt"], block_size=c["bs"], _mutation=mutation)


@pytest.mark.parametrize("name", GOLDEN_ATTN)
def test_attention_matches_brute_force_fixture(name):
    c, out = _run_golden(name)
    np.testing.assert_allclose(out, c["expect"], rtol=1e-5, atol=1e-5)


def test_decode_minimal_case_structure():
    ex = known()["decode_minimal"]
    c = _golden_attn("decode_minimal")
    assert list(c["bt"][0]) == ex["tables"][0] and list(c["lens_k"]) == ex["context_lens"]


def _sdpa_ref(q, k, v, scale, causal):
    """torch CPU SDPA on [L, H, D] float32 arrays with GQA by head repetition."""
    g = q.shape[1] // k.shape[1]
    qt = torch.from_numpy(q).permute(1, 0, 2)
    kt = torch.from_numpy(k).repeat_interleave(g, dim=1).permute(1, 0, 2)
    vt = torch.from_numpy(v).repeat_interleave(g, dim=1).permute(1, 0, 2)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, scale=scale)
    return o.permute(1, 0, 2).numpy()


@pytest.mark.parametrize("hq,hkv", [(4, 4), (4, 2), (8, 2)])
def test_dense_self_attention_equals_torch_sdpa(hq, hkv):
    # Lq == Lk: bottom-right and top-left causal alignment coincide.
    rng = np.random.default_rng(1)
    lens = [5, 17, 1]
    tq = sum(lens)
    q = rng.standard_normal((tq, hq, 32)).astype(np.float32)
    k = rng.standard_normal((tq, hkv, 32)).astype(np.float32)
    v = rng.standard_normal((tq, hkv, 32)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)])
    out = orc.paged_attention(q, k, v, cu, lens, 0.3, cu_seqlens_k=cu)
    for s in range(3):
        a, b = cu[s], cu[s + 1]
        np.testing.assert_allclose(out[a:b], _sdpa_ref(q[a:b], k[a:b], v[a:b], 0.3, True),
                                   rtol=1e-5, atol=1e-5)


def test_decode_equals_torch_sdpa_without_mask():
    rng = np.random.default_rng(2)
    hq, hkv, d, bs = 8, 2, 16, 4
    kc = rng.standard_normal((6, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((6, bs, hkv, d)).astype(np.float32)
    tables = np.array([[4, 1, 0], [2, 5, -1]], np.int32)
    lens = [11, 6]
    q = rng.standard_normal((2, hq, d)).astype(np.float32)
    out = orc.paged_attention(q, kc, vc, [0, 1, 2], lens, 0.25, block_tables=tables, block_size=bs)
    for b in range(2):
        k = orc.gather_rows(kc, tables[b], lens[b], bs)
        v = orc.gather_rows(vc, tables[b], lens[b], bs)
        np.testing.assert_allclose(out[b:b + 1], _sdpa_ref(q[b:b + 1], k, v, 0.25, False),
                                   rtol=1e-5, atol=1e-5)


def test_zero_query_gives_mean_of_visible_values():
    # q = 0 -> uniform weights over exactly the visible keys: row i of a
    # sequence with Lq queries and Lk keys averages V[0 .. i + Lk - Lq].
    rng = np.random.default_rng(3)
    lq, lk, hkv, d = 4, 10, 2, 8
    v = rng.standard_normal((lk, hkv, d)).astype(np.float32)
    k = rng.standard_normal((lk, hkv, d)).astype(np.float32)
    q = np.zeros((lq, 4, d), np.float32)
    out = orc.paged_attention(q, k, v, [0, lq], [lk], 1.0, cu_seqlens_k=[0, lk])
    for i in range(lq):
        for h in range(4):
            np.testing.assert_allclose(out[i, h], v[: i + lk - lq + 1, h // 2].mean(0), atol=1e-6)


def test_single_key_returns_its_value_and_constant_v():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 2, 8)).astype(np.float32)
    k = rng.standard_normal((1, 1, 8)).astype(np.float32)
    v = rng.standard_normal((1, 1, 8)).astype(np.float32)
    out = orc.paged_attention(q, k, v, [0, 1], [1], 0.5, cu_seqlens_k=[0, 1])
    np.testing.assert_allclose(out[0], np.repeat(v[0], 2, 0), atol=1e-7)
    kk = rng.standard_normal((9, 1, 8)).astype(np.float32)
    vv = np.full((9, 1, 8), 1.25, np.float32)
    out = orc.paged_attention(q, kk, vv, [0, 1], [9], 0.5, cu_seqlens_k=[0, 9])
    np.testing.assert_allclose(out, 1.25, atol=1e-6)


def test_block_table_permutation_invariance_and_empty_context():
    rng = np.random.default_rng(5)
    bs, hkv, d = 4, 1, 8
    kc = rng.standard_normal((5, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((5, bs, hkv, d)).astype(np.float32)
    q = rng.standard_normal((2, 2, d)).astype(np.float32)
    t1 = np.array([[0, 1, 2], [3, 4, -1]], np.int32)
    perm = np.array([4, 2, 0, 1, 3])             # page p moves to perm[p]
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    t2 = np.where(t1 >= 0, perm[np.maximum(t1, 0)], -1).astype(np.int32)
    a = orc.paged_attention(q, kc, vc, [0, 1, 2], [10, 0], 0.4, block_tables=t1, block_size=bs)
    b = orc.paged_attention(q, kc2, vc2, [0, 1, 2], [10, 0], 0.4, block_tables=t2, block_size=bs)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a[1], 0.0)     # context 0 -> zeros


def test_bf16_helpers_round_trip_and_round_to_nearest_even():
    x = np.array([1.0, -2.5, 3.140625, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9], np.float32)
    bits = orc.f32_to_bf16(x)
    back = orc.bf16_to_f32(bits)
    np.testing.assert_array_equal(back[:3], x[:3])
    assert back[3] == 1.0                         # tie -> even mantissa
    assert back[4] == 1.0 + 2 ** -7               # above the tie -> rounds up
    t = torch.tensor(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, t)


# ---------------------------------------------------------------------------
# planted mistakes must be caught
# ---------------------------------------------------------------------------
def _pinning_checks_pass(mutation) -> bool:
    try:
        for name in GOLDEN_ATTN:
            c, out = _run_golden(name, mutation)
            np.testing.assert_allclose(out, c["expect"], rtol=1e-5, atol=1e-5)
        rng = np.random.default_rng(3)
        lq, lk = 4, 10
        v = rng.standard_normal((lk, 2, 8)).astype(np.float32)
        out = orc.paged_attention(np.zeros((lq, 4, 8), np.float32),
                                  rng.standard_normal((lk, 2, 8)).astype(np.float32), v,
                                  [0, lq], [lk], 1.0, cu_seqlens_k=[0, lk], _mutation=mutation)
        for i in range(lq):
            for h in range(4):
                np.testing.assert_allclose(out[i, h], v[: i + lk - lq + 1, h // 2].mean(0),
                                           atol=1e-6)
    except AssertionError:
        return False
    return True


def test_unmutated_oracle_passes_the_pinning_checks():
    assert _pinning_checks_pass(None)


@pytest.mark.parametrize("mutation", ["top_left", "strict", "gqa_mod", "no_scale"])
def test_planted_mistake_is_caught(mutation):
    assert not _pinning_checks_pass(mutation)
