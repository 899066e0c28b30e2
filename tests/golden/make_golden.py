"""Writes the committed golden fixtures of the KV-cache path.

Run from the repo root:  python tests/golden/make_golden.py

Two kinds of data, neither produced by the oracle under test:

* guide_known_answers.json — worked answers transcribed from the reference's
  study guide (master_nano-vllm-v2.md): the slot formula example (:2766-2776),
  the tiny store example (:2830-2852), the store test matrix (:2895-2921), the
  LM-head index example (:1222) and the decode minimal / shared-prefix cases
  (:4345-4391).
* store_small.npz / attn_small.npz — seeded small cases whose expected outputs
  come from the scalar brute force below: per-token copies for the store, and
  per-(row, head, key) Python-float loops with math.exp for attention.  They
  pin the numpy oracle and are inputs of the GPU parity tests.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern (round to nearest even), no NaNs expected."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# guide known answers
# ---------------------------------------------------------------------------
KNOWN = {
    "slot_example": {"block_size": 4, "block_table": [3, 0, 5], "positions": [2, 3, 4, 7, 8, 9],
                     "slots": [14, 15, 0, 3, 20, 21]},
    "store_tiny": {"N": 3, "Hkv": 1, "D": 2, "block_size": 4, "num_blocks": 2,
                   "slots": [5, 0, -1], "key": [[10, 11], [20, 21], [30, 31]],
                   "fill": -999,
                   # token0 -> [block1, offset1]; token1 -> [block0, offset0]; token2 skipped
                   "changed": [[1, 1, 0, 0, 10], [1, 1, 0, 1, 11], [0, 0, 0, 0, 20],
                               [0, 0, 0, 1, 21]]},
    "store_matrix": {"slots": [[0], [3, 4], [513, 12, 1024, -1, 255, 256]], "N": [1, 3, 17],
                     "hkv_d": [[1, 2], [8, 128], [4, 64]], "block_size": 256},
    "lm_head_example": {"query_lens": [2, 1, 4], "cu_seqlens_q": [0, 2, 3, 7],
                        "last_indices": [1, 2, 6]},
    "decode_minimal": {"context_lens": [5], "tables": [[2, 0]], "num_blocks": 4, "hq": 1,
                       "hkv": 1, "d": 128, "block_size": 4},
    "decode_shared_prefix": {"context_lens": [5, 5], "tables": [[2, 0], [2, 3]], "num_blocks": 4,
                             "hq": 1, "hkv": 1, "d": 128, "block_size": 4},
}


# ---------------------------------------------------------------------------
# scalar brute force
# ---------------------------------------------------------------------------
def store_brute(key, value, k_cache, v_cache, slots, block_size):
    """Per-token copy, the guide's store_ref loop (master_nano-vllm-v2.md:2834-2843)."""
    for t in range(key.shape[0]):
        s = int(slots[t])
        if s == -1:
            continue
        k_cache[s // block_size, s % block_size] = key[t]
        v_cache[s // block_size, s % block_size] = value[t]


def attn_brute(q, k_cache, v_cache, tables, lens_q, lens_k, block_size, scale):
    """q [Tq,Hq,D] float32 values, caches [NB,bs,Hkv,D]; returns float64 [Tq,Hq,D]."""
    tq, hq, d = q.shape
    hkv = k_cache.shape[2]
    g = hq // hkv
    out = np.zeros((tq, hq, d), dtype=np.float64)
    row0 = 0
    for s, (lq, lk) in enumerate(zip(lens_q, lens_k)):
        for i in range(lq):
            for h in range(hq):
                kvh = h // g
                qv = [float(x) for x in q[row0 + i, h]]
                scores, vals = [], []
                for j in range(lk):
                    if j > i + lk - lq:
                        continue
                    page = tables[s][j // block_size]
                    kv = k_cache[page, j % block_size, kvh]
                    dot = 0.0
                    for e in range(d):
                        dot += qv[e] * float(kv[e])
                    scores.append(dot * scale)
                    vals.append(v_cache[page, j % block_size, kvh])
                if not scores:
                    continue
                m = max(scores)
                ws = [math.exp(x - m) for x in scores]
                tot = sum(ws)
                for e in range(d):
                    out[row0 + i, h, e] = sum(w * float(v[e]) for w, v in zip(ws, vals)) / tot
        row0 += lq
    return out


def make_store_cases(rng):
    cases = {}
    for ci, (slots, n, (hkv, d)) in enumerate([
        ([0], 1, (1, 2)),
        ([3, 4], 3, (8, 128)),
        ([513, 12, 1024, -1, 255, 256], 17, (4, 64)),
    ]):
        n = max(n, len(slots))
        s = list(slots)
        extra = [x for x in rng.permutation(5 * 256) if x not in s][: n - len(s)]
        s = np.array(s + list(extra), dtype=np.int32)
        key = bf16_round(rng.standard_normal((n, hkv, d)).astype(np.float32))
        value = bf16_round(rng.standard_normal((n, hkv, d)).astype(np.float32))
        kc = np.full((5, 256, hkv, d), 0x7F7F, dtype=np.uint16)  # recognisable fill
        vc = np.full((5, 256, hkv, d), 0x3F3F, dtype=np.uint16)
        ek, ev = kc.copy(), vc.copy()
        store_brute(key, value, ek, ev, s, 256)
        cases[f"c{ci}_key"] = key
        cases[f"c{ci}_value"] = value
        cases[f"c{ci}_slots"] = s
        cases[f"c{ci}_k_cache"] = kc
        cases[f"c{ci}_v_cache"] = vc
        cases[f"c{ci}_expect_k"] = ek
        cases[f"c{ci}_expect_v"] = ev
    return cases


def make_attn_case(rng, name, hq, hkv, d, block_size, num_blocks, tables, lens_q, lens_k):
    tq = sum(lens_q)
    q = bf16_round(rng.standard_normal((tq, hq, d)).astype(np.float32))
    kc = bf16_round(rng.standard_normal((num_blocks, block_size, hkv, d)).astype(np.float32))
    vc = bf16_round(rng.standard_normal((num_blocks, block_size, hkv, d)).astype(np.float32))
    # rows no sequence reads are zero (keeps the fixture small once compressed)
    used = np.zeros((num_blocks, block_size), dtype=bool)
    for t, lk in zip(tables, lens_k):
        for j in range(lk):
            used[t[j // block_size], j % block_size] = True
    kc[~used] = 0
    vc[~used] = 0
    scale = d ** -0.5
    expect = attn_brute(bf16_value(q), bf16_value(kc), bf16_value(vc), tables, lens_q, lens_k,
                        block_size, scale)
    width = max(len(t) for t in tables)
    bt = np.full((len(tables), width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    return {f"{name}_q": q, f"{name}_k_cache": kc, f"{name}_v_cache": vc,
            f"{name}_block_tables": bt, f"{name}_lens_q": np.array(lens_q, dtype=np.int32),
            f"{name}_lens_k": np.array(lens_k, dtype=np.int32),
            f"{name}_meta": np.array([hq, hkv, d, block_size], dtype=np.int32),
            f"{name}_expect": expect.astype(np.float32)}


def main():
    rng = np.random.default_rng(20260101)
    with open(os.path.join(HERE, "guide_known_answers.json"), "w") as f:
        json.dump(KNOWN, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "store_small.npz"), **make_store_cases(rng))
    attn = {}
    dm = KNOWN["decode_minimal"]
    attn.update(make_attn_case(rng, "decode_minimal", 1, 1, 128, 4, 4, dm["tables"], [1],
                               dm["context_lens"]))
    ds = KNOWN["decode_shared_prefix"]
    attn.update(make_attn_case(rng, "decode_shared", 1, 1, 128, 4, 4, ds["tables"], [1, 1],
                               ds["context_lens"]))
    # GQA decode (G=2), reversed and random tables across a 256-token page edge
    attn.update(make_attn_case(rng, "decode_gqa", 4, 2, 128, 256, 6, [[5, 4], [1], [3, 0, 2]],
                               [1, 1, 1], [257, 1, 513]))
    # prefill with a cached prefix (Lk > Lq) and one without (Lk == Lq), bs=4
    attn.update(make_attn_case(rng, "prefill_prefix", 4, 2, 128, 4, 8, [[6, 1, 3], [0, 5]],
                               [3, 6], [9, 6]))
    # prefill at the real page size (G=4): 40 new tokens after a 256-token prefix
    attn.update(make_attn_case(rng, "prefill_page", 8, 2, 128, 256, 3, [[2, 0]], [40], [296]))
    np.savez_compressed(os.path.join(HERE, "attn_small.npz"), **attn)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
