"""Pins the oracle's LM-head selection and sampler (CPU): the guide's LM-head
example, the exponential-race theorem by chi-square, closed forms, and
planted mistakes that must fail."""
import json
import os

import numpy as np
import pytest
from scipy import stats

from oracle import kv_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_last_token_rows_reproduce_guide_example():
    with open(os.path.join(GOLDEN, "guide_known_answers.json")) as f:
        ex = json.load(f)["lm_head_example"]
    x = np.arange(7 * 3).reshape(7, 3)
    rows = orc.last_token_rows(x, ex["cu_seqlens_q"])
    assert rows.tolist() == x[ex["last_indices"]].tolist()


def _race_counts(logits, temp, n_draws, seed, mutation=None):
    rng = np.random.default_rng(seed)
    v = logits.shape[0]
    rows = np.broadcast_to(logits, (n_draws, v))
    noise = rng.exponential(1.0, size=(n_draws, v)).astype(np.float32)
    tok = orc.sample_tokens(rows, np.full(n_draws, temp), noise, _mutation=mutation)
    return np.bincount(tok, minlength=v)


def _softmax(x, t):
    z = np.exp((x - x.max()) / t)
    return z / z.sum()


@pytest.mark.parametrize("temp", [1.0, 0.5, 2.0])
def test_sampler_draws_follow_softmax(temp):
    logits = np.linspace(-2.0, 1.5, 12).astype(np.float32)
    counts = _race_counts(logits, temp, 60000, seed=int(temp * 10))
    p = _softmax(logits.astype(np.float64), temp)
    assert stats.chisquare(counts, p * counts.sum()).pvalue > 1e-3


@pytest.mark.parametrize("mutation", ["noise_mul", "temp_mul"])
def test_sampler_planted_mistakes_fail_chisquare(mutation):
    logits = np.linspace(-2.0, 1.5, 12).astype(np.float32)
    counts = _race_counts(logits, 0.5, 60000, seed=3, mutation=mutation)
    p = _softmax(logits.astype(np.float64), 0.5)
    assert stats.chisquare(counts, p * counts.sum()).pvalue < 1e-6


def test_sampler_unit_noise_is_greedy_and_noise_clamped():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((64, 1000)).astype(np.float32)
    tok = orc.sample_tokens(logits, np.full(64, 0.7), np.ones((64, 1000), np.float32))
    assert np.array_equal(tok, logits.argmax(axis=1))
    # a zero draw is clamped to 1e-10 and wins its row unless the probability underflowed
    noise = np.ones((64, 1000), np.float32)
    noise[np.arange(64), 5] = 0.0
    assert np.all(orc.sample_tokens(logits, np.full(64, 1.0), noise) == 5)
    # bf16 bit patterns are read as bf16
    bits = orc.f32_to_bf16(logits)
    tb = orc.sample_tokens(bits, np.full(64, 1.0), np.ones((64, 1000), np.float32))
    assert np.array_equal(tb, orc.bf16_to_f32(bits).argmax(axis=1))
