"""GPU parity of the LM-head last-token gather (nvk_gather_last_tokens) and
the sampler (nvk_sample) against the oracle: with the caller's noise the
token must equal the reference formula's argmax (a different index only at a
near-tie of the two best scores, within 1e-5 relative); with the kernel's
Philox noise the draws must follow softmax(logits / T) (chi-square) and be
repeatable for a given seed and offset."""

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import kv_oracle as orc
from nanovllm_amd import _lib
from nanovllm_amd.layers.sampler import Sampler, compute_logits, last_token_hidden
from nanovllm_amd.utils.context import reset_context, set_context
from tests.gpu_utils import bits, say

pytestmark = pytest.mark.gpu


def _check_tokens(got, logits_np, temps, noise):
    ref = orc.sample_tokens(logits_np, temps, noise)
    bad = np.nonzero(got != ref)[0]
    if bad.size:
        x = orc.bf16_to_f32(logits_np) if logits_np.dtype == np.uint16 else logits_np
        x = x.astype(np.float64) / np.asarray(temps, np.float64)[:, None]
        s = x - np.log(np.maximum(noise.astype(np.float64), 1e-10))
        for r in bad:
            assert abs(s[r, got[r]] - s[r, ref[r]]) <= 1e-5 * max(1.0, abs(s[r, ref[r]])), \
                f"row {r}: {got[r]} vs {ref[r]} is not a near-tie"
    assert bad.size <= max(1, got.size // 100)


@pytest.mark.parametrize("b,v,dtype", [(64, 151936, torch.bfloat16), (5, 1000, torch.float32),
                                       (3, 7, torch.bfloat16), (512, 4099, torch.bfloat16),
                                       (64, 151936, torch.float16), (7, 300, torch.float16)])
def test_sampler_with_given_noise_matches_reference_formula(b, v, dtype):
    say(f"sampler given noise b={b} v={v} {dtype}")
    g = torch.Generator().manual_seed(b * 31 + v)
    logits = (torch.randn(b, v, generator=g) * 3.0).to(dtype)
    temps = (0.5 + torch.rand(b, generator=g)).to(torch.float32)
    noise = torch.empty(b, v).exponential_(1.0, generator=g)
    noise[0, 0] = 0.0                                      # clamped at 1e-10
    tok = Sampler()(logits.cuda(), temps.cuda(), noise=noise.cuda()).cpu().numpy()
    ln = bits(logits) if dtype == torch.bfloat16 else logits.numpy()
    _check_tokens(tok, ln, temps.numpy(), noise.numpy())
    assert tok.min() >= 0 and tok.max() < v


def test_sampler_padded_row_stride():
    say("sampler padded row stride")
    g = torch.Generator().manual_seed(2)
    full = (torch.randn(16, 1032, generator=g) * 2).to(torch.bfloat16).cuda()
    logits = full[:, :1000]
    temps = torch.full((16,), 0.8)
    noise = torch.empty(16, 1000).exponential_(1.0, generator=g)
    tok = Sampler()(logits, temps.cuda(), noise=noise.cuda()).cpu().numpy()
    _check_tokens(tok, bits(logits.cpu()), temps.numpy(), noise.numpy())


def test_sampler_whole_chunks_with_unaligned_noise_rows():
    """Logits rows 16-byte aligned (a padded view) over two whole 8192-token
    chunks plus 5 tokens, the caller's noise contiguous with an odd row length,
    so every other noise row starts 4 bytes past a 16-byte boundary."""
    say("sampler whole chunks, unaligned noise rows")
    g = torch.Generator().manual_seed(5)
    v = 2 * 8192 + 5
    full = (torch.randn(6, 16400, generator=g) * 2).to(torch.bfloat16).cuda()
    logits = full[:, :v]
    temps = (0.5 + torch.rand(6, generator=g)).to(torch.float32)
    noise = torch.empty(6, v).exponential_(1.0, generator=g)
    tok = Sampler()(logits, temps.cuda(), noise=noise.cuda()).cpu().numpy()
    _check_tokens(tok, bits(logits.cpu()), temps.numpy(), noise.numpy())


def _raw_sample(logits, temps, seed, offset):
    lib = _lib.load()
    out = torch.empty(logits.shape[0], dtype=torch.int64, device="cuda")
    wsb = lib.nvk_sample_workspace_size(logits.shape[0], logits.shape[1])
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    rc = lib.nvk_sample(logits.data_ptr(), logits.stride(0), logits.shape[0], logits.shape[1],
                        _lib.dtype_code(logits), temps.data_ptr(), None, 0, seed, offset,
                        out.data_ptr(), ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


def test_philox_draws_repeat_for_a_seed_and_offset():
    say("sampler philox determinism")
    logits = torch.zeros(256, 5000, dtype=torch.bfloat16, device="cuda")   # uniform
    temps = torch.ones(256, device="cuda")
    a = _raw_sample(logits, temps, 1234, 0)
    b = _raw_sample(logits, temps, 1234, 0)
    c = _raw_sample(logits, temps, 1234, 5000)
    d = _raw_sample(logits, temps, 99, 0)
    assert torch.equal(a, b)
    assert not torch.equal(a, c) and not torch.equal(a, d)
    # uniform logits: every token equally likely
    toks = torch.cat([_raw_sample(logits, temps, 7, k * 1251) for k in range(40)]).cpu().numpy()
    counts = np.bincount(toks // 500, minlength=10)       # 10 bins of 500 tokens
    assert stats.chisquare(counts).pvalue > 1e-4


@pytest.mark.parametrize("temp", [1.0, 0.5, 2.0])
def test_philox_draws_follow_softmax(temp):
    say(f"sampler philox distribution T={temp}")
    torch.manual_seed(11)
    v, rows, calls = 12, 4096, 15
    base = torch.linspace(-2.0, 1.5, v).to(torch.bfloat16)
    logits = base.repeat(rows, 1).cuda()
    temps = torch.full((rows,), temp, device="cuda")
    sampler = Sampler()
    toks = torch.cat([sampler(logits, temps) for _ in range(calls)]).cpu().numpy()
    counts = np.bincount(toks, minlength=v)
    x = base.float().numpy().astype(np.float64) / temp
    p = np.exp(x - x.max())
    p /= p.sum()
    assert stats.chisquare(counts, p * counts.sum()).pvalue > 1e-4


def test_draws_across_vocab_chunks_follow_softmax():
    # mass spread over five 8192-token chunks of the row (chunk edges included):
    # the chunk is drawn by its mass, then the token inside it
    say("sampler draws across chunks")
    v, rows, calls = 40000, 4096, 10
    hot = [5, 8191, 8192, 12000, 16383, 20000, 24576, 30000, 35000, 39999]
    vals = torch.linspace(-1.0, 1.2, len(hot))
    base = torch.full((v,), -40.0)
    base[hot] = vals
    logits = base.to(torch.bfloat16).repeat(rows, 1).cuda()
    temps = torch.ones(rows, device="cuda")
    toks = torch.cat([_raw_sample(logits, temps, 5, k * 10007) for k in range(calls)]).cpu().numpy()
    assert np.isin(toks, hot).all()
    counts = np.array([(toks == h).sum() for h in hot])
    x = base.to(torch.bfloat16).float().numpy()[hot].astype(np.float64)
    p = np.exp(x - x.max())
    p /= p.sum()
    assert stats.chisquare(counts, p * counts.sum()).pvalue > 1e-4


def test_draws_over_more_than_128_wave_chunks():
    """A 300000-token vocabulary (147 wave chunks of 2048 logits: the choose
    kernel's registers hold 128, the rest go through its loop), mass on
    tokens on both sides of the 128-chunk edge (262144) and at the last one."""
    say("sampler draws past 128 wave chunks")
    v, rows, calls = 300000, 1024, 10
    hot = [5, 100000, 262143, 262144, 270000, 299999]
    vals = torch.linspace(-0.8, 0.9, len(hot))
    base = torch.full((v,), -40.0)
    base[hot] = vals
    logits = base.to(torch.bfloat16).repeat(rows, 1).cuda()
    temps = torch.ones(rows, device="cuda")
    toks = torch.cat([_raw_sample(logits, temps, 13, k * 7919) for k in range(calls)]).cpu().numpy()
    assert np.isin(toks, hot).all()
    counts = np.array([(toks == h).sum() for h in hot])
    x = base.to(torch.bfloat16).float().numpy()[hot].astype(np.float64)
    p = np.exp(x - x.max())
    p /= p.sum()
    assert stats.chisquare(counts, p * counts.sum()).pvalue > 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_draws_inside_one_chunk_follow_softmax(dtype):
    """Mass over every token of one 8192-token chunk, shuffled so that each
    thread and pass of the chunk's workgroup holds some of it: the chunk's
    own inverse-CDF draw follows the softmax (16 bins of 512 tokens), for
    bf16 and fp16 logits."""
    say(f"sampler draws inside one chunk {dtype}")
    v, rows, calls, temp = 8192, 4096, 10, 1.3
    perm = torch.randperm(v, generator=torch.Generator().manual_seed(3))
    base = torch.linspace(-3.0, 3.0, v)[perm].to(dtype)
    logits = base.repeat(rows, 1).cuda()
    temps = torch.full((rows,), temp, device="cuda")
    toks = torch.cat([_raw_sample(logits, temps, 21, k * 3001) for k in range(calls)]).cpu().numpy()
    x = base.float().numpy().astype(np.float64) / temp
    p = np.exp(x - x.max())
    p /= p.sum()
    counts = np.bincount(toks // 512, minlength=16)
    expected = np.bincount(np.arange(v) // 512, weights=p, minlength=16) * toks.size
    assert stats.chisquare(counts, expected).pvalue > 1e-4


def test_draws_over_a_full_vocabulary_follow_softmax():
    """Qwen3-sized rows (151936 logits: 19 workgroups and 75 wave chunks of
    2048 logits per row, the last ones partial), 10240 draws: the counts per
    2048-token bin match the bins' softmax mass (chi-square: a dropped or
    doubled bin fails it), the draws' summed log-probability matches minus
    the rows' entropy (z-test: tokens mapped to the wrong index inside a bin
    fail it), and the randomised probability integral transform of each draw,
    F(token - 1) + v p(token) with v uniform, is uniform on (0, 1) (KS test)."""
    say("sampler full-vocabulary draws")
    v, rows, calls, temp = 151936, 512, 20, 1.0
    gen = torch.Generator(device="cuda").manual_seed(31)
    logits = (torch.randn(rows, v, generator=gen, device="cuda") * 2).to(torch.bfloat16)
    temps = torch.full((rows,), temp, device="cuda")
    toks = torch.stack([_raw_sample(logits, temps, 41, k * 40000) for k in range(calls)], 1)
    p = torch.softmax(logits.double() / temp, dim=-1)
    nb = (v + 2047) // 2048
    bin_of = torch.arange(v, device="cuda") // 2048
    mass = torch.zeros(nb, dtype=torch.float64, device="cuda").index_add_(0, bin_of, p.sum(0))
    counts = torch.bincount(bin_of[toks.flatten()], minlength=nb)
    assert stats.chisquare(counts.cpu().numpy(), (mass * calls).cpu().numpy()).pvalue > 1e-4
    lp = torch.log(p.clamp_min(1e-300))
    ent = -(p * lp).sum(-1)
    var = (p * lp * lp).sum(-1) - ent * ent
    z = (lp.gather(1, toks).sum() + ent.sum() * calls) / torch.sqrt(var.sum() * calls)
    assert abs(z.item()) < 5, z.item()
    before = (torch.cumsum(p, dim=-1) - p).gather(1, toks)
    vv = torch.rand(toks.shape, generator=torch.Generator(device="cuda").manual_seed(5),
                    device="cuda", dtype=torch.float64)
    pit = (before + vv * p.gather(1, toks)).flatten().cpu().numpy()
    assert stats.kstest(pit, "uniform").pvalue > 1e-4


def test_draws_uniform_over_a_partial_last_chunk():
    say("sampler partial last chunk")
    v = 8197                                                  # 8192 + 5
    logits = torch.zeros(2048, v, dtype=torch.float32, device="cuda")
    temps = torch.ones(2048, device="cuda")
    toks = torch.cat([_raw_sample(logits, temps, 9, k * 4099) for k in range(20)]).cpu().numpy()
    assert toks.min() >= 0 and toks.max() < v
    counts = np.bincount(toks * 11 // v, minlength=11)       # 11 equal bins
    expected = np.bincount(np.arange(v) * 11 // v, minlength=11) / v * toks.size
    assert stats.chisquare(counts, expected).pvalue > 1e-4
    # the last chunk's five tokens are drawn at their share
    assert abs((toks >= 8192).mean() - 5 / v) < 5 * np.sqrt(5 / v / toks.size)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rows_without_finite_logits_give_token_zero(dtype):
    """Rows of -inf give token 0; NaN and +inf logits carry no mass (row 3:
    its one finite logit is drawn)."""
    logits = torch.full((4, 100), float("-inf"), device="cuda", dtype=dtype)
    logits[1, 37] = 0.0
    logits[3, 5] = float("nan")
    logits[3, 50] = float("inf")
    logits[3, 60] = 0.5
    for seed in (1, 2, 3):
        out = _raw_sample(logits, torch.ones(4, device="cuda"), seed, 0).cpu().tolist()
        assert out == [0, 37, 0, 60]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_last_token_gather_and_lm_head(dtype):
    say(f"lm head gather {dtype}")
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 1024, generator=g).to(dtype).cuda()
    w = torch.randn(300, 1024, generator=g).to(dtype).cuda()
    cu = torch.tensor([0, 2, 3, 7], dtype=torch.int32, device="cuda")
    rows = last_token_hidden(x, cu)
    assert torch.equal(rows.cpu(), x.cpu()[[1, 2, 6]])
    set_context(True, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=4, max_seqlen_k=4)
    try:
        logits = compute_logits(x, w)
    finally:
        reset_context()
    torch.testing.assert_close(logits.float().cpu(),
                               (x.float().cpu()[[1, 2, 6]] @ w.float().cpu().T), atol=0.5, rtol=2e-2)
    set_context(False)
    try:
        assert compute_logits(x, w).shape == (7, 300)     # decode: every row
    finally:
        reset_context()
