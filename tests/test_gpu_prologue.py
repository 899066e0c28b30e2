"""GPU parity of the fused q/k RMSNorm + RoPE + KV-store prologue
(nvk_qk_norm_rope_store) against the oracle's restatement of qwen3.py:79-86
and attention.py:62-63.

Bar: the v rows reach the cache bit for bit, the cached k rows are bit for
bit the returned k, untouched cache rows keep their bytes.  q and k agree with
the oracle bit for bit except where the sum of squares / rsqrt rounding (a few
f32 ulps; the kernel's reduction order and v_rsq_f32 against the oracle's
pairwise mean and float64 rsqrt) moves a normed value across a bf16 rounding
boundary: such elements are at most 2 bf16 ulps of the normed value away,
carried through the rotation, i.e. |diff| <= 2^-6 * (|x1| + |x2|) of the
rotated pair, and fewer than 1 in 1000.
"""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from nanovllm_amd import attention_with_prologue, qk_norm_rope_store, rope_cos_sin_cache
from nanovllm_amd.layers.attention import Attention
from nanovllm_amd.utils.context import reset_context, set_context
from tests.gpu_utils import (assert_attn_close, assert_rotated_close, bits, from_bits,
                             oracle_decode, say)

pytestmark = pytest.mark.gpu

D = 128
MAX_POS = 40960
THETA = 1_000_000.0
EPS = 1e-6


@pytest.fixture(scope="module")
def cos_sin():
    return rope_cos_sin_cache(D, MAX_POS, THETA)          # CPU [MAX_POS, 1, D] f32


def _case(t, hq, hkv, nb, bs, seed, row_pad=0):
    g = torch.Generator().manual_seed(seed)
    r = hq + 2 * hkv
    qkv_full = (torch.randn(t, r * D + row_pad, generator=g) * 2.0).to(torch.bfloat16)
    qkv = qkv_full[:, :r * D]
    qw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, MAX_POS, (t,), generator=g, dtype=torch.int64)
    if t:
        pos[0] = 0
        pos[-1] = MAX_POS - 1
    kc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    if t > 2:
        perm[torch.randperm(t, generator=g)[: max(1, t // 20)]] = -1
        perm[1] = nb * bs + 5          # outside the cache: skipped
    return qkv_full, qkv, qw, kw, pos, kc, vc, perm


def _oracle(qkv, qw, kw, pos, kc, vc, slots, cos_sin, hq, hkv):
    kc_ref, vc_ref = bits(kc).copy(), bits(vc).copy()
    sl = slots.numpy().astype(np.int64)
    sl = np.where(sl >= kc.shape[0] * kc.shape[1], -1, sl)      # skipped like -1
    q, k, v = orc.qk_norm_rope_store(bits(qkv), pos.numpy(), bits(qw), bits(kw), EPS,
                                     cos_sin.reshape(MAX_POS, D).numpy(), hq, hkv, D,
                                     kc_ref, vc_ref, sl)
    return q, k, v, kc_ref, vc_ref


@pytest.mark.parametrize("t,hq,hkv", [(1, 16, 8), (7, 16, 8), (300, 16, 8), (4288, 16, 8),
                                      (513, 8, 4), (129, 4, 2)])
def test_prologue_matches_oracle(cos_sin, t, hq, hkv):
    say(f"prologue t={t} hq={hq} hkv={hkv}")
    nb, bs = 32, 256
    qkv_full, qkv, qw, kw, pos, kc, vc, slots = _case(t, hq, hkv, nb, bs, seed=t + hq)
    q_ref, k_ref, v_ref, kc_ref, vc_ref = _oracle(qkv, qw, kw, pos, kc, vc, slots, cos_sin, hq, hkv)
    dev = torch.device("cuda:0")
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    q, k, v = qk_norm_rope_store(pos.to(dev), qkv.to(dev), hq, hkv, D, qw.to(dev), kw.to(dev),
                                 EPS, cos_sin.to(dev), kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    assert_rotated_close(bits(q), q_ref, "q")
    assert_rotated_close(bits(k), k_ref, "k")
    assert np.array_equal(bits(v), v_ref)
    # caches: v rows bit-exact, k rows equal to the returned k, the rest untouched
    sl = slots.numpy().astype(np.int64)
    valid = (sl >= 0) & (sl < nb * bs)
    kc_got = bits(kc_d).reshape(nb * bs, hkv, D)
    vc_got = bits(vc_d).reshape(nb * bs, hkv, D)
    assert np.array_equal(vc_got, vc_ref.reshape(nb * bs, hkv, D))
    assert np.array_equal(kc_got[sl[valid]], bits(k)[valid])
    untouched = np.ones(nb * bs, dtype=bool)
    untouched[sl[valid]] = False
    assert np.array_equal(kc_got[untouched], bits(kc).reshape(nb * bs, hkv, D)[untouched])


def test_prologue_padded_rows_no_store_no_k(cos_sin):
    say("prologue padded qkv rows, no store, no k")
    t, hq, hkv = 65, 16, 8
    qkv_full, qkv, qw, kw, pos, kc, vc, slots = _case(t, hq, hkv, 4, 256, seed=3, row_pad=24)
    q_ref, _, _, _, _ = _oracle(qkv, qw, kw, pos, kc, vc, slots, cos_sin, hq, hkv)
    dev = torch.device("cuda:0")
    qkv_d = qkv_full.to(dev)[:, :(hq + 2 * hkv) * D]
    assert qkv_d.stride(0) == (hq + 2 * hkv) * D + 24
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    q, k, v = qk_norm_rope_store(pos.to(dev), qkv_d, hq, hkv, D, qw.to(dev), kw.to(dev), EPS,
                                 cos_sin.to(dev), return_k=False)
    torch.cuda.synchronize()
    assert k is None
    assert_rotated_close(bits(q), q_ref, "q")
    assert torch.equal(kc_d.cpu(), kc) and torch.equal(vc_d.cpu(), vc)


def test_prologue_empty_batch(cos_sin):
    dev = torch.device("cuda:0")
    qkv = torch.empty(0, 32 * D, dtype=torch.bfloat16, device=dev)
    w = torch.ones(D, dtype=torch.bfloat16, device=dev)
    q, k, v = qk_norm_rope_store(torch.empty(0, dtype=torch.int64, device=dev), qkv, 16, 8, D, w,
                                 w, EPS, cos_sin.to(dev))
    assert q.shape == (0, 16, D) and k.shape == (0, 8, D) and v.shape == (0, 8, D)


class _Norm:
    def __init__(self, w):
        self.weight, self.eps = w, EPS


class _Rope:
    def __init__(self, cache):
        self.cos_sin_cache = cache


def test_attention_with_prologue_decode_matches_oracle_chain(cos_sin):
    """Qwen3Attention.forward's prologue + Attention on a decode step: the
    fused path against oracle prologue -> oracle decode attention."""
    say("attention_with_prologue decode B=16")
    dev = torch.device("cuda:0")
    b, hq, hkv, bs, nb = 16, 16, 8, 256, 100
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(1, 1500, (b,), generator=g, dtype=torch.int32)
    pages = torch.randperm(nb, generator=g)
    w = (lens.max().item() + bs - 1) // bs
    bt = torch.full((b, w), -1, dtype=torch.int32)
    used = 0
    for i in range(b):
        n = (int(lens[i]) + bs - 1) // bs
        bt[i, :n] = pages[used:used + n]
        used += n
    assert used <= nb
    slots = torch.tensor([int(bt[i, (int(lens[i]) - 1) // bs]) * bs + (int(lens[i]) - 1) % bs
                          for i in range(b)], dtype=torch.int32)
    pos = (lens - 1).to(torch.int64)
    qkv = (torch.randn(b, (hq + 2 * hkv) * D, generator=g) * 2.0).to(torch.bfloat16)
    qw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    # oracle chain
    q_ref, _, _, kc_ref, vc_ref = _oracle(qkv, qw, kw, pos, kc, vc, slots, cos_sin, hq, hkv)
    scale = D ** -0.5
    ref = oracle_decode(from_bits(q_ref, "cpu"), from_bits(kc_ref, "cpu"), from_bits(vc_ref, "cpu"),
                        bt, lens, bs, scale)
    # fused path
    attn = Attention(hq, D, scale, hkv)
    attn.k_cache, attn.v_cache = kc.to(dev), vc.to(dev)
    set_context(False, slot_mapping=slots.to(dev), context_lens=lens.to(dev),
                block_tables=bt.to(dev))
    try:
        o = attention_with_prologue(attn, pos.to(dev), qkv.to(dev), _Norm(qw.to(dev)),
                                    _Norm(kw.to(dev)), _Rope(cos_sin.to(dev)))
        torch.cuda.synchronize()
    finally:
        reset_context()
    assert o.shape == (b, 1, hq, D)
    assert_attn_close(o.reshape(b, hq, D), ref, "decode after fused prologue")
    assert np.array_equal(bits(attn.v_cache), vc_ref)
