"""The attention prologue in float16, the element type the reference runs in
when hf_config.dtype is float16 (model_runner.py:29 sets torch's default
dtype from it, so the qkv rows, the norm weights and the caches all are).

* nvk_qk_norm_rope_store against the oracle's f16 restatement of
  qwen3.py:79-86 + attention.py:62-63 (pinned against transformers' Qwen3
  RMSNorm and rotary in float16, tests/test_prologue_oracle.py): v rows and
  cached k rows bit-exact; q and k bit-exact but for < 0.1 % of elements
  within 2 f16 ulps of the rotated pair (the sum-of-squares / rsqrt rounding
  of the kernel against the oracle's).
* nvk_paged_decode_prologue against the two calls it replaces, bit for bit
  (outputs and caches), and the decode output against the oracle within
  2e-2 abs / 1e-2 rel.
* Mixed element types are rejected before any launch.
"""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, assert_rotated_close, bits, oracle_decode, say
from oracle import kv_oracle as orc
from nanovllm_amd import (_lib, paged_decode, paged_decode_with_prologue, qk_norm_rope_store,
                          rope_cos_sin_cache)

pytestmark = pytest.mark.gpu

D = 128
MAX_POS = 40960
EPS = 1e-6
F16 = torch.float16


@pytest.fixture(scope="module")
def cos_sin():
    return rope_cos_sin_cache(D, MAX_POS, 1_000_000.0)     # CPU [MAX_POS, 1, D] f32


def _prologue_case(t, hq, hkv, nb, bs, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(t, (hq + 2 * hkv) * D, generator=g) * 2.0).to(F16)
    qw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(F16)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(F16)
    pos = torch.randint(0, MAX_POS, (t,), generator=g, dtype=torch.int64)
    kc = torch.randn(nb, bs, hkv, D, generator=g).to(F16)
    vc = torch.randn(nb, bs, hkv, D, generator=g).to(F16)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    if t > 2:
        slots[torch.randperm(t, generator=g)[: max(1, t // 20)]] = -1
    return qkv, qw, kw, pos, kc, vc, slots


@pytest.mark.parametrize("t,hq,hkv", [(7, 16, 8), (300, 16, 8), (4288, 16, 8), (129, 8, 4)])
def test_prologue_f16_matches_oracle(cos_sin, t, hq, hkv):
    say(f"f16 prologue t={t} hq={hq} hkv={hkv}")
    nb, bs = 24, 256
    qkv, qw, kw, pos, kc, vc, slots = _prologue_case(t, hq, hkv, nb, bs, seed=50 + t)
    kc_ref, vc_ref = bits(kc).copy(), bits(vc).copy()
    q_ref, k_ref, v_ref = orc.qk_norm_rope_store(
        bits(qkv), pos.numpy(), bits(qw), bits(kw), EPS, cos_sin.reshape(MAX_POS, D).numpy(),
        hq, hkv, D, kc_ref, vc_ref, slots.numpy().astype(np.int64), elt="f16")
    dev = torch.device("cuda:0")
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    q, k, v = qk_norm_rope_store(pos.to(dev), qkv.to(dev), hq, hkv, D, qw.to(dev), kw.to(dev),
                                 EPS, cos_sin.to(dev), kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    assert q.dtype == F16 and k.dtype == F16
    assert_rotated_close(bits(q), q_ref, "f16 q", elt="f16")
    assert_rotated_close(bits(k), k_ref, "f16 k", elt="f16")
    assert np.array_equal(bits(v), v_ref)
    sl = slots.numpy().astype(np.int64)
    valid = sl >= 0
    assert np.array_equal(bits(vc_d).reshape(nb * bs, hkv, D), vc_ref.reshape(nb * bs, hkv, D))
    assert np.array_equal(bits(kc_d).reshape(nb * bs, hkv, D)[sl[valid]], bits(k)[valid])


@pytest.mark.parametrize("hq,hkv,bs", [(16, 8, 256), (16, 2, 64), (16, 16, 16)])
def test_fused_decode_prologue_f16_equals_two_calls(cos_sin, hq, hkv, bs):
    lens = [1, 31, 32, 33, 255, 256, 257, 700, 2048, 3000]
    g = torch.Generator().manual_seed(60 + hkv + bs)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 3
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32)
    nxt = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[nxt:nxt + p].to(torch.int32)
        nxt += p
    slots = torch.tensor([int(bt[i, (n - 1) // bs]) * bs + (n - 1) % bs
                          for i, n in enumerate(lens)], dtype=torch.int32)
    pos = torch.tensor([n - 1 for n in lens], dtype=torch.int64)
    qkv = (torch.randn(len(lens), (hq + 2 * hkv) * D, generator=g) * 2.0).to(F16)
    qw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(F16)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(F16)
    kc = torch.randn(nb, bs, hkv, D, generator=g).to(F16)
    vc = torch.randn(nb, bs, hkv, D, generator=g).to(F16)
    d = lambda x: x.cuda()
    cs = cos_sin.cuda()
    lens_t = torch.tensor(lens, dtype=torch.int32)
    kc1, vc1, kc2, vc2 = d(kc), d(vc), d(kc), d(vc)
    say(f"f16 decode prologue two calls G={hq // hkv} page {bs}")
    q, _, _ = qk_norm_rope_store(d(pos), d(qkv), hq, hkv, D, d(qw), d(kw), EPS, cs, kc1, vc1,
                                 d(slots), return_k=False)
    ref = paged_decode(q, kc1, vc1, d(lens_t), d(bt), D ** -0.5)
    torch.cuda.synchronize()
    say(f"f16 decode prologue fused G={hq // hkv} page {bs}")
    out = paged_decode_with_prologue(d(pos), d(qkv), hq, hkv, D, d(qw), d(kw), EPS, cs, kc2, vc2,
                                     d(slots), d(lens_t), d(bt), D ** -0.5)
    torch.cuda.synchronize()
    assert out.dtype == F16
    assert torch.equal(out, ref) and torch.equal(kc2, kc1) and torch.equal(vc2, vc1)
    exp = oracle_decode(q.cpu(), kc1.cpu(), vc1.cpu(), bt, lens_t, bs, D ** -0.5)
    assert_attn_close(out, exp, f"f16 fused decode G={hq // hkv}")


def test_prologue_mixed_dtypes_rejected(cos_sin):
    qkv, qw, kw, pos, kc, vc, slots = _prologue_case(4, 16, 8, 2, 256, seed=70)
    d = lambda x: x.cuda()
    with pytest.raises(_lib.NvkError, match="share one dtype"):
        qk_norm_rope_store(d(pos), d(qkv), 16, 8, D, d(qw.to(torch.bfloat16)), d(kw), EPS,
                           d(cos_sin))
    with pytest.raises(_lib.NvkError, match="share one dtype"):
        qk_norm_rope_store(d(pos), d(qkv), 16, 8, D, d(qw), d(kw), EPS, d(cos_sin),
                           d(kc.to(torch.bfloat16)), d(vc.to(torch.bfloat16)), d(slots))
