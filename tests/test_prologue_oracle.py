"""Pins the oracle's attention prologue (RMSNorm, RoPE, their composition with
the KV store) without the reference: against transformers' Qwen3 routines
(independent implementations of the same definitions), closed forms and
invariants, and planted mistakes that must fail.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from nanovllm_amd.layers.prologue import rope_cos_sin_cache

D = 128
MAX_POS = 40960
THETA = 1_000_000.0     # Qwen3-0.6B rope_theta


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _weight(seed):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)


@pytest.fixture(scope="module")
def cos_sin():
    return rope_cos_sin_cache(D, MAX_POS, THETA).reshape(MAX_POS, D).numpy()


def _transformers():
    return pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


# --------------------------------------------------------------------------- RMSNorm
def test_rms_norm_matches_transformers_qwen3_rmsnorm():
    m = _transformers()
    x = _rand_bf16((257, 4, D), 0, scale=3.0)
    w = _weight(1)
    norm = m.Qwen3RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w.float())
        norm = norm.to(torch.bfloat16)
        ref = _bits(norm(x))
    got = orc.rms_norm(_bits(x), _bits(w), 1e-6)
    same = got == ref
    # mean / rsqrt rounding may move the normed value across a bf16 rounding
    # boundary (one bf16 ulp), which the weight product carries to at most two
    assert same.mean() > 0.999
    diff = np.abs(orc.bf16_to_f32(got) - orc.bf16_to_f32(ref))
    assert np.all(diff <= np.abs(orc.bf16_to_f32(ref)) * 2.0 ** -6)


def test_rms_norm_closed_forms():
    x = _bits(_rand_bf16((64, D), 2))
    one = _bits(torch.ones(D, dtype=torch.bfloat16))
    # scaling a row by a power of two is exact in bf16 and cancels exactly (eps = 0)
    x2 = orc.f32_to_bf16(orc.bf16_to_f32(x) * 4.0)
    assert np.array_equal(orc.rms_norm(x2, one, 0.0), orc.rms_norm(x, one, 0.0))
    # sign symmetry
    xn = x ^ np.uint16(0x8000)
    assert np.array_equal(orc.rms_norm(xn, one, 0.0), orc.rms_norm(x, one, 0.0) ^ np.uint16(0x8000))
    # unit weights: each output row has mean square 1 (up to bf16 rounding)
    y = orc.bf16_to_f32(orc.rms_norm(x, one, 1e-6))
    np.testing.assert_allclose(np.mean(y * y, axis=-1), 1.0, rtol=1e-2)
    # weights scale the output elementwise: weight 2 doubles every value exactly
    two = _bits(torch.full((D,), 2.0, dtype=torch.bfloat16))
    assert np.array_equal(orc.bf16_to_f32(orc.rms_norm(x, two, 1e-6)),
                          2 * orc.bf16_to_f32(orc.rms_norm(x, one, 1e-6)))


def test_rms_norm_planted_sum_instead_of_mean_fails():
    x = _bits(_rand_bf16((16, D), 3))
    one = _bits(torch.ones(D, dtype=torch.bfloat16))
    y = orc.bf16_to_f32(orc.rms_norm(x, one, 1e-6, _mutation="sum"))
    assert not np.allclose(np.mean(y * y, axis=-1), 1.0, rtol=1e-2)


# --------------------------------------------------------------------------- RoPE
def test_cos_sin_cache_matches_transformers_rotary_embedding(cos_sin):
    m = _transformers()
    from transformers import Qwen3Config
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8,
                      head_dim=D, rope_theta=THETA, max_position_embeddings=MAX_POS)
    rot = m.Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 2, 17, 4095, 12345, MAX_POS - 1]])
    cos, sin = rot(torch.zeros(1, dtype=torch.float32), pos)
    np.testing.assert_array_equal(cos[0, :, :D // 2].numpy(), cos_sin[pos[0], :D // 2])
    np.testing.assert_array_equal(sin[0, :, :D // 2].numpy(), cos_sin[pos[0], D // 2:])


def _rope_transformers(x_bf16, positions, cos_sin):
    m = _transformers()
    cs = torch.from_numpy(cos_sin[positions])
    c, s = cs[:, :D // 2], cs[:, D // 2:]
    cos = torch.cat((c, c), -1)
    sin = torch.cat((s, s), -1)
    xf = x_bf16.float()
    q_embed, _ = m.apply_rotary_pos_emb(xf, xf, cos, sin, unsqueeze_dim=1)
    return _bits(q_embed.to(torch.bfloat16))


def _rope_oracle(x_bits, positions, cos_sin, mutation=None):
    cs = cos_sin[positions]
    return orc.apply_rotary_emb(x_bits, cs[:, None, :D // 2], cs[:, None, D // 2:],
                                _mutation=mutation)


def test_rope_matches_transformers_bit_for_bit(cos_sin):
    x = _rand_bf16((300, 3, D), 4)
    pos = np.random.default_rng(5).integers(0, MAX_POS, 300)
    assert np.array_equal(_rope_oracle(_bits(x), pos, cos_sin), _rope_transformers(x, pos, cos_sin))


def test_rope_identity_at_position_zero(cos_sin):
    x = _bits(_rand_bf16((8, 2, D), 6))
    assert np.array_equal(_rope_oracle(x, np.zeros(8, dtype=np.int64), cos_sin), x)


def test_rope_relative_position_and_pair_norm(cos_sin):
    rng = np.random.default_rng(7)
    q = _bits(_rand_bf16((1, 1, D), 8))
    k = _bits(_rand_bf16((1, 1, D), 9))
    nq = np.linalg.norm(orc.bf16_to_f32(q))
    nk = np.linalg.norm(orc.bf16_to_f32(k))
    for _ in range(20):
        m, n, s = (int(v) for v in rng.integers(0, 8000, 3))
        a = orc.bf16_to_f32(_rope_oracle(q, np.array([m]), cos_sin)).ravel()
        b = orc.bf16_to_f32(_rope_oracle(k, np.array([n]), cos_sin)).ravel()
        c = orc.bf16_to_f32(_rope_oracle(q, np.array([m + s]), cos_sin)).ravel()
        d = orc.bf16_to_f32(_rope_oracle(k, np.array([n + s]), cos_sin)).ravel()
        assert abs(a @ b - c @ d) <= 2e-2 * nq * nk
        assert abs(np.linalg.norm(a) - nq) <= 1e-2 * nq


@pytest.mark.parametrize("mutation", ["swap", "sign", "interleaved"])
def test_rope_planted_mistakes_fail(cos_sin, mutation):
    x = _rand_bf16((64, 2, D), 10)
    pos = np.random.default_rng(11).integers(1, 4096, 64)
    bad = _rope_oracle(_bits(x), pos, cos_sin, mutation)
    ident = _rope_oracle(_bits(x), np.zeros(64, dtype=np.int64), cos_sin, mutation)
    caught = (not np.array_equal(bad, _rope_transformers(x, pos, cos_sin))
              or not np.array_equal(ident, _bits(x)))
    assert caught


# --------------------------------------------------------------------------- composition
def test_qk_norm_rope_store_matches_per_token_loop(cos_sin):
    hq, hkv, t = 4, 2, 9
    qkv = _bits(_rand_bf16((t, (hq + 2 * hkv) * D), 12, scale=2.0))
    qw, kw = _bits(_weight(13)), _bits(_weight(14))
    pos = np.array([5, 6, 7, 0, 1, 2, 3, 100, 39999])
    nb, bs = 2, 8
    kc = np.zeros((nb, bs, hkv, D), dtype=np.uint16)
    vc = np.zeros_like(kc)
    slots = np.array([3, -1, 15, 0, 7, -1, 9, 1, 2])
    q, k, v = orc.qk_norm_rope_store(qkv, pos, qw, kw, 1e-6, cos_sin, hq, hkv, D, kc, vc, slots)
    assert q.shape == (t, hq, D) and k.shape == (t, hkv, D) and v.shape == (t, hkv, D)
    exp_kc = np.zeros_like(kc).reshape(nb * bs, hkv, D)
    exp_vc = np.zeros_like(exp_kc)
    for i in range(t):
        row = qkv[i].reshape(hq + 2 * hkv, D)
        cs = cos_sin[pos[i]]
        for h in range(hq + hkv):
            w = qw if h < hq else kw
            n = orc.rms_norm(row[h][None], w, 1e-6)
            r = orc.apply_rotary_emb(n, cs[None, :D // 2], cs[None, D // 2:])[0]
            got = q[i, h] if h < hq else k[i, h - hq]
            assert np.array_equal(got, r), (i, h)
        assert np.array_equal(v[i], row[hq + hkv:])
        if slots[i] >= 0:
            exp_kc[slots[i]] = k[i]
            exp_vc[slots[i]] = row[hq + hkv:]
    assert np.array_equal(kc.reshape(nb * bs, hkv, D), exp_kc)
    assert np.array_equal(vc.reshape(nb * bs, hkv, D), exp_vc)


# --------------------------------------------------------------------------- f16
# The reference runs the model in hf_config.dtype (model_runner.py:29), so the
# prologue also exists for float16: the same operations with every rounding
# to T done to float16.
def _rand_f16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.float16)


def test_rms_norm_f16_matches_transformers_qwen3_rmsnorm():
    m = _transformers()
    x = _rand_f16((257, 4, D), 20, scale=3.0)
    w = _weight(21).to(torch.float16)
    norm = m.Qwen3RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w.float())
        norm = norm.to(torch.float16)
        ref = _bits(norm(x))
    got = orc.rms_norm(_bits(x), _bits(w), 1e-6, elt="f16")
    same = got == ref
    assert same.mean() > 0.999
    diff = np.abs(orc.f16_to_f32(got) - orc.f16_to_f32(ref))
    assert np.all(diff <= np.abs(orc.f16_to_f32(ref)) * 2.0 ** -9)
    # rounding to bf16 instead of f16 (a planted mistake) is far from it
    wrong = orc.rms_norm(_bits(x), _bits(w.to(torch.bfloat16)), 1e-6)
    assert (orc.bf16_to_f32(wrong) != orc.f16_to_f32(ref)).mean() > 0.5


def test_rms_norm_f16_closed_forms():
    x = _bits(_rand_f16((64, D), 22))
    one = _bits(torch.ones(D, dtype=torch.float16))
    x2 = orc.f32_to_f16(orc.f16_to_f32(x) * 4.0)          # exact in f16
    assert np.array_equal(orc.rms_norm(x2, one, 0.0, elt="f16"),
                          orc.rms_norm(x, one, 0.0, elt="f16"))
    xn = x ^ np.uint16(0x8000)
    assert np.array_equal(orc.rms_norm(xn, one, 0.0, elt="f16"),
                          orc.rms_norm(x, one, 0.0, elt="f16") ^ np.uint16(0x8000))
    y = orc.f16_to_f32(orc.rms_norm(x, one, 1e-6, elt="f16"))
    np.testing.assert_allclose(np.mean(y * y, axis=-1), 1.0, rtol=2e-3)


def test_rope_f16_matches_transformers_bit_for_bit(cos_sin):
    m = _transformers()
    x = _rand_f16((300, 3, D), 23)
    pos = np.random.default_rng(24).integers(0, MAX_POS, 300)
    cs = torch.from_numpy(cos_sin[pos])
    c, s = cs[:, :D // 2], cs[:, D // 2:]
    xf = x.float()
    q_embed, _ = m.apply_rotary_pos_emb(xf, xf, torch.cat((c, c), -1), torch.cat((s, s), -1),
                                        unsqueeze_dim=1)
    got = orc.apply_rotary_emb(_bits(x), cos_sin[pos][:, None, :D // 2],
                               cos_sin[pos][:, None, D // 2:], elt="f16")
    assert np.array_equal(got, _bits(q_embed.to(torch.float16)))
    ident = orc.apply_rotary_emb(_bits(x), cos_sin[[0] * 300][:, None, :D // 2],
                                 cos_sin[[0] * 300][:, None, D // 2:], elt="f16")
    assert np.array_equal(ident, _bits(x))


def test_qk_norm_rope_store_f16_matches_per_token_loop(cos_sin):
    hq, hkv, t = 4, 2, 7
    qkv = _bits(_rand_f16((t, (hq + 2 * hkv) * D), 25, scale=2.0))
    qw, kw = _bits(_weight(26).to(torch.float16)), _bits(_weight(27).to(torch.float16))
    pos = np.array([5, 6, 7, 0, 1, 300, 39999])
    kc = np.zeros((2, 8, hkv, D), dtype=np.uint16)
    vc = np.zeros_like(kc)
    slots = np.array([3, -1, 15, 0, 7, 9, 1])
    q, k, v = orc.qk_norm_rope_store(qkv, pos, qw, kw, 1e-6, cos_sin, hq, hkv, D, kc, vc, slots,
                                     elt="f16")
    for i in range(t):
        row = qkv[i].reshape(hq + 2 * hkv, D)
        cs = cos_sin[pos[i]]
        for h in range(hq + hkv):
            n = orc.rms_norm(row[h][None], qw if h < hq else kw, 1e-6, elt="f16")
            r = orc.apply_rotary_emb(n, cs[None, :D // 2], cs[None, D // 2:], elt="f16")[0]
            assert np.array_equal(q[i, h] if h < hq else k[i, h - hq], r), (i, h)
        if slots[i] >= 0:
            assert np.array_equal(kc.reshape(16, hkv, D)[slots[i]], k[i])
            assert np.array_equal(vc.reshape(16, hkv, D)[slots[i]], row[hq + hkv:])
