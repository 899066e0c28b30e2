"""Pins oracle/torch_cpu.py (the PyTorch CPU path bench.py times as its CPU
baseline) against oracle/kv_oracle.py, which tests/test_oracle.py pins against
golden vectors and closed forms: the store bit for bit, attention to float32
rounding, on the cases the reference's shapes produce (prefix + new tokens
with bottom-right causal alignment, decode, rows and sequences without keys,
GQA group sizes 1-8, several page sizes), and the q/k norm + rotary + store
prologue (v rows bit for bit; q and k bit for bit but where the sum of
squares rounds differently, within 2 bf16 ulps)."""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from oracle import torch_cpu

HD = 128


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(seed, lens_q, lens_k, bs, hq, hkv):
    g = torch.Generator().manual_seed(seed)
    pages = [(k + bs - 1) // bs for k in lens_k]
    perm = torch.randperm(sum(pages) + 2, generator=g)
    w = max(max(pages), 1)
    bt = torch.full((len(lens_k), w), -1, dtype=torch.int32)
    nxt = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[nxt:nxt + p].to(torch.int32)
        nxt += p
    nb = int(perm.numel())
    kc = torch.randn(nb, bs, hkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, HD, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(lens_q), hq, HD, generator=g).to(torch.bfloat16)
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int64)
    return q, kc, vc, bt, cu_q


def test_store_bit_exact_with_skips_and_value_row_stride():
    g = torch.Generator().manual_seed(3)
    n, nb, bs, hkv = 300, 4, 256, 8
    qkv = torch.randn(n, (16 + 2 * hkv) * HD, generator=g).to(torch.bfloat16)
    key = torch.randn(n, hkv, HD, generator=g).to(torch.bfloat16)
    value = qkv[:, (16 + hkv) * HD:].view(n, hkv, HD)            # row stride 4096, as qwen3.py:78-81
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[torch.randperm(n, generator=g)[:15]] = -1
    kc = torch.randn(nb, bs, hkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, HD, generator=g).to(torch.bfloat16)
    kc_ref, vc_ref = _bits(kc).copy(), _bits(vc).copy()
    orc.kv_store(_bits(key), _bits(value), kc_ref, vc_ref, slots.numpy())
    torch_cpu.store_kvcache_cpu(key, value, kc, vc, slots)
    assert np.array_equal(_bits(kc), kc_ref) and np.array_equal(_bits(vc), vc_ref)


@pytest.mark.parametrize("lens_q,lens_k,bs,hq,hkv", [
    ([100, 37, 1], [612, 549, 513], 256, 16, 8),        # 512-token prefix + new tokens
    ([1] * 6, [1, 255, 256, 257, 700, 2048], 256, 16, 8),  # decode
    ([5, 0, 3], [3, 800, 300], 256, 16, 8),             # rows without keys, no queries
    ([64, 20], [64, 530], 16, 16, 16),                  # G = 1, small pages
    ([9, 12], [700, 12], 64, 16, 2),                    # G = 8
])
def test_attention_matches_numpy_oracle(lens_q, lens_k, bs, hq, hkv):
    q, kc, vc, bt, cu_q = _case(sum(lens_q) + bs + hkv, lens_q, lens_k, bs, hq, hkv)
    scale = HD ** -0.5
    got = torch_cpu.paged_attention_cpu(q, kc, vc, cu_q, lens_k, scale, bt).numpy()
    ref = orc.paged_attention(_bits(q), _bits(kc), _bits(vc), cu_q, np.array(lens_k), scale,
                              block_tables=bt.numpy(), block_size=bs)
    np.testing.assert_allclose(got, ref, atol=2e-5, rtol=1e-4)
    # rows that see no key are zeros in both
    for s, (lq, lk) in enumerate(zip(lens_q, lens_k)):
        for i in range(max(0, lq - lk)):
            assert not got[cu_q[s] + i].any()


def test_bottom_right_alignment_is_what_is_timed():
    # A mutation of the CPU path's mask (top-left alignment) is caught by the
    # numpy oracle on a prefix case, so the comparison above has teeth.
    q, kc, vc, bt, cu_q = _case(9, [40], [300], 256, 16, 8)
    scale = HD ** -0.5
    ref = orc.paged_attention(_bits(q), _bits(kc), _bits(vc), cu_q, np.array([300]), scale,
                              block_tables=bt.numpy(), block_size=256)
    k = torch_cpu._gather(kc, bt[0], 300).float().transpose(0, 1)
    v = torch_cpu._gather(vc, bt[0], 300).float().transpose(0, 1)
    top_left = torch.nn.functional.scaled_dot_product_attention(
        q.float().transpose(0, 1), k, v, is_causal=True, scale=scale, enable_gqa=True)
    assert not np.allclose(top_left.transpose(0, 1).numpy(), ref, atol=2e-2, rtol=1e-2)


def test_prologue_matches_numpy_oracle():
    from nanovllm_amd.layers.prologue import rope_cos_sin_cache
    g = torch.Generator().manual_seed(11)
    t, hq, hkv, nb, bs = 300, 16, 8, 4, 256
    qkv = (torch.randn(t, (hq + 2 * hkv) * HD, generator=g) * 2).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (t,), generator=g)
    qw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    cs = rope_cos_sin_cache(HD, 4096, 1e6).reshape(4096, HD)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    slots[:7] = -1
    kc = torch.zeros(nb, bs, hkv, HD, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc_ref, vc_ref = _bits(kc).copy(), _bits(vc).copy()
    q, k, v = torch_cpu.qk_norm_rope_store_cpu(pos, qkv, hq, hkv, HD, qw, kw, 1e-6, cs, kc, vc,
                                               slots)
    q_ref, k_ref, _ = orc.qk_norm_rope_store(_bits(qkv), pos.numpy(), _bits(qw), _bits(kw), 1e-6,
                                             cs.numpy(), hq, hkv, HD, kc_ref, vc_ref,
                                             slots.numpy())
    assert np.array_equal(_bits(vc), vc_ref)                 # v rows are a bit copy
    for got, ref in ((q, q_ref), (k, k_ref), (kc, kc_ref)):
        gb, rb = _bits(got), np.asarray(ref)
        same = gb == rb
        assert same.mean() > 0.999                           # sum-of-squares rounding only
        diff = np.abs(orc.bf16_to_f32(gb) - orc.bf16_to_f32(rb))
        assert float(diff.max()) <= 2 ** -5 * max(1.0, float(np.abs(orc.bf16_to_f32(rb)).max()))
