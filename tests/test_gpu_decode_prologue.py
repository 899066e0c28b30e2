"""Decode step with the prologue inside the decode kernel
(nvk_paged_decode_prologue) against the two-call path it replaces: the fused
q/k RMSNorm + RoPE + store (nvk_qk_norm_rope_store, itself checked against the
oracle in test_gpu_prologue.py) followed by the paged decode (checked against
the oracle in test_gpu_decode.py).  Bar: the outputs and both caches are equal
bit for bit.  Cases: GQA groups 1-8, pages that hold whole 32-token chunks
and pages that do not, contexts on and around chunk and page edges, contexts
of one token, graph-padding rows (slot -1, context 0), a padded qkv row
stride, and the routing of attention_with_prologue in decode steps on both
sides of its batch threshold."""
import pytest
import torch

from gpu_utils import assert_attn_close, oracle_decode, say
from nanovllm_amd import (attention_with_prologue, paged_decode, paged_decode_with_prologue,
                          qk_norm_rope_store, rope_cos_sin_cache)
from nanovllm_amd.layers.attention import Attention
from nanovllm_amd.utils.context import reset_context, set_context
from nanovllm_amd.workloads import _Norm, _Rope

pytestmark = pytest.mark.gpu

D = 128
MAX_POS = 40960
EPS = 1e-6


def _case(seed, lens, hq, hkv, bs, row_pad=0, pad_rows=0):
    """lens: context lengths including the new token; pad_rows graph-padding
    rows appended (slot -1, context 0)."""
    g = torch.Generator().manual_seed(seed)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 4
    perm = torch.randperm(nb, generator=g)
    b = len(lens) + pad_rows
    w = max(pages)
    bt = torch.full((b, w), -1, dtype=torch.int32)
    nxt = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[nxt:nxt + p].to(torch.int32)
        nxt += p
    lens_t = torch.tensor(list(lens) + [0] * pad_rows, dtype=torch.int32)
    slots = torch.full((b,), -1, dtype=torch.int32)
    for i, n in enumerate(lens):
        slots[i] = bt[i, (n - 1) // bs] * bs + (n - 1) % bs
    pos = torch.tensor([max(n - 1, 0) for n in lens] + [0] * pad_rows, dtype=torch.int64)
    r = hq + 2 * hkv
    qkv_full = (torch.randn(b, r * D + row_pad, generator=g) * 2.0).to(torch.bfloat16)
    qw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16)
    return dict(qkv=qkv_full.cuda()[:, :r * D], qw=qw.cuda(), kw=kw.cuda(), pos=pos.cuda(),
                kc=kc.cuda(), vc=vc.cuda(), bt=bt.cuda(), lens=lens_t.cuda(), slots=slots.cuda())


@pytest.fixture(scope="module")
def cos_sin():
    return rope_cos_sin_cache(D, MAX_POS, 1_000_000.0, device="cuda")


def _both(c, hq, hkv, cos_sin, what):
    scale = D ** -0.5
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    say(f"decode prologue two calls: {what}")
    q, _, _ = qk_norm_rope_store(c["pos"], c["qkv"], hq, hkv, D, c["qw"], c["kw"], EPS, cos_sin,
                                 kc1, vc1, c["slots"], return_k=False)
    ref = paged_decode(q, kc1, vc1, c["lens"], c["bt"], scale)
    torch.cuda.synchronize()
    say(f"decode prologue fused: {what}")
    out = paged_decode_with_prologue(c["pos"], c["qkv"], hq, hkv, D, c["qw"], c["kw"], EPS,
                                     cos_sin, kc2, vc2, c["slots"], c["lens"], c["bt"], scale)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"{what}: output"
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), f"{what}: caches"
    return out, q, kc1, vc1


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 8), (16, 4), (16, 2)])
def test_fused_equals_two_calls_group_sizes(hq, hkv, cos_sin):
    lens = [1, 31, 32, 33, 255, 256, 257, 700, 2048, 3000]
    c = _case(20 + hkv, lens, hq, hkv, 256)
    _both(c, hq, hkv, cos_sin, f"G={hq // hkv}")


@pytest.mark.parametrize("bs", [16, 64, 512])
def test_fused_equals_two_calls_page_sizes(bs, cos_sin):
    lens = [1, 15, 16, 17, 63, 64, 65, 513, 1500]
    c = _case(30 + bs, lens, 16, 8, bs)
    _both(c, 16, 8, cos_sin, f"page {bs}")


def test_fused_qwen3_batch64_with_padding_rows_and_row_stride(cos_sin):
    g = torch.Generator().manual_seed(40)
    lens = torch.randint(100, 2049, (57,), generator=g).tolist()
    c = _case(41, lens, 16, 8, 256, row_pad=64, pad_rows=7)
    out, q, kc, vc = _both(c, 16, 8, cos_sin, "B=57 + 7 padding rows, padded qkv rows")
    assert not out[57:].any()                                    # padded rows: zeros
    ref = oracle_decode(q.cpu(), kc.cpu(), vc.cpu(), c["bt"].cpu(), c["lens"].cpu(), 256,
                        D ** -0.5)
    assert_attn_close(out, ref, "fused decode vs oracle")


@pytest.mark.parametrize("batch", [4, 32, 33, 40])
def test_attention_with_prologue_decode_routes(batch, cos_sin, monkeypatch):
    """Batches up to FUSED_DECODE_MAX_BATCH take the fused kernel, larger ones
    the two calls; both give the two calls' bits."""
    import nanovllm_amd.layers.prologue as prologue
    taken = []
    real = prologue.paged_decode_with_prologue
    monkeypatch.setattr(prologue, "paged_decode_with_prologue",
                        lambda *a, **k: taken.append(1) or real(*a, **k))
    g = torch.Generator().manual_seed(50 + batch)
    lens = torch.randint(1, 2049, (batch,), generator=g).tolist()
    c = _case(50, lens, 16, 8, 256)
    attn = Attention(16, D, D ** -0.5, 8)
    attn.k_cache, attn.v_cache = c["kc"].clone(), c["vc"].clone()
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    set_context(False, slot_mapping=c["slots"], context_lens=c["lens"], block_tables=c["bt"])
    try:
        say(f"attention_with_prologue decode step, batch {batch}")
        o = attention_with_prologue(attn, c["pos"], c["qkv"], _Norm(c["qw"], EPS),
                                    _Norm(c["kw"], EPS), _Rope(cos_sin))
        q, _, _ = qk_norm_rope_store(c["pos"], c["qkv"], 16, 8, D, c["qw"], c["kw"], EPS,
                                     cos_sin, kc1, vc1, c["slots"], return_k=False)
        ref = paged_decode(q, kc1, vc1, c["lens"], c["bt"], D ** -0.5).unsqueeze(1)
        torch.cuda.synchronize()
    finally:
        reset_context()
    assert o.shape == (batch, 1, 16, D)
    assert torch.equal(o, ref)
    assert torch.equal(attn.k_cache, kc1) and torch.equal(attn.v_cache, vc1)
    assert bool(taken) == (batch <= prologue.FUSED_DECODE_MAX_BATCH)
