"""The Attention module as a drop-in: driven the way the reference drives it.

q/k/v come from a packed qkv projection as in Qwen3Attention.forward
(qwen3.py:77-86: q, k contiguous after the per-head norms, v a strided view),
the metadata from the runner-equivalent builders (model_runner.py:123-188), and
the caches are per-layer views of one [2, L, NB, 256, Hkv, D] allocation
(model_runner.py:115-121).  Steps: warmup with an empty cache, prefill without
prefix, decode, and a prefix-cache hit.
"""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, f32, say
from oracle import kv_oracle as orc
from nanovllm_amd import Attention
from oracle import step_metadata as metadata
from oracle.sequence import Sequence
from nanovllm_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

HQ, HKV, HD, BS = 16, 8, 128, 256


def _qkv(n, gen):
    qkv = torch.randn(n, (HQ + 2 * HKV) * HD, generator=gen).to(torch.bfloat16).cuda()
    q, k, v = qkv.split([HQ * HD, HKV * HD, HKV * HD], dim=-1)
    return (q.reshape(n, HQ, HD).contiguous(), k.reshape(n, HKV, HD).contiguous(),
            v.view(n, HKV, HD))


def _oracle_paged(q, kc, vc, tables, lens_q, lens_k):
    cu_q = np.concatenate([[0], np.cumsum(lens_q)])
    bt = np.full((len(tables), max(len(t) for t in tables)), -1, np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    return orc.paged_attention(f32(q), f32(kc), f32(vc), cu_q, lens_k, HD ** -0.5,
                               block_tables=bt, block_size=BS)


def test_attention_module_end_to_end():
    gen = torch.Generator().manual_seed(31)
    Sequence.block_size = BS
    attn = Attention(HQ, HD, HD ** -0.5, HKV)

    # 1. warmup: empty cache -> no store, dense attention (model_runner.py:91-101)
    warm = [Sequence([0] * 300, num_scheduled_tokens=300)]
    metadata.prepare_prefill(warm, BS)
    q, k, v = _qkv(300, gen)
    say("module warmup (dense)")
    o = attn(q, k, v)
    torch.cuda.synchronize()
    ref = orc.paged_attention(f32(q), f32(k), f32(v), [0, 300], [300], HD ** -0.5,
                              cu_seqlens_k=[0, 300])
    assert o.shape == (300, HQ, HD)
    assert_attn_close(o, ref, "warmup")
    reset_context()

    # 2. caches as per-layer views of one allocation
    nb = 16
    kv_cache = torch.zeros(2, 2, nb, BS, HKV, HD, dtype=torch.bfloat16, device="cuda")
    attn.k_cache, attn.v_cache = kv_cache[0, 1], kv_cache[1, 1]

    # 3. prefill of two fresh sequences (no prefix -> block_tables None)
    lens = [300, 40]
    seqs = [Sequence(list(range(n)), block_table=t, num_scheduled_tokens=n)
            for n, t in zip(lens, [[7, 2], [11]])]
    metadata.prepare_prefill(seqs, BS)
    assert get_context().block_tables is None
    q, k, v = _qkv(sum(lens), gen)
    say("module prefill (store + dense)")
    o = attn(q, k, v)
    torch.cuda.synchronize()
    kc_cpu, vc_cpu = attn.k_cache.cpu(), attn.v_cache.cpu()
    row = 0
    for s, n in zip(seqs, lens):
        slots = orc.slots_for(s.block_table, range(n), BS)
        assert torch.equal(kc_cpu.view(-1, HKV, HD)[slots], k[row:row + n].cpu())
        assert torch.equal(vc_cpu.view(-1, HKV, HD)[slots], v[row:row + n].cpu())
        row += n
    cu = [0, 300, 340]
    ref = orc.paged_attention(f32(q), f32(k), f32(v), cu, lens, HD ** -0.5, cu_seqlens_k=cu)
    assert_attn_close(o, ref, "prefill")
    reset_context()

    # 4. decode: one new token each (context_lens counts it)
    for s in seqs:
        s.num_cached_tokens = len(s)
        s.append_token(1)
    metadata.prepare_decode(seqs, BS)
    q, k, v = _qkv(2, gen)
    say("module decode")
    o = attn(q, k, v)
    torch.cuda.synchronize()
    assert o.shape == (2, 1, HQ, HD)
    kc_cpu, vc_cpu = attn.k_cache.cpu(), attn.v_cache.cpu()
    ref = _oracle_paged(q, kc_cpu, vc_cpu, [s.block_table for s in seqs], [1, 1],
                        [len(s) for s in seqs])
    assert_attn_close(o[:, 0], ref, "decode")
    reset_context()

    # 5. prefix-cache hit: a new sequence reuses page 7 (first 256 tokens of seq 0)
    hit = Sequence(list(range(256)) + [5] * 60, block_table=[7, 3], num_cached_tokens=256,
                   num_scheduled_tokens=60)
    metadata.prepare_prefill([hit], BS)
    assert get_context().block_tables is not None
    q, k, v = _qkv(60, gen)
    say("module prefill with prefix hit (paged)")
    o = attn(q, k, v)
    torch.cuda.synchronize()
    kc_cpu, vc_cpu = attn.k_cache.cpu(), attn.v_cache.cpu()
    ref = _oracle_paged(q, kc_cpu, vc_cpu, [[7, 3]], [60], [316])
    assert_attn_close(o, ref, "prefix hit")
    reset_context()
    # the other layer's cache view was never written
    assert kv_cache[:, 0].eq(0).all()


def test_layers_of_a_step_share_one_tile_order():
    """A chunked-prefill step through three Attention layers (their own cache
    views, one Context): the first layer ranks the query tiles, the other
    two reuse that order, and each output equals varlen_prefill ranking its
    own tiles, bit for bit.  A new step (new Context) ranks again."""
    from nanovllm_amd import varlen_prefill
    from nanovllm_amd.layers import attention as attn_mod
    gen = torch.Generator().manual_seed(33)
    Sequence.block_size = BS
    nb, layers = 120, 3
    kv_cache = torch.randn(2, layers, nb, BS, HKV, HD, generator=gen).to(torch.bfloat16).cuda()
    mods = []
    for i in range(layers):
        m = Attention(HQ, HD, HD ** -0.5, HKV)
        m.k_cache, m.v_cache = kv_cache[0, i], kv_cache[1, i]
        mods.append(m)
    rng = np.random.default_rng(34)
    perm = rng.permutation(nb).tolist()
    seqs, nxt = [], 0
    for _ in range(24):
        cached = int(rng.integers(1, 3)) * BS
        new = int(rng.integers(40, 500)) if seqs else 500
        pages = (cached + new + BS - 1) // BS
        seqs.append(Sequence(list(range(cached + new)), block_table=perm[nxt:nxt + pages],
                             num_cached_tokens=cached, num_scheduled_tokens=new))
        nxt += pages
    metadata.prepare_prefill(seqs, BS)
    ctx = get_context()
    assert ctx.block_tables is not None
    # enough query tiles (24 sequences x 8 tiles x 8 kv heads) for a ranked order
    assert len(seqs) == 24 and ctx.max_seqlen_q > 7 * 64
    n = sum(s.num_scheduled_tokens for s in seqs)
    orders = []
    try:
        for i, m in enumerate(mods):
            q, k, v = _qkv(n, gen)
            say(f"module layer {i} of a chunked-prefill step")
            o = m(q, k, v)
            orders.append(attn_mod._step_order[1])
            ref = varlen_prefill(q, m.k_cache, m.v_cache, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                 ctx.max_seqlen_q, HD ** -0.5, block_table=ctx.block_tables,
                                 max_seqlen_k=ctx.max_seqlen_k)
            torch.cuda.synchronize()
            assert torch.equal(o, ref), f"layer {i}"
        assert orders[0] is not None and orders[1] is orders[0] and orders[2] is orders[0]
        metadata.prepare_prefill(seqs, BS)       # the next step: new cu_seqlens tensors
        mods[0](*_qkv(n, gen))
        assert attn_mod._step_order[1] is not orders[0]
    finally:
        reset_context()
