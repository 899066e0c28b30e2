"""Seeded synthetic inputs of the KV-cache path at Qwen3-0.6B shape.

Five workloads (16 q heads, 8 kv heads, head_dim 128, bf16, 256-token pages):

  kv_store_case     4096 new tokens scattered into a 64-page cache; the slots are
                    the first 4096 of a random permutation of the 16384 slots, with
                    205 (5 %) of them set to -1.
  decode_case       64 sequences, context U{100..2048}, pages drawn without
                    sharing from a shuffled 1024-page pool, tables padded with -1.
  prefill_case      32 sequences = a shared 512-token prefix (2 common pages) plus
                    U{100..1024} new tokens in fresh pages; the new K/V are stored
                    through slot_mapping before attention.
  spec_verify_case  32 sequences, context U{1024..8192} of which the last 6 are
                    queries; the last 5 (draft tokens) are stored in the step.
  mixed_layer_case  one layer of a chunked-prefill + decode step: 8 chunks of 512
                    new tokens after U{0..1536} cached ones, plus 192 decodes with
                    context U{256..4096}.

Every tensor is produced on the CPU from ``torch.Generator().manual_seed(seed)``
in a fixed order, so a case is identical wherever it is built; ``.to(device)``
moves it.  Values are N(0,1) rounded to bf16.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

HQ, HKV, HD, BLOCK = 16, 8, 128, 256


def _randn(gen, *shape):
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)


def _randint(gen, lo, hi, n):
    """n integers uniform in [lo, hi] (inclusive)."""
    return torch.randint(lo, hi + 1, (n,), generator=gen).tolist()


def _pad_tables(tables, width=None):
    w = width if width is not None else max(len(t) for t in tables)
    out = torch.full((len(tables), w), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return out


@dataclass
class Case:
    tensors: dict = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    def __getattr__(self, name):
        t = self.__dict__.get("tensors", {})
        if name in t:
            return t[name]
        m = self.__dict__.get("meta", {})
        if name in m:
            return m[name]
        raise AttributeError(name)

    def to(self, device):
        return Case({k: (v.to(device) if isinstance(v, torch.Tensor) else v)
                     for k, v in self.tensors.items()}, dict(self.meta))


def kv_store_case(seed=0, n_tokens=4096, num_blocks=64, block_size=BLOCK, hkv=HKV, hd=HD,
                  skip=205, value_row_stride=None):
    gen = torch.Generator().manual_seed(seed)
    key = _randn(gen, n_tokens, hkv, hd)
    value_full = _randn(gen, n_tokens, (value_row_stride or hkv * hd) // hd, hd)
    value = value_full[:, :hkv]  # row stride value_row_stride when given (packed-qkv view)
    slots = torch.randperm(num_blocks * block_size, generator=gen)[:n_tokens].to(torch.int32)
    skip_pos = torch.randperm(n_tokens, generator=gen)[:skip]
    slots[skip_pos] = -1
    k_cache = torch.zeros(num_blocks, block_size, hkv, hd, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    return Case(dict(key=key, value=value, k_cache=k_cache, v_cache=v_cache, slot_mapping=slots),
                dict(block_size=block_size, n_valid=n_tokens - skip))


def _fill_pool(gen, pool_blocks, block_size, hkv, hd):
    k_cache = _randn(gen, pool_blocks, block_size, hkv, hd)
    v_cache = _randn(gen, pool_blocks, block_size, hkv, hd)
    return k_cache, v_cache


def decode_case(seed=1, batch=64, hq=HQ, hkv=HKV, hd=HD, block_size=BLOCK, ctx_lo=100,
                ctx_hi=2048, pool_blocks=1024, ctx=None, width=None):
    gen = torch.Generator().manual_seed(seed)
    lens = list(ctx) if ctx is not None else _randint(gen, ctx_lo, ctx_hi, batch)
    batch = len(lens)
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    tables, nxt = [], 0
    for n in lens:
        need = (n + block_size - 1) // block_size
        tables.append(perm[nxt:nxt + need])
        nxt += need
    assert nxt <= pool_blocks, "pool too small"
    q = _randn(gen, batch, hq, hd)
    k_cache, v_cache = _fill_pool(gen, pool_blocks, block_size, hkv, hd)
    bt = _pad_tables(tables, width)
    return Case(dict(q=q, k_cache=k_cache, v_cache=v_cache, block_tables=bt,
                     context_lens=torch.tensor(lens, dtype=torch.int32)),
                dict(block_size=block_size, scale=hd ** -0.5, lens=lens, tables=tables))


def _prefix_batch(gen, lens_new, cached, block_size, pool_blocks, shared_prefix_pages):
    """Block tables for sequences with `cached[i]` cached tokens then `lens_new[i]` new ones.
    The first `shared_prefix_pages` pages are common to every sequence."""
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    shared = perm[:shared_prefix_pages]
    nxt = shared_prefix_pages
    tables, slots = [], []
    for n_new, c in zip(lens_new, cached):
        total = c + n_new
        need = (total + block_size - 1) // block_size
        own = need - shared_prefix_pages
        table = shared + perm[nxt:nxt + own]
        nxt += own
        tables.append(table)
        for p in range(c, total):
            slots.append(table[p // block_size] * block_size + p % block_size)
    assert nxt <= pool_blocks, "pool too small"
    return tables, slots


def prefill_case(seed=2, nseq=32, prefix=512, new_lo=100, new_hi=1024, hq=HQ, hkv=HKV, hd=HD,
                 block_size=BLOCK, pool_blocks=256, lens_new=None):
    gen = torch.Generator().manual_seed(seed)
    lens_new = list(lens_new) if lens_new is not None else _randint(gen, new_lo, new_hi, nseq)
    nseq = len(lens_new)
    assert prefix % block_size == 0
    tables, slots = _prefix_batch(gen, lens_new, [prefix] * nseq, block_size, pool_blocks,
                                  prefix // block_size)
    tq = sum(lens_new)
    q = _randn(gen, tq, hq, hd)
    key = _randn(gen, tq, hkv, hd)
    value = _randn(gen, tq, hkv, hd)
    k_cache, v_cache = _fill_pool(gen, pool_blocks, block_size, hkv, hd)
    cu_q = torch.tensor([0] + list(torch.tensor(lens_new).cumsum(0).tolist()), dtype=torch.int32)
    lens_k = [prefix + n for n in lens_new]
    cu_k = torch.tensor([0] + list(torch.tensor(lens_k).cumsum(0).tolist()), dtype=torch.int32)
    return Case(dict(q=q, key=key, value=value, k_cache=k_cache, v_cache=v_cache,
                     slot_mapping=torch.tensor(slots, dtype=torch.int32),
                     block_tables=_pad_tables(tables), cu_seqlens_q=cu_q, cu_seqlens_k=cu_k),
                dict(block_size=block_size, scale=hd ** -0.5, lens_q=lens_new, lens_k=lens_k,
                     max_seqlen_q=max(lens_new), max_seqlen_k=max(lens_k), tables=tables))


def spec_verify_case(seed=4, batch=32, n_query=6, n_draft=5, ctx_lo=1024, ctx_hi=8192, hq=HQ,
                     hkv=HKV, hd=HD, block_size=BLOCK, pool_blocks=1100):
    """The last `n_query` of each context are queries; the last `n_draft` of
    those (the draft tokens) are stored in the step, the first query (the last
    accepted token) is already cached."""
    gen = torch.Generator().manual_seed(seed)
    lens = _randint(gen, ctx_lo, ctx_hi, batch)
    cached = [n - n_draft for n in lens]
    tables, slots = _prefix_batch(gen, [n_draft] * batch, cached, block_size, pool_blocks, 0)
    q = _randn(gen, batch * n_query, hq, hd)
    key = _randn(gen, batch * n_draft, hkv, hd)
    value = _randn(gen, batch * n_draft, hkv, hd)
    k_cache, v_cache = _fill_pool(gen, pool_blocks, block_size, hkv, hd)
    cu_q = torch.arange(0, (batch + 1) * n_query, n_query, dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    return Case(dict(q=q, key=key, value=value, k_cache=k_cache, v_cache=v_cache,
                     slot_mapping=torch.tensor(slots, dtype=torch.int32),
                     block_tables=_pad_tables(tables), cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                     context_lens=torch.tensor(lens, dtype=torch.int32)),
                dict(block_size=block_size, scale=hd ** -0.5, lens_q=[n_query] * batch,
                     lens_k=lens, max_seqlen_q=n_query, max_seqlen_k=max(lens), tables=tables))


def mixed_step_metadata(seed=3, n_chunks=8, chunk=512, cached_lo=0, cached_hi=1536, n_decode=192,
                        ctx_lo=256, ctx_hi=4096, block_size=BLOCK, pool_blocks=3300, gen=None):
    """Block tables, slots and lengths of one mixed step (shared by every layer):
    prefill chunks (paged, mid-page starts allowed) and decodes in one pool."""
    gen = gen if gen is not None else torch.Generator().manual_seed(seed)
    cached = _randint(gen, cached_lo, cached_hi, n_chunks)
    dec_lens = _randint(gen, ctx_lo, ctx_hi, n_decode)
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    nxt = 0
    pf_tables, pf_slots = [], []
    for c in cached:
        total = c + chunk
        need = (total + block_size - 1) // block_size
        t = perm[nxt:nxt + need]
        nxt += need
        pf_tables.append(t)
        for p in range(c, total):
            pf_slots.append(t[p // block_size] * block_size + p % block_size)
    dec_tables, dec_slots = [], []
    for n in dec_lens:
        need = (n + block_size - 1) // block_size
        t = perm[nxt:nxt + need]
        nxt += need
        dec_tables.append(t)
        dec_slots.append(t[(n - 1) // block_size] * block_size + (n - 1) % block_size)
    assert nxt <= pool_blocks, "pool too small"
    lens_k = [c + chunk for c in cached]
    cu_q = torch.arange(0, (n_chunks + 1) * chunk, chunk, dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lens_k).cumsum(0).tolist()), dtype=torch.int32)
    return dict(slot_mapping=torch.tensor(pf_slots + dec_slots, dtype=torch.int32),
                prefill_block_tables=_pad_tables(pf_tables), cu_seqlens_q=cu_q,
                cu_seqlens_k=cu_k, decode_block_tables=_pad_tables(dec_tables),
                context_lens=torch.tensor(dec_lens, dtype=torch.int32)), \
        dict(block_size=block_size, lens_q=[chunk] * n_chunks, lens_k=lens_k, max_seqlen_q=chunk,
             max_seqlen_k=max(lens_k), dec_lens=dec_lens, n_tokens=n_chunks * chunk + n_decode,
             pool_blocks=pool_blocks)


def mixed_layer_case(seed=3, n_chunks=8, chunk=512, cached_lo=0, cached_hi=1536, n_decode=192,
                     ctx_lo=256, ctx_hi=4096, hq=HQ, hkv=HKV, hd=HD, block_size=BLOCK,
                     pool_blocks=3300):
    """One layer of a mixed step: prefill chunks (paged, mid-page starts allowed)
    and decode sequences share one cache pool."""
    gen = torch.Generator().manual_seed(seed)
    tensors, meta = mixed_step_metadata(seed, n_chunks, chunk, cached_lo, cached_hi, n_decode,
                                        ctx_lo, ctx_hi, block_size, pool_blocks, gen=gen)
    tq = n_chunks * chunk
    q_pf = _randn(gen, tq, hq, hd)
    q_dec = _randn(gen, n_decode, hq, hd)
    key = _randn(gen, tq + n_decode, hkv, hd)
    value = _randn(gen, tq + n_decode, hkv, hd)
    k_cache, v_cache = _fill_pool(gen, pool_blocks, block_size, hkv, hd)
    tensors.update(q_prefill=q_pf, q_decode=q_dec, key=key, value=value, k_cache=k_cache,
                   v_cache=v_cache)
    meta.update(scale=hd ** -0.5)
    return Case(tensors, meta)


def prologue_case(seed=5, hq=HQ, hkv=HKV, hd=HD, max_position=40960, rope_theta=1_000_000.0):
    """The fused attention prologue over one layer of the mixed step: the 4288
    new tokens (8 prefill chunks of 512 after U{0..1536} cached tokens + 192
    decodes over U{256..4096}) with their positions and slots in a 3300-page
    pool (the caches themselves are left to the caller: 1.7 GB each);
    qkv ~ N(0, 2^2) bf16, norm weights ~ 1 + N(0, 0.2^2)."""
    from nanovllm_amd.layers.prologue import rope_cos_sin_cache
    tensors, meta = mixed_step_metadata()
    gen = torch.Generator().manual_seed(seed)
    chunk = meta["lens_q"][0]
    pos = [p for lk in meta["lens_k"] for p in range(lk - chunk, lk)]
    pos += [n - 1 for n in meta["dec_lens"]]
    n = meta["n_tokens"]
    assert len(pos) == n
    qkv = (torch.randn(n, (hq + 2 * hkv) * hd, generator=gen) * 2.0).to(torch.bfloat16)
    qw = (1.0 + 0.2 * torch.randn(hd, generator=gen)).to(torch.bfloat16)
    kw = (1.0 + 0.2 * torch.randn(hd, generator=gen)).to(torch.bfloat16)
    return Case(dict(qkv=qkv, positions=torch.tensor(pos, dtype=torch.int64), q_weight=qw,
                     k_weight=kw, cos_sin=rope_cos_sin_cache(hd, max_position, rope_theta),
                     slot_mapping=tensors["slot_mapping"]),
                dict(n_tokens=n, hq=hq, hkv=hkv, hd=hd, eps=1e-6, pool_blocks=meta["pool_blocks"],
                     block_size=meta["block_size"], n_unique_positions=len(set(pos))))


class _Norm:
    """The two attributes of layernorm.RMSNorm the fused prologue reads."""

    def __init__(self, weight, eps):
        self.weight, self.eps = weight, eps


class _Rope:
    """The attribute of rotary_embedding.RotaryEmbedding the fused prologue reads."""

    def __init__(self, cos_sin_cache):
        self.cos_sin_cache = cos_sin_cache


def decode_stack(num_layers, num_blocks, device, seed=6, hq=HQ, hkv=HKV, hd=HD,
                 block_size=BLOCK, max_position=40960, rope_theta=1_000_000.0, eps=1e-6):
    """The attention path of a Qwen3 decoder stack on one device: per layer an
    Attention whose caches are views of one [2, L, NB, bs, Hkv, D] allocation
    (allocate_kv_cache, model_runner.py:103-121; filled with N(0,1) bf16),
    q/k norm weights ~ 1 + N(0, 0.2^2), one shared rotary cache.  Returns
    (layers, rope, kv_cache, step): layers[i] = (attn, q_norm, k_norm) and
    step(positions [bs], qkv [bs, L, (Hq+2Hkv)*D]) -> [bs, L, Hq*D] runs, per
    layer, the fused prologue (norms, rotation, store) and the attention of
    the current Context."""
    from nanovllm_amd.layers.attention import Attention
    from nanovllm_amd.layers.prologue import attention_with_prologue, rope_cos_sin_cache
    gen = torch.Generator(device=device).manual_seed(seed)
    kv_cache = torch.empty(2, num_layers, num_blocks, block_size, hkv, hd, dtype=torch.bfloat16,
                           device=device)
    for i in range(num_layers):
        for j in range(2):
            for b in range(0, num_blocks, 256):
                n = min(256, num_blocks - b)
                kv_cache[j, i, b:b + n].copy_(torch.randn(n, block_size, hkv, hd, generator=gen,
                                                          device=device))
    rope = _Rope(rope_cos_sin_cache(hd, max_position, rope_theta, device=device))
    layers = []
    for i in range(num_layers):
        attn = Attention(hq, hd, hd ** -0.5, hkv)
        attn.k_cache, attn.v_cache = kv_cache[0, i], kv_cache[1, i]
        w = lambda: (1.0 + 0.2 * torch.randn(hd, generator=gen, device=device)).to(torch.bfloat16)
        layers.append((attn, _Norm(w(), eps), _Norm(w(), eps)))

    def step(positions, qkv):
        outs = [attention_with_prologue(attn, positions, qkv[:, i], qn, kn, rope)
                .reshape(positions.numel(), hq * hd)
                for i, (attn, qn, kn) in enumerate(layers)]
        return torch.stack(outs, dim=1)

    return layers, rope, kv_cache, step


# ---------------------------------------------------------------------------
# Algorithmic work of a call (the numerators of the rooflines)
# ---------------------------------------------------------------------------
def attention_bytes(seqlens_k, num_kv_heads: int, head_dim: int, n_q_rows: int, num_q_heads: int,
                    elem_bytes: int = 2) -> int:
    """Unique K+V bytes of every sequence's keys + q read + out written."""
    kv = 2 * sum(int(n) for n in seqlens_k) * num_kv_heads * head_dim * elem_bytes
    return kv + 2 * n_q_rows * num_q_heads * head_dim * elem_bytes


def prefill_flops(seqlens_q, seqlens_k, num_q_heads: int, head_dim: int) -> int:
    """4 * Hq * D * (number of unmasked (query, key) pairs): QK^T plus PV.
    Query row i of a sequence with Lq queries and Lk keys sees
    min(Lk, i + Lk - Lq + 1) keys (bottom-right aligned causal mask)."""
    pairs = 0
    for lq, lk in zip(seqlens_q, seqlens_k):
        lq, lk = int(lq), int(lk)
        diag = lk - lq
        for i in range(lq):
            pairs += max(0, min(lk, i + diag + 1))
    return 4 * num_q_heads * head_dim * pairs


def prologue_bytes(n_tokens: int, n_valid_slots: int, n_unique_positions: int,
                   num_q_heads: int, num_kv_heads: int, head_dim: int, write_k: bool) -> int:
    """HBM bytes the fused prologue must move: the qkv rows, positions and
    slots read, one cos/sin row per distinct position, q written, k and v
    rows written to the caches for valid slots (and k written out if asked)."""
    row = head_dim * 2
    rd = n_tokens * (num_q_heads + 2 * num_kv_heads) * row + n_tokens * (8 + 4)
    rd += n_unique_positions * head_dim * 4
    wr = n_tokens * num_q_heads * row + n_valid_slots * 2 * num_kv_heads * row
    if write_k:
        wr += n_tokens * num_kv_heads * row
    return rd + wr
