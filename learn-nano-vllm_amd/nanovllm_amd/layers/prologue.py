"""Fused attention prologue of a Qwen3 decoder layer on MI355X.

Between the qkv projection and the attention kernels the reference runs
(nanovllm/models/qwen3.py:79-86, then attention.py:62-63):

    q, k, v = qkv.split([q_size, kv_size, kv_size], dim=-1)   # views [T, H, D]
    q = self.q_norm(q); k = self.k_norm(k)                    # layernorm.py:16-26
    q, k = self.rotary_emb(positions, q, k)                   # rotary_embedding.py:37-48
    store_kvcache(k, v, k_cache, v_cache, slot_mapping)       # attention.py:62-63

``qk_norm_rope_store`` does all of it in one libnvk.so kernel
(``nvk_qk_norm_rope_store``): every head row is read once, q comes out
normed and rotated, the rotated k and the raw v rows go straight into the
caches.  In a decode step ``paged_decode_with_prologue`` goes one step
further: the decode kernel itself norms and rotates q and the new k, stores
the new k and v and attends (``nvk_paged_decode_prologue``), one launch
fewer and q never written.  ``attention_with_prologue`` is the matching
replacement for the body of ``Qwen3Attention.forward`` up to
``self.attn(q, k, v)`` and takes the decode-step form for batches of up to
``FUSED_DECODE_MAX_BATCH`` sequences.
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import get_context

# Largest decode batch routed to the decode kernel with the prologue inside.
# Measured on MI355X, 28-layer Qwen3-0.6B decode step (16/8 heads, contexts
# U{100..2048}, graph replay): the fused kernel is 11 % faster at B = 1, 9 %
# at B = 4, 1-2 % at B = 16-32, and 0.4-2 % slower from B = 40 to 64, where
# the decode is bandwidth-bound and the per-wave prologue arithmetic costs
# more than the separate prologue launch.
FUSED_DECODE_MAX_BATCH = 32


def rope_cos_sin_cache(head_size: int, max_position: int, base: float,
                       device=None) -> torch.Tensor:
    """The reference's RotaryEmbedding buffer (rotary_embedding.py:27-34):
    float32 [max_position, 1, head_size] = cat(cos(t*inv_freq), sin(t*inv_freq))."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
    return cache if device is None else cache.to(device)


def _same_dtype(*ts: torch.Tensor) -> None:
    """qkv, the norm weights and the caches share the model's dtype (bf16 or
    f16; model_runner.py:29 sets it for every parameter and the caches)."""
    dt = ts[0].dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise _lib.NvkError(f"the prologue is built for bfloat16 and float16, got {dt}")
    for t in ts[1:]:
        if t.dtype != dt:
            raise _lib.NvkError(f"qkv, norm weights and caches must share one dtype: "
                                f"{dt} and {t.dtype}")


def qk_norm_rope_store(positions: torch.Tensor, qkv: torch.Tensor, num_heads: int,
                       num_kv_heads: int, head_dim: int, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, eps: float, cos_sin_cache: torch.Tensor,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, return_k: bool = True):
    """q/k RMSNorm + RoPE + KV-store in one kernel.

    positions: int64 [T]; qkv: bf16 or f16 (the model's dtype; the norm weights
    and caches share it) [T, (num_heads + 2*num_kv_heads) * head_dim] (last
    dim contiguous, any row stride).  Returns (q [T, Hq, D] new tensor,
    k [T, Hkv, D] new tensor or None when return_k is False, v = the view of
    qkv the reference passes on).  With slot_mapping given, the rotated k and
    the raw v rows are stored into the caches (slot -1 skipped), as
    store_kvcache does; without it nothing is stored.
    """
    T = qkv.shape[0]
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    assert qkv.dim() == 2 and qkv.shape[1] == q_size + 2 * kv_size and qkv.stride(-1) == 1
    assert positions.numel() == T
    assert q_norm_weight.numel() == head_dim and k_norm_weight.numel() == head_dim
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    assert cs.shape[1] == head_dim and cs.stride(-1) == 1 and cs.dtype == torch.float32
    _same_dtype(qkv, q_norm_weight, k_norm_weight)
    v = qkv[:, q_size + kv_size:].view(-1, num_kv_heads, head_dim)
    store = slot_mapping is not None
    if store:
        D = kv_size
        assert k_cache is not None and v_cache is not None
        assert k_cache.stride(1) == D and v_cache.stride(1) == D      # attention.py:38
        assert slot_mapping.numel() == T                               # attention.py:39
        assert k_cache.stride(0) == k_cache.shape[1] * D and v_cache.stride(0) == v_cache.shape[1] * D
        assert k_cache.shape == v_cache.shape
        _same_dtype(qkv, k_cache, v_cache)
    dev = _lib.require_gpu(qkv, positions, q_norm_weight, k_norm_weight, cs,
                           k_cache if store else None, v_cache if store else None, slot_mapping)
    q = torch.empty(T, num_heads, head_dim, dtype=qkv.dtype, device=dev)
    k = torch.empty(T, num_kv_heads, head_dim, dtype=qkv.dtype, device=dev) if return_k else None
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    pos = pos.contiguous()
    qw, kw = q_norm_weight.contiguous(), k_norm_weight.contiguous()
    slots = None
    cache_slots = 0
    if store:
        slots = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
        slots = slots.contiguous()
        cache_slots = k_cache.shape[0] * k_cache.shape[1]
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.nvk_qk_norm_rope_store(
            qkv.data_ptr(), qkv.stride(0), T, pos.data_ptr(), qw.data_ptr(), kw.data_ptr(),
            float(eps), cs.data_ptr(), cs.stride(0), cs.shape[0], num_heads, num_kv_heads, head_dim,
            q.data_ptr(), q.stride(0), q.stride(1),
            _lib.ptr(k), k.stride(0) if k is not None else 0, k.stride(1) if k is not None else 0,
            _lib.ptr(k_cache) if store else None, _lib.ptr(v_cache) if store else None,
            _lib.ptr(slots), cache_slots, _lib.dtype_code(qkv), _lib.stream_ptr(dev))
    _lib.check(code)
    return q, k, v


def paged_decode_with_prologue(positions: torch.Tensor, qkv: torch.Tensor, num_heads: int,
                               num_kv_heads: int, head_dim: int, q_norm_weight: torch.Tensor,
                               k_norm_weight: torch.Tensor, eps: float,
                               cos_sin_cache: torch.Tensor, k_cache: torch.Tensor,
                               v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                               context_lens: torch.Tensor, block_tables: torch.Tensor,
                               scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """A decode step's prologue and attention in one decode kernel: the same
    results, bit for bit, as ``qk_norm_rope_store(...)`` (storing the new k and
    v at ``slot_mapping``) followed by ``paged_decode(q, k_cache, v_cache,
    context_lens, block_tables, scale)``.  Row b of qkv is sequence b's new
    token; ``slot_mapping[b]`` must be the cache row of key
    ``context_lens[b] - 1`` (as model_runner.prepare_decode builds them).
    Returns [B, Hq, D] (or fills ``out``)."""
    B = qkv.shape[0]
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    assert qkv.dim() == 2 and qkv.shape[1] == q_size + 2 * kv_size and qkv.stride(-1) == 1
    assert positions.numel() == B and slot_mapping.numel() == B and context_lens.numel() == B
    assert q_norm_weight.numel() == head_dim and k_norm_weight.numel() == head_dim
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    assert cs.shape[1] == head_dim and cs.stride(-1) == 1 and cs.dtype == torch.float32
    _same_dtype(qkv, q_norm_weight, k_norm_weight, k_cache, v_cache)
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or k_cache.shape != v_cache.shape:
        raise _lib.NvkError("k_cache/v_cache must be contiguous [num_blocks, block_size, Hkv, D]")
    num_blocks, block_size, hkv, dk = k_cache.shape
    if hkv != num_kv_heads or dk != head_dim:
        raise _lib.NvkError("cache shape and head counts differ")
    dev = _lib.require_gpu(qkv, positions, q_norm_weight, k_norm_weight, cs, k_cache, v_cache,
                           slot_mapping, context_lens, block_tables)
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    pos = pos.contiguous()
    slots = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
    slots = slots.contiguous()
    lens = context_lens if context_lens.dtype == torch.int32 else context_lens.to(torch.int32)
    lens = lens.contiguous()
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    if bt.dim() != 2 or bt.shape[0] != B or bt.stride(-1) != 1:
        raise _lib.NvkError("block_table must be [batch, max_blocks]")
    qw, kw = q_norm_weight.contiguous(), k_norm_weight.contiguous()
    if out is None:
        out = torch.empty((B, num_heads, head_dim), dtype=qkv.dtype, device=dev)
    lib = _lib.load()
    max_blocks = bt.shape[1]
    ws_bytes = lib.nvk_paged_decode_workspace_size(B, num_heads, num_kv_heads, head_dim,
                                                   block_size, max_blocks)
    ws = _lib.workspace(dev, ws_bytes)
    with torch.cuda.device(dev):
        code = lib.nvk_paged_decode_prologue(
            qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), qw.data_ptr(), kw.data_ptr(),
            float(eps), cs.data_ptr(), cs.stride(0), cs.shape[0], k_cache.data_ptr(),
            v_cache.data_ptr(), slots.data_ptr(), num_blocks * block_size, bt.data_ptr(),
            bt.stride(0), lens.data_ptr(), B, num_heads, num_kv_heads, head_dim, block_size,
            max_blocks, num_blocks, float(scale), out.data_ptr(), out.stride(0), out.stride(1),
            _lib.ptr(ws), ws_bytes, _lib.dtype_code(qkv), _lib.stream_ptr(dev))
    _lib.check(code)
    return out


def attention_with_prologue(attn, positions: torch.Tensor, qkv: torch.Tensor, q_norm, k_norm,
                            rotary_emb) -> torch.Tensor:
    """Qwen3Attention.forward up to and including ``self.attn(q, k, v)``
    (qwen3.py:79-86) with the prologue fused: ``attn`` is an
    nanovllm_amd Attention, q_norm / k_norm expose ``weight`` and ``eps``
    (layernorm.RMSNorm), rotary_emb exposes ``cos_sin_cache``.  Returns what
    ``attn(q, k, v)`` returns ([T, Hq, D] prefill, [B, 1, Hq, D] decode)."""
    assert q_norm.eps == k_norm.eps    # one eps for both norms (qwen3.py:70-71)
    context = get_context()
    store = bool(attn.k_cache.numel() and attn.v_cache.numel())
    if (store and not context.is_prefill and attn.head_dim == 128
            and qkv.shape[0] <= FUSED_DECODE_MAX_BATCH):
        # small decode step: prologue, store and attention in the decode kernel
        return paged_decode_with_prologue(
            positions, qkv, attn.num_heads, attn.num_kv_heads, attn.head_dim, q_norm.weight,
            k_norm.weight, q_norm.eps, rotary_emb.cos_sin_cache, attn.k_cache, attn.v_cache,
            context.slot_mapping, context.context_lens, context.block_tables,
            attn.scale).unsqueeze(1)
    # k itself is read only by the dense (no block table) prefill
    need_k = context.is_prefill and context.block_tables is None
    q, k, v = qk_norm_rope_store(
        positions, qkv, attn.num_heads, attn.num_kv_heads, attn.head_dim, q_norm.weight,
        k_norm.weight, q_norm.eps, rotary_emb.cos_sin_cache,
        attn.k_cache if store else None, attn.v_cache if store else None,
        context.slot_mapping if store else None, return_k=need_k)
    return attn(q, k, v, kv_stored=True)
