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
caches.  ``attention_with_prologue`` is the matching replacement for the
body of ``Qwen3Attention.forward`` up to ``self.attn(q, k, v)``.
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import get_context


def rope_cos_sin_cache(head_size: int, max_position: int, base: float,
                       device=None) -> torch.Tensor:
    """The reference's RotaryEmbedding buffer (rotary_embedding.py:27-34):
    float32 [max_position, 1, head_size] = cat(cos(t*inv_freq), sin(t*inv_freq))."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
    return cache if device is None else cache.to(device)


def qk_norm_rope_store(positions: torch.Tensor, qkv: torch.Tensor, num_heads: int,
                       num_kv_heads: int, head_dim: int, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, eps: float, cos_sin_cache: torch.Tensor,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, return_k: bool = True):
    """q/k RMSNorm + RoPE + KV-store in one kernel.

    positions: int64 [T]; qkv: bf16 [T, (num_heads + 2*num_kv_heads) * head_dim]
    (last dim contiguous, any row stride).  Returns (q [T, Hq, D] new tensor,
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
    v = qkv[:, q_size + kv_size:].view(-1, num_kv_heads, head_dim)
    store = slot_mapping is not None
    if store:
        D = kv_size
        assert k_cache is not None and v_cache is not None
        assert k_cache.stride(1) == D and v_cache.stride(1) == D      # attention.py:38
        assert slot_mapping.numel() == T                               # attention.py:39
        assert k_cache.stride(0) == k_cache.shape[1] * D and v_cache.stride(0) == v_cache.shape[1] * D
        assert k_cache.shape == v_cache.shape and k_cache.dtype == qkv.dtype == v_cache.dtype
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
    # k itself is read only by the dense (no block table) prefill
    need_k = context.is_prefill and context.block_tables is None
    q, k, v = qk_norm_rope_store(
        positions, qkv, attn.num_heads, attn.num_kv_heads, attn.head_dim, q_norm.weight,
        k_norm.weight, q_norm.eps, rotary_emb.cos_sin_cache,
        attn.k_cache if store else None, attn.v_cache if store else None,
        context.slot_mapping if store else None, return_k=need_k)
    return attn(q, k, v, kv_stored=True)
