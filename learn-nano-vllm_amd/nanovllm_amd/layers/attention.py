"""Drop-in for nanovllm/layers/attention.py on MI355X.

``store_kvcache`` and ``Attention`` keep the reference's names, signatures,
argument checks and control flow (attention.py:33-75); the Triton store
kernel and the two flash-attn calls are replaced by libnvk.so entry points.
"""
from __future__ import annotations

import torch
from torch import nn

from nanovllm_amd import _lib
from nanovllm_amd.flash_api import paged_decode, prefill_tile_order, varlen_prefill
from nanovllm_amd.utils.context import get_context


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter new K/V rows into the paged caches (attention.py:33-40).

    key/value: [N, num_kv_heads, head_dim]; each token row contiguous
    (row stride free: value is a view of the packed qkv).  Caches
    [num_blocks, block_size, num_kv_heads, head_dim]; slot -1 skips the token.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    # The flat slot*D addressing of the reference kernel needs whole pages.
    assert k_cache.stride(0) == k_cache.shape[1] * D and v_cache.stride(0) == v_cache.shape[1] * D
    assert k_cache.shape == v_cache.shape and key.dtype == k_cache.dtype == value.dtype == v_cache.dtype
    dev = _lib.require_gpu(key, value, k_cache, v_cache, slot_mapping)
    slots = slot_mapping
    if slots.dtype != torch.int32:
        slots = slots.to(torch.int32)
    slots = slots.contiguous()
    cache_slots = k_cache.shape[0] * k_cache.shape[1]
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.nvk_kv_store(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                                k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(), N, D,
                                key.element_size(), cache_slots, _lib.stream_ptr(dev))
    _lib.check(code)


# The longest-first tile order of the current step's prefill, ranked by the
# first layer and reused by the others: every layer of a step reads the same
# Context (one set_context per step, model_runner.py:132-169), so the order
# is keyed on the step's cu_seqlens tensors and the call's sizes.  Any order
# gives the same output bits (an order of other sizes is ignored by the
# kernel), so a stale entry can only cost time.
_step_order: list = [None, None]     # [key, order tensor or None]


def _prefill_order(context, q, k, block_table):
    if torch.cuda.is_current_stream_capturing():
        return None                      # no cached device buffer inside a graph
    hkv = k.shape[2] if block_table is not None else k.shape[1]
    key = (context.cu_seqlens_q, context.cu_seqlens_k, context.max_seqlen_q,
           context.max_seqlen_k, q.shape[1], hkv, k.shape[1] if block_table is not None else 0,
           block_table.shape[1] if block_table is not None else k.shape[0], q.device)
    cached = _step_order[0]
    if cached is not None and len(cached) == len(key) and all(
            a is b if isinstance(a, torch.Tensor) else a == b for a, b in zip(cached, key)):
        return _step_order[1]
    order = prefill_tile_order(context.cu_seqlens_q, context.cu_seqlens_k, context.max_seqlen_q,
                               k, q.shape[1], block_table=block_table,
                               max_seqlen_k=context.max_seqlen_k)
    _step_order[0], _step_order[1] = key, order
    return order


class Attention(nn.Module):
    """Same constructor and forward as nanovllm.layers.attention.Attention.

    forward(q [T,Hq,D], k [T,Hkv,D], v [T,Hkv,D]) reads the step metadata from
    get_context(); prefill returns [T,Hq,D], decode returns [B,1,Hq,D].
    kv_stored=True (an addition; the reference has no such argument) skips the
    store because the fused prologue (layers/prologue.py) already wrote the
    caches; k may then be None unless the step is a dense prefill.
    """

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_stored: bool = False):
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() and v_cache.numel() and not kv_stored:
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        if context.is_prefill:
            if context.block_tables is not None:    # prefix cache / later chunk
                k, v = k_cache, v_cache
            order = _prefill_order(context, q, k, context.block_tables)
            o = varlen_prefill(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k,
                               context.max_seqlen_q, self.scale, block_table=context.block_tables,
                               max_seqlen_k=context.max_seqlen_k, order=order)
        else:    # decode
            o = paged_decode(q, k_cache, v_cache, context.context_lens, context.block_tables,
                             self.scale).unsqueeze(1)
        return o
