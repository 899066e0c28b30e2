"""flash-attn-compatible entry points backed by libnvk.so.

nanovllm/layers/attention.py:6 imports ``flash_attn_varlen_func`` and
``flash_attn_with_kvcache`` from flash-attn (an un-vendored CUDA extension).
The two functions below accept the same arguments for the forms the
reference uses, so that import line is the only change a CUDA-free build of
the reference needs.  Unsupported flash-attn options (dropout, sliding window,
softcap, ALiBi, returning probabilities / LSE, in-call cache append, rotary)
raise NotImplementedError instead of being silently ignored.
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib


def _unsupported(**opts) -> None:
    for name, (value, default) in opts.items():
        if value != default:
            raise NotImplementedError(f"nanovllm_amd: {name}={value!r} is not supported")


def _attn_dtype(*ts: torch.Tensor) -> int:
    """The library's code for the one 16-bit type (bf16 or fp16) of q, k, v."""
    dt = ts[0].dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise _lib.NvkError(f"attention kernels are built for bfloat16 and float16, got {dt}")
    for t in ts[1:]:
        if t.dtype != dt:
            raise _lib.NvkError(f"q, k and v must share one dtype: {dt} and {t.dtype}")
    return _lib.dtype_code(ts[0])


def _int32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _key_bound(k, block_table, max_seqlen_k):
    """The per-sequence key bound the library plans a prefill with."""
    bound = (block_table.shape[1] * k.shape[1]) if block_table is not None else k.shape[0]
    return min(int(max_seqlen_k), bound) if max_seqlen_k else bound


def prefill_tile_order(cu_seqlens_q, cu_seqlens_k, max_seqlen_q, k, num_q_heads,
                       block_table=None, max_seqlen_k=None):
    """The longest-first order of a prefill's query tiles, for every layer of a
    step (they share cu_seqlens): pass it as ``order`` to varlen_prefill to
    skip the per-call ranking kernel.  k: the layer's keys or cache (only its
    shape is read); num_q_heads: the q heads the prefill calls will have.
    Returns an int32 device tensor, or None when the prefill runs in grid
    order anyway."""
    dev = _lib.require_gpu(cu_seqlens_q, cu_seqlens_k)
    cu_q, cu_k = _int32(cu_seqlens_q), _int32(cu_seqlens_k)
    batch = cu_q.numel() - 1
    hkv = k.shape[2] if block_table is not None else k.shape[1]
    bs = k.shape[1] if block_table is not None else 0
    mk = _key_bound(k, block_table, max_seqlen_k)
    lib = _lib.load()
    nbytes = lib.nvk_prefill_tile_order_size(batch, int(max_seqlen_q), mk, num_q_heads, hkv, bs)
    if nbytes == 0:
        return None
    order = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        code = lib.nvk_prefill_tile_order(cu_q.data_ptr(), cu_k.data_ptr(), batch,
                                          int(max_seqlen_q), mk, num_q_heads, hkv, bs,
                                          order.data_ptr(), nbytes, _lib.stream_ptr(dev))
    _lib.check(code)
    return order


def varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, softmax_scale,
                   block_table=None, out=None, max_seqlen_k=None, order=None):
    """Causal varlen attention (bottom-right aligned), dense or paged keys.

    q: [Tq, Hq, D]; dense k/v: [Tk, Hkv, D]; paged k/v: [NB, bs, Hkv, D] caches
    with ``block_table`` [B, W] int32.  Returns [Tq, Hq, D] (or fills ``out``).
    ``max_seqlen_k`` (host int, optional) bounds the keys of a sequence; the
    library uses it to decide whether to split long key ranges across
    workgroups (its workspace is this stream's cached buffer).  ``order``:
    from prefill_tile_order with the same metadata (ranked once per step).
    """
    dev = _lib.require_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k, block_table)
    dtype = _attn_dtype(q, k, v)
    if q.dim() != 3 or q.stride(-1) != 1:
        raise _lib.NvkError("q must be [tokens, heads, head_dim] with unit last stride")
    tq, hq, d = q.shape
    cu_q = _int32(cu_seqlens_q)
    cu_k = _int32(cu_seqlens_k)
    batch = cu_q.numel() - 1
    if cu_k.numel() != batch + 1:
        raise _lib.NvkError("cu_seqlens_q and cu_seqlens_k disagree on the batch size")
    if out is None:
        out = torch.empty((tq, hq, d), dtype=q.dtype, device=dev)
    if block_table is not None:
        if k.dim() != 4 or not k.is_contiguous() or not v.is_contiguous() or k.shape != v.shape:
            raise _lib.NvkError("paged k/v must be contiguous [num_blocks, block_size, Hkv, D] caches")
        num_blocks, block_size, hkv, dk = k.shape
        bt = _int32(block_table)
        if bt.dim() != 2 or bt.shape[0] != batch:
            raise _lib.NvkError("block_table must be [batch, max_blocks]")
        k_st = v_st = kv_sh = 0
        total_k = num_blocks * block_size
        max_blocks, bt_stride = bt.shape[1], bt.stride(0)
    else:
        if k.dim() != 3 or k.stride(-1) != 1 or v.stride(-1) != 1 or k.shape != v.shape:
            raise _lib.NvkError("dense k/v must be [tokens, Hkv, D] with unit last stride")
        if k.stride(1) != v.stride(1):
            raise _lib.NvkError("k and v must share the head stride")
        total_k, hkv, dk = k.shape
        k_st, v_st, kv_sh = k.stride(0), v.stride(0), k.stride(1)
        num_blocks = block_size = max_blocks = bt_stride = 0
        bt = None
    if dk != d:
        raise _lib.NvkError("q and k head_dim differ")
    scale = float(softmax_scale) if softmax_scale is not None else d ** -0.5
    lib = _lib.load()
    key_bound = max_blocks * block_size if bt is not None else total_k
    msk = min(int(max_seqlen_k), key_bound) if max_seqlen_k else key_bound
    ws_bytes = lib.nvk_varlen_prefill_workspace_size(batch, int(max_seqlen_q), msk, hq, hkv, d)
    ws = _lib.workspace(dev, ws_bytes)
    order_bytes = 0
    if order is not None:
        if order.dtype != torch.int32 or order.device != dev or not order.is_contiguous():
            raise _lib.NvkError("order must be the int32 device tensor prefill_tile_order returns")
        order_bytes = order.numel() * 4
        need = lib.nvk_prefill_tile_order_size(batch, int(max_seqlen_q), msk, hq, hkv,
                                               block_size if bt is not None else 0)
        if need == 0:
            order = None          # this call runs its tiles in grid order
        elif order_bytes < need:
            raise _lib.NvkError(f"order holds {order_bytes} bytes; a prefill of these sizes "
                                f"needs {need} (rank it with this call's sizes and head counts)")
    with torch.cuda.device(dev):
        code = lib.nvk_varlen_prefill_ordered(
            q.data_ptr(), q.stride(0), q.stride(1), tq,
            k.data_ptr(), v.data_ptr(), k_st, v_st, kv_sh, total_k,
            cu_q.data_ptr(), cu_k.data_ptr(), batch, int(max_seqlen_q), msk,
            _lib.ptr(bt), bt_stride, max_blocks, block_size, num_blocks,
            hq, hkv, d, scale,
            out.data_ptr(), out.stride(0), out.stride(1),
            _lib.ptr(ws), ws_bytes, _lib.ptr(order), order_bytes,
            dtype, _lib.stream_ptr(dev))
    _lib.check(code)
    return out


def paged_decode(q, k_cache, v_cache, context_lens, block_table, softmax_scale, out=None):
    """One query per sequence over its paged cache.  q: [B, Hq, D] (any token /
    head strides).  Returns [B, Hq, D] (or fills ``out``)."""
    dev = _lib.require_gpu(q, k_cache, v_cache, context_lens, block_table)
    dtype = _attn_dtype(q, k_cache, v_cache)
    if q.dim() != 3 or q.stride(-1) != 1:
        raise _lib.NvkError("q must be [batch, heads, head_dim] with unit last stride")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or k_cache.shape != v_cache.shape:
        raise _lib.NvkError("k_cache/v_cache must be contiguous [num_blocks, block_size, Hkv, D]")
    b, hq, d = q.shape
    num_blocks, block_size, hkv, dk = k_cache.shape
    if dk != d:
        raise _lib.NvkError("q and cache head_dim differ")
    bt = _int32(block_table)
    lens = _int32(context_lens)
    if bt.dim() != 2 or bt.shape[0] != b or lens.numel() != b:
        raise _lib.NvkError("block_table must be [batch, max_blocks] and cache_seqlens [batch]")
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=dev)
    scale = float(softmax_scale) if softmax_scale is not None else d ** -0.5
    lib = _lib.load()
    max_blocks = bt.shape[1]
    ws_bytes = lib.nvk_paged_decode_workspace_size(b, hq, hkv, d, block_size, max_blocks)
    ws = _lib.workspace(dev, ws_bytes)
    with torch.cuda.device(dev):
        code = lib.nvk_paged_decode(
            q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
            bt.data_ptr(), bt.stride(0), lens.data_ptr(), b, hq, hkv, d, block_size, max_blocks,
            num_blocks, scale, out.data_ptr(), out.stride(0), out.stride(1),
            _lib.ptr(ws), ws_bytes, dtype, _lib.stream_ptr(dev))
    _lib.check(code)
    return out


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                           softcap=0.0, alibi_slopes=None, deterministic=False,
                           return_attn_probs=False, block_table=None):
    """Drop-in for flash_attn.flash_attn_varlen_func as used at
    nanovllm/layers/attention.py:67-70 (causal=True, optional block_table)."""
    _unsupported(dropout_p=(dropout_p, 0.0), causal=(causal, True),
                 window_size=(tuple(window_size), (-1, -1)), softcap=(softcap, 0.0),
                 alibi_slopes=(alibi_slopes, None), return_attn_probs=(return_attn_probs, False))
    return varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, softmax_scale,
                          block_table=block_table, max_seqlen_k=max_seqlen_k)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None,
                            block_table=None, softmax_scale=None, causal=False,
                            window_size=(-1, -1), softcap=0.0, rotary_interleaved=True,
                            alibi_slopes=None, num_splits=0, return_softmax_lse=False):
    """Drop-in for flash_attn.flash_attn_with_kvcache as used at
    nanovllm/layers/attention.py:72-74.

    q: [B, Sq, Hq, D].  Sq == 1 runs the split-K decode kernel.  Sq > 1 (e.g.
    speculative-decode verification) runs the causal varlen kernel with the
    query block aligned to the end of each sequence's cache_seqlens keys.
    Without block_table the caches are [B, S, Hkv, D]: sequence b is then one
    page of S slots.
    """
    _unsupported(k=(k, None), v=(v, None), rotary_cos=(rotary_cos, None),
                 rotary_sin=(rotary_sin, None), cache_batch_idx=(cache_batch_idx, None),
                 cache_leftpad=(cache_leftpad, None), window_size=(tuple(window_size), (-1, -1)),
                 softcap=(softcap, 0.0), alibi_slopes=(alibi_slopes, None),
                 return_softmax_lse=(return_softmax_lse, False))
    if q.dim() != 4:
        raise _lib.NvkError("q must be [batch, seqlen_q, heads, head_dim]")
    b, sq, hq, d = q.shape
    dev = _lib.require_gpu(q, k_cache, v_cache)
    if cache_seqlens is None:
        raise NotImplementedError("nanovllm_amd: cache_seqlens is required")
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((b,), cache_seqlens, dtype=torch.int32, device=dev)
    if block_table is None:
        block_table = torch.arange(b, dtype=torch.int32, device=dev).view(b, 1)
    if sq == 1:
        out = paged_decode(q[:, 0], k_cache, v_cache, cache_seqlens, block_table, softmax_scale)
        return out.view(b, 1, hq, d)
    if not causal:
        raise NotImplementedError("nanovllm_amd: seqlen_q > 1 needs causal=True")
    lens = _int32(cache_seqlens)
    cu = torch.empty(2, b + 1, dtype=torch.int32, device=dev)   # cu_seqlens_q, cu_seqlens_k
    with torch.cuda.device(dev):
        code = _lib.load().nvk_uniform_cu_seqlens(lens.data_ptr(), b, sq, cu[0].data_ptr(),
                                                  cu[1].data_ptr(), _lib.stream_ptr(dev))
    _lib.check(code)
    cu_q, cu_k = cu[0], cu[1]
    qf = q.reshape(b * sq, hq, d)
    out = varlen_prefill(qf, k_cache, v_cache, cu_q, cu_k, sq, softmax_scale,
                         block_table=block_table)
    return out.view(b, sq, hq, d)
