"""Device-side builders of the step metadata (the reference's prepare_prefill /
prepare_decode, model_runner.py:123-188, without their per-token loops).

The host gathers per-sequence numbers only -- cached and scheduled token
counts (prefill) or lengths (decode) -- and the block tables as one
concatenated id list with row offsets, uploads them in a single pinned copy,
and one libnvk.so kernel (``nvk_prefill_metadata`` / ``nvk_decode_metadata``)
expands them into exactly the reference's tensors: cu_seqlens_q/k, positions
(int64), slot_mapping, the -1 padded block tables, context_lens.  The token
ids themselves (input_ids) are sequence data and are still gathered on the
host, by slices into a typed array instead of a Python loop per token.

``prepare_decode_device(..., into=runner)`` writes the decode metadata
straight into a DecodeGraphRunner's static buffers with the graph padding of
run_model (model_runner.py:204-210) for the rows up to the replayed bucket.
"""
from __future__ import annotations

from array import array
from itertools import accumulate, chain

import torch

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import set_context


def pack_block_tables(seqs):
    """(row offsets [B+1], concatenated page ids, table width) of the
    sequences' block tables: the compressed form of prepare_block_tables."""
    lens = [len(s.block_table) for s in seqs]
    offsets = [0] + list(accumulate(lens))
    ids = list(chain.from_iterable(s.block_table for s in seqs))
    return offsets, ids, max(lens) if lens else 0


def _upload(values: array, device):
    """One pinned host-to-device copy of a typed array ('i' int32 / 'q' int64)."""
    dtype = torch.int32 if values.typecode == "i" else torch.int64
    if len(values) == 0:
        return torch.empty(0, dtype=dtype, device=device)
    host = torch.frombuffer(values, dtype=dtype)
    return host.pin_memory().to(device, non_blocking=True)


def prepare_prefill_device(seqs, block_size, device="cuda"):
    """prepare_prefill (model_runner.py:129-170) with the expansion on the GPU.
    Sets the Context and returns (input_ids, positions) like the reference."""
    dev = torch.device(device)
    b = len(seqs)
    cached = [s.num_cached_tokens for s in seqs]
    new = [s.num_scheduled_tokens for s in seqs]
    offsets, ids, width = pack_block_tables(seqs)
    n_tokens = sum(new)
    max_q = max(new)
    max_k = max(c + n for c, n in zip(cached, new))
    packed = _upload(array("i", cached + new + offsets + ids), dev)
    tokens = array("q")
    for s, c, n in zip(seqs, cached, new):
        tokens.extend(s[c:c + n])
    input_ids = _upload(tokens, dev)
    cu_q = torch.empty(b + 1, dtype=torch.int32, device=dev)
    cu_k = torch.empty(b + 1, dtype=torch.int32, device=dev)
    positions = torch.empty(n_tokens, dtype=torch.int64, device=dev)
    slots = torch.empty(n_tokens, dtype=torch.int32, device=dev)
    # block_tables only with a cached prefix (cu_seqlens_k[-1] > cu_seqlens_q[-1], line 162)
    tables = torch.empty(b, width, dtype=torch.int32, device=dev) if sum(cached) > 0 else None
    p = packed.data_ptr()
    i32 = packed.element_size()
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.nvk_prefill_metadata(
            p, p + b * i32, p + 2 * b * i32, p + (3 * b + 1) * i32 if ids else None, b, block_size,
            width, n_tokens, cu_q.data_ptr(), cu_k.data_ptr(), positions.data_ptr(),
            slots.data_ptr(), _lib.ptr(tables), _lib.stream_ptr(dev))
    _lib.check(code)
    if not ids:      # warmup: no sequence has pages, the reference gathers no slots (line 149)
        slots = slots[:0]
    set_context(True, cu_q, cu_k, max_q, max_k, slots, None, tables)
    return input_ids, positions


def prepare_decode_device(seqs, block_size, device="cuda", into=None):
    """prepare_decode (model_runner.py:172-188) with the expansion on the GPU.

    Without ``into``: fresh tensors, Context set, returns (input_ids, positions).
    With ``into`` (a DecodeGraphRunner): the metadata lands in its static
    buffers, rows up to the bucket of this batch padded (slot -1, context 0),
    the table written only in its live [:bs, :w] rectangle; the Context points
    at the live rows of the buffers (full table width, as during capture);
    replay with runner.replay(bs); returns (input_ids, runner.positions[:bs])."""
    dev = torch.device(device)
    b = len(seqs)
    lens = [len(s) for s in seqs]
    offsets, ids, width = pack_block_tables(seqs)
    packed = _upload(array("i", lens + offsets + ids), dev)
    input_ids = _upload(array("q", [s.last_token for s in seqs]), dev)
    if into is None:
        padded = b
        context_lens = torch.empty(b, dtype=torch.int32, device=dev)
        positions = torch.empty(b, dtype=torch.int64, device=dev)
        slots = torch.empty(b, dtype=torch.int32, device=dev)
        tables = torch.empty(b, width, dtype=torch.int32, device=dev)
    else:
        padded = into.bucket(b)
        context_lens, positions = into.context_lens, into.positions
        slots, tables = into.slot_mapping, into.block_tables
        if width > tables.shape[1]:
            raise ValueError(f"block table width {width} above the captured {tables.shape[1]}")
    p = packed.data_ptr()
    i32 = packed.element_size()
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.nvk_decode_metadata(
            p, p + b * i32, p + (2 * b + 1) * i32, b, padded, block_size, width, tables.stride(0),
            context_lens.data_ptr(), positions.data_ptr(), slots.data_ptr(), tables.data_ptr(),
            _lib.stream_ptr(dev))
    _lib.check(code)
    set_context(False, slot_mapping=slots[:b], context_lens=context_lens[:b],
                block_tables=tables[:b])
    return input_ids, positions[:b]
