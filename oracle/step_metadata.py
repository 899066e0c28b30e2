"""Host restatement of the reference's attention-metadata builders.

TEST INFRASTRUCTURE ONLY, like the rest of oracle/: tests/ and the
cpu_baseline leg of bench.py use it as the parity reference of the device builders
(nanovllm_amd/engine/device_metadata.py) and as the timed host path; the
product never imports it.

Same outputs, dtypes and conventions as ModelRunner.prepare_block_tables /
prepare_prefill / prepare_decode (nanovllm/engine/model_runner.py:123-188)
and the graph-replay padding of run_model (model_runner.py:200-211):

* block tables are int32 [B, W], each row padded with -1 to the batch max;
* prefill: cu_seqlens_q over the scheduled (new) tokens, cu_seqlens_k over
  cached + new tokens, slot_mapping by page-range expansion, block_tables
  only when some sequence has cached tokens (cu_seqlens_k[-1] > cu_seqlens_q[-1]);
  sequences without a block table (warmup) contribute no slots;
* decode: slot = block_table[-1]*block_size + last_block_num_tokens - 1 and
  context_lens = len(seq), which counts the token being stored;
* graph replay: rows past the live batch get slot -1 and context length 0,
  and only the live [:bs, :w] rectangle of the table is refreshed.

The per-token Python loops are the reference's; they run on the host.
"""
from __future__ import annotations

import torch

from nanovllm_amd.utils.context import set_context


def _to_device(values, dtype, device):
    t = torch.tensor(values, dtype=dtype)
    if device is not None and torch.device(device).type == "cuda":
        t = t.pin_memory().to(device, non_blocking=True)
    elif device is not None:
        t = t.to(device)
    return t


def prepare_block_tables(seqs, device="cuda"):
    max_len = max(len(seq.block_table) for seq in seqs)
    block_tables = [seq.block_table + [-1] * (max_len - len(seq.block_table)) for seq in seqs]
    return _to_device(block_tables, torch.int32, device)


def prefill_slots(seq, block_size):
    """Cache slots of tokens [num_cached_tokens, num_cached+num_scheduled) of seq."""
    start = seq.num_cached_tokens
    end = start + seq.num_scheduled_tokens
    slots = []
    if not seq.block_table:
        return slots
    start_block = start // block_size
    end_block = (end + block_size - 1) // block_size
    for i in range(start_block, end_block):
        first = start % block_size if i == start_block else 0
        last = end - i * block_size if i == end_block - 1 else block_size
        base = seq.block_table[i] * block_size
        slots.extend(range(base + first, base + last))
    return slots


def prepare_prefill(seqs, block_size, device="cuda"):
    input_ids, positions, slot_mapping = [], [], []
    cu_seqlens_q, cu_seqlens_k = [0], [0]
    max_seqlen_q = max_seqlen_k = 0
    block_tables = None
    for seq in seqs:
        start = seq.num_cached_tokens
        seqlen_q = seq.num_scheduled_tokens
        end = start + seqlen_q
        input_ids.extend(seq[start:end])
        positions.extend(range(start, end))
        cu_seqlens_q.append(cu_seqlens_q[-1] + seqlen_q)
        cu_seqlens_k.append(cu_seqlens_k[-1] + end)
        max_seqlen_q = max(seqlen_q, max_seqlen_q)
        max_seqlen_k = max(end, max_seqlen_k)
        slot_mapping.extend(prefill_slots(seq, block_size))
    if cu_seqlens_k[-1] > cu_seqlens_q[-1]:    # some sequence has cached tokens
        block_tables = prepare_block_tables(seqs, device)
    input_ids = _to_device(input_ids, torch.int64, device)
    positions = _to_device(positions, torch.int64, device)
    cu_q = _to_device(cu_seqlens_q, torch.int32, device)
    cu_k = _to_device(cu_seqlens_k, torch.int32, device)
    slots = _to_device(slot_mapping, torch.int32, device)
    set_context(True, cu_q, cu_k, max_seqlen_q, max_seqlen_k, slots, None, block_tables)
    return input_ids, positions


def prepare_decode(seqs, block_size, device="cuda"):
    input_ids, positions, slot_mapping, context_lens = [], [], [], []
    for seq in seqs:
        input_ids.append(seq.last_token)
        positions.append(len(seq) - 1)
        context_lens.append(len(seq))
        slot_mapping.append(seq.block_table[-1] * block_size + seq.last_block_num_tokens - 1)
    input_ids = _to_device(input_ids, torch.int64, device)
    positions = _to_device(positions, torch.int64, device)
    slots = _to_device(slot_mapping, torch.int32, device)
    lens = _to_device(context_lens, torch.int32, device)
    block_tables = prepare_block_tables(seqs, device)
    set_context(False, slot_mapping=slots, context_lens=lens, block_tables=block_tables)
    return input_ids, positions


class DecodeGraphBuffers:
    """Static decode metadata of a captured decode step (model_runner.py:228-232).

    ``load`` refreshes them before a replay the way run_model does
    (model_runner.py:204-210): slots of padded rows -1, their context length
    0, and only the live [:bs, :w] rectangle of the block table rewritten.
    """

    def __init__(self, max_bs, max_num_blocks, device="cuda"):
        self.slot_mapping = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.context_lens = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.block_tables = torch.zeros(max_bs, max_num_blocks, dtype=torch.int32, device=device)

    def load(self, slot_mapping, context_lens, block_tables):
        bs = slot_mapping.numel()
        self.slot_mapping.fill_(-1)
        self.slot_mapping[:bs] = slot_mapping
        self.context_lens.zero_()
        self.context_lens[:bs] = context_lens
        self.block_tables[:bs, :block_tables.size(1)] = block_tables
