"""Per-forward attention metadata, the side channel between the runner and
``Attention.forward``.

Same record, same module-global lifecycle and same function signatures as
nanovllm/utils/context.py:5-27, because two readers depend on them:
``Attention.forward`` (nanovllm/layers/attention.py:60) and the LM head's
last-token selection (nanovllm/layers/embed_head.py:57-60).

Fields (all device tensors are int32):
  is_prefill      True for a prefill / chunked-prefill step, False for decode.
  cu_seqlens_q    [B+1] prefix sums of the new (query) tokens per sequence.
  cu_seqlens_k    [B+1] prefix sums of cached + new tokens per sequence.
  max_seqlen_q/k  host ints; max_seqlen_q sizes the prefill grid.
  slot_mapping    [N] flat cache slot of every new token, -1 = do not store.
  context_lens    [B] decode only: tokens in the cache, counting the new one.
  block_tables    [B, W] page ids padded with -1, or None (no cached prefix).
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
