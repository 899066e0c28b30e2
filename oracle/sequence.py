"""Token-sequence record with the block arithmetic the metadata builders use.

TEST INFRASTRUCTURE ONLY (see oracle/step_metadata.py): the input record of
the metadata tests.  The device builders take any object with these fields,
e.g. the reference's own Sequence.

Mirrors the fields and properties of nanovllm/engine/sequence.py:14-65 that
the KV-cache path reads: the token list, ``num_cached_tokens`` /
``num_scheduled_tokens`` (chunked prefill), the page list ``block_table`` and
the block math ``num_blocks`` / ``last_block_num_tokens``.  Scheduling state,
sampling parameters and pickling stay with the reference engine.
"""
from __future__ import annotations

from copy import copy
from itertools import count


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], block_table: list[int] | None = None,
                 num_cached_tokens: int = 0, num_scheduled_tokens: int = 0):
        self.seq_id = next(Sequence.counter)
        self.token_ids = copy(token_ids)
        self.last_token = token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(token_ids)
        self.num_cached_tokens = num_cached_tokens
        self.num_scheduled_tokens = num_scheduled_tokens
        self.block_table = list(block_table) if block_table else []

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self):
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
