"""Bucketed HIP-graph capture and replay of a decode step.

The reference captures one CUDA graph per batch-size bucket and replays the
smallest bucket that holds the live batch (ModelRunner.capture_cudagraph /
run_model, nanovllm/engine/model_runner.py:195-257):

* buckets [1, 2, 4, 8, 16, 32, ..., max_bs], captured largest first, all in
  one graph memory pool;
* static metadata buffers (slot_mapping, context_lens, block_tables) sized for
  max_bs, all zero while capturing (a warmup run precedes each capture);
* before a replay: live rows copied in, slot_mapping of the padded rows set to
  -1, their context length to 0, and only the live [:bs, :w] rectangle of the
  block table rewritten (the rest keeps stale entries).

``DecodeGraphRunner`` does the same for any decode step function, so the
attention path of this package (the fused prologue, the store and the paged
decode of every layer) runs under exactly that capture / padding contract.
The kernels allocate nothing, read no metadata on the host and skip padded
rows (slot -1 writes nothing, context 0 writes zeros, table entries past a
context are never read), which is what makes the replay valid.
"""
from __future__ import annotations

from typing import Callable

import torch

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import get_context, reset_context, set_context


def graph_buckets(max_bs: int) -> list[int]:
    """model_runner.py:234: [1, 2, 4, 8] + multiples of 16 up to max_bs."""
    return [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 16))


class DecodeGraphRunner:
    """step(positions [bs], **inputs [bs, ...]) -> tensor [bs, ...] is captured
    once per bucket; ``run`` replays the bucket that holds the live batch.

    inputs: name -> (per-row shape, dtype) of the static input buffers;
    output: (per-row shape, dtype) of the static output buffer.
    """

    def __init__(self, step: Callable[..., torch.Tensor], max_bs: int, max_num_blocks: int,
                 inputs: dict[str, tuple[tuple[int, ...], torch.dtype]],
                 output: tuple[tuple[int, ...], torch.dtype], device="cuda"):
        self.step = step
        self.max_bs = max_bs
        self.buckets = graph_buckets(max_bs)
        if self.buckets[-1] != max_bs:
            self.buckets.append(max_bs)
        z = lambda *shape, dtype: torch.zeros(*shape, dtype=dtype, device=device)
        self.positions = z(max_bs, dtype=torch.int64)
        self.slot_mapping = z(max_bs, dtype=torch.int32)
        self.context_lens = z(max_bs, dtype=torch.int32)
        self.block_tables = z(max_bs, max_num_blocks, dtype=torch.int32)
        self.inputs = {name: z(max_bs, *shape, dtype=dt) for name, (shape, dt) in inputs.items()}
        self.outputs = z(max_bs, *output[0], dtype=output[1])
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        pool = None
        for bs in reversed(self.buckets):                   # model_runner.py:236-248
            graph = torch.cuda.CUDAGraph()
            set_context(False, slot_mapping=self.slot_mapping[:bs],
                        context_lens=self.context_lens[:bs], block_tables=self.block_tables[:bs])
            self.outputs[:bs] = self._call(bs)              # warmup
            with torch.cuda.graph(graph, pool):
                self.outputs[:bs] = self._call(bs)          # capture
            if pool is None:
                pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
            reset_context()

    def _call(self, bs: int) -> torch.Tensor:
        return self.step(self.positions[:bs], **{k: v[:bs] for k, v in self.inputs.items()})

    def bucket(self, bs: int) -> int:
        return next(x for x in self.buckets if x >= bs)

    def replay(self, bs: int, **inputs: torch.Tensor) -> torch.Tensor:
        """Replay the bucket of a live batch of bs whose metadata and positions
        are already in the static buffers (written by
        device_metadata.prepare_decode_device(..., into=self)); ``inputs``
        are copied into the live rows first.  Returns outputs[:bs]."""
        if bs > self.max_bs:
            raise ValueError(f"batch {bs} above the largest captured bucket {self.max_bs}")
        for name, value in inputs.items():
            self.inputs[name][:bs] = value
        self.graphs[self.bucket(bs)].replay()
        return self.outputs[:bs]

    def run(self, positions: torch.Tensor, **inputs: torch.Tensor) -> torch.Tensor:
        """Replay for the live batch; metadata from get_context() (prepare_decode),
        as run_model does (model_runner.py:200-211).  Returns outputs[:bs] (a
        view of the static buffer, overwritten by the next replay)."""
        bs = positions.numel()
        if bs > self.max_bs:
            raise ValueError(f"batch {bs} above the largest captured bucket {self.max_bs}")
        context = get_context()
        graph = self.graphs[self.bucket(bs)]
        for name, value in inputs.items():
            self.inputs[name][:bs] = value
        # run_model's refresh (slots -1 and contexts 0 past the live batch, the
        # live block-table rectangle copied) in one kernel
        # the refresh kernel reads these through raw pointers: they must live on
        # the graph's GPU (the copies run_model makes would also accept host or
        # other-device tensors; those are moved first)
        dev = self.positions.device
        pos = positions.to(device=dev, dtype=torch.int64).contiguous()
        slots = context.slot_mapping.to(device=dev, dtype=torch.int32).contiguous()
        lens = context.context_lens.to(device=dev, dtype=torch.int32).contiguous()
        bt = context.block_tables.to(device=dev, dtype=torch.int32)
        _lib.require_gpu(pos, slots, lens, bt)
        if bt.dim() != 2 or bt.size(0) != bs or bt.size(1) > self.block_tables.size(1):
            raise ValueError(f"block_tables {tuple(bt.shape)} for batch {bs} and a static "
                             f"width of {self.block_tables.size(1)}")
        if bt.stride(1) != 1:
            bt = bt.contiguous()
        if slots.numel() != bs or lens.numel() != bs:
            raise ValueError("slot_mapping and context_lens need one entry per sequence")
        _lib.check(_lib.load().nvk_decode_graph_refresh(
            pos.data_ptr(), slots.data_ptr(), lens.data_ptr(), bt.data_ptr(), bt.stride(0), bs,
            bt.size(1), self.positions.data_ptr(), self.slot_mapping.data_ptr(),
            self.context_lens.data_ptr(), self.block_tables.data_ptr(), self.block_tables.stride(0),
            self.max_bs, _lib.stream_ptr(self.positions.device)))
        graph.replay()
        return self.outputs[:bs]
