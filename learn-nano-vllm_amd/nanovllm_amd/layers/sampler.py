"""Drop-in for nanovllm/layers/sampler.py and the last-token selection of
nanovllm/layers/embed_head.py:56-60 on MI355X.

``Sampler().forward(logits, temperatures)`` keeps the reference's signature
and distribution: token i with probability softmax(logits / T)_i, drawn by
libnvk.so (``nvk_sample``) in a single read of the logits.  Without the
caller's noise the draw is an inverse transform with uniforms from a Philox
stream seeded from torch's CPU generator (so torch.manual_seed makes runs
repeatable); with it (for checking against a reference draw) the reference's
argmax softmax(logits / T) / noise itself is evaluated.

``last_token_hidden`` / ``compute_logits`` are ParallelLMHead.forward for one
rank: in a prefill step only each sequence's last new token reaches the LM
head GEMM (a plain library GEMM, F.linear).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import get_context


class Sampler(nn.Module):
    """forward(logits [B, V] bf16/f32, temperatures [B] f32) -> int64 [B]."""

    def __init__(self):
        super().__init__()
        self._offset = 0

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor,
                noise: torch.Tensor | None = None) -> torch.Tensor:
        assert logits.dim() == 2 and logits.stride(-1) == 1
        b, v = logits.shape
        dev = _lib.require_gpu(logits, temperatures, noise)
        temps = temperatures.to(torch.float32).contiguous()
        assert temps.numel() == b
        if noise is not None:
            assert noise.shape == (b, v) and noise.dtype == torch.float32 and noise.stride(-1) == 1
        tokens = torch.empty(b, dtype=torch.int64, device=dev)
        seed = int(torch.randint(0, 2 ** 62, (1,)).item()) if noise is None else 0
        offset = self._offset
        self._offset += 1
        lib = _lib.load()
        ws_bytes = lib.nvk_sample_workspace_size(b, v)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            code = lib.nvk_sample(logits.data_ptr(), logits.stride(0), b, v, _lib.dtype_code(logits),
                                  temps.data_ptr(), _lib.ptr(noise),
                                  noise.stride(0) if noise is not None else 0, seed, offset,
                                  tokens.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev))
        _lib.check(code)
        return tokens


def last_token_hidden(x: torch.Tensor, cu_seqlens_q: torch.Tensor) -> torch.Tensor:
    """x[cu_seqlens_q[1:] - 1] (embed_head.py:57-59) by nvk_gather_last_tokens."""
    assert x.dim() == 2 and x.stride(-1) == 1
    b = cu_seqlens_q.numel() - 1
    dev = _lib.require_gpu(x, cu_seqlens_q)
    cu = cu_seqlens_q if cu_seqlens_q.dtype == torch.int32 else cu_seqlens_q.to(torch.int32)
    cu = cu.contiguous()
    out = torch.empty(b, x.shape[1], dtype=x.dtype, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        code = lib.nvk_gather_last_tokens(x.data_ptr(), x.stride(0), cu.data_ptr(), b, x.shape[1],
                                          _lib.dtype_code(x), out.data_ptr(), out.stride(0),
                                          _lib.stream_ptr(dev))
    _lib.check(code)
    return out


def compute_logits(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """ParallelLMHead.forward on one rank (embed_head.py:56-66)."""
    context = get_context()
    if context.is_prefill:
        x = last_token_hidden(x, context.cu_seqlens_q)
    return F.linear(x, weight)
