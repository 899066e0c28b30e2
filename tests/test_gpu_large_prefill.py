"""The reference's largest prefill calls, checked on the GPU.

* Warmup (ModelRunner.warmup_model, model_runner.py:91-101): with
  max_num_batched_tokens 16384 and max_model_len 4096 (config.py:9,11) the
  engine runs max(16384 // 4096, 1) = 4 sequences of 4096 tokens through the
  dense path (empty caches, block_tables None).  Each sequence then has 64
  query tiles per kv head, and the longest-first tile order spans many rounds
  of workgroups.
* A full chunked-prefill step of 16384 new tokens over a paged prefix
  (prepare_prefill, model_runner.py:129-170): 4 x 4096 new tokens after
  U{0..2048} cached, and 32 x 512 after U{0..3584} cached (mid-page starts).

Closed-form needles (tests/needles.py) need no oracle, so these run at the
full 16/8-head shape and put a needle on both sides of every 64-key tile edge
and every page edge.  The same lengths at 2/1 heads (G = 2, as Qwen3) are
also checked against the oracle within 2e-2 abs / 1e-2 rel, on random data
and through the Attention module for the warmup.
"""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, f32, oracle_prefill_paged, say
from needles import NeedleCase, run_schedule
from oracle import kv_oracle as orc
from oracle import step_metadata as metadata
from oracle.sequence import Sequence
from nanovllm_amd import Attention, varlen_prefill
from nanovllm_amd.utils.context import reset_context
from test_gpu_prefill_split import _paged_case

pytestmark = pytest.mark.gpu

WARMUP = [4096] * 4    # model_runner.py:91-101 with config.py's defaults


def _lens(seed, n, lo, hi):
    return [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, n)]


STEPS = {
    "4 x 4096 new after U{0..2048} cached": ([4096] * 4, _lens(90, 4, 0, 2048)),
    "32 x 512 new after U{0..3584} cached": ([512] * 32, _lens(91, 32, 0, 3584)),
}


def _prefill(case):
    return varlen_prefill(case.q, case.k, case.v, case.cu_q, case.cu_k, max(case.lens_q),
                          case.scale, block_table=case.block_tables,
                          max_seqlen_k=max(case.lens_k))


def test_warmup_shape_dense_needles():
    case = NeedleCase(20, WARMUP, WARMUP, block_size=0)
    run_schedule(case, _prefill, 64, "warmup 4 x 4096 dense")


@pytest.mark.parametrize("name", list(STEPS))
def test_16k_token_paged_step_needles(name):
    lens_q, cached = STEPS[name]
    lens_k = [q + c for q, c in zip(lens_q, cached)]
    assert sum(lens_q) == 16384
    case = NeedleCase(21, lens_q, lens_k, block_size=256)
    run_schedule(case, _prefill, 64, f"paged step {name}")


@pytest.mark.parametrize("name", list(STEPS))
def test_16k_token_paged_step_oracle_two_heads(name):
    lens_q, cached = STEPS[name]
    lens_k = [q + c for q, c in zip(lens_q, cached)]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(22, lens_q, lens_k, hq=2, hkv=1)
    say(f"paged step {name}, 2/1 heads, against the oracle")
    out = varlen_prefill(q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q),
                         128 ** -0.5, block_table=bt.cuda(), max_seqlen_k=max(lens_k))
    torch.cuda.synchronize()
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, 256, 128 ** -0.5)
    assert_attn_close(out, ref, f"paged step {name}, 2/1 heads")


def test_warmup_through_attention_module_two_heads():
    """Attention.forward in the warmup step: empty caches, so no store and the
    dense varlen call (attention.py:59-70), at the warmup's 4 x 4096 tokens."""
    hq, hkv, hd = 2, 1, 128
    Sequence.block_size = 256
    seqs = [Sequence([0] * n, num_scheduled_tokens=n) for n in WARMUP]
    metadata.prepare_prefill(seqs, 256)
    gen = torch.Generator().manual_seed(23)
    n = sum(WARMUP)
    q = torch.randn(n, hq, hd, generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn(n, hkv, hd, generator=gen).to(torch.bfloat16).cuda()
    v = torch.randn(n, hkv, hd, generator=gen).to(torch.bfloat16).cuda()
    attn = Attention(hq, hd, hd ** -0.5, hkv)
    say("warmup 4 x 4096 through Attention, 2/1 heads")
    try:
        o = attn(q, k, v)
        torch.cuda.synchronize()
    finally:
        reset_context()
    cu = np.concatenate([[0], np.cumsum(WARMUP)])
    ref = orc.paged_attention(f32(q), f32(k), f32(v), cu, WARMUP, hd ** -0.5, cu_seqlens_k=cu)
    assert o.shape == (n, hq, hd)
    assert_attn_close(o, ref, "warmup through the module")
