"""The configurations at their full size on the GPU, against the oracle.

* One layer of the mixed chunked-prefill + decode step at its size: 8 chunks
  of 512 new tokens after U{0..1536} cached ones plus 192 decodes over
  U{256..4096}, 4288 tokens stored first into a 3300-page pool (the same
  block tables and slots every layer of the step uses).  Store bit for bit
  (the oracle's index assignment over the whole cache), attention within
  2e-2 abs / 1e-2 rel.
* Decode at the reference's larger graph batches (model_runner.py:226,234:
  up to 512 sequences) with contexts up to max_model_len 4096 (config.py:11).

Data are N(0, 1) bf16 drawn on the GPU from a seeded generator; the oracle
reads bit patterns and widens only the rows a sequence uses.
"""
import numpy as np
import pytest
import torch

from gpu_utils import assert_attn_close, bits, oracle_paged_bits, say
from oracle import kv_oracle as orc
from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill
from nanovllm_amd.workloads import mixed_step_metadata

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 16, 8, 128, 256


def _randn(gen, *shape):
    return torch.randn(*shape, generator=gen, device="cuda").to(torch.bfloat16)


def _pool(gen, nb):
    kc = torch.empty(nb, BS, HKV, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    for x in (kc, vc):
        for i in range(0, nb, 512):
            x[i:i + 512] = _randn(gen, min(512, nb - i), BS, HKV, D)
    return kc, vc


def test_mixed_step_layer_at_full_size():
    tens, meta = mixed_step_metadata()             # 8 x 512 after U{0..1536}; 192 x U{256..4096}
    t = {k: v.cuda() for k, v in tens.items()}
    gen = torch.Generator(device="cuda").manual_seed(30)
    n_tok = meta["n_tokens"]
    assert n_tok == 8 * 512 + 192 and len(meta["dec_lens"]) == 192
    kc, vc = _pool(gen, meta["pool_blocks"])
    q_pf, q_dec = _randn(gen, 8 * 512, HQ, D), _randn(gen, 192, HQ, D)
    key, value = _randn(gen, n_tok, HKV, D), _randn(gen, n_tok, HKV, D)
    kc0, vc0 = bits(kc), bits(vc)
    say("mixed layer at full size: store 4288 tokens")
    store_kvcache(key, value, kc, vc, t["slot_mapping"])
    say("mixed layer at full size: 8 prefill chunks of 512")
    o_pf = varlen_prefill(q_pf, kc, vc, t["cu_seqlens_q"], t["cu_seqlens_k"],
                          meta["max_seqlen_q"], 128 ** -0.5,
                          block_table=t["prefill_block_tables"],
                          max_seqlen_k=meta["max_seqlen_k"])
    say("mixed layer at full size: 192 decodes")
    o_dec = paged_decode(q_dec, kc, vc, t["context_lens"], t["decode_block_tables"],
                         128 ** -0.5)
    torch.cuda.synchronize()
    orc.kv_store(bits(key), bits(value), kc0, vc0, tens["slot_mapping"].numpy())
    assert np.array_equal(bits(kc), kc0), "k cache differs from the oracle's store"
    assert np.array_equal(bits(vc), vc0), "v cache differs from the oracle's store"
    ref_pf = oracle_paged_bits(q_pf, kc, vc, tens["prefill_block_tables"],
                               tens["cu_seqlens_q"], np.asarray(meta["lens_k"]), BS, 128 ** -0.5)
    assert_attn_close(o_pf, ref_pf, "mixed step: prefill chunks")
    ref_dec = oracle_paged_bits(q_dec, kc, vc, tens["decode_block_tables"], np.arange(193),
                                tens["context_lens"], BS, 128 ** -0.5)
    assert_attn_close(o_dec, ref_dec, "mixed step: decodes")


def _decode_batch(seed, batch, lo, hi, nb=1024):
    """batch sequences over U{lo..hi} keys; pages drawn from a shared read-only
    pool (distinct inside a sequence, shared across sequences as prefix
    caching shares them)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, batch)
    w = int(-(-int(lens.max()) // BS))
    bt = np.full((batch, w), -1, np.int32)
    for i, n in enumerate(lens):
        need = -(-int(n) // BS)
        bt[i, :need] = rng.choice(nb, need, replace=False)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    kc, vc = _pool(gen, nb)
    q = _randn(gen, batch, HQ, D)
    return q, kc, vc, torch.from_numpy(bt), torch.from_numpy(lens.astype(np.int32))


@pytest.mark.parametrize("batch,lo,hi", [(128, 1, 4096), (256, 1024, 4096), (512, 256, 4096)])
def test_decode_large_batches_long_contexts(batch, lo, hi):
    q, kc, vc, bt, lens = _decode_batch(60 + batch, batch, lo, hi)
    say(f"decode batch {batch} over U{{{lo}..{hi}}}")
    out = paged_decode(q, kc, vc, lens.cuda(), bt.cuda(), 128 ** -0.5)
    torch.cuda.synchronize()
    ref = oracle_paged_bits(q, kc, vc, bt, np.arange(batch + 1), lens, BS, 128 ** -0.5)
    assert_attn_close(out, ref, f"decode batch {batch}")
