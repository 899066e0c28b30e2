"""float16 attention on the GPU.  The reference runs attention in the model's
dtype (nanovllm/engine/model_runner.py:29 sets torch's default dtype from
hf_config.dtype) and flash-attn takes bf16 and fp16 alike, so the
decode, varlen prefill (paged, dense, split-K, short-query) and KV-store
accept fp16 tensors too: against the oracle within 2e-2 abs / 1e-2 rel, the
store bit for bit, and the closed-form needle checks, which must hold exactly.
Inputs are the bf16 workloads converted to fp16 (exact at these magnitudes)."""
import numpy as np
import pytest
import torch

from gpu_utils import (assert_attn_close, oracle_decode, oracle_prefill_dense,
                       oracle_prefill_paged, say)
from needles import NeedleCase, run_schedule
from oracle import kv_oracle as orc
from nanovllm_amd import (_lib, flash_attn_varlen_func, flash_attn_with_kvcache, paged_decode,
                          store_kvcache, varlen_prefill)
from nanovllm_amd.workloads import decode_case, prefill_case, spec_verify_case

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _h(t):
    return t.to(F16)


def test_fp16_decode_batch64():
    case = decode_case(seed=90, pool_blocks=600)
    c = case.to("cuda")
    say("fp16 decode B=64")
    out = paged_decode(_h(c.q), _h(c.k_cache), _h(c.v_cache), c.context_lens, c.block_tables,
                       case.scale)
    torch.cuda.synchronize()
    assert out.dtype == F16
    ref = oracle_decode(_h(case.q), _h(case.k_cache), _h(case.v_cache), case.block_tables,
                        case.context_lens, case.block_size, case.scale)
    assert_attn_close(out, ref, "fp16 decode")


@pytest.mark.parametrize("hq,hkv,hd", [(16, 16, 128), (16, 2, 128), (8, 2, 64)])
def test_fp16_decode_groups_and_head_dim_64(hq, hkv, hd):
    case = decode_case(seed=91, hq=hq, hkv=hkv, hd=hd, ctx=[1, 33, 700, 2500], pool_blocks=20)
    c = case.to("cuda")
    say(f"fp16 decode {hq}/{hkv} d={hd}")
    out = paged_decode(_h(c.q), _h(c.k_cache), _h(c.v_cache), c.context_lens, c.block_tables,
                       case.scale)
    torch.cuda.synchronize()
    ref = oracle_decode(_h(case.q), _h(case.k_cache), _h(case.v_cache), case.block_tables,
                        case.context_lens, case.block_size, case.scale)
    assert_attn_close(out, ref, f"fp16 decode {hq}/{hkv}")


def test_fp16_store_then_paged_prefill():
    case = prefill_case(seed=92)              # 32 seqs: 512-token prefix + U{100..1024}
    c = case.to("cuda")
    kc, vc = _h(c.k_cache), _h(c.v_cache)
    say("fp16 store + prefill 32 seqs")
    store_kvcache(_h(c.key), _h(c.value), kc, vc, c.slot_mapping)
    out = flash_attn_varlen_func(_h(c.q), kc, vc, c.cu_seqlens_q, c.cu_seqlens_k,
                                 case.max_seqlen_q, case.max_seqlen_k, softmax_scale=case.scale,
                                 causal=True, block_table=c.block_tables)
    torch.cuda.synchronize()
    assert out.dtype == F16
    # the store is a bit copy whatever the 16-bit type
    kc_ref = _h(case.k_cache).clone().view(-1, 8, 128)
    vc_ref = _h(case.v_cache).clone().view(-1, 8, 128)
    sl = case.slot_mapping.long()
    kc_ref[sl] = _h(case.key)
    vc_ref[sl] = _h(case.value)
    assert torch.equal(kc.cpu().view(-1, 8, 128), kc_ref)
    assert torch.equal(vc.cpu().view(-1, 8, 128), vc_ref)
    ref = oracle_prefill_paged(_h(case.q), kc_ref.view(kc.shape), vc_ref.view(vc.shape),
                               case.block_tables, case.cu_seqlens_q, case.cu_seqlens_k,
                               case.block_size, case.scale)
    assert_attn_close(out, ref, "fp16 paged prefill")


def test_fp16_dense_prefill_and_split_k():
    gen = torch.Generator().manual_seed(93)
    lens = [1, 127, 128, 129, 300]
    tq = sum(lens)
    q, k, v = (torch.randn(tq, h, 128, generator=gen).to(F16) for h in (16, 8, 8))
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    say("fp16 dense prefill")
    out = flash_attn_varlen_func(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), max(lens),
                                 max(lens), softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_prefill_dense(q, k, v, cu, cu, 128 ** -0.5), "fp16 dense")
    # two short query ranges over long dense keys: the split-K path and its merge
    lq, lk = [20, 7], [5000, 3000]
    q = torch.randn(sum(lq), 16, 128, generator=gen).to(F16)
    k, v = (torch.randn(sum(lk), 8, 128, generator=gen).to(F16) for _ in range(2))
    cu_q = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32)
    say("fp16 dense split-K")
    out = varlen_prefill(q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), max(lq),
                         128 ** -0.5, max_seqlen_k=max(lk))
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_prefill_dense(q, k, v, cu_q, cu_k, 128 ** -0.5), "fp16 split")


def test_fp16_spec_verify_short_query_kernels():
    case = spec_verify_case(batch=8, ctx_hi=4096, pool_blocks=140)
    c = case.to("cuda")
    kc, vc = _h(c.k_cache), _h(c.v_cache)
    store_kvcache(_h(c.key), _h(c.value), kc, vc, c.slot_mapping)
    say("fp16 spec verify")
    out = flash_attn_with_kvcache(_h(c.q).view(8, 6, 16, 128), kc, vc,
                                  cache_seqlens=c.context_lens, block_table=c.block_tables,
                                  softmax_scale=case.scale, causal=True)
    torch.cuda.synchronize()
    ref = oracle_prefill_paged(_h(c.q).cpu(), kc.cpu(), vc.cpu(), case.block_tables,
                               case.cu_seqlens_q, case.cu_seqlens_k, 256, case.scale)
    assert_attn_close(out.view(-1, 16, 128), ref, "fp16 spec verify")


def test_fp16_needles_decode_prefill_short_query():
    def dec(c):
        lens = c.cu_k[1:] - c.cu_k[:-1]
        return paged_decode(c.q, c.k, c.v, lens, c.block_tables, c.scale)

    def pre(c):
        return varlen_prefill(c.q, c.k, c.v, c.cu_q, c.cu_k, max(c.lens_q), c.scale,
                              block_table=c.block_tables, max_seqlen_k=max(c.lens_k))

    rng = np.random.default_rng(94)
    lens = [int(x) for x in rng.integers(100, 2049, 64)]
    run_schedule(NeedleCase(95, [1] * 64, lens, dtype=F16), dec, 32, "fp16 decode")
    lq = [int(x) for x in rng.integers(100, 700, 12)]
    run_schedule(NeedleCase(96, lq, [512 + x for x in lq], dtype=F16), pre, 64, "fp16 prefill")
    lk = [int(x) for x in rng.integers(1024, 6000, 12)]
    run_schedule(NeedleCase(97, [6] * 12, lk, dtype=F16), pre, 64, "fp16 short query")
    # 32 x 6 over contexts up to 8192: the short-query kernel with K staged in LDS
    lk = [int(x) for x in rng.integers(1024, 8193, 32)]
    run_schedule(NeedleCase(100, [6] * 32, lk, dtype=F16), pre, 64, "fp16 short query, K in LDS")
    # 2 x 6 over long contexts: every group cut into ~64 parts, sliced combine
    run_schedule(NeedleCase(101, [6] * 2, [9000, 12000], dtype=F16), pre, 64,
                 "fp16 short query, sliced combine")


def test_fp16_noalloc_decode_matches_workspace_decode():
    case = decode_case(seed=98, ctx=[5, 2000, 0, 777], pool_blocks=16)
    c = case.to("cuda")
    q, kc, vc = _h(c.q), _h(c.k_cache), _h(c.v_cache)
    ref = paged_decode(q, kc, vc, c.context_lens, c.block_tables, case.scale)
    out = torch.full_like(ref, float("nan"))
    lib = _lib.load()
    bt = c.block_tables
    say("fp16 no-alloc decode")
    rc = lib.nvk_paged_decode_noalloc(q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(),
                                      vc.data_ptr(), bt.data_ptr(), bt.stride(0),
                                      c.context_lens.data_ptr(), 4, 16, 8, 128, 256, bt.shape[1],
                                      kc.shape[0], case.scale, out.data_ptr(), out.stride(0),
                                      out.stride(1), _lib.NVK_DTYPE_F16,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_mixed_dtypes_are_rejected():
    case = decode_case(seed=99, ctx=[10], pool_blocks=2).to("cuda")
    with pytest.raises(_lib.NvkError):
        paged_decode(_h(case.q), case.k_cache, case.v_cache, case.context_lens,
                     case.block_tables, case.scale)
    with pytest.raises(_lib.NvkError):
        paged_decode(case.q.float(), case.k_cache.float(), case.v_cache.float(),
                     case.context_lens, case.block_tables, case.scale)
