"""Varlen causal prefill on the GPU against the oracle (flash_attn_varlen_func
as called at attention.py:64-70), within 2e-2 abs / 1e-2 rel.  Covers the
paged prefix path, the dense path (warmup / no prefix, strided v) and
speculative-decode verification through flash_attn_with_kvcache."""
import numpy as np
import pytest
import torch

from gpu_utils import (GOLDEN, assert_attn_close, from_bits, oracle_prefill_dense,
                       oracle_prefill_paged, oracle_store, say)
from oracle import kv_oracle as orc
from nanovllm_amd import flash_attn_varlen_func, flash_attn_with_kvcache, store_kvcache
from nanovllm_amd.workloads import prefill_case, spec_verify_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["prefill_prefix", "prefill_page"])
def test_prefill_golden_fixture(name):
    data = np.load(f"{GOLDEN}/attn_small.npz")
    hq, hkv, d, bs = [int(x) for x in data[f"{name}_meta"]]
    q = from_bits(data[f"{name}_q"])
    kc, vc = from_bits(data[f"{name}_k_cache"]), from_bits(data[f"{name}_v_cache"])
    bt = torch.from_numpy(data[f"{name}_block_tables"]).cuda()
    lq, lk = data[f"{name}_lens_q"], data[f"{name}_lens_k"]
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32, device="cuda")
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device="cuda")
    say(f"prefill golden {name}")
    out = flash_attn_varlen_func(q, kc, vc, cu_q, cu_k, int(lq.max()), int(lk.max()),
                                 softmax_scale=d ** -0.5, causal=True, block_table=bt)
    torch.cuda.synchronize()
    assert_attn_close(out, data[f"{name}_expect"], name)


def _run_paged_case(case, what):
    c = case.to("cuda")
    say(what + " (store)")
    store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
    say(what + " (attention)")
    out = flash_attn_varlen_func(c.q, c.k_cache, c.v_cache, c.cu_seqlens_q, c.cu_seqlens_k,
                                 case.max_seqlen_q, case.max_seqlen_k, softmax_scale=case.scale,
                                 causal=True, block_table=c.block_tables)
    torch.cuda.synchronize()
    ek, ev = oracle_store(case.key, case.value, case.k_cache, case.v_cache, case.slot_mapping)
    kc = torch.from_numpy(ek.view(np.int16)).view(torch.bfloat16)
    vc = torch.from_numpy(ev.view(np.int16)).view(torch.bfloat16)
    ref = oracle_prefill_paged(case.q, kc, vc, case.block_tables, case.cu_seqlens_q,
                               case.cu_seqlens_k, case.block_size, case.scale)
    assert_attn_close(out, ref, what)


def test_prefill_qwen3_prefix_cache_32_seqs():
    case = prefill_case()        # 32 seqs: 512-token shared prefix + U{100..1024} new
    _run_paged_case(case, "prefill 32 seqs prefix 512")


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 4), (16, 2)])
def test_prefill_paged_group_sizes(hq, hkv):
    case = prefill_case(seed=21, hq=hq, hkv=hkv, lens_new=[1, 63, 64, 65, 200, 129], prefix=256,
                        pool_blocks=24)
    _run_paged_case(case, f"prefill paged G={hq // hkv}")


def test_prefill_paged_small_pages():
    case = prefill_case(seed=22, block_size=16, prefix=48, lens_new=[5, 77, 160], pool_blocks=64)
    _run_paged_case(case, "prefill block_size 16")


def test_prefill_chunk_mid_page_start():
    # a later chunk: 300 new tokens after 100 cached ones (the chunk starts mid-page)
    gen = torch.Generator().manual_seed(23)
    bs, cached, new = 256, 100, 300
    pages = [5, 2]
    kc = torch.randn(8, bs, 8, 128, generator=gen).to(torch.bfloat16)
    vc = torch.randn(8, bs, 8, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(new, 16, 128, generator=gen).to(torch.bfloat16)
    bt = torch.tensor([pages], dtype=torch.int32)
    cu_q = torch.tensor([0, new], dtype=torch.int32)
    cu_k = torch.tensor([0, cached + new], dtype=torch.int32)
    say("prefill chunk mid-page")
    out = flash_attn_varlen_func(q.cuda(), kc.cuda(), vc.cuda(), cu_q.cuda(), cu_k.cuda(), new,
                                 cached + new, softmax_scale=128 ** -0.5, causal=True,
                                 block_table=bt.cuda())
    torch.cuda.synchronize()
    ref = oracle_prefill_paged(q, kc, vc, bt, cu_q, cu_k, bs, 128 ** -0.5)
    assert_attn_close(out, ref, "chunk mid-page")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 16), (8, 1)])
def test_prefill_dense_no_prefix_strided_v(hq, hkv):
    # warmup / no-prefix path: k, v are the step's own rows; v is a view of the
    # packed qkv (row stride (hq + 2*hkv) * 128) as in qwen3.py:77-81.
    gen = torch.Generator().manual_seed(24)
    lens = [1, 127, 128, 129, 300, 64]
    tq = sum(lens)
    width = (hq + 2 * hkv) * 128
    qkv = torch.randn(tq, width, generator=gen).to(torch.bfloat16)
    q = qkv[:, :hq * 128].reshape(tq, hq, 128).contiguous()
    k = qkv[:, hq * 128:(hq + hkv) * 128].reshape(tq, hkv, 128).contiguous()
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    g = qkv.cuda()
    v_view = g[:, (hq + hkv) * 128:].view(tq, hkv, 128)
    assert v_view.stride(0) == width
    say(f"prefill dense G={hq // hkv}")
    out = flash_attn_varlen_func(q.cuda(), k.cuda(), v_view, cu.cuda(), cu.cuda(), max(lens),
                                 max(lens), softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    v = qkv[:, (hq + hkv) * 128:].reshape(tq, hkv, 128)
    ref = oracle_prefill_dense(q, k, v, cu, cu, 128 ** -0.5)
    assert_attn_close(out, ref, "dense")


def test_prefill_grid_larger_than_batch_and_empty_sequences():
    # max_seqlen_q larger than any sequence, and a sequence with no new tokens
    gen = torch.Generator().manual_seed(25)
    lens = [0, 70, 3]
    tq = sum(lens)
    q = torch.randn(tq, 16, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(tq, 8, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(tq, 8, 128, generator=gen).to(torch.bfloat16)
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    say("prefill oversize grid")
    out = flash_attn_varlen_func(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), cu.cuda(), 500, 500,
                                 softmax_scale=0.1, causal=True)
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_prefill_dense(q, k, v, cu, cu, 0.1), "oversize grid")


def test_spec_verify_six_queries_over_long_context():
    case = spec_verify_case(batch=8, ctx_hi=4096, pool_blocks=140)
    c = case.to("cuda")
    say("spec-verify store")
    store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
    q4 = c.q.view(8, 6, 16, 128)
    say("spec-verify attention")
    out = flash_attn_with_kvcache(q4, c.k_cache, c.v_cache, cache_seqlens=c.context_lens,
                                  block_table=c.block_tables, softmax_scale=case.scale, causal=True)
    torch.cuda.synchronize()
    ek, ev = oracle_store(case.key, case.value, case.k_cache, case.v_cache, case.slot_mapping)
    kc = torch.from_numpy(ek.view(np.int16)).view(torch.bfloat16)
    vc = torch.from_numpy(ev.view(np.int16)).view(torch.bfloat16)
    ref = oracle_prefill_paged(case.q, kc, vc, case.block_tables, case.cu_seqlens_q,
                               case.cu_seqlens_k, 256, case.scale)
    assert_attn_close(out.view(-1, 16, 128), ref, "spec-verify")
