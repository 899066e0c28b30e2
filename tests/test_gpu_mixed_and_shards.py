"""A mixed chunked-prefill + decode layer, and the path at the head counts of a
tensor-parallel shard (Qwen3-0.6B's 16/8 heads split over 2 and 4 GPUs: 8/4
and 4/2, cache rows of 512 and 256 elements), on the GPU against the oracle:
KV-store bit-exact, attention within 2e-2 abs / 1e-2 rel."""
import numpy as np
import pytest
import torch

from gpu_utils import (assert_attn_close, bits, oracle_decode, oracle_prefill_paged,
                       oracle_store, say)
from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill
from nanovllm_amd.workloads import decode_case, mixed_layer_case, prefill_case

pytestmark = pytest.mark.gpu


def _stored(case):
    ek, ev = oracle_store(case.key, case.value, case.k_cache, case.v_cache, case.slot_mapping)
    return (torch.from_numpy(ek.view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(ev.view(np.int16)).view(torch.bfloat16), ek, ev)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 4), (4, 2)])
def test_mixed_layer_store_then_prefill_chunks_and_decodes(hq, hkv):
    case = mixed_layer_case(seed=41, n_chunks=3, chunk=200, cached_hi=600, n_decode=16,
                            ctx_hi=1500, hq=hq, hkv=hkv, pool_blocks=120)
    c = case.to("cuda")
    say(f"mixed layer {hq}/{hkv}: store")
    store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
    say(f"mixed layer {hq}/{hkv}: prefill chunks")
    o_pf = varlen_prefill(c.q_prefill, c.k_cache, c.v_cache, c.cu_seqlens_q, c.cu_seqlens_k,
                          case.max_seqlen_q, case.scale, block_table=c.prefill_block_tables,
                          max_seqlen_k=case.max_seqlen_k)
    say(f"mixed layer {hq}/{hkv}: decodes")
    o_dec = paged_decode(c.q_decode, c.k_cache, c.v_cache, c.context_lens,
                         c.decode_block_tables, case.scale)
    torch.cuda.synchronize()
    kc, vc, ek, ev = _stored(case)
    np.testing.assert_array_equal(bits(c.k_cache), ek)
    np.testing.assert_array_equal(bits(c.v_cache), ev)
    ref_pf = oracle_prefill_paged(case.q_prefill, kc, vc, case.prefill_block_tables,
                                  case.cu_seqlens_q, case.cu_seqlens_k, case.block_size,
                                  case.scale)
    assert_attn_close(o_pf, ref_pf, "mixed prefill chunks")
    ref_dec = oracle_decode(case.q_decode, kc, vc, case.decode_block_tables, case.context_lens,
                            case.block_size, case.scale)
    assert_attn_close(o_dec, ref_dec, "mixed decodes")


@pytest.mark.parametrize("hq,hkv", [(8, 4), (4, 2)])
def test_tensor_parallel_shard_shapes(hq, hkv):
    dc = decode_case(seed=42, hq=hq, hkv=hkv, batch=24, pool_blocks=200)
    c = dc.to("cuda")
    say(f"shard {hq}/{hkv}: decode")
    out = paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens, c.block_tables, dc.scale)
    torch.cuda.synchronize()
    assert_attn_close(out, oracle_decode(dc.q, dc.k_cache, dc.v_cache, dc.block_tables,
                                         dc.context_lens, dc.block_size, dc.scale),
                      f"shard decode {hq}/{hkv}")
    pc = prefill_case(seed=43, hq=hq, hkv=hkv, lens_new=[3, 100, 513], prefix=256,
                      pool_blocks=20)
    p = pc.to("cuda")
    say(f"shard {hq}/{hkv}: store + prefill")
    store_kvcache(p.key, p.value, p.k_cache, p.v_cache, p.slot_mapping)
    o = varlen_prefill(p.q, p.k_cache, p.v_cache, p.cu_seqlens_q, p.cu_seqlens_k,
                       pc.max_seqlen_q, pc.scale, block_table=p.block_tables)
    torch.cuda.synchronize()
    kc, vc, ek, ev = _stored(pc)
    np.testing.assert_array_equal(bits(p.k_cache), ek)
    assert_attn_close(o, oracle_prefill_paged(pc.q, kc, vc, pc.block_tables, pc.cu_seqlens_q,
                                              pc.cu_seqlens_k, 256, pc.scale),
                      f"shard prefill {hq}/{hkv}")


def test_mixed_layer_decode_and_prefill_on_two_streams_match_sequential():
    """The overlapped order of a mixed step (the decodes on the main stream, the
    prefill chunks on a second stream after the store, joined afterwards; a
    graph replays it) gives the sequential order's outputs bit for bit."""
    case = mixed_layer_case(seed=44, n_chunks=4, chunk=256, cached_hi=800, n_decode=48,
                            ctx_hi=2000, pool_blocks=420)
    c = case.to("cuda")
    say("mixed layer, two streams: store")
    store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)

    def prefill(out):
        return varlen_prefill(c.q_prefill, c.k_cache, c.v_cache, c.cu_seqlens_q, c.cu_seqlens_k,
                              case.max_seqlen_q, case.scale, block_table=c.prefill_block_tables,
                              max_seqlen_k=case.max_seqlen_k, out=out)

    def decode(out):
        return paged_decode(c.q_decode, c.k_cache, c.v_cache, c.context_lens,
                            c.decode_block_tables, case.scale, out=out)

    say("mixed layer, two streams: sequential reference")
    ref_pf, ref_dec = prefill(None), decode(None)
    torch.cuda.synchronize()
    o_pf, o_dec = torch.full_like(ref_pf, float("nan")), torch.full_like(ref_dec, float("nan"))
    side = torch.cuda.Stream()

    def overlapped():
        main = torch.cuda.current_stream()
        side.wait_stream(main)
        decode(o_dec)
        with torch.cuda.stream(side):
            prefill(o_pf)
        main.wait_stream(side)

    say("mixed layer, two streams: eager")
    overlapped()
    torch.cuda.synchronize()
    assert torch.equal(o_pf, ref_pf) and torch.equal(o_dec, ref_dec)
    say("mixed layer, two streams: graph, three replays")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        overlapped()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        overlapped()
    for _ in range(3):
        o_pf.fill_(float("nan"))
        o_dec.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_pf, ref_pf) and torch.equal(o_dec, ref_dec)
