"""CPU tests of the host side: the C-ABI library surface, argument validation
(no kernel launch), the Context record and the metadata builders."""
import dataclasses
import json
import os
import re

import pytest
import torch

from nanovllm_amd import _lib
from oracle import step_metadata as metadata
from oracle.sequence import Sequence
from nanovllm_amd.utils import context as ctx_mod

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nvk.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nvk_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = header_functions()
    assert {"nvk_kv_store", "nvk_paged_decode", "nvk_varlen_prefill"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with nvk.h"
    assert lib.nvk_build_target() == b"gfx950"


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="passes fake device pointers; a validation regression must not be "
                           "able to launch a kernel on them, so it only runs without a GPU")
def test_error_codes_without_launching():
    lib = _lib.load()
    assert lib.nvk_strerror(0) == b"ok"
    for code in (-1, -2, -3, -4):
        assert lib.nvk_strerror(code).startswith(b"nvk:")
    # unsupported element size / negative count / zero tokens (nothing launched)
    assert lib.nvk_kv_store(1, 8, 1, 8, 1, 1, 1, 4, 8, 3, 100, None) == -2
    assert lib.nvk_kv_store(1, 8, 1, 8, 1, 1, 1, -1, 8, 2, 100, None) == -1
    assert lib.nvk_kv_store(None, 8, None, 8, None, None, None, 0, 8, 2, 100, None) == 0
    # decode: f32 not built (bf16 and fp16 are), head_dim 96 not built, G=3 not
    # built, bad scale
    args = [16, 16 * 128, 128, 16, 16, 16, 8, 16, 4, 16, 8, 128, 256, 8, 1024, 0.088, 16, 16 * 128,
            128, 16, 1 << 30]
    assert lib.nvk_paged_decode(*args, 2, None) == -2
    bad_hd = list(args); bad_hd[11] = 96
    assert lib.nvk_paged_decode(*bad_hd, 0, None) == -2
    bad_g = list(args); bad_g[9] = 12; bad_g[10] = 4
    assert lib.nvk_paged_decode(*bad_g, 0, None) == -2
    bad_scale = list(args); bad_scale[15] = 0.0
    assert lib.nvk_paged_decode(*bad_scale, 0, None) == -1
    # workspace too small
    small_ws = list(args); small_ws[20] = 16
    assert lib.nvk_paged_decode(*small_ws, 0, None) == -4
    # group descriptors (8 bytes per (sequence, kv head), 256-byte padded) + 2
    # records per wave of the persistent grid, each holding 1 kv head x 2 q
    # heads; B=64, 8 kv heads, 2048-token tables: 512 workgroups x 4 waves
    assert lib.nvk_paged_decode_workspace_size(64, 16, 8, 128, 256, 8) == \
        4096 + 2048 * 2 * 1 * 2 * (128 + 4) * 4
    # tiny problem: one wave per chunk (B=1, 1 kv head, 64-token table: 2 chunks -> 1 WG)
    assert lib.nvk_paged_decode_workspace_size(1, 2, 1, 128, 64, 1) == 256 + 4 * 2 * 2 * 132 * 4
    assert lib.nvk_paged_decode_workspace_size(4, 16, 5, 128, 256, 1) == 0   # 16 % 5 != 0
    # the no-allocation decode: the same argument checks, and sizes whose
    # workspace exceeds its 20 MiB static scratch rejected before any launch
    assert lib.nvk_strerror(-5).startswith(b"nvk:")
    assert lib.nvk_paged_decode_noalloc(*args[:19], 2, None) == -2          # f32
    assert lib.nvk_paged_decode_noalloc(*bad_scale[:19], 0, None) == -1
    huge = list(args); huge[8], huge[9], huge[10] = 2048, 8192, 1024
    assert lib.nvk_paged_decode_workspace_size(2048, 8192, 1024, 128, 256, 8) > 20 << 20
    assert lib.nvk_paged_decode_noalloc(*huge[:19], 0, None) == -5
    # prefill: head_dim 64 not built
    assert lib.nvk_varlen_prefill(16, 2048, 128, 4, 16, 16, 1024, 1024, 128, 4, 16, 16, 1, 4, 4,
                                  None, 0, 0, 0, 0, 16, 8, 64, 0.1, 16, 2048, 128, None, 0, 0,
                                  None) == -2
    # 32 sequences of 6 queries over <= 8192 keys: the larger of the split-K records of
    # the tile kernel (8 kv heads x 32 x 1 query tile = 256 workgroups, split 4 ways,
    # 128 rows x (128 + 4) floats) and the short-query kernels' (descriptors + 2
    # records of 16 rows per wave of a 2048-wave grid)
    split = 8 * 32 * 1 * 4 * 128 * 132 * 4
    short = 32 * 8 * 8 + 2048 * 2 * 16 * 132 * 4
    assert lib.nvk_varlen_prefill_workspace_size(32, 6, 8192, 16, 8, 128) == max(split, short)
    # enough query tiles to fill the GPU and too many rows for the short path: the
    # longest-first tile order only, one int32 per (sequence, query tile) pair
    # (32 x 1024/64) and the order's tag, rounded up to 256 bytes
    assert lib.nvk_varlen_prefill_workspace_size(32, 1024, 1536, 16, 8, 128) == \
        (32 * 16 + 1) * 4 // 256 * 256 + 256
    assert lib.nvk_prefill_tile_order_size(32, 1024, 1536, 16, 8, 256) == 2304
    # a grid of one round of workgroups (3 x 2 query tiles x 8 kv heads): no order
    assert lib.nvk_varlen_prefill_workspace_size(3, 100, 1536, 16, 8, 128) == 0
    # one sequence of 6 queries over 512 keys: no split; the short-query kernels'
    # records for 8 kv heads x 16 chunks of 32 keys / 2 per wave = 64 waves
    assert lib.nvk_varlen_prefill_workspace_size(1, 6, 512, 16, 8, 128) == \
        256 + 64 * 2 * 16 * 132 * 4
    # 9 queries x G 2 = 18 rows: too many for the short path
    assert lib.nvk_varlen_prefill_workspace_size(1, 9, 512, 16, 8, 128) == 0
    # fused prologue: (qkv, stride, T, pos, qw, kw, eps, cos_sin, cs_stride, max_pos, Hq, Hkv,
    # D, q_out, strides, k_out, strides, k_cache, v_cache, slots, cache_slots, dtype, stream)
    pro = [16, 32 * 128, 4, 16, 16, 16, 1e-6, 16, 128, 4096, 16, 8, 128, 16, 16 * 128, 128,
           None, 0, 0, 16, 16, 16, 1 << 20, 0, None]
    assert lib.nvk_qk_norm_rope_store(*pro[:12], 64, *pro[13:]) == -2     # head_dim 64
    assert lib.nvk_qk_norm_rope_store(*pro[:23], 2, None) == -2           # f32 (bf16, f16 built)
    zero = list(pro); zero[2] = 0
    assert lib.nvk_qk_norm_rope_store(*zero) == 0                          # nothing to do
    no_q = list(pro); no_q[13] = None
    assert lib.nvk_qk_norm_rope_store(*no_q) == -1
    narrow = list(pro); narrow[1] = 31 * 128                               # row < Hq+2Hkv heads
    assert lib.nvk_qk_norm_rope_store(*narrow) == -1
    mis = list(pro); mis[0] = 24                                           # qkv not 16-B aligned
    assert lib.nvk_qk_norm_rope_store(*mis) == -3
    no_cache = list(pro); no_cache[19] = None                              # slots without caches
    assert lib.nvk_qk_norm_rope_store(*no_cache) == -1
    huge = list(pro); huge[2] = 1 << 31                                    # grid > 2^31 - 1
    assert lib.nvk_qk_norm_rope_store(*huge) == -1
    # decode with the prologue: (qkv, stride, pos, qw, kw, eps, cos_sin, cs_stride, max_pos,
    # k_cache, v_cache, slots, cache_slots, tables, bt_stride, lens, B, Hq, Hkv, D, bs,
    # max_blocks, num_blocks, scale, out, out strides, ws, ws_bytes, dtype, stream)
    dp = [16, 32 * 128, 16, 16, 16, 1e-6, 16, 128, 4096, 16, 16, 16, 1 << 20, 16, 8, 16, 4, 16, 8,
          128, 256, 8, 1024, 0.088, 16, 16 * 128, 128, 16, 1 << 30, 0, None]
    hd64 = list(dp); hd64[19] = 64
    assert lib.nvk_paged_decode_prologue(*hd64) == -2                     # head_dim 64
    f32 = list(dp); f32[29] = 2
    assert lib.nvk_paged_decode_prologue(*f32) == -2                      # f32 (bf16, f16 built)
    none = list(dp); none[16] = 0
    assert lib.nvk_paged_decode_prologue(*none) == 0                      # empty batch
    no_slots = list(dp); no_slots[11] = None
    assert lib.nvk_paged_decode_prologue(*no_slots) == -1
    narrow = list(dp); narrow[1] = 31 * 128
    assert lib.nvk_paged_decode_prologue(*narrow) == -1                   # row < Hq+2Hkv heads
    mis = list(dp); mis[0] = 24
    assert lib.nvk_paged_decode_prologue(*mis) == -3
    small = list(dp); small[28] = 16
    assert lib.nvk_paged_decode_prologue(*small) == -4                    # workspace too small
    # step metadata: (cached, new, offsets, ids, B, bs, width, T, cu_q, cu_k, pos, slots, tables)
    assert lib.nvk_prefill_metadata(16, 16, 16, 16, 9000, 256, 4, 10, 16, 16, 16, 16, 16,
                                    None) == -2                            # batch > 8192
    assert lib.nvk_prefill_metadata(None, None, None, None, 0, 256, 0, 0, None, None, None, None,
                                    None, None) == 0                       # empty step
    assert lib.nvk_prefill_metadata(16, 16, 16, 16, 4, 0, 4, 10, 16, 16, 16, 16, 16,
                                    None) == -1                            # block size 0
    assert lib.nvk_prefill_metadata(16, 16, 16, 16, 4, 256, 4, 10, 16, 16, None, 16, 16,
                                    None) == -1                            # no positions
    # (lens, offsets, ids, B, padded, bs, width, stride, ctx, pos, slots, tables)
    assert lib.nvk_decode_metadata(16, 16, 16, 8, 4, 256, 4, 4, 16, 16, 16, 16, None) == -1
    assert lib.nvk_decode_metadata(16, 16, 16, 4, 8, 256, 4, 2, 16, 16, 16, 16, None) == -1
    assert lib.nvk_decode_metadata(None, None, None, 0, 0, 256, 0, 0, None, None, None, None,
                                   None) == 0
    # sampler: three 4-byte slots per row and 2048-element wave chunk
    assert lib.nvk_sample_workspace_size(64, 151936) == 64 * 19 * 4 * 12
    assert lib.nvk_sample_workspace_size(0, 10) == 0
    smp = [16, 151936, 64, 151936, 0, 16, None, 0, 1, 0, 16, 16, 64 * 19 * 48, None]
    assert lib.nvk_sample(*smp[:4], 7, *smp[5:]) == -2                     # unknown dtype
    small = list(smp); small[12] = 8
    assert lib.nvk_sample(*small) == -4                                    # workspace too small
    narrow = list(smp); narrow[1] = 100
    assert lib.nvk_sample(*narrow) == -1                                   # row stride < vocab
    # gather: (x, stride, cu, B, hidden, dtype, out, out_stride, stream)
    assert lib.nvk_gather_last_tokens(16, 1024, 16, 4, 1024, 2, 16, 1024, None) == -2
    assert lib.nvk_gather_last_tokens(16, 1024, 16, 4, 1020, 0, 16, 1024, None) == -3
    assert lib.nvk_gather_last_tokens(None, 1024, None, 0, 1024, 0, None, 1024, None) == 0


def test_cpu_tensors_are_rejected_not_served():
    k = torch.zeros(2, 1, 8, dtype=torch.bfloat16)
    kc = torch.zeros(1, 4, 1, 8, dtype=torch.bfloat16)
    with pytest.raises(_lib.NvkError):
        ctx_mod.set_context(False)
        from nanovllm_amd import store_kvcache
        store_kvcache(k, k, kc, kc.clone(), torch.tensor([0, 1], dtype=torch.int32))


def test_context_record_matches_reference_fields():
    fields = [(f.name, f.default) for f in dataclasses.fields(ctx_mod.Context)]
    assert fields == [("is_prefill", False), ("cu_seqlens_q", None), ("cu_seqlens_k", None),
                      ("max_seqlen_q", 0), ("max_seqlen_k", 0), ("slot_mapping", None),
                      ("context_lens", None), ("block_tables", None)]
    ctx_mod.set_context(True, max_seqlen_q=3)
    assert ctx_mod.get_context().is_prefill and ctx_mod.get_context().max_seqlen_q == 3
    ctx_mod.reset_context()
    assert ctx_mod.get_context() == ctx_mod.Context()


def _known():
    with open(os.path.join(GOLDEN, "guide_known_answers.json")) as f:
        return json.load(f)


def test_prefill_slots_reproduce_guide_example():
    ex = _known()["slot_example"]
    bs = ex["block_size"]
    seq = Sequence(list(range(12)), block_table=ex["block_table"], num_cached_tokens=2,
                   num_scheduled_tokens=8)
    slots = metadata.prefill_slots(seq, bs)
    by_pos = dict(zip(range(2, 10), slots))
    assert [by_pos[p] for p in ex["positions"]] == ex["slots"]


def test_prepare_prefill_lm_head_example_and_no_prefix():
    ex = _known()["lm_head_example"]
    seqs = []
    nxt = 0
    for n in ex["query_lens"]:
        seqs.append(Sequence(list(range(n)), block_table=[nxt], num_scheduled_tokens=n))
        nxt += 1
    metadata.prepare_prefill(seqs, 256, device="cpu")
    c = ctx_mod.get_context()
    assert c.cu_seqlens_q.tolist() == ex["cu_seqlens_q"]
    assert (c.cu_seqlens_q[1:] - 1).tolist() == ex["last_indices"]
    assert c.block_tables is None                       # nothing cached
    assert c.cu_seqlens_q.dtype == torch.int32 and c.slot_mapping.dtype == torch.int32
    assert c.slot_mapping.tolist() == [0, 1, 256, 512, 513, 514, 515]


def test_prepare_prefill_chunk_with_prefix_and_warmup():
    bs = 4
    a = Sequence(list(range(10)), block_table=[7, 2, 9], num_cached_tokens=4,
                 num_scheduled_tokens=5)               # chunk of 5 after a cached page
    warm = Sequence([0] * 3, num_scheduled_tokens=3)    # warmup: no block table, no slots
    warm.block_table = []
    metadata.prepare_prefill([a, warm], bs, device="cpu")
    c = ctx_mod.get_context()
    assert c.cu_seqlens_q.tolist() == [0, 5, 8]
    assert c.cu_seqlens_k.tolist() == [0, 9, 12]
    assert c.max_seqlen_q == 5 and c.max_seqlen_k == 9
    assert c.slot_mapping.tolist() == [8, 9, 10, 11, 36]
    assert c.block_tables.tolist() == [[7, 2, 9], [-1, -1, -1]]


def test_prepare_decode_slot_and_context_lens(monkeypatch):
    bs = 4
    monkeypatch.setattr(Sequence, "block_size", bs)       # as LLMEngine does (llm_engine.py:21)
    a = Sequence(list(range(9)), block_table=[3, 0, 5])   # 9 tokens: last in page 5 offset 0
    b = Sequence(list(range(4)), block_table=[1])
    metadata.prepare_decode([a, b], bs, device="cpu")
    c = ctx_mod.get_context()
    assert c.slot_mapping.tolist() == [20, 7]
    assert c.context_lens.tolist() == [9, 4]
    assert c.block_tables.tolist() == [[3, 0, 5], [1, -1, -1]]
    assert not c.is_prefill


def test_graph_buffers_pad_rows_like_run_model():
    g = metadata.DecodeGraphBuffers(8, 4, device="cpu")
    g.block_tables.fill_(77)                            # stale content from an earlier step
    g.load(torch.tensor([5, 9], dtype=torch.int32), torch.tensor([6, 10], dtype=torch.int32),
           torch.tensor([[1, -1], [2, 3]], dtype=torch.int32))
    assert g.slot_mapping.tolist() == [5, 9] + [-1] * 6
    assert g.context_lens.tolist() == [6, 10] + [0] * 6
    assert g.block_tables[:2].tolist() == [[1, -1, 77, 77], [2, 3, 77, 77]]
    assert g.block_tables[2:].eq(77).all()


def test_pack_block_tables_is_the_compressed_table():
    from nanovllm_amd.engine.device_metadata import pack_block_tables
    seqs = [Sequence([1, 2, 3], block_table=[4, 5]), Sequence([1], block_table=[]),
            Sequence([1] * 9, block_table=[7, 8, 9])]
    assert pack_block_tables(seqs) == ([0, 2, 2, 5], [4, 5, 7, 8, 9], 3)


def test_work_counts():
    from nanovllm_amd.workloads import attention_bytes, prefill_flops, prologue_bytes
    assert prefill_flops([2], [2], 1, 1) == 4 * 3
    assert prefill_flops([1], [5], 2, 4) == 4 * 2 * 4 * 5
    # brute force over the bottom-right causal mask, ragged and empty sequences
    lq, lk = [3, 0, 7, 5], [10, 4, 7, 5]
    pairs = sum(1 for q, k in zip(lq, lk) for i in range(q) for j in range(k) if j <= i + k - q)
    assert prefill_flops(lq, lk, 3, 8) == 4 * 3 * 8 * pairs
    assert attention_bytes([3, 4], 2, 8, 2, 4) == 2 * 7 * 2 * 8 * 2 + 2 * 2 * 4 * 8 * 2
    # prologue: 10 tokens, 8 valid slots, 6 distinct positions, Qwen3 heads, k written out
    D = 128
    row = D * 2
    assert prologue_bytes(10, 8, 6, 16, 8, D, write_k=True) == (
        10 * 32 * row + 10 * 12 + 6 * D * 4 + 10 * 16 * row + 8 * 16 * row + 10 * 8 * row)
