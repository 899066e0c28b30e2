"""Paged GQA decode on the GPU against the oracle (flash_attn_with_kvcache as
called at attention.py:72-74), within 2e-2 abs / 1e-2 rel."""
import numpy as np
import pytest
import torch

from gpu_utils import GOLDEN, assert_attn_close, from_bits, oracle_decode, say
from nanovllm_amd import flash_attn_with_kvcache, paged_decode
from nanovllm_amd.workloads import decode_case

pytestmark = pytest.mark.gpu


def _check(case, what, q=None):
    c = case.to("cuda")
    q_gpu = c.q if q is None else q
    say(what)
    out = paged_decode(q_gpu, c.k_cache, c.v_cache, c.context_lens, c.block_tables, case.scale)
    torch.cuda.synchronize()
    ref = oracle_decode(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                        case.block_size, case.scale)
    assert_attn_close(out, ref, what)
    return out


@pytest.mark.parametrize("name", ["decode_minimal", "decode_shared", "decode_gqa"])
def test_decode_golden_fixture(name):
    data = np.load(f"{GOLDEN}/attn_small.npz")
    hq, hkv, d, bs = [int(x) for x in data[f"{name}_meta"]]
    q = from_bits(data[f"{name}_q"])
    kc, vc = from_bits(data[f"{name}_k_cache"]), from_bits(data[f"{name}_v_cache"])
    bt = torch.from_numpy(data[f"{name}_block_tables"]).cuda()
    lens = torch.from_numpy(data[f"{name}_lens_k"]).cuda()
    say(f"decode golden {name}")
    out = paged_decode(q, kc, vc, lens, bt, d ** -0.5)
    torch.cuda.synchronize()
    assert_attn_close(out, data[f"{name}_expect"], name)


def test_decode_qwen3_batch64():
    case = decode_case(pool_blocks=600)   # B=64, ctx U{100..2048}, 16/8 heads
    out = _check(case, "decode B=64 ctx<=2048")
    assert out.shape == (64, 16, 128) and out.dtype == torch.bfloat16


@pytest.mark.parametrize("hq,hkv", [(16, 16), (16, 8), (16, 4), (16, 2)])
def test_decode_context_ladder_and_group_sizes(hq, hkv):
    ctx = [1, 5, 255, 256, 257, 513, 1024, 4096]
    case = decode_case(seed=7, hq=hq, hkv=hkv, ctx=ctx, pool_blocks=40)
    _check(case, f"decode ladder G={hq // hkv}")


def test_decode_groups_cut_into_many_parts():
    """Two sequences over 1500 and 3000 keys: the stream-K split cuts each
    (sequence, kv head) group into ~24 and ~47 wave parts; the grid has more
    than 32 waves per group, so the combine folds them in sixteen interleaved
    slices (one per wave of a 1024-thread workgroup) merged through LDS."""
    case = decode_case(seed=11, ctx=[1500, 3000], pool_blocks=24)
    _check(case, "decode groups of 24 and 47 parts")


@pytest.mark.parametrize("bs", [16, 64, 512])
def test_decode_other_block_sizes(bs):
    ctx = [1, 63, 64, 65, 700, 1500]
    case = decode_case(seed=8, block_size=bs, ctx=ctx, pool_blocks=4000 // bs + 16)
    _check(case, f"decode block_size={bs}")


def test_decode_head_dim_64():
    case = decode_case(seed=9, hq=8, hkv=2, hd=64, ctx=[3, 300, 1000], pool_blocks=12)
    _check(case, "decode head_dim=64")


def test_decode_reversed_and_shared_tables_and_stale_padding():
    case = decode_case(seed=10, ctx=[600, 600, 3, 257], pool_blocks=12, width=6)
    bt = case.block_tables
    bt[1, :3] = bt[0, :3].flip(0)          # same pages, reversed order
    bt[3, 0] = bt[0, 0]                    # shares the first page of sequence 0
    # stale tails: valid page ids that must not be read
    for b, n in enumerate([600, 600, 3, 257]):
        need = (n + 255) // 256
        bt[b, need:] = 11
    case.tensors["block_tables"] = bt
    _check(case, "decode reversed/shared/stale tables")


def test_decode_zero_context_rows_write_zeros():
    case = decode_case(seed=12, ctx=[0, 700, 0, 1], pool_blocks=8)
    c = case.to("cuda")
    out = torch.full((4, 16, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    say("decode zero-context rows")
    paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens, c.block_tables, case.scale, out=out)
    torch.cuda.synchronize()
    assert out[0].eq(0).all() and out[2].eq(0).all()
    ref = oracle_decode(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                        256, case.scale)
    assert_attn_close(out, ref, "zero-context")


def test_decode_zero_context_row_beside_a_long_context():
    """An empty context next to one of 16000 keys: the grid has far more than
    32 waves per group, so the sliced combine writes the zero rows."""
    case = decode_case(seed=13, ctx=[0, 16000], pool_blocks=70)
    c = case.to("cuda")
    out = torch.full((2, 16, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    say("decode zero-context row, sliced combine")
    paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens, c.block_tables, case.scale, out=out)
    torch.cuda.synchronize()
    assert out[0].eq(0).all()
    ref = oracle_decode(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                        256, case.scale)
    assert_attn_close(out, ref, "zero-context beside 16000 keys")


def test_decode_strided_query_and_flash_api_shape():
    case = decode_case(seed=13, ctx=[100, 2000, 37], pool_blocks=12)
    c = case.to("cuda")
    packed = torch.zeros(3, 4096, dtype=torch.bfloat16, device="cuda")
    q = packed[:, :2048].view(3, 16, 128)
    q.copy_(c.q)
    assert q.stride(0) == 4096
    say("decode strided q via flash_attn_with_kvcache")
    out = flash_attn_with_kvcache(q.unsqueeze(1), c.k_cache, c.v_cache,
                                  cache_seqlens=c.context_lens, block_table=c.block_tables,
                                  softmax_scale=case.scale, causal=True)
    torch.cuda.synchronize()
    assert out.shape == (3, 1, 16, 128)
    ref = oracle_decode(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                        256, case.scale)
    assert_attn_close(out[:, 0], ref, "strided q")


def test_decode_graph_capture_replays_with_padded_rows():
    # Capture store + decode once at batch 8 with all-zero metadata (as
    # capture_cudagraph does), then replay with live rows and padded rows.
    from nanovllm_amd import store_kvcache
    from oracle.step_metadata import DecodeGraphBuffers
    bs_graph, width = 8, 8
    pool = decode_case(seed=14, ctx=[1] * 8, pool_blocks=64)
    k_cache, v_cache = pool.k_cache.cuda(), pool.v_cache.cuda()
    bufs = DecodeGraphBuffers(bs_graph, width)
    q = torch.zeros(bs_graph, 16, 128, dtype=torch.bfloat16, device="cuda")
    key = torch.zeros(bs_graph, 8, 128, dtype=torch.bfloat16, device="cuda")
    value = torch.zeros_like(key)
    out = torch.zeros(bs_graph, 16, 128, dtype=torch.bfloat16, device="cuda")
    scale = 128 ** -0.5

    def step():
        store_kvcache(key, value, k_cache, v_cache, bufs.slot_mapping)
        paged_decode(q, k_cache, v_cache, bufs.context_lens, bufs.block_tables, scale, out=out)

    say("decode graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()                                   # warmup outside the graph
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()

    gen = torch.Generator().manual_seed(15)
    perm = torch.randperm(64, generator=gen).tolist()
    for rep, live in enumerate([5, 8, 3]):
        lens = torch.randint(200, 2000, (live,), generator=gen).to(torch.int32)
        tables, nxt = [], 0
        for n in lens.tolist():
            need = (n + 255) // 256
            tables.append(perm[nxt:nxt + need]); nxt += need
        w = max(len(t) for t in tables)
        bt = torch.full((live, w), -1, dtype=torch.int32)
        for i, t in enumerate(tables):
            bt[i, :len(t)] = torch.tensor(t)
        slots = torch.tensor([t[(n - 1) // 256] * 256 + (n - 1) % 256
                              for t, n in zip(tables, lens.tolist())], dtype=torch.int32)
        qh = torch.randn(bs_graph, 16, 128, generator=gen).to(torch.bfloat16)
        kh = torch.randn(bs_graph, 8, 128, generator=gen).to(torch.bfloat16)
        vh = torch.randn(bs_graph, 8, 128, generator=gen).to(torch.bfloat16)
        q.copy_(qh); key.copy_(kh); value.copy_(vh)
        bufs.load(slots.cuda(), lens.cuda(), bt.cuda())
        say(f"decode graph replay {rep} live={live}")
        g.replay()
        torch.cuda.synchronize()
        kc_cpu, vc_cpu = k_cache.cpu(), v_cache.cpu()
        # the replay stored the live rows' new K/V at their slots
        for i in range(live):
            s_ = int(slots[i])
            assert torch.equal(kc_cpu.view(-1, 8, 128)[s_], kh[i])
            assert torch.equal(vc_cpu.view(-1, 8, 128)[s_], vh[i])
        ref = oracle_decode(qh[:live], kc_cpu, vc_cpu, bt, lens, 256, scale)
        assert_attn_close(out[:live], ref, f"graph replay {rep}")
        assert out[live:].eq(0).all(), "padded rows must be zero"
