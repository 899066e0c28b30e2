"""Bucketed HIP-graph decode of a multi-layer attention stack, replayed the way
the reference's run_model does (model_runner.py:195-257): graphs captured per
bucket with all-zero metadata, live batches smaller than their bucket, padded
rows with slot -1 and context 0, stale block-table tails from earlier
replays.  Every layer runs the fused prologue (norms, rotation, store) and the
paged decode; the result is checked against the oracle per layer."""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc
from nanovllm_amd.engine.graph_runner import DecodeGraphRunner, graph_buckets
from nanovllm_amd.utils.context import reset_context, set_context
from nanovllm_amd.workloads import decode_stack
from tests.gpu_utils import (assert_attn_close, assert_rotated_close, bits, from_bits,
                             oracle_decode, say)

L, NB, BS, W, MAX_BS = 2, 128, 256, 8, 32
HQ, HKV, D = 16, 8, 128


def test_graph_buckets_follow_the_reference():
    assert graph_buckets(512)[:6] == [1, 2, 4, 8, 16, 32] and graph_buckets(512)[-1] == 512
    assert graph_buckets(8) == [1, 2, 4, 8]


@pytest.mark.gpu
def test_bucketed_decode_graph_replays_match_oracle():
    say("decode graph: capture buckets")
    dev = torch.device("cuda:0")
    layers, rope, kv_cache, step = decode_stack(L, NB, dev, seed=31)
    runner = DecodeGraphRunner(step, MAX_BS, W, inputs={"qkv": ((L, (HQ + 2 * HKV) * D),
                                                                torch.bfloat16)},
                               output=((L, HQ * D), torch.bfloat16), device=dev)
    assert runner.buckets == [1, 2, 4, 8, 16, 32]
    cos_sin = rope.cos_sin_cache.reshape(-1, D).cpu().numpy()
    gen = torch.Generator().manual_seed(32)
    for rep, live in enumerate([5, 16, 20, 1, 32]):
        perm = torch.randperm(NB, generator=gen).tolist()
        lens = torch.randint(1, 1500, (live,), generator=gen, dtype=torch.int32)
        tables, nxt = [], 0
        for n in lens.tolist():
            need = (n + BS - 1) // BS
            tables.append(perm[nxt:nxt + need])
            nxt += need
        assert nxt <= NB
        w = max(len(t) for t in tables)
        bt = torch.full((live, w), -1, dtype=torch.int32)
        for i, t in enumerate(tables):
            bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
        slots = torch.tensor([t[(n - 1) // BS] * BS + (n - 1) % BS for t, n in zip(tables, lens.tolist())],
                             dtype=torch.int32)
        pos = (lens - 1).to(torch.int64)
        qkv = (torch.randn(live, L, (HQ + 2 * HKV) * D, generator=gen) * 2.0).to(torch.bfloat16)
        before = bits(kv_cache).copy()
        say(f"decode graph replay {rep}: live={live} bucket={runner.bucket(live)}")
        set_context(False, slot_mapping=slots.to(dev), context_lens=lens.to(dev),
                    block_tables=bt.to(dev))
        try:
            out = runner.run(pos.to(dev), qkv=qkv.to(dev)).clone()
            padded = runner.outputs[live:runner.bucket(live)].clone()
            torch.cuda.synchronize()
        finally:
            reset_context()
        assert out.shape == (live, L, HQ * D)
        assert padded.eq(0).all(), "padded rows must be zero"
        after = bits(kv_cache)
        sl = slots.numpy().astype(np.int64)
        for i, (attn, qn, kn) in enumerate(layers):
            kc_ref, vc_ref = before[0, i].copy(), before[1, i].copy()
            q_ref, k_ref, _ = orc.qk_norm_rope_store(
                bits(qkv[:, i]), pos.numpy(), bits(qn.weight), bits(kn.weight), qn.eps, cos_sin,
                HQ, HKV, D, kc_ref, vc_ref, sl)
            # v rows bit-exact, every other cache row untouched
            assert np.array_equal(after[1, i], vc_ref), f"layer {i}: v cache"
            kc_got = after[0, i].reshape(NB * BS, HKV, D)
            untouched = np.ones(NB * BS, dtype=bool)
            untouched[sl] = False
            assert np.array_equal(kc_got[untouched],
                                  before[0, i].reshape(NB * BS, HKV, D)[untouched])
            assert_rotated_close(kc_got[sl], k_ref, f"layer {i}: cached k")
            ref = oracle_decode(from_bits(q_ref, "cpu"), from_bits(after[0, i], "cpu"),
                                from_bits(after[1, i], "cpu"), bt, lens, BS, D ** -0.5)
            assert_attn_close(out[:, i].reshape(live, HQ, D), ref, f"replay {rep} layer {i}")
    with pytest.raises(ValueError):
        runner.run(torch.zeros(MAX_BS + 1, dtype=torch.int64, device=dev),
                   qkv=torch.zeros(MAX_BS + 1, L, (HQ + 2 * HKV) * D, dtype=torch.bfloat16,
                                   device=dev))


@pytest.mark.gpu
def test_large_buckets_replay_live_batches_below_their_bucket():
    """Buckets 48..512 of the reference's list (model_runner.py:234) with live
    batches of 33, 40, 100, 250 and 500 sequences (padded rows in every
    replay, a smaller batch after a larger one leaves stale table rows and
    columns) over contexts U{1..4096} (max_model_len, config.py:11).  Pages
    before a sequence's last one come from 64 pages shared read-only across
    sequences; the last page, where the new token is stored, is private."""
    nb, w, max_bs = 64 + 512, 16, 512
    say("decode graph, large buckets: capture 1..512")
    dev = torch.device("cuda:0")
    layers, rope, kv_cache, step = decode_stack(L, nb, dev, seed=33)
    runner = DecodeGraphRunner(step, max_bs, w, inputs={"qkv": ((L, (HQ + 2 * HKV) * D),
                                                                torch.bfloat16)},
                               output=((L, HQ * D), torch.bfloat16), device=dev)
    assert runner.buckets[:7] == [1, 2, 4, 8, 16, 32, 48] and runner.buckets[-1] == 512
    cos_sin = rope.cos_sin_cache.reshape(-1, D).cpu().numpy()
    rng = np.random.default_rng(34)
    gen = torch.Generator().manual_seed(35)
    for rep, live in enumerate([500, 40, 250, 33, 100]):
        lens = rng.integers(1, 4097, live).astype(np.int32)
        private = rng.permutation(512)[:live] + 64
        bt = np.full((live, w), -1, np.int32)
        for i, n in enumerate(lens):
            need = -(-int(n) // BS)
            bt[i, :need - 1] = rng.choice(64, need - 1, replace=False)
            bt[i, need - 1] = private[i]
        slots = (private * BS + (lens - 1) % BS).astype(np.int32)
        pos = torch.from_numpy(lens.astype(np.int64) - 1)
        qkv = (torch.randn(live, L, (HQ + 2 * HKV) * D, generator=gen) * 2.0).to(torch.bfloat16)
        before = bits(kv_cache).copy()
        say(f"decode graph replay {rep}: live={live} bucket={runner.bucket(live)}")
        set_context(False, slot_mapping=torch.from_numpy(slots).to(dev),
                    context_lens=torch.from_numpy(lens).to(dev),
                    block_tables=torch.from_numpy(bt).to(dev))
        try:
            out = runner.run(pos.to(dev), qkv=qkv.to(dev)).clone()
            padded = runner.outputs[live:runner.bucket(live)].clone()
            torch.cuda.synchronize()
        finally:
            reset_context()
        assert padded.eq(0).all(), "padded rows must be zero"
        after = bits(kv_cache)
        sl = slots.astype(np.int64)
        for i, (attn, qn, kn) in enumerate(layers):
            kc_ref, vc_ref = before[0, i].copy(), before[1, i].copy()
            q_ref, k_ref, _ = orc.qk_norm_rope_store(
                bits(qkv[:, i]), pos.numpy(), bits(qn.weight), bits(kn.weight), qn.eps, cos_sin,
                HQ, HKV, D, kc_ref, vc_ref, sl)
            assert np.array_equal(after[1, i], vc_ref), f"replay {rep} layer {i}: v cache"
            kc_got = after[0, i].reshape(nb * BS, HKV, D)
            untouched = np.ones(nb * BS, dtype=bool)
            untouched[sl] = False
            assert np.array_equal(kc_got[untouched],
                                  before[0, i].reshape(nb * BS, HKV, D)[untouched])
            assert_rotated_close(kc_got[sl], k_ref, f"replay {rep} layer {i}: cached k")
            ref = orc.paged_attention(q_ref, after[0, i], after[1, i], np.arange(live + 1), lens,
                                      D ** -0.5, block_tables=bt, block_size=BS)
            assert_attn_close(out[:, i].reshape(live, HQ, D), ref, f"replay {rep} layer {i}")


@pytest.mark.gpu
@pytest.mark.parametrize("bs,width", [(3, 5), (8, 7), (0, 5), (1, 1)])
def test_graph_refresh_kernel_equals_run_model_copies(bs, width):
    """nvk_decode_graph_refresh against run_model's tensor copies
    (model_runner.py:200-211) on static buffers holding stale values: slots -1
    and contexts 0 past the live batch, positions and block-table cells outside
    the live rectangle untouched; the source table is a strided view."""
    from nanovllm_amd import _lib
    say(f"graph refresh kernel bs={bs} width={width}")
    dev = torch.device("cuda:0")
    rows, cols = 8, 7
    g = torch.Generator().manual_seed(bs * 10 + width)
    stale = lambda *shape, dt: torch.randint(-50, 50, shape, generator=g, dtype=dt).to(dev)
    pos0, slot0 = stale(rows, dt=torch.int64), stale(rows, dt=torch.int32)
    ctx0, bt0 = stale(rows, dt=torch.int32), stale(rows, cols, dt=torch.int32)
    src_pos = torch.randint(0, 4096, (bs,), generator=g, dtype=torch.int64).to(dev)
    src_slot = torch.randint(-1, 9000, (bs,), generator=g, dtype=torch.int32).to(dev)
    src_ctx = torch.randint(0, 4096, (bs,), generator=g, dtype=torch.int32).to(dev)
    src_bt = torch.randint(-1, 300, (bs, width + 2), generator=g, dtype=torch.int32).to(dev)[:, :width]
    # reference: the copies of run_model
    pos_r, slot_r, ctx_r, bt_r = pos0.clone(), slot0.clone(), ctx0.clone(), bt0.clone()
    pos_r[:bs] = src_pos
    slot_r.fill_(-1)
    slot_r[:bs] = src_slot
    ctx_r.zero_()
    ctx_r[:bs] = src_ctx
    bt_r[:bs, :width] = src_bt
    pos, slot, ctx, bt = pos0.clone(), slot0.clone(), ctx0.clone(), bt0.clone()
    lib = _lib.load()
    rc = lib.nvk_decode_graph_refresh(src_pos.data_ptr(), src_slot.data_ptr(), src_ctx.data_ptr(),
                                      src_bt.data_ptr(), src_bt.stride(0), bs, width,
                                      pos.data_ptr(), slot.data_ptr(), ctx.data_ptr(),
                                      bt.data_ptr(), bt.stride(0), rows,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    for got, ref, what in ((pos, pos_r, "positions"), (slot, slot_r, "slot_mapping"),
                           (ctx, ctx_r, "context_lens"), (bt, bt_r, "block_tables")):
        assert torch.equal(got, ref), what
    # a batch above the static rows and a table wider than its stride are refused
    assert lib.nvk_decode_graph_refresh(src_pos.data_ptr(), src_slot.data_ptr(),
                                        src_ctx.data_ptr(), src_bt.data_ptr(), src_bt.stride(0),
                                        rows + 1, width, pos.data_ptr(), slot.data_ptr(),
                                        ctx.data_ptr(), bt.data_ptr(), bt.stride(0), rows,
                                        torch.cuda.current_stream().cuda_stream) != 0
    assert lib.nvk_decode_graph_refresh(src_pos.data_ptr(), src_slot.data_ptr(),
                                        src_ctx.data_ptr(), src_bt.data_ptr(), src_bt.stride(0),
                                        max(bs, 1), cols + 1, pos.data_ptr(), slot.data_ptr(),
                                        ctx.data_ptr(), bt.data_ptr(), bt.stride(0), rows,
                                        torch.cuda.current_stream().cuda_stream) != 0
