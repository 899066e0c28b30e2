#!/usr/bin/env python3
"""Benchmark of the nano-vLLM KV-cache hot path on one MI355X.

Headline (`value`): paged GQA decode attention, Qwen3-0.6B shape: batch 64,
16 q / 8 kv heads, head_dim 128, bf16, 256-token pages, context U{100..2048}
(seeded).  A step is one decode-attention call over the batch (the split-K
kernel and its combine pass).  `value` = algorithmic bytes of a step (unique
K+V bytes of every context + q read + output written) / wall time per step,
with every input resident in HBM.  More legs ride along in the same JSON
line: the KV-store scatter (4096 tokens into a 64-page cache, 5 % slots -1)
in GB/s, the fused q/k RMSNorm + RoPE + KV-store prologue over one layer's
4288 new tokens of the mixed step in GB/s (with the same steps as eager
torch operations timed beside it), the varlen prefill over a 512-token
shared prefix (32 sequences, U{100..1024} new tokens) in TFLOP/s of unmasked QK^T + PV work, the
speculative-decode verification (32 sequences, 6 queries over U{1024..8192}
keys, split-K) in GB/s, the decode attention path of a 28-layer stack
(fused prologue + paged decode per layer, B = 64) replayed from bucketed HIP
graphs as the reference's run_model does, in GB/s, the step metadata built
by the reference's host loops against the device builders (ms per call), the
sampler over Qwen3-sized logits against the reference's torch operations, and
a mixed step of 28 layers (per layer: KV-store of 4288 tokens, 8 prefill chunks of 512 after U{0..1536} cached tokens, 192
decodes over U{256..4096}; a separate KV pool per layer) as the fraction of
its roofline time (decode and store bytes at HBM peak + prefill FLOPs at MFMA
peak).

Timing: each leg builds K steps into one HIP graph cycling over copies of its
inputs (as many as make one cycle touch >= 1 GiB, 4x the 256 MB Infinity
Cache, so no step finds its working set cached from the previous use of its
copy), replays a W-step graph first as warmup, then
brackets one replay of the K-step graph with device synchronisation (wall
clock -> ms_per_step) and HIP events on the launch stream (-> roofline
achieved).  The CPU baseline of the store, decode and prefill legs is the
reference's path on the host CPU in PyTorch (index_put, block-table gather +
scaled_dot_product_attention; oracle/torch_cpu.py) on up to 16 host threads;
the prologue's is the numpy oracle on one thread.  Both run on the same inputs.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                  [--legs decode,store,prologue,prefill,spec,graph,metadata,sampler,mixed]
                  [--eager]

--eager launches the steps one by one instead of replaying a graph (for
counter collection with rocprofv3, which profiles individual dispatches).
--copy-calibration MiB only runs a plain device-to-device copy of that size
(5 launches) and exits: the reference kernel of known traffic against which
the HBM counters (FETCH_SIZE / WRITE_SIZE) of the legs are scaled.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "learn-nano-vllm_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "decode-attn + KV-store HBM GB/s (% peak); prefill MFMA util; Qwen3-0.6B shape"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--legs",
                   default="decode,store,prologue,prefill,spec,graph,metadata,sampler,mixed",
                   help="comma list of legs to run (decode, the headline, always runs)")
    p.add_argument("--eager", action="store_true",
                   help="launch steps one by one (no graph), e.g. under rocprofv3 --pmc")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MiB",
                   help="only run a plain device copy of MiB mebibytes (counter calibration)")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_eager(torch, step_fns, steps, warmup):
    """Launch `steps` calls (cycling over step_fns) one by one; return
    (wall seconds per step, event seconds per step)."""
    for i in range(max(1, warmup)):
        step_fns[i % len(step_fns)]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        step_fns[i % len(step_fns)]()
    end.record()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, start.elapsed_time(end) / 1e3 / steps


def time_graph(torch, step_fns, steps, warmup, eager=False):
    """Capture `steps` calls (cycling over step_fns) in one graph; return
    (wall seconds per step, event seconds per step)."""
    if eager:
        return time_eager(torch, step_fns, steps, warmup)
    def capture(n, start):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(len(step_fns)):          # eager warmup of every variant
                step_fns[i]()
        torch.cuda.current_stream().wait_stream(s)
        with torch.cuda.graph(g):
            for i in range(n):
                step_fns[(start + i) % len(step_fns)]()
        return g

    # the timed steps continue the cycle where the warmup stopped
    g_warm = capture(max(1, warmup), 0)
    g = capture(steps, max(1, warmup) % len(step_fns))
    g_warm.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ev = start.elapsed_time(end) / 1e3 / steps
    return wall, ev


def cpu_time(fn, reps):
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


MALL_CYCLE_BYTES = 1 << 30   # 4x the 256 MB Infinity Cache


def rotation(bytes_per_call, least=2):
    """Copies of a leg's inputs to cycle over so that one cycle touches at least
    1 GiB of distinct data: no call finds its working set still in the 256 MB
    Infinity Cache from the previous use of the same copy."""
    return max(least, -(-MALL_CYCLE_BYTES // max(1, int(bytes_per_call))))


def host_threads(torch):
    """Host threads the CPU baseline runs on: the CPUs this process may use,
    at most 16 (the host cores that go with one GPU of an 8-GPU node)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(max(1, min(16, n or 1)))
    return torch.get_num_threads()


def traffic_for(leg):
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(leg, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def mixed_leg(torch, dev, args, orc, layers=28):
    """28 layers of one mixed step, each with its own KV pool (random bf16 made on
    the GPU) and the same block tables / slots; a layer = KV-store of every new
    token, the prefill chunks, the decodes."""
    from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill
    from nanovllm_amd.workloads import mixed_step_metadata

    log(f"building mixed step ({layers} layers, ~3.5 GB of KV pool per layer)")
    tens, meta = mixed_step_metadata()
    t = {k: v.to(dev) for k, v in tens.items()}
    gen = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev,
                                     dtype=torch.float32).to(torch.bfloat16)
    n_tok, nb = meta["n_tokens"], meta["pool_blocks"]
    q_pf, q_dec = rnd(4096, 16, 128), rnd(192, 16, 128)
    key, value = rnd(n_tok, 8, 128), rnd(n_tok, 8, 128)
    pools = []
    for _ in range(layers):
        kc = torch.empty(nb, 256, 8, 128, dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        for x in (kc, vc):
            for i in range(0, nb, 256):
                x[i:i + 256].copy_(rnd(min(256, nb - i), 256, 8, 128))
        pools.append((kc, vc))
    o_pf, o_dec = torch.empty_like(q_pf), torch.empty_like(q_dec)
    scale = 128 ** -0.5

    def step():
        for kc, vc in pools:
            store_kvcache(key, value, kc, vc, t["slot_mapping"])
            varlen_prefill(q_pf, kc, vc, t["cu_seqlens_q"], t["cu_seqlens_k"],
                           meta["max_seqlen_q"], scale, block_table=t["prefill_block_tables"],
                           out=o_pf, max_seqlen_k=meta["max_seqlen_k"])
            paged_decode(q_dec, kc, vc, t["context_lens"], t["decode_block_tables"], scale,
                         out=o_dec)

    steps, warm = min(args.steps, 10), min(args.warmup, 2)
    log("timing mixed step")
    wall, ev = time_graph(torch, [step], steps, warm, args.eager)
    dec_bytes = orc.attention_bytes(meta["dec_lens"], 8, 128, 192, 16)
    pf_flops = orc.prefill_flops(meta["lens_q"], meta["lens_k"], 16, 128)
    st_bytes = int((tens["slot_mapping"] >= 0).sum()) * 2 * 2 * 2048 + 4 * n_tok
    t_roof = layers * ((dec_bytes + st_bytes) / (HBM_PEAK_GBS * 1e9) +
                       pf_flops / (BF16_PEAK_TFLOPS * 1e12))
    del pools
    return dict(ms_per_step=wall * 1e3, layers=layers, steps=steps,
                workload="28 layers x (KV-store 4288 tokens + 8 prefill chunks of 512 after "
                         "U{0..1536} cached + 192 decodes over U{256..4096}), 3300-page pool "
                         "per layer",
                per_layer={"decode_bytes": dec_bytes, "prefill_flops": pf_flops,
                           "store_bytes": st_bytes},
                roofline={"bound": "mixed", "t_roof_ms": round(t_roof * 1e3, 4),
                          "t_measured_ms": round(ev * 1e3, 4),
                          "frac": round(t_roof / ev, 4)})


def prologue_leg(torch, dev, args, orc, bits):
    """Fused q/k RMSNorm + RoPE + KV-store over the mixed step's 4288 new tokens
    of one layer (rotated copies of the inputs storing into one 3300-page pool), and the
    same steps as separate eager torch operations (the reference's
    layernorm.py:16-26 / rotary_embedding.py:6-14 code, then the store) for
    comparison."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from nanovllm_amd import qk_norm_rope_store, store_kvcache
    from nanovllm_amd.workloads import prologue_case

    log("building prologue workload (4288 tokens of the mixed step, 3300-page pool)")
    pc = prologue_case()
    hq, hkv, hd, eps = pc.hq, pc.hkv, pc.hd, pc.eps
    n_valid = int((pc.slot_mapping >= 0).sum())
    pbytes = orc.prologue_bytes(pc.n_tokens, n_valid, pc.n_unique_positions, hq, hkv, hd,
                                write_k=False)
    # copies of the step's inputs; every copy stores into other rows of one
    # shared pool (its slots shifted by a multiple of 53 pages, mod the pool)
    kc = torch.zeros(pc.pool_blocks, pc.block_size, hkv, hd, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    n_slots = pc.pool_blocks * pc.block_size
    copies = []
    for i in range(rotation(pbytes)):
        c = pc.to(dev)
        sm = c.slot_mapping
        c.tensors["slot_mapping"] = torch.where(sm >= 0, (sm + i * 53 * pc.block_size) % n_slots,
                                                sm)
        copies.append((c, kc, vc))
    fused = [(lambda c=c, kc=kc, vc=vc: qk_norm_rope_store(
        c.positions, c.qkv, hq, hkv, hd, c.q_weight, c.k_weight, eps, c.cos_sin, kc, vc,
        c.slot_mapping, return_k=False)) for c, kc, vc in copies]

    def rms(x, w):                                        # layernorm.py:16-26, eager
        dt = x.dtype
        x = x.float()
        var = x.pow(2).mean(dim=-1, keepdim=True)
        x.mul_(torch.rsqrt(var + eps))
        return x.to(dt).mul_(w)

    def rope(x, cos, sin):                                # rotary_embedding.py:6-14, eager
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    def unfused_step(c, kc, vc):
        q, k, v = c.qkv.split([hq * hd, hkv * hd, hkv * hd], dim=-1)
        q, k, v = q.view(-1, hq, hd), k.view(-1, hkv, hd), v.view(-1, hkv, hd)
        q, k = rms(q, c.q_weight), rms(k, c.k_weight)
        cos, sin = c.cos_sin[c.positions].chunk(2, dim=-1)
        q, k = rope(q, cos, sin), rope(k, cos, sin)
        store_kvcache(k, v, kc, vc, c.slot_mapping)
        return q

    unfused = [(lambda c=c, kc=kc, vc=vc: unfused_step(c, kc, vc)) for c, kc, vc in copies]
    log("timing fused prologue")
    wall, ev = time_graph(torch, fused, args.steps, args.warmup, args.eager)
    log("timing the same steps as eager torch operations")
    wall_u, _ = time_graph(torch, unfused, min(args.steps, 20), min(args.warmup, 3), args.eager)
    leg = dict(ms_per_step=wall * 1e3, bytes_per_step=pbytes,
               workload="q/k RMSNorm + RoPE + KV-store of one layer's 4288 new tokens "
                        "(Qwen3-0.6B heads 16/8, head_dim 128; 8 prefill chunks of 512 + 192 "
                        "decodes; 3300-page pool)",
               unfused_torch_ms=round(wall_u * 1e3, 5),
               roofline={"bound": "hbm", "achieved": round(pbytes / ev / 1e9, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": traffic_for("prologue")})
    if not args.no_cpu_baseline:
        qkv_b, pos = bits(pc.qkv), pc.positions.numpy()
        qw, kw, cs = bits(pc.q_weight), bits(pc.k_weight), pc.cos_sin.reshape(-1, hd).numpy()
        sl = pc.slot_mapping.numpy()
        kc_h = np.zeros((pc.pool_blocks, pc.block_size, hkv, hd), dtype=np.uint16)
        vc_h = np.zeros_like(kc_h)
        with threadpool_limits(1):
            t = cpu_time(lambda: orc.qk_norm_rope_store(qkv_b, pos, qw, kw, eps, cs, hq, hkv, hd,
                                                        kc_h, vc_h, sl), 5)
        leg["cpu_baseline"] = {"value": round(pbytes / t / 1e9, 4), "unit": "GB/s", "cores": 1,
                               "kind": "port",
                               "sample": "the full 4288-token prologue through the numpy oracle "
                                         "(norms, rotation, store), median of 5 reps on 1 host "
                                         "thread"}
    del copies, fused, unfused
    return leg


def decode_graph_leg(torch, dev, args, orc, layers=28):
    """The decode attention path of a 28-layer Qwen3-0.6B stack, captured per
    batch bucket and replayed as the reference's run_model does: per layer the
    fused prologue (q/k norms, rotation, store of the new token) and the paged
    decode over the headline decode contexts (B = 64, U{100..2048}; the B = 4 line
    runs both inside the decode kernel, as attention_with_prologue routes
    batches of up to 32); every layer has
    its own 1024-page cache (views of one [2, 28, 1024, 256, 8, 128]
    allocation).  Timed as graph replays (run() with its host-side buffer
    refresh) and as the same step launched eagerly."""
    from nanovllm_amd.engine.graph_runner import DecodeGraphRunner
    from nanovllm_amd.utils.context import reset_context, set_context
    from nanovllm_amd.workloads import decode_case, decode_stack

    dc = decode_case()
    b, nb, w = 64, dc.k_cache.shape[0], dc.block_tables.shape[1]
    log(f"building {layers}-layer decode stack (30 GB of KV cache) and capturing buckets")
    stack, _, kv_cache, step = decode_stack(layers, nb, dev)
    r = 16 + 2 * 8
    runner = DecodeGraphRunner(step, b, w, inputs={"qkv": ((layers, r * 128), torch.bfloat16)},
                               output=((layers, 16 * 128), torch.bfloat16), device=dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    qkv = (torch.randn(b, layers, r * 128, generator=gen, device=dev) * 2.0).to(torch.bfloat16)
    lens = dc.context_lens.to(dev)
    slots = torch.tensor([int(dc.block_tables[i, (n - 1) // 256]) * 256 + (n - 1) % 256
                          for i, n in enumerate(dc.lens)], dtype=torch.int32, device=dev)
    pos = (lens - 1).to(torch.int64)
    steps, warm = min(args.steps, 20), min(args.warmup, 3)

    def timed(n):
        """(graph replay, eager) seconds per step for the first n sequences."""
        set_context(False, slot_mapping=slots[:n], context_lens=lens[:n],
                    block_tables=dc.block_tables[:n].to(dev))
        try:
            out = []
            for fn in (lambda: runner.run(pos[:n], qkv=qkv[:n]), lambda: step(pos[:n], qkv[:n])):
                for _ in range(warm):
                    fn()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(steps):
                    fn()
                torch.cuda.synchronize()
                out.append((time.perf_counter() - t0) / steps)
            return out
        finally:
            reset_context()

    log("timing graph replays and eager launches, B = 64 and B = 4")
    t_graph, t_eager = timed(b)
    t_graph4, t_eager4 = timed(4)
    per_layer = (orc.attention_bytes(dc.lens, 8, 128, b, 16) +
                 orc.prologue_bytes(b, b, b, 16, 8, 128, write_k=False))
    total = layers * per_layer
    del runner, stack, kv_cache
    return dict(ms_per_step=round(t_graph * 1e3, 4), eager_ms_per_step=round(t_eager * 1e3, 4),
                batch4={"ms_per_step": round(t_graph4 * 1e3, 4),
                        "eager_ms_per_step": round(t_eager4 * 1e3, 4),
                        "contexts": dc.lens[:4]},
                layers=layers, bytes_per_step=total,
                workload=f"{layers} layers x (fused q/k norm + RoPE + store of 64 new tokens, "
                         "paged decode B=64 over U{100..2048}), bucket 64 of "
                         "[1, 2, 4, 8, 16, 32, 48, 64], graph replays",
                roofline={"bound": "hbm", "achieved": round(total / t_graph / 1e9, 2),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(total / t_graph / 1e9 / HBM_PEAK_GBS, 4)})


def metadata_leg(torch, dev, args):
    """Step metadata built by the reference's host loops (restated in
    engine/metadata.py) against the device builders, wall time per call
    including the upload and a device synchronisation: a chunked-prefill step
    of 64 sequences (U{0..1536} cached + U{100..1024} new tokens) and a
    512-sequence decode step over U{256..4096}."""
    import random
    from nanovllm_amd.engine import metadata
    from nanovllm_amd.engine.device_metadata import prepare_decode_device, prepare_prefill_device
    from nanovllm_amd.engine.sequence import Sequence
    from nanovllm_amd.utils.context import reset_context

    rng = random.Random(8)
    bs = 256
    pages = list(range(64 * 11 + 512 * 17))
    rng.shuffle(pages)
    nxt = 0
    pf = []
    for _ in range(64):
        c, m = rng.randint(0, 1536), rng.randint(100, 1024)
        need = (c + m + bs - 1) // bs
        pf.append(Sequence([rng.randint(0, 150000) for _ in range(c + m)],
                           block_table=pages[nxt:nxt + need], num_cached_tokens=c,
                           num_scheduled_tokens=m))
        nxt += need
    dc = []
    for _ in range(512):
        n = rng.randint(256, 4096)
        need = (n + bs - 1) // bs
        dc.append(Sequence([rng.randint(0, 150000) for _ in range(n)],
                           block_table=pages[nxt:nxt + need]))
        nxt += need

    def wall(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
            reset_context()
        return statistics.median(ts)

    log("timing step metadata builders (host loops vs device kernel)")
    reps = 20
    res = {
        "prefill_64_seqs": {
            "tokens": sum(q.num_scheduled_tokens for q in pf),
            "host_loops_ms": round(wall(lambda: metadata.prepare_prefill(pf, bs, dev), reps) * 1e3, 3),
            "device_ms": round(wall(lambda: prepare_prefill_device(pf, bs, dev), reps) * 1e3, 3)},
        "decode_512_seqs": {
            "host_loops_ms": round(wall(lambda: metadata.prepare_decode(dc, bs, dev), reps) * 1e3, 3),
            "device_ms": round(wall(lambda: prepare_decode_device(dc, bs, dev), reps) * 1e3, 3)},
    }
    res["workload"] = ("slot_mapping / positions / cu_seqlens / padded block tables of a "
                       "64-sequence chunked prefill and a 512-sequence decode, median of "
                       f"{reps} calls, wall time with the device synchronised")
    return res


def sampler_leg(torch, dev, args):
    """Temperature sampling of the next tokens from Qwen3-0.6B-sized logits
    (vocab 151936, bf16) for 64 and 512 sequences: the fused kernel (one read
    of the logits, Philox noise) against the reference's torch operations
    (sampler.py:7-12 without torch.compile: float, div, softmax, exponential_,
    clamp_min_, div_, argmax), each timed as a 20-call HIP graph."""
    from nanovllm_amd.layers.sampler import Sampler

    vocab = 151936
    out = {}
    sampler = Sampler()

    def torch_sampler(logits, temps):
        x = logits.float().div_(temps.unsqueeze(dim=1))
        probs = torch.softmax(x, dim=-1)
        return probs.div_(torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)).argmax(dim=-1)

    for b in (64, 512):
        gen = torch.Generator(device=dev).manual_seed(b)
        nbytes = b * vocab * 2 + b * 8
        logits = [(torch.randn(b, vocab, generator=gen, device=dev) * 3).to(torch.bfloat16)
                  for _ in range(rotation(nbytes))]
        temps = torch.full((b,), 0.8, device=dev)
        fused = [(lambda x=x: sampler(x, temps)) for x in logits]
        ref = [(lambda x=x: torch_sampler(x, temps)) for x in logits]
        log(f"timing sampler B={b}")
        _, ev = time_graph(torch, fused, 20, 3, args.eager)
        _, ev_ref = time_graph(torch, ref, 20, 3, args.eager)
        out[f"batch_{b}"] = {"ms_per_call": round(ev * 1e3, 4),
                             "torch_ops_ms_per_call": round(ev_ref * 1e3, 4),
                             "bytes_per_call": nbytes,
                             "roofline": {"bound": "hbm", "achieved": round(nbytes / ev / 1e9, 2),
                                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                          "frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4)}}
        del logits, fused, ref
    out["workload"] = "next-token sampling over bf16 logits [B, 151936], temperature 0.8"
    return out


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV-cache path runs on a single MI355X "
              "(no sharding is built); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return

    from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill
    from nanovllm_amd.workloads import (decode_case, kv_store_case, prefill_case,
                                        spec_verify_case)
    from oracle import kv_oracle as orc
    from oracle import torch_cpu as tcpu

    legs = set(args.legs.split(","))
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    result = {}

    # ------------------------------------------------------------------ decode
    log("building decode workload (B=64, ctx U{100..2048}, 1024-page pool)")
    dc = decode_case()
    dec_bytes = orc.attention_bytes(dc.lens, 8, 128, 64, 16)
    pools = [dc.to(dev) for _ in range(rotation(dec_bytes))]   # separate copies of the pool
    outs = [torch.empty(64, 16, 128, dtype=torch.bfloat16, device=dev) for _ in pools]
    dec_fns = [
        (lambda c=c, o=o: paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens,
                                       c.block_tables, dc.scale, out=o))
        for c, o in zip(pools, outs)]
    log("timing decode")
    wall, ev = time_graph(torch, dec_fns, args.steps, args.warmup, args.eager)
    dec_gbs = dec_bytes / wall / 1e9
    dec_ach = dec_bytes / ev / 1e9
    result["decode"] = dict(ms_per_step=wall * 1e3, gbs=dec_gbs, event_gbs=dec_ach,
                            bytes_per_step=dec_bytes)
    cpu = None
    if not args.no_cpu_baseline:
        threads = host_threads(torch)
        log(f"cpu baseline: decode on the PyTorch CPU path, {threads} threads")
        t = cpu_time(lambda: tcpu.paged_attention_cpu(dc.q, dc.k_cache, dc.v_cache, range(65),
                                                      dc.context_lens, dc.scale,
                                                      dc.block_tables), 10)
        cpu = {"value": round(dec_bytes / t / 1e9, 4), "unit": "GB/s", "cores": threads,
               "kind": "port",
               "sample": "the full 64-sequence decode batch through the PyTorch CPU path "
                         "(block-table gather + f32 scaled_dot_product_attention), median of "
                         f"10 reps on {threads} host threads "
                         f"(os.cpu_count() = {os.cpu_count()})"}
    del pools, outs, dec_fns

    # ------------------------------------------------------------------ store
    if "store" in legs:
        log("building kv-store workload (4096 tokens, 64 pages, 205 slots -1)")
        sc = kv_store_case()
        n_valid = int((sc.slot_mapping >= 0).sum())
        st_bytes = n_valid * 2 * 2 * 8 * 128 * 2 + 4 * 4096
        copies = [sc.to(dev) for _ in range(rotation(st_bytes))]
        st_fns = [(lambda c=c: store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping))
                  for c in copies]
        log("timing kv-store")
        wall_s, ev_s = time_graph(torch, st_fns, args.steps, args.warmup, args.eager)
        leg = dict(ms_per_step=wall_s * 1e3, bytes_per_step=st_bytes,
                   roofline={"bound": "hbm", "achieved": round(st_bytes / ev_s / 1e9, 2),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(st_bytes / ev_s / 1e9 / HBM_PEAK_GBS, 4),
                             "traffic": traffic_for("kv_store")})
        if not args.no_cpu_baseline:
            threads = host_threads(torch)
            kc, vc = sc.k_cache.clone(), sc.v_cache.clone()
            t = cpu_time(lambda: tcpu.store_kvcache_cpu(sc.key, sc.value, kc, vc,
                                                        sc.slot_mapping), 50)
            leg["cpu_baseline"] = {"value": round(st_bytes / t / 1e9, 3), "unit": "GB/s",
                                   "cores": threads, "kind": "port",
                                   "sample": "full 4096-token store through the PyTorch CPU "
                                             "path (index_put on the flat cache views), median "
                                             f"of 50 reps on {threads} host threads "
                                             f"(os.cpu_count() = {os.cpu_count()})"}
        result["kv_store"] = leg
        del copies, st_fns

    # ------------------------------------------------------------------ prologue
    if "prologue" in legs:
        result["prologue"] = prologue_leg(torch, dev, args, orc, bits)

    # ------------------------------------------------------------------ prefill
    if "prefill" in legs:
        log("building prefill workload (32 seqs, 512-token shared prefix)")
        pc = prefill_case()
        touched = orc.attention_bytes(pc.lens_k, 8, 128, sum(pc.lens_q), 16)
        copies = [pc.to(dev) for _ in range(rotation(touched))]
        for c in copies:   # the new tokens' K/V are in the cache before attention
            store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
        outs = [torch.empty_like(c.q) for c in copies]
        pf_fns = [(lambda c=c, o=o: varlen_prefill(c.q, c.k_cache, c.v_cache, c.cu_seqlens_q,
                                                   c.cu_seqlens_k, pc.max_seqlen_q, pc.scale,
                                                   block_table=c.block_tables, out=o))
                  for c, o in zip(copies, outs)]
        flops = orc.prefill_flops(pc.lens_q, pc.lens_k, 16, 128)
        log("timing prefill")
        wall_p, ev_p = time_graph(torch, pf_fns, args.steps, args.warmup, args.eager)
        tf = flops / ev_p / 1e12
        leg = dict(ms_per_step=wall_p * 1e3, flops_per_step=flops,
                   roofline={"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                             "traffic": traffic_for("prefill")})
        if not args.no_cpu_baseline:
            threads = host_threads(torch)
            kc, vc = pc.k_cache.clone(), pc.v_cache.clone()
            tcpu.store_kvcache_cpu(pc.key, pc.value, kc, vc, pc.slot_mapping)
            t = cpu_time(lambda: tcpu.paged_attention_cpu(pc.q, kc, vc, pc.cu_seqlens_q,
                                                          pc.lens_k, pc.scale,
                                                          pc.block_tables), 5)
            leg["cpu_baseline"] = {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s",
                                   "cores": threads, "kind": "port",
                                   "sample": "the full 32-sequence prefill through the PyTorch "
                                             "CPU path (block-table gather + f32 "
                                             "scaled_dot_product_attention with the "
                                             "bottom-right causal mask), median of 5 reps on "
                                             f"{threads} host threads "
                                             f"(os.cpu_count() = {os.cpu_count()})"}
        result["prefill"] = leg
        del copies, outs, pf_fns

    # ------------------------------------------------------------------ spec verify
    if "spec" in legs:
        log("building spec-verify workload (32 seqs, 6 queries, ctx U{1024..8192})")
        vc_ = spec_verify_case()
        sv_bytes = orc.attention_bytes(vc_.lens_k, 8, 128, 32 * 6, 16)
        copies = [vc_.to(dev) for _ in range(rotation(sv_bytes))]
        for c in copies:   # the 5 draft tokens of every sequence are stored first
            store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
        outs = [torch.empty_like(c.q) for c in copies]
        sv_fns = [(lambda c=c, o=o: varlen_prefill(c.q, c.k_cache, c.v_cache, c.cu_seqlens_q,
                                                   c.cu_seqlens_k, vc_.max_seqlen_q, vc_.scale,
                                                   block_table=c.block_tables, out=o,
                                                   max_seqlen_k=vc_.max_seqlen_k))
                  for c, o in zip(copies, outs)]
        log("timing spec verify")
        wall_v, ev_v = time_graph(torch, sv_fns, args.steps, args.warmup, args.eager)
        result["spec_verify"] = dict(
            ms_per_step=wall_v * 1e3, bytes_per_step=sv_bytes,
            workload="32 sequences x 6 query tokens (5 drafts + the last accepted token) over "
                     "U{1024..8192} paged keys (short-query stream-K kernels)",
            roofline={"bound": "hbm", "achieved": round(sv_bytes / ev_v / 1e9, 2),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(sv_bytes / ev_v / 1e9 / HBM_PEAK_GBS, 4),
                      "traffic": traffic_for("spec_verify")})
        del copies, outs, sv_fns

    # ------------------------------------------------------------------ decode graphs
    if "graph" in legs:
        result["decode_graph"] = decode_graph_leg(torch, dev, args, orc)

    # ------------------------------------------------------------------ step metadata
    if "metadata" in legs:
        result["step_metadata"] = metadata_leg(torch, dev, args)

    # ------------------------------------------------------------------ sampler
    if "sampler" in legs:
        result["sampler"] = sampler_leg(torch, dev, args)

    # ------------------------------------------------------------------ mixed step
    if "mixed" in legs:
        result["mixed_step"] = mixed_leg(torch, dev, args, orc)

    d = result["decode"]
    line = {
        "metric": METRIC,
        "value": round(d["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "paged GQA decode attention: batch 64, 16 q / 8 kv heads, "
                               "head_dim 128, bf16, 256-token pages, context U{100..2048} (seed 1)",
                   "batch": 64, "num_q_heads": 16, "num_kv_heads": 8, "head_dim": 128,
                   "block_size": 256, "context": "U{100..2048}",
                   "bytes_per_step": d["bytes_per_step"]},
        "roofline": {"bound": "hbm", "achieved": round(d["event_gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(d["event_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("decode")},
        "cpu_baseline": cpu,
    }
    for k in ("kv_store", "prologue", "prefill", "spec_verify", "decode_graph", "step_metadata",
              "sampler", "mixed_step"):
        if k in result:
            line[k] = result[k]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
