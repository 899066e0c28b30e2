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
copy), launches the K-step graph once untimed (its first launch uploads it),
replays a W-step graph as warmup and keeps replaying it until at least 50 ms
of warm replays have run (so the clocks are up whatever W is), then times
the K-step graph TIMED_REPS times, each replay bracketed by device
synchronisation (wall clock), alternating with as many replays bracketed by
HIP events on the launch stream; ms_per_step is the median wall time and
roofline achieved uses the median event time (a single ~1 ms replay moved
by 5-10 % with host-side jitter).  Beside the store, a device copy of the same bytes (and one of 512
MiB) under the same rotation gives the copy rate this box reaches.

CPU baselines run after every GPU leg: the reference's path on the host CPU
in PyTorch (oracle/torch_cpu.py: index_put for the store, block-table gather +
scaled_dot_product_attention for decode, prefill, spec-verify and the mixed
step, the eager RMSNorm / rotary / store tensor operations for the prologue)
on up to 16 host threads, on the same inputs (the mixed step on one layer,
scaled by 28).

roofline.traffic (HBM bytes per step behind the L2) comes from
profiles/hbm_traffic.json, written by --collect-traffic from rocprofv3
FETCH_SIZE / WRITE_SIZE runs; it is reported only when the file was measured
on the kernel sources being timed (a hash of csrc/ and include/), else null.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                  [--legs decode,store,prologue,prefill,spec,graph,metadata,sampler,mixed]
                  [--eager]

--eager launches the steps one by one instead of replaying a graph (for
counter collection with rocprofv3, which profiles individual dispatches).
--copy-calibration MiB only runs a plain device-to-device copy of that size
(5 launches) and exits: the reference kernel of known traffic against which
the HBM counters (FETCH_SIZE / WRITE_SIZE) of the legs are scaled.
--collect-traffic DIR OUT reads the counter runs under DIR (named
<COUNTER>_copy and <COUNTER>_<leg>, see profiles/hbm_traffic_counters.md) and
writes the traffic file OUT.
"""
from __future__ import annotations

import argparse
import csv
import glob
import hashlib
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
    p.add_argument("--collect-traffic", nargs=2, metavar=("DIR", "OUT"),
                   help="write the traffic file OUT from the rocprofv3 counter runs under DIR")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


MIN_WARM_S = 0.05   # every leg warms for at least this long before its timed replays
TIMED_REPS = 5      # timed replays of the K steps; the medians are reported


def time_eager(torch, step_fns, steps, warmup):
    """Launch `steps` calls (cycling over step_fns) one by one; return
    (wall seconds per step, event seconds per step)."""
    t_warm = time.perf_counter()
    i = 0
    while i < max(1, warmup) or time.perf_counter() - t_warm < MIN_WARM_S:
        step_fns[i % len(step_fns)]()
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()

    def run():
        for i in range(steps):
            step_fns[i % len(step_fns)]()
    return timed_reps(torch, run, steps)


def timed_reps(torch, run, steps):
    """TIMED_REPS wall-clock timings of run() (K steps) bracketed by device
    synchronisation, alternating with TIMED_REPS timings by HIP events on the
    current stream; returns the medians per step (wall s, event s)."""
    # The first record of a new event costs ~200 us of host time on MI355X,
    # which would sit inside the event interval: both are recorded once first.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    end.record()
    walls, evs = [], []
    for _ in range(TIMED_REPS):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run()
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) / steps)
        start.record()
        run()
        end.record()
        torch.cuda.synchronize()
        evs.append(start.elapsed_time(end) / 1e3 / steps)
    return statistics.median(walls), statistics.median(evs)


def time_graph(torch, step_fns, steps, warmup, eager=False):
    """Capture `steps` calls (cycling over step_fns) in one graph; return
    (wall seconds per step, event seconds per step).  The warmup graph of
    `warmup` steps is replayed until at least MIN_WARM_S of replays ran."""
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
    # The first launch of a graph uploads it (measured on MI355X: ~250 us of
    # host time for a 40-node graph): it happens here, untimed.
    g.replay()
    torch.cuda.synchronize()
    t_warm = time.perf_counter()
    g_warm.replay()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t_warm, 1e-6)
    for _ in range(int((MIN_WARM_S - one) / one) + 1 if one < MIN_WARM_S else 0):
        g_warm.replay()
    torch.cuda.synchronize()
    return timed_reps(torch, g.replay, steps)


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


def kernel_source_hash():
    """sha256 over the kernel sources (learn-nano-vllm_amd/csrc/*, include/*.h):
    the traffic file is valid only for the sources it was measured on."""
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(ROOT, "learn-nano-vllm_amd", "csrc", "*")) +
                   glob.glob(os.path.join(ROOT, "include", "*.h")))
    for f in files:
        h.update(os.path.relpath(f, ROOT).encode())
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def traffic_for(leg):
    """HBM bytes per step of a leg, or None when the traffic file is missing or
    was measured on other kernel sources than the ones built here."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    if data.get("source_sha256") != kernel_source_hash():
        return None
    return data.get("legs", {}).get(leg, {}).get("bytes_per_launch")


# Traffic collection: per leg, the bench run that holds it (--legs), the
# kernels of one step, and the kernel launched once per step.
TRAFFIC_LEGS = {
    "decode": ("decode", ("paged_decode_kernel", "paged_decode_combine_kernel"),
               "paged_decode_kernel"),
    "kv_store": ("store", ("kv_store_rows_kernel",), "kv_store_rows_kernel"),
    "prologue": ("prologue", ("qk_prologue_kernel",), "qk_prologue_kernel"),
    "prefill": ("prefill", ("varlen_prefill_kernel",), "varlen_prefill_kernel"),
    "spec_verify": ("spec", ("short_query_kernel", "short_query_combine_kernel"),
                    "short_query_kernel"),
}


def _base_name(kernel_name):
    """'void (anonymous namespace)::foo<1, 2>((anonymous namespace)::Args)' -> 'foo'."""
    head = kernel_name.replace("(anonymous namespace)::", "")
    head = head[5:] if head.startswith("void ") else head
    for sep in ("<", "("):
        head = head.split(sep)[0]
    return head.strip()


def _counter_rows(run_dir):
    files = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {run_dir}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def collect_traffic(run_root, out_path):
    """Per leg, mean HBM bytes per step from the FETCH_SIZE and WRITE_SIZE runs,
    each counter scaled by what it reads for the 512 MiB calibration copy."""
    scale = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [float(r["Counter_Value"]) for r in _counter_rows(f"{run_root}/{counter}_copy")
                if r["Counter_Name"] == counter and "copyBuffer" in r["Kernel_Name"]]
        if not vals:
            raise SystemExit(f"{counter}: no copy dispatch in the calibration run")
        scale[counter] = (512 << 20) / (statistics.mean(vals) * 1024.0)
    legs = {}
    for leg, (run, kernels, main_kernel) in TRAFFIC_LEGS.items():
        per = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            sums, counts = {}, {}
            for r in _counter_rows(f"{run_root}/{counter}_{run}"):
                name = r["Kernel_Name"]
                if r["Counter_Name"] != counter or _base_name(name) not in kernels:
                    continue
                sums[name] = sums.get(name, 0.0) + float(r["Counter_Value"])
                counts[name] = counts.get(name, 0) + 1
            steps = sum(c for n, c in counts.items() if _base_name(n) == main_kernel)
            if not steps:
                raise SystemExit(f"{leg}: no {main_kernel} dispatch in {counter}_{run}")
            for name in sums:
                per.setdefault(name, {"dispatches": counts[name]})
                key = "read_bytes" if counter == "FETCH_SIZE" else "write_bytes"
                per[name][key] = int(sums[name] * 1024.0 * scale[counter] / steps)
        rd = sum(k.get("read_bytes", 0) for k in per.values())
        wr = sum(k.get("write_bytes", 0) for k in per.values())
        legs[leg] = {"bytes_per_launch": rd + wr, "read_bytes": rd, "write_bytes": wr,
                     "kernels": per}
    data = {"_note": "HBM-side bytes per step (every kernel of the operator, per eager step), "
                     "from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of bench.py --eager, "
                     "each scaled by what the counter reads for a 512 MiB device copy",
            "source_sha256": kernel_source_hash(),
            "scale": {k: round(v, 4) for k, v in scale.items()},
            "legs": legs}
    with open(out_path, "w") as f:
        json.dump(data, f, indent=1)
    print(json.dumps({k: v["bytes_per_launch"] for k, v in legs.items()}), flush=True)


def mixed_leg(torch, dev, args, cpu_jobs, layers=28):
    """28 layers of one mixed step, each with its own KV pool (random bf16 made on
    the GPU) and the same block tables / slots; a layer = KV-store of every new
    token, then the decodes with the prefill chunks beside them on a second
    stream, joined before the next layer."""
    from nanovllm_amd import paged_decode, store_kvcache, varlen_prefill
    from nanovllm_amd.flash_api import prefill_tile_order
    from nanovllm_amd.workloads import attention_bytes, mixed_step_metadata, prefill_flops

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

    side = torch.cuda.Stream()   # default priority

    def step():
        # the layers share the step's metadata: the prefill tiles are ranked once
        order = prefill_tile_order(t["cu_seqlens_q"], t["cu_seqlens_k"], meta["max_seqlen_q"],
                                   pools[0][0], 16, block_table=t["prefill_block_tables"],
                                   max_seqlen_k=meta["max_seqlen_k"])
        main = torch.cuda.current_stream()
        for kc, vc in pools:
            store_kvcache(key, value, kc, vc, t["slot_mapping"])
            # After the store, the decode takes every workgroup slot first and the
            # prefill chunks, on a side stream, fill the slots its waves leave as
            # they finish; the layer ends when both have (321 -> 306 us per layer
            # on MI355X; the prefill first delays the decode's persistent waves:
            # 383 us).
            side.wait_stream(main)
            paged_decode(q_dec, kc, vc, t["context_lens"], t["decode_block_tables"], scale,
                         out=o_dec)
            with torch.cuda.stream(side):
                varlen_prefill(q_pf, kc, vc, t["cu_seqlens_q"], t["cu_seqlens_k"],
                               meta["max_seqlen_q"], scale, block_table=t["prefill_block_tables"],
                               out=o_pf, max_seqlen_k=meta["max_seqlen_k"], order=order)
            main.wait_stream(side)

    steps, warm = min(args.steps, 10), min(args.warmup, 2)
    log("timing mixed step")
    wall, ev = time_graph(torch, [step], steps, warm, args.eager)
    dec_bytes = attention_bytes(meta["dec_lens"], 8, 128, 192, 16)
    pf_flops = prefill_flops(meta["lens_q"], meta["lens_k"], 16, 128)
    st_bytes = int((tens["slot_mapping"] >= 0).sum()) * 2 * 2 * 2048 + 4 * n_tok
    t_roof = layers * ((dec_bytes + st_bytes) / (HBM_PEAK_GBS * 1e9) +
                       pf_flops / (BF16_PEAK_TFLOPS * 1e12))
    del pools
    if not args.no_cpu_baseline:
        cpu_jobs.append(("mixed_step", lambda: mixed_cpu_baseline(torch, layers)))
    return dict(ms_per_step=wall * 1e3, layers=layers, steps=steps,
                workload="28 layers x (KV-store 4288 tokens + 8 prefill chunks of 512 after "
                         "U{0..1536} cached + 192 decodes over U{256..4096}), 3300-page pool "
                         "per layer; prefill tiles ranked once per step; in each layer the "
                         "decodes run with the prefill chunks beside them on a second stream",
                per_layer={"decode_bytes": dec_bytes, "prefill_flops": pf_flops,
                           "store_bytes": st_bytes},
                roofline={"bound": "mixed", "t_roof_ms": round(t_roof * 1e3, 4),
                          "t_measured_ms": round(ev * 1e3, 4),
                          "frac": round(t_roof / ev, 4)})


def mixed_cpu_baseline(torch, layers):
    """One layer of the mixed step through the PyTorch CPU path (index_put store
    of the 4288 new tokens, then gather + SDPA attention of the 8 prefill
    chunks and of the 192 decodes) on the same metadata, scaled by the layers
    of the step."""
    from oracle import torch_cpu as tcpu
    from nanovllm_amd.workloads import mixed_layer_case

    threads = host_threads(torch)
    log(f"cpu baseline: one mixed-step layer on the PyTorch CPU path, {threads} threads")
    mc = mixed_layer_case()
    kc, vc = mc.k_cache, mc.v_cache

    def layer():
        tcpu.store_kvcache_cpu(mc.key, mc.value, kc, vc, mc.slot_mapping)
        tcpu.paged_attention_cpu(mc.q_prefill, kc, vc, mc.cu_seqlens_q, mc.lens_k, mc.scale,
                                 mc.prefill_block_tables)
        tcpu.paged_attention_cpu(mc.q_decode, kc, vc, range(len(mc.dec_lens) + 1),
                                 mc.context_lens, mc.scale, mc.decode_block_tables)

    t = cpu_time(layer, 3)
    return {"value": round(t * layers * 1e3, 2), "unit": "ms/step", "cores": threads,
            "kind": "port",
            "sample": f"one of the {layers} layers (store of 4288 tokens, 8 prefill chunks of 512, "
                      "192 decodes) through the PyTorch CPU path, median of 3 reps on "
                      f"{threads} host threads (os.cpu_count() = {os.cpu_count()}), times "
                      f"{layers}"}


def prologue_leg(torch, dev, args, cpu_jobs):
    """Fused q/k RMSNorm + RoPE + KV-store over the mixed step's 4288 new tokens
    of one layer (rotated copies of the inputs storing into one 3300-page pool), and the
    same steps as separate eager torch operations (the reference's
    layernorm.py:16-26 / rotary_embedding.py:6-14 code, then the store) for
    comparison."""
    from nanovllm_amd import qk_norm_rope_store, store_kvcache
    from nanovllm_amd.workloads import prologue_bytes, prologue_case

    log("building prologue workload (4288 tokens of the mixed step, 3300-page pool)")
    pc = prologue_case()
    hq, hkv, hd, eps = pc.hq, pc.hkv, pc.hd, pc.eps
    n_valid = int((pc.slot_mapping >= 0).sum())
    pbytes = prologue_bytes(pc.n_tokens, n_valid, pc.n_unique_positions, hq, hkv, hd,
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
        def prologue_cpu():
            from oracle import torch_cpu as tcpu
            threads = host_threads(torch)
            log(f"cpu baseline: prologue on the PyTorch CPU path, {threads} threads")
            kc_h = torch.zeros(pc.pool_blocks, pc.block_size, hkv, hd, dtype=torch.bfloat16)
            vc_h = torch.zeros_like(kc_h)
            cs = pc.cos_sin.reshape(-1, hd)
            t = cpu_time(lambda: tcpu.qk_norm_rope_store_cpu(
                pc.positions, pc.qkv, hq, hkv, hd, pc.q_weight, pc.k_weight, eps, cs, kc_h, vc_h,
                pc.slot_mapping), 10)
            return {"value": round(pbytes / t / 1e9, 4), "unit": "GB/s", "cores": threads,
                    "kind": "port",
                    "sample": "the full 4288-token prologue through the PyTorch CPU path (the "
                              "reference's RMSNorm and rotary tensor operations, then index_put "
                              f"into the caches), median of 10 reps on {threads} host threads "
                              f"(os.cpu_count() = {os.cpu_count()})"}
        cpu_jobs.append(("prologue", prologue_cpu))
    del copies, fused, unfused
    return leg


def decode_graph_leg(torch, dev, args, layers=28):
    """The decode attention path of a 28-layer Qwen3-0.6B stack, captured per
    batch bucket and replayed as the reference's run_model does: per layer the
    fused prologue (q/k norms, rotation, store of the new token) and the paged
    decode over the headline decode contexts (B = 64, U{100..2048}; the B = 4 line
    runs both inside the decode kernel, as attention_with_prologue routes
    batches of up to 32); every layer has
    its own 1024-page cache (views of one [2, 28, 1024, 256, 8, 128]
    allocation).  Timed as graph replays (run() with its refresh of the step
    metadata; the qkv rows sit in the graph's input buffer, as the projection
    would write them inside the graph) and as the same step launched eagerly."""
    from nanovllm_amd.engine.graph_runner import DecodeGraphRunner
    from nanovllm_amd.utils.context import reset_context, set_context
    from nanovllm_amd.workloads import attention_bytes, decode_case, decode_stack, prologue_bytes

    from nanovllm_amd.layers.prologue import attention_with_prologue

    dc = decode_case()
    b, nb, w = 64, dc.k_cache.shape[0], dc.block_tables.shape[1]
    log(f"building {layers}-layer decode stack (30 GB of KV cache) and capturing buckets")
    stack, rope, kv_cache, _ = decode_stack(layers, nb, dev)

    def step(positions, qkv):
        # every layer's kernels run; the step returns the last layer's output,
        # as a model step returns its last hidden state (run_model copies that
        # one tensor into the graph's output buffer, model_runner.py:245)
        out = None
        for i, (attn, qn, kn) in enumerate(stack):
            out = attention_with_prologue(attn, positions, qkv[:, i], qn, kn, rope)
        return out.reshape(positions.numel(), 16 * 128)

    r = 16 + 2 * 8
    runner = DecodeGraphRunner(step, b, w, inputs={"qkv": ((layers, r * 128), torch.bfloat16)},
                               output=((16 * 128,), torch.bfloat16), device=dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    qkv = (torch.randn(b, layers, r * 128, generator=gen, device=dev) * 2.0).to(torch.bfloat16)
    lens = dc.context_lens.to(dev)
    slots = torch.tensor([int(dc.block_tables[i, (n - 1) // 256]) * 256 + (n - 1) % 256
                          for i, n in enumerate(dc.lens)], dtype=torch.int32, device=dev)
    pos = (lens - 1).to(torch.int64)
    steps = min(args.steps, 10)

    def timed(n):
        """(graph replay, eager) seconds per step for the first n sequences:
        medians of TIMED_REPS + 2 rounds, each round timing `steps` replays
        (run(): refresh + replay) and `steps` eager steps by HIP events, one
        after the other, after a time-based warm-up of both."""
        set_context(False, slot_mapping=slots[:n], context_lens=lens[:n],
                    block_tables=dc.block_tables[:n].to(dev))
        # In the model the qkv rows are made inside the graph (the projection
        # precedes attention in every layer); the replay copies only the step
        # metadata, as run_model does (model_runner.py:200-211).  So the rows
        # are put in the graph's input buffer once, not copied every step.
        runner.inputs["qkv"][:n] = qkv[:n]
        fns = (lambda: runner.run(pos[:n]), lambda: step(pos[:n], qkv[:n]))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        e1.record()
        try:
            t_warm = time.perf_counter()
            while time.perf_counter() - t_warm < MIN_WARM_S:
                for fn in fns:
                    fn()
                torch.cuda.synchronize()
            out = ([], [])
            for _ in range(TIMED_REPS + 2):
                for fn, ts in zip(fns, out):
                    torch.cuda.synchronize()
                    e0.record()
                    for _ in range(steps):
                        fn()
                    e1.record()
                    torch.cuda.synchronize()
                    ts.append(e0.elapsed_time(e1) / 1e3 / steps)
            return [statistics.median(ts) for ts in out]
        finally:
            reset_context()

    log("timing graph replays and eager launches, B = 64 and B = 4")
    t_graph, t_eager = timed(b)
    t_graph4, t_eager4 = timed(4)
    per_layer = (attention_bytes(dc.lens, 8, 128, b, 16) +
                 prologue_bytes(b, b, b, 16, 8, 128, write_k=False))
    total = layers * per_layer
    del runner, stack, kv_cache
    return dict(ms_per_step=round(t_graph * 1e3, 4), eager_ms_per_step=round(t_eager * 1e3, 4),
                batch4={"ms_per_step": round(t_graph4 * 1e3, 4),
                        "eager_ms_per_step": round(t_eager4 * 1e3, 4),
                        "contexts": dc.lens[:4]},
                layers=layers, bytes_per_step=total,
                workload=f"{layers} layers x (fused q/k norm + RoPE + store of 64 new tokens, "
                         "paged decode B=64 over U{100..2048}), bucket 64 of "
                         "[1, 2, 4, 8, 16, 32, 48, 64], graph replays (refresh + replay) "
                         "against the same step launched eagerly, HIP-event medians of "
                         "interleaved rounds",
                roofline={"bound": "hbm", "achieved": round(total / t_graph / 1e9, 2),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(total / t_graph / 1e9 / HBM_PEAK_GBS, 4)})


class _SeqRecord:
    """The fields of a scheduled sequence that the step-metadata builders read
    (the reference's Sequence carries them, nanovllm/engine/sequence.py)."""

    def __init__(self, token_ids, block_table, num_cached_tokens=0, num_scheduled_tokens=0):
        self.token_ids = token_ids
        self.block_table = block_table
        self.num_cached_tokens = num_cached_tokens
        self.num_scheduled_tokens = num_scheduled_tokens

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def last_token(self):
        return self.token_ids[-1]


def metadata_leg(torch, dev, args, cpu_jobs):
    """Step metadata built by the device builders, wall time per call including
    the upload and a device synchronisation: a chunked-prefill step of 64
    sequences (U{0..1536} cached + U{100..1024} new tokens) and a 512-sequence
    decode step over U{256..4096}.  The CPU baseline runs the reference's host
    loops (restated in oracle/step_metadata.py) on the same sequences, with the
    same upload and synchronisation."""
    import random
    from nanovllm_amd.engine.device_metadata import prepare_decode_device, prepare_prefill_device
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
        pf.append(_SeqRecord([rng.randint(0, 150000) for _ in range(c + m)],
                             block_table=pages[nxt:nxt + need], num_cached_tokens=c,
                             num_scheduled_tokens=m))
        nxt += need
    dc = []
    for _ in range(512):
        n = rng.randint(256, 4096)
        need = (n + bs - 1) // bs
        dc.append(_SeqRecord([rng.randint(0, 150000) for _ in range(n)],
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

    log("timing step metadata builders (device kernels)")
    reps = 20
    res = {
        "prefill_64_seqs": {
            "tokens": sum(q.num_scheduled_tokens for q in pf),
            "device_ms": round(wall(lambda: prepare_prefill_device(pf, bs, dev), reps) * 1e3, 3)},
        "decode_512_seqs": {
            "device_ms": round(wall(lambda: prepare_decode_device(dc, bs, dev), reps) * 1e3, 3)},
    }
    res["workload"] = ("slot_mapping / positions / cu_seqlens / padded block tables of a "
                       "64-sequence chunked prefill and a 512-sequence decode, median of "
                       f"{reps} calls, wall time with the device synchronised")
    if not args.no_cpu_baseline:
        def metadata_cpu():
            from oracle import step_metadata as host
            from oracle.sequence import Sequence
            log("cpu baseline: step metadata by the reference's host loops")
            pf_h = [Sequence(s.token_ids, s.block_table, s.num_cached_tokens,
                             s.num_scheduled_tokens) for s in pf]
            dc_h = [Sequence(s.token_ids, s.block_table) for s in dc]
            return {"prefill_64_seqs_ms": round(wall(lambda: host.prepare_prefill(pf_h, bs, dev),
                                                     reps) * 1e3, 3),
                    "decode_512_seqs_ms": round(wall(lambda: host.prepare_decode(dc_h, bs, dev),
                                                     reps) * 1e3, 3),
                    "unit": "ms/call", "cores": 1, "kind": "port",
                    "sample": "the same two steps through the reference's per-token host loops "
                              "(one Python thread), upload and device synchronisation included, "
                              f"median of {reps} calls"}
        cpu_jobs.append(("step_metadata", metadata_cpu))
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


def copy_ceiling(torch, dev, nbytes, args):
    """GB/s of torch's device-to-device copy of nbytes (read nbytes + write
    nbytes) under the same >= 1 GiB rotation as the legs: the read + write rate
    this box reaches for a transfer of that size."""
    n = rotation(2 * nbytes)
    src = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(n)]
    dst = [torch.empty_like(x) for x in src]
    fns = [(lambda a=a, b=b: b.copy_(a)) for a, b in zip(src, dst)]
    _, ev = time_graph(torch, fns, 20, 3, args.eager)
    del src, dst, fns
    return round(2 * nbytes / ev / 1e9, 1)


PROBE_LIB = os.path.join(ROOT, "learn-nano-vllm_amd", "bench_probe", "libnvk_probe.so")


def stream_probe_rate(torch, dev, args, mode, nbytes, moved):
    """GB/s (of `moved` bytes per launch) of one hand-written streaming kernel
    (learn-nano-vllm_amd/bench_probe/stream_probe.hip: 16 B per lane,
    non-temporal): mode 0 reads `nbytes`, 1 writes them, 2 copies them; timed
    like the legs, over buffers rotated past the >= 1 GiB of the caches."""
    import ctypes
    lib = ctypes.CDLL(PROBE_LIB)
    lib.nvk_probe_stream.restype = ctypes.c_int
    lib.nvk_probe_stream.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]

    def call(a, b):
        rc = lib.nvk_probe_stream(mode, a.data_ptr() if a is not None else None, b.data_ptr(),
                                  nbytes, torch.cuda.current_stream(dev).cuda_stream)
        if rc != 0:
            raise RuntimeError(f"stream probe mode {mode}: error {rc}")

    n = rotation(moved)
    src = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(n)] \
        if mode != 1 else [None] * n
    dst = [torch.empty(nbytes if mode else 4096, dtype=torch.uint8, device=dev)
           for _ in range(n)]
    fns = [(lambda a=a, b=b: call(a, b)) for a, b in zip(src, dst)]
    _, ev = time_graph(torch, fns, 20, 3, args.eager)
    del src, dst, fns
    return round(moved / ev / 1e9, 1)


def copy_probe_rate(torch, dev, args, moved):
    """The copy probe over `moved` bytes of read + write (half each)."""
    half = (moved // 2 + 15) // 16 * 16
    return stream_probe_rate(torch, dev, args, 2, half, 2 * half)


def stream_ceilings(torch, dev, args, store_bytes=None):
    """GB/s that plain streaming kernels reach on this box: read-only,
    write-only and copy over 512 MiB buffers, and a copy of the store's own
    byte count (the prologue leg adds one of its own byte count).  These are the rates a read + write kernel (the store, the
    prologue) and a read kernel (the decode) can be held against, besides the
    8 TB/s peak."""
    big = 512 << 20
    out = {"read_512mib_gbs": stream_probe_rate(torch, dev, args, 0, big, big),
           "write_512mib_gbs": stream_probe_rate(torch, dev, args, 1, big, big),
           "copy_512mib_gbs": stream_probe_rate(torch, dev, args, 2, big, 2 * big)}
    if store_bytes:
        out["copy_store_bytes_gbs"] = copy_probe_rate(torch, dev, args, store_bytes)
    out["what"] = ("hand-written streaming kernels (16-byte non-temporal accesses, 4 per lane "
                   "in flight): GB/s of bytes read, written, or read + written (copy)")
    return out


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV-cache path runs on a single MI355X "
              "(no sharding is built); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.collect_traffic:
        collect_traffic(*args.collect_traffic)
        return

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
    from nanovllm_amd.workloads import (attention_bytes, decode_case, kv_store_case,
                                        prefill_case, prefill_flops,
                                        spec_verify_case)

    legs = set(args.legs.split(","))
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    result = {}
    # CPU baselines: (result key, fn -> cpu_baseline dict), run after every GPU leg
    cpu_jobs = []

    def cpu_sample(n_reps, what, threads):
        return (f"{what}, median of {n_reps} reps on {threads} host threads "
                f"(os.cpu_count() = {os.cpu_count()})")

    # ------------------------------------------------------------------ decode
    log("building decode workload (B=64, ctx U{100..2048}, 1024-page pool)")
    dc = decode_case()
    dec_bytes = attention_bytes(dc.lens, 8, 128, 64, 16)
    pools = [dc.to(dev) for _ in range(rotation(dec_bytes))]   # separate copies of the pool
    outs = [torch.empty(64, 16, 128, dtype=torch.bfloat16, device=dev) for _ in pools]
    dec_fns = [
        (lambda c=c, o=o: paged_decode(c.q, c.k_cache, c.v_cache, c.context_lens,
                                       c.block_tables, dc.scale, out=o))
        for c, o in zip(pools, outs)]
    log("timing decode")
    wall, ev = time_graph(torch, dec_fns, args.steps, args.warmup, args.eager)
    result["decode"] = dict(ms_per_step=wall * 1e3, gbs=dec_bytes / wall / 1e9,
                            event_gbs=dec_bytes / ev / 1e9, bytes_per_step=dec_bytes)
    del pools, outs, dec_fns
    if not args.no_cpu_baseline:
        def decode_cpu():
            from oracle import torch_cpu as tcpu
            threads = host_threads(torch)
            log(f"cpu baseline: decode on the PyTorch CPU path, {threads} threads")
            t = cpu_time(lambda: tcpu.paged_attention_cpu(dc.q, dc.k_cache, dc.v_cache, range(65),
                                                          dc.context_lens, dc.scale,
                                                          dc.block_tables), 10)
            return {"value": round(dec_bytes / t / 1e9, 4), "unit": "GB/s", "cores": threads,
                    "kind": "port",
                    "sample": cpu_sample(10, "the full 64-sequence decode batch through the "
                                             "PyTorch CPU path (block-table gather + f32 "
                                             "scaled_dot_product_attention)", threads)}
        cpu_jobs.append(("decode", decode_cpu))

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
        del copies, st_fns
        log("timing device copies of the same bytes and of 512 MiB")
        same = copy_ceiling(torch, dev, st_bytes // 2, args)
        big = copy_ceiling(torch, dev, 512 << 20, args)
        log("timing streaming probes (read, write, copy)")
        streams = stream_ceilings(torch, dev, args, st_bytes)
        result["stream_ceiling"] = streams
        ach = st_bytes / ev_s / 1e9
        result["kv_store"] = dict(
            ms_per_step=wall_s * 1e3, bytes_per_step=st_bytes,
            roofline={"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                      "traffic": traffic_for("kv_store")},
            copy_ceiling={"same_bytes_copy_gbs": same, "copy_512mib_gbs": big,
                          "frac_of_same_bytes_copy": round(ach / same, 4),
                          "frac_of_512mib_copy": round(ach / big, 4),
                          "frac_of_copy_probe_512mib": round(ach / streams["copy_512mib_gbs"], 4),
                          "frac_of_copy_probe_same_bytes":
                              round(ach / streams["copy_store_bytes_gbs"], 4),
                          "what": "torch device-to-device copy reading and writing the store's "
                                  "bytes (and 512 MiB), same rotation, GB/s of read + write; "
                                  "the probes' figures are in stream_ceiling"})
        if not args.no_cpu_baseline:
            def store_cpu():
                from oracle import torch_cpu as tcpu
                threads = host_threads(torch)
                log(f"cpu baseline: kv-store on the PyTorch CPU path, {threads} threads")
                kc, vc = sc.k_cache.clone(), sc.v_cache.clone()
                t = cpu_time(lambda: tcpu.store_kvcache_cpu(sc.key, sc.value, kc, vc,
                                                            sc.slot_mapping), 50)
                return {"value": round(st_bytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
                        "kind": "port",
                        "sample": cpu_sample(50, "full 4096-token store through the PyTorch CPU "
                                                 "path (index_put on the flat cache views)",
                                             threads)}
            cpu_jobs.append(("kv_store", store_cpu))

    # ------------------------------------------------------------------ prologue
    if "prologue" in legs:
        result["prologue"] = prologue_leg(torch, dev, args, cpu_jobs)
        if "stream_ceiling" in result:   # a read + write stream, like a copy
            r = result["prologue"]["roofline"]
            r["frac_of_copy_probe"] = round(
                r["achieved"] / result["stream_ceiling"]["copy_512mib_gbs"], 4)
            log("timing the copy probe over the prologue's bytes")
            same = copy_probe_rate(torch, dev, args, result["prologue"]["bytes_per_step"])
            result["stream_ceiling"]["copy_prologue_bytes_gbs"] = same
            r["frac_of_copy_probe_same_bytes"] = round(r["achieved"] / same, 4)

    # ------------------------------------------------------------------ prefill
    if "prefill" in legs:
        log("building prefill workload (32 seqs, 512-token shared prefix)")
        pc = prefill_case()
        touched = attention_bytes(pc.lens_k, 8, 128, sum(pc.lens_q), 16)
        copies = [pc.to(dev) for _ in range(rotation(touched))]
        for c in copies:   # the new tokens' K/V are in the cache before attention
            store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
        outs = [torch.empty_like(c.q) for c in copies]
        # The tiles are ranked once per model step, as Attention.forward does
        # for every layer of a step (they share cu_seqlens), so a step of the
        # leg is the attention kernel alone; the same call ranking its own
        # tiles (one more small kernel) is timed beside it.
        from nanovllm_amd.flash_api import prefill_tile_order
        c0 = copies[0]
        order = prefill_tile_order(c0.cu_seqlens_q, c0.cu_seqlens_k, pc.max_seqlen_q, c0.k_cache,
                                   16, block_table=c0.block_tables)
        assert order is not None
        pf_fns = [(lambda c=c, o=o: varlen_prefill(c.q, c.k_cache, c.v_cache, c.cu_seqlens_q,
                                                   c.cu_seqlens_k, pc.max_seqlen_q, pc.scale,
                                                   block_table=c.block_tables, out=o,
                                                   order=order))
                  for c, o in zip(copies, outs)]
        ranked_fns = [(lambda c=c, o=o: varlen_prefill(c.q, c.k_cache, c.v_cache, c.cu_seqlens_q,
                                                       c.cu_seqlens_k, pc.max_seqlen_q, pc.scale,
                                                       block_table=c.block_tables, out=o))
                      for c, o in zip(copies, outs)]
        flops = prefill_flops(pc.lens_q, pc.lens_k, 16, 128)
        log("timing prefill")
        wall_p, ev_p = time_graph(torch, pf_fns, args.steps, args.warmup, args.eager)
        wall_r, ev_r = time_graph(torch, ranked_fns, args.steps, args.warmup, args.eager)
        tf = flops / ev_p / 1e12
        result["prefill"] = dict(
            ms_per_step=wall_p * 1e3, flops_per_step=flops,
            step="one layer's varlen_prefill with the step's tile order (ranked once per step)",
            ranked_per_call={"ms_per_step": round(wall_r * 1e3, 5),
                             "tflops": round(flops / ev_r / 1e12, 2),
                             "what": "the same call ranking its own tiles first"},
            roofline={"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                      "traffic": traffic_for("prefill")})
        del copies, outs, pf_fns, ranked_fns, order
        if not args.no_cpu_baseline:
            def prefill_cpu():
                from oracle import torch_cpu as tcpu
                threads = host_threads(torch)
                log(f"cpu baseline: prefill on the PyTorch CPU path, {threads} threads")
                kc, vc = pc.k_cache.clone(), pc.v_cache.clone()
                tcpu.store_kvcache_cpu(pc.key, pc.value, kc, vc, pc.slot_mapping)
                t = cpu_time(lambda: tcpu.paged_attention_cpu(pc.q, kc, vc, pc.cu_seqlens_q,
                                                              pc.lens_k, pc.scale,
                                                              pc.block_tables), 5)
                return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s",
                        "cores": threads, "kind": "port",
                        "sample": cpu_sample(5, "the full 32-sequence prefill through the "
                                                "PyTorch CPU path (block-table gather + f32 "
                                                "scaled_dot_product_attention with the "
                                                "bottom-right causal mask)", threads)}
            cpu_jobs.append(("prefill", prefill_cpu))

    # ------------------------------------------------------------------ spec verify
    if "spec" in legs:
        log("building spec-verify workload (32 seqs, 6 queries, ctx U{1024..8192})")
        vc_ = spec_verify_case()
        sv_bytes = attention_bytes(vc_.lens_k, 8, 128, 32 * 6, 16)
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
        if not args.no_cpu_baseline:
            def spec_cpu():
                from oracle import torch_cpu as tcpu
                threads = host_threads(torch)
                log(f"cpu baseline: spec verify on the PyTorch CPU path, {threads} threads")
                kc, vc = vc_.k_cache.clone(), vc_.v_cache.clone()
                tcpu.store_kvcache_cpu(vc_.key, vc_.value, kc, vc, vc_.slot_mapping)
                t = cpu_time(lambda: tcpu.paged_attention_cpu(vc_.q, kc, vc, vc_.cu_seqlens_q,
                                                              vc_.lens_k, vc_.scale,
                                                              vc_.block_tables), 5)
                return {"value": round(sv_bytes / t / 1e9, 4), "unit": "GB/s", "cores": threads,
                        "kind": "port",
                        "sample": cpu_sample(5, "the full 32 x 6-query verification through "
                                                "the PyTorch CPU path (block-table gather + f32 "
                                                "scaled_dot_product_attention with the "
                                                "bottom-right causal mask)", threads)}
            cpu_jobs.append(("spec_verify", spec_cpu))

    # ------------------------------------------------------------------ decode graphs
    if "graph" in legs:
        result["decode_graph"] = decode_graph_leg(torch, dev, args)

    # ------------------------------------------------------------------ step metadata
    if "metadata" in legs:
        result["step_metadata"] = metadata_leg(torch, dev, args, cpu_jobs)

    # ------------------------------------------------------------------ sampler
    if "sampler" in legs:
        result["sampler"] = sampler_leg(torch, dev, args)

    # ------------------------------------------------------------------ mixed step
    if "mixed" in legs:
        result["mixed_step"] = mixed_leg(torch, dev, args, cpu_jobs)

    # ------------------------------------------------------------------ CPU baselines
    torch.cuda.synchronize()
    cpu = None
    for key, fn in cpu_jobs:
        base = fn()
        if key == "decode":
            cpu = base
        else:
            result[key]["cpu_baseline"] = base

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
    if "stream_ceiling" in result:   # the decode is a read stream
        line["roofline"]["frac_of_read_probe"] = round(
            d["event_gbs"] / result["stream_ceiling"]["read_512mib_gbs"], 4)
    for k in ("kv_store", "prologue", "prefill", "spec_verify", "decode_graph", "step_metadata",
              "sampler", "mixed_step", "stream_ceiling"):
        if k in result:
            line[k] = result[k]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
