"""Benchmark: 64-request ragged talker decode step on one MI355X.

Workload (the talker decode-attention step): 64 concurrent requests with context lengths
c_b = torch.randint(64, 1025, (64,)) under seed 0 (sum 32,718), a packed bf16 KV arena
(2*28 planes, 64 slots, 8 KV heads, capacity 1024, head_dim 128), 16 query heads, RoPE
theta 1e6.  One step = the ranking of the 64 requests by length (one small launch, read by
every layer) and 28 layers; each layer is one fused HIP launch doing RoPE of q and of the new
key, the paired K/V write at position c_b and ragged GQA decode attention over c_b + 1 keys.
The 29 launches of a step are captured once into a HIP graph and replayed.
Inputs are synthetic (seeded random, resident in HBM before timing).

Prints one JSON line: tokens/s (64 tokens per step), the dominant kernel's roofline
(algorithmic bytes per launch / average launch time against 8 TB/s) and the CPU baseline
(the reference's torch decode layer on this host's cores, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

LAYERS, BATCH, HQ, HKV, D, CAPACITY = 28, 64, 16, 8, 128, 1024
PEAK_HBM_GBS = 8000.0
TRAFFIC_SUMMARY = ROOT / "profiles" / "decode_step_talker64_hbm_traffic.md"


def algorithmic_bytes(contexts: torch.Tensor) -> int:
    """Bytes one fused layer launch must move: arena K/V rows 0..c_b-1 read, the new K/V rows
    read from the QKV projection and written to the arena, Q read, O written, cos/sin rows
    read, positions read."""
    row = HKV * D * 2                       # one token of one plane, bf16
    arena_read = int(contexts.sum()) * row * 2
    new_kv = BATCH * row * 2 * 2            # read + write, K and V
    q_o = BATCH * HQ * D * 2 * 2
    cos_sin = BATCH * D * 2 * 2
    return arena_read + new_kv + q_o + cos_sin + BATCH * 8


def attention_bytes(contexts: torch.Tensor) -> int:
    """Bytes of the non-fused attention launch: arena K/V rows 0..c_b read, Q read, O written."""
    return (int(contexts.sum()) + BATCH) * HKV * D * 2 * 2 + BATCH * HQ * D * 2 * 2 + BATCH * 8


def calibration_copy(pkg, device, nbytes, stream):
    """The plain copy kernel over ``nbytes`` (three launches), so that rocprofv3's
    FETCH_SIZE / WRITE_SIZE of a run can be scaled by what they read for a copy of known size."""
    if nbytes <= 0:
        return
    n = nbytes // 16 * 16
    src = torch.empty(n, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        status = pkg.library().q3t_copy_bytes(dst.data_ptr(), src.data_ptr(), n, stream.cuda_stream)
        if status != 0:
            raise RuntimeError("calibration copy failed")
    torch.cuda.synchronize()


def prefill_detail(pkg, device, reps=20):
    """The prefill workload: 16 prompts, lengths randint(32, 513, (16,)) under seed 0
    (sum 4790), 28 layers of RoPE + arena write + varlen causal GQA in one graph.
    Returns per-layer times and the MFMA rate of the attention kernel."""
    gen = torch.Generator().manual_seed(0)
    lengths = torch.randint(32, 513, (16,), generator=gen)
    total, longest = int(lengths.sum()), int(lengths.max())
    cu = torch.zeros(17, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    positions = torch.cat([torch.arange(int(n)) for n in lengths]).to(device)
    dgen = torch.Generator(device=device).manual_seed(2)
    qkv = torch.randn(LAYERS, total, HQ + 2 * HKV, D, generator=dgen, device=device, dtype=torch.bfloat16)
    arena = torch.zeros(2 * LAYERS, 16, HKV, 512, D, device=device, dtype=torch.bfloat16)
    cos, sin = pkg.rope_tables(positions, D)
    dcu = cu.to(device)
    out = torch.empty(LAYERS, total, HQ, D, device=device, dtype=torch.bfloat16)

    def step(attention_only):
        # prefill_step's kernels: the key prologue, then attention rotating the raw queries,
        # reading the values from the projection rows and copying them into the arena
        for layer in range(LAYERS):
            row = qkv[layer]
            q, k, v = row[:, :HQ], row[:, HQ:HQ + HKV], row[:, HQ + HKV:]
            if not attention_only:
                pkg.prefill_rope_write(q, k, None, cos, sin, dcu, arena[layer], arena[LAYERS + layer],
                                       rotate_query=False)
            pkg.prefill_attention(q, arena[layer], arena[LAYERS + layer], dcu, longest,
                                  out=out[layer], cos=cos, sin=sin, new_values=v)

    times = {}
    for attention_only in (False, True):
        step(attention_only)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(attention_only)
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        times[attention_only] = start.elapsed_time(stop) * 1e3 / (reps * LAYERS)
    flops = 2 * D * HQ * int((lengths * (lengths + 1)).sum())
    # the step's query, key, value and output rows (T x (Hq + 2 Hkv + Hq) x D bf16)
    row_bytes = total * (2 * HQ + 2 * HKV) * D * 2
    return {"workload": "16 prompts, lengths randint(32,513) seed 0, sum %d, 28 layers" % total,
            "lengths": lengths.tolist(),
            "us_per_layer_rope_write_attention": times[False],
            "us_per_layer_attention": times[True],
            "attention_flops_per_layer": flops,
            "attention_TFLOPs": flops / (times[True] * 1e-6) / 1e12,
            "mfma_frac_of_2500_TFLOPs": flops / (times[True] * 1e-6) / 2.5e15,
            "qkvo_bytes_per_layer": row_bytes,
            "step_GBs": row_bytes / (times[False] * 1e-6) / 1e9}


def predictor_detail(pkg, device, reps=20):
    """The code predictor's attention: 64 requests, 5 layers, 15 steps over a 16-position
    cache (PredictorCache windows: step 0 writes positions 0-1 and attends them causally,
    step s writes s+1 and attends 0..s+1).  Every layer-step is one fused launch (two tokens
    at step 0, one after); all 75 in one graph."""
    layers, steps, batch, cap = 5, 15, BATCH, 16
    dgen = torch.Generator(device=device).manual_seed(3)
    arena = torch.zeros(2 * layers, batch, HKV, cap, D, device=device, dtype=torch.bfloat16)
    rows = torch.randn(steps, layers, batch, 2, HQ + 2 * HKV, D, generator=dgen, device=device,
                       dtype=torch.bfloat16)
    positions = [torch.full((batch,), max(s + 1, 1), device=device, dtype=torch.int64) for s in range(steps)]
    tables = [pkg.rope_tables(positions[s], D) for s in range(steps)]
    cos0, sin0 = pkg.rope_tables(torch.arange(2, device=device).expand(batch, 2).contiguous(), D)
    out = torch.empty(batch, 2, HQ, D, device=device, dtype=torch.bfloat16)

    def chain():
        for s in range(steps):
            for layer in range(layers):
                r = rows[s, layer]
                keys, values = arena[layer], arena[layers + layer]
                if s == 0:
                    pkg.decode_step(r[:, :, :HQ], r[:, :, HQ:HQ + HKV], r[:, :, HQ + HKV:], keys, values,
                                    positions[0], cos0, sin0, out=out)
                else:
                    q, k, v = r[:, :1, :HQ], r[:, :1, HQ:HQ + HKV], r[:, :1, HQ + HKV:]
                    pkg.decode_step(q, k, v, keys, values, positions[s], *tables[s], out=out[:, :1])

    chain()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    chain_us = start.elapsed_time(stop) * 1e3 / reps
    return {"workload": "code predictor: 64 requests, 5 layers, 15 steps, 16-position cache",
            "us_per_15_step_chain": chain_us, "us_per_step": chain_us / steps,
            "us_per_layer_step": chain_us / (steps * layers)}


def _replay_us(fn, calls=1, reps=100):
    """Mean time per call of a graph holding ``calls`` calls of ``fn``, over ``reps`` replays
    after warm-up, launch included.  With one call this is the method of the reference's
    operator probes (tools/probe_attention_context.py:48-65, tools/probe_rotary_exact.py:69-74);
    more calls per graph spread the graph launch over them."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    for _ in range(10):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return round(start.elapsed_time(stop) * 1e3 / (reps * calls), 2)


def reference_probe_detail(pkg, device):
    """The reference's own operator probes at their B=64 shapes (its Ascend 910B1 figures in
    ``reference_910b1_us``), same inputs, timed as one call per graph (the reference's method)
    and as 20 calls per graph:

    * decode GQA, 16/8 heads, D 128, a 512-row arena, positions (7 b) mod L
      (tools/probe_attention_context.py:20-36): with the boolean mask over all 512 keys
      (``full_arena``), with the mask and L valid keys (``valid_length``), and through
      positions alone (``positions``, the form the slot cache uses); all three give the
      same output;
    * the paired K/V write from strided projection views, capacity 512
      (tools/probe_paired_kv.py:24-38);
    * exact bf16 RoPE of q and k, BSND, cos/sin from random phases
      (tools/probe_rotary_exact.py:23-37);
    * predictor-shape attention, D 64 in a 16-row cache with L valid keys, the 2x2 causal
      step at L = 2 (tools/probe_predictor_padded_kv.py:20-35).

    ``graph_replay_floor_us`` is one replay of a graph holding a single one-element add."""
    gen = torch.Generator(device=device).manual_seed(42)
    probes = {}
    diffs = {}
    for batch, lengths in ((64, (64, 128, 256, 512)), (32, (512,)), (8, (512,)), (1, (512,))):
        q = torch.randn(batch, 1, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
        keys = torch.randn(batch, HKV, 512, D, generator=gen, device=device, dtype=torch.bfloat16)
        values = torch.randn_like(keys)
        for length in lengths:
            positions = (torch.arange(batch, device=device) * 7) % length
            keep = (torch.arange(512, device=device)[None, :] <= positions[:, None])[:, None, None, :]
            full = torch.full((batch,), 511, device=device, dtype=torch.int64)
            valid = torch.full((batch,), length - 1, device=device, dtype=torch.int64)
            calls = {"full_arena": (pkg.decode_attention, (q, keys, values, full), {"mask": keep}),
                     "valid_length": (pkg.decode_attention, (q, keys, values, valid), {"mask": keep}),
                     "positions": (pkg.decode_attention, (q, keys, values, positions), {})}
            outs = [fn(*a, **kw).float() for fn, a, kw in calls.values()]
            diffs[f"decode_gqa_b{batch}_L{length}"] = max(float((o - outs[0]).abs().max()) for o in outs[1:])
            for name, call in calls.items():
                probes[f"decode_gqa_b{batch}_L{length}_{name}"] = call
    batch, capacity = 64, 512
    packed = torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=gen, device=device, dtype=torch.bfloat16)
    k = packed[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D).transpose(1, 2)
    v = packed[..., (HQ + HKV) * D:].view(batch, 1, HKV, D).transpose(1, 2)
    cache = [torch.randn(batch, HKV, capacity, D, generator=gen, device=device, dtype=torch.bfloat16)
             for _ in range(2)]
    positions = torch.arange(batch, device=device) % capacity
    probes["paired_kv_write_b64_cap512"] = (pkg.write, (k, v, *cache, positions), {"row_tiled": True})
    for length in (1, 64):
        query = torch.randn(batch, length, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
        key = torch.randn(batch, length, HKV, D, generator=gen, device=device, dtype=torch.bfloat16)
        phase = torch.randn(batch, length, D // 2, generator=gen, device=device).repeat(1, 1, 2)
        cos, sin = phase.cos().bfloat16(), phase.sin().bfloat16()
        probes[f"rope_qk_b64_s{length}"] = (
            lambda qq, kk, c, s: (pkg.rotary(qq, c, s), pkg.rotary(kk, c, s)), (query, key, cos, sin), {})
    for length in (2, 3, 8, 16):
        qlen = 2 if length == 2 else 1
        q = torch.randn(batch, qlen, HQ, 64, generator=gen, device=device, dtype=torch.bfloat16)
        keys = torch.randn(batch, HKV, 16, 64, generator=gen, device=device, dtype=torch.bfloat16)
        values = torch.randn_like(keys)
        valid = torch.full((batch,), length - 1, device=device, dtype=torch.int64)
        probes[f"predictor_attention_b64_L{length}"] = (pkg.decode_attention, (q, keys, values, valid), {})
    out = {}
    for calls in (1, 20):
        out[f"{calls}_call_per_graph_us" if calls == 1 else f"{calls}_calls_per_graph_us"] = {
            name: _replay_us(lambda: fn(*a, **kw), calls=calls) for name, (fn, a, kw) in probes.items()}
    one = torch.zeros(1, device=device)
    out["graph_replay_floor_us"] = _replay_us(lambda: one.add_(1))
    out["decode_gqa_max_abs_diff_between_forms"] = diffs
    out["reference_910b1_us"] = {
        "decode_gqa_b64_L512": {"full_arena": 99.13, "valid_length": 99.16},
        "decode_gqa_b64_L64/128/256_valid_length": [86.70, 86.50, 90.31],
        "decode_gqa_b32/b8/b1_L512_full_arena": [64.98, 43.73, 22.91],
        "paired_kv_write_b64_cap512": 11.54, "rope_qk_b64_s1": 23.61, "rope_qk_b64_s64": 90.57,
        "predictor_attention_b64_L2/3/8/16": [77.19, 77.28, 76.84, 79.23]}
    return out


def read_traffic():
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (committed summary)."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    text = TRAFFIC_SUMMARY.read_text()
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def cpu_baseline(seconds: float, threads: int = 0, dtype=torch.bfloat16):
    """The reference's torch decode layer (scatter_ write, eager RoPE, SDPA under the
    0/finfo.min context mask) on this host, one layer of the same 64-request workload, in
    bf16 (the GPU path's arithmetic type) or fp32."""
    from oracle import torch_path

    previous = torch.get_num_threads()
    if threads:
        torch.set_num_threads(threads)
    threads = torch.get_num_threads()
    gen = torch.Generator().manual_seed(0)
    contexts = torch.randint(64, 1025, (BATCH,), generator=gen)
    arena_k = torch.randn(BATCH, HKV, CAPACITY, D, generator=gen).to(dtype)
    arena_v = torch.randn(BATCH, HKV, CAPACITY, D, generator=gen).to(dtype)
    qkv = torch.randn(BATCH, 1, (HQ + 2 * HKV) * D, generator=gen).to(dtype)
    q = qkv[..., :HQ * D].view(BATCH, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(BATCH, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(BATCH, 1, HKV, D)
    angle = (contexts.float()[:, None] * (1.0 / (1e6 ** (torch.arange(0, D, 2).float() / D)))[None])
    emb = torch.cat([angle, angle], -1)
    cos, sin = emb.cos().to(dtype)[:, None], emb.sin().to(dtype)[:, None]
    times = []
    deadline = time.perf_counter() + seconds
    with torch.inference_mode():
        torch_path.decode_layer(q, k, v, cos, sin, arena_k, arena_v, contexts)  # warm-up
        while time.perf_counter() < deadline or len(times) < 3:
            t0 = time.perf_counter()
            torch_path.decode_layer(q, k, v, cos, sin, arena_k, arena_v, contexts)
            times.append(time.perf_counter() - t0)
            if len(times) >= 200:
                break
    times.sort()
    layer_s = times[len(times) // 2]
    torch.set_num_threads(previous)
    return {"value": BATCH / (LAYERS * layer_s), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": (f"median of {len(times)} runs of one talker layer (64 requests, capacity "
                       f"{CAPACITY}, {str(dtype).split('.')[-1]}, torch {threads} threads, {len(os.sched_getaffinity(0))} "
                       f"cores in the affinity mask) = {layer_s * 1e3:.2f} ms, scaled to a 28-layer step")}


def arena_move_detail(pkg, arena, contexts, reps=20):
    """One compaction move on the talker arena (all 56 planes, capacity 1024): the whole slot
    row, as the reference copies it, against the moved request's prefix [:position + 1]
    (SlotArena.move(length=...)).  Moves the last slot into slot 0 (after all timing)."""
    last = arena.shape[1] - 1
    length = int(contexts[last]) + 1
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {}
    for name, n in (("full_row", arena.shape[3]), ("prefix", length)):
        dst, src = arena[:, 0, :, :n], arena[:, last, :, :n]
        pkg.copy_rows(dst, src)
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            pkg.copy_rows(dst, src)
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) * 1e3 / reps
        nbytes = 2 * dst.numel() * dst.element_size()  # read + write
        out[name] = {"rows": n, "us": us, "bytes": nbytes, "GBs": nbytes / (us * 1e-6) / 1e9}
    return out


def trace_detail(pkg, device, iterations=200, slots=128):
    """The mixed continuous-batching trace at talker shape: 128 slots, 200 iterations of
    seeded Poisson arrivals (mean 2 per iteration), prompts U{32..512}, frame limits
    U{200..2000}, a cancellation of the oldest request with probability 0.2 per iteration,
    decode bucket step 16 with bucket_kv (continuous.py:425-473, 541-657), over a 28-layer
    packed arena (capacity 512, growing).  Per iteration: the admissions' prefix loads, the
    compaction moves and any regrowth (the arena operations), then the 28 fused decode
    launches at the scheduled positions (zero-position rows of the graph batch included).
    Reports the decode launches' total time and algorithmic GB/s over the trace, and the
    arena operations' time.  The scheduler's integer state runs on the host between them."""
    import numpy as np

    class _Config:
        num_key_value_heads, head_dim, num_hidden_layers = HKV, D, LAYERS

    class _Talker(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = _Config()
            self.layers = torch.nn.ModuleList([torch.nn.Identity() for _ in range(LAYERS)])
            self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16, device=device))

    rng = np.random.default_rng(0)
    arrivals, cancels, ident = [], [], 0
    for _ in range(iterations):
        batch = []
        for _ in range(int(rng.poisson(2.0))):
            batch.append((ident, int(rng.integers(32, 513)), int(rng.integers(200, 2001))))
            ident += 1
        arrivals.append(batch)
        cancels.append(float(rng.random()))
    arena = pkg.SlotArena(_Talker(), slots, 512, packed_kv=True)
    sched = pkg.SlotScheduler(slots, 512, 16, True, arena=arena)
    dgen = torch.Generator(device=device).manual_seed(3)
    qkv = torch.randn(LAYERS, slots, 1, (HQ + 2 * HKV) * D, generator=dgen, device=device, dtype=torch.bfloat16)
    prefill = torch.randn(2 * LAYERS, 16, HKV, 512, D, generator=dgen, device=device, dtype=torch.bfloat16)
    out = torch.empty(slots, 1, HQ, D, device=device, dtype=torch.bfloat16)
    decode_events, arena_events, decode_bytes, launches = [], [], 0, 0
    queue, active = [], []
    for it in range(iterations):
        queue.extend(arrivals[it])
        cancelled = [active[0]] if active and cancels[it] < 0.2 else []
        free = slots - (len(active) - len(cancelled))
        subs, queue = queue[:min(free, prefill.shape[1])], queue[min(free, prefill.shape[1]):]
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()
        sched.ops = []
        sched.cancel(cancelled)
        sched.admit(subs, prefill)
        record = sched.decode_batch()
        ev[1].record()
        done = []
        if record is not None:
            positions = record.positions_tensor(device)
            cos, sin = pkg.rope_tables(positions, D)
            b = record.batch
            ev[2].record()
            for layer in range(LAYERS):
                row = qkv[layer, :b]
                pkg.decode_step(row[..., :HQ * D].view(b, 1, HQ, D),
                                row[..., HQ * D:(HQ + HKV) * D].view(b, 1, HKV, D),
                                row[..., (HQ + HKV) * D:].view(b, 1, HKV, D),
                                sched.arena.keys[layer], sched.arena.values[layer], positions, cos, sin,
                                out=out[:b])
            ev[3].record()
            decode_events.append((ev[2], ev[3]))
            row_bytes = HKV * D * 2
            decode_bytes += LAYERS * (sum(record.positions) * row_bytes * 2 + b * row_bytes * 4
                                      + b * HQ * D * 4 + b * D * 4 + b * 8)
            launches += LAYERS
            done = sched.advance()
        arena_events.append((ev[0], ev[1]))
        active = [i for i in active if i not in cancelled and i not in done]
        active.extend(i for i, _, _ in subs if i not in done)
    torch.cuda.synchronize()
    decode_us = sum(a.elapsed_time(b) for a, b in decode_events) * 1e3
    arena_us = sum(a.elapsed_time(b) for a, b in arena_events) * 1e3
    return {"workload": "128-slot, 200-iteration mixed trace, 28-layer talker arena (8 KV heads, "
                        "head_dim 128, bf16), eager launches",
            "final_capacity": sched.capacity, "decode_launches": launches,
            "decode_us_total": decode_us, "decode_algorithmic_bytes": decode_bytes,
            "decode_GBs": decode_bytes / (decode_us * 1e-6) / 1e9,
            "arena_ops_us_total": arena_us}


KERNELS = {"bundled": "decode_bundled_kernel<G2,fused,streamed,no norm>",
           "balanced": "decode_balanced_kernel<bf16,128,G2,SQ1,fused,streamed>",
           "chunked": "decode_chunks_kernel<bf16,128,G2,SQ1,fused,streamed>"}


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--max-chunks", type=int, default=0,
                        help="chunked grid: 64-key chunks per request and KV head (0 = default)")
    parser.add_argument("--splits", type=int, default=0,
                        help="balanced grid: workgroups per KV head (0: the default); under the "
                             "automatic grid, > 0 selects balanced and < 0 chunked")
    parser.add_argument("--grid", choices=["bundled", "balanced", "chunked"], default=None,
                        help="decode grid by name (default: the library's choice, bundled for "
                             "this workload)")
    parser.add_argument("--no-plan", action="store_true",
                        help="every layer launch ranks the requests itself instead of reading the "
                             "step's decode plan")
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--calibrate-bytes", type=int, default=0,
                        help="after timing, launch the plain copy kernel on this many bytes "
                             "(HBM counter calibration under rocprofv3)")
    parser.add_argument("--decode-only", action="store_true",
                        help="skip the prefill, predictor, arena-move and talker-step details "
                             "(per-kernel profiling of the headline launches alone)")
    parser.add_argument("--prefill-only", action="store_true",
                        help="run only the prefill workload and print its detail line "
                             "(for per-kernel profiling of the prefill kernels)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the package has no multi-GPU path "
              "(decode would shard by request slot, one arena per GPU)", file=sys.stderr)
        sys.exit(2)

    pkg = __graft_entry__.import_package()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_detail(pkg, device)}), flush=True)
        calibration_copy(pkg, device, args.calibrate_bytes, torch.cuda.current_stream(device))
        return
    gen = torch.Generator().manual_seed(0)
    contexts = torch.randint(64, 1025, (BATCH,), generator=gen)
    positions = contexts.to(device)
    dgen = torch.Generator(device=device).manual_seed(1)
    arena = torch.randn(2 * LAYERS, BATCH, HKV, CAPACITY, D, generator=dgen, device=device,
                        dtype=torch.bfloat16)
    qkv = torch.randn(LAYERS, BATCH, 1, (HQ + 2 * HKV) * D, generator=dgen, device=device,
                      dtype=torch.bfloat16)
    cos, sin = pkg.rope_tables(positions, D)
    out = torch.empty(LAYERS, BATCH, 1, HQ, D, device=device, dtype=torch.bfloat16)
    views = []
    for layer in range(LAYERS):
        row = qkv[layer]
        views.append((row[..., :HQ * D].view(BATCH, 1, HQ, D),
                      row[..., HQ * D:(HQ + HKV) * D].view(BATCH, 1, HKV, D),
                      row[..., (HQ + HKV) * D:].view(BATCH, 1, HKV, D),
                      arena[layer], arena[LAYERS + layer], out[layer]))

    plan_buf = torch.empty(pkg.plan_shape(BATCH, HQ, HKV), device=device, dtype=torch.int32)

    def step():
        # one ranking per step (all layers attend the same lengths), inside the timed graph
        plan = None if args.no_plan else pkg.decode_plan(positions, CAPACITY, HQ, HKV, out=plan_buf)
        for q, k, v, ak, av, o in views:
            pkg.decode_step(q, k, v, ak, av, positions, cos, sin, out=o, max_chunks=args.max_chunks,
                            splits=args.splits, grid=args.grid, plan=plan)

    step()  # eager: sizes the workspace before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    launch_us = ms_per_step * 1e3 / LAYERS
    bytes_per_launch = algorithmic_bytes(contexts)
    achieved = bytes_per_launch / (launch_us * 1e-6) / 1e9

    # attention alone: the non-fused kernel over the already-written arena, same graph method
    q0 = views[0][0].contiguous()
    attn_graph = torch.cuda.CUDAGraph()
    pkg.decode_attention(q0, arena[0], arena[LAYERS], positions, max_chunks=args.max_chunks,
                         splits=args.splits, grid=args.grid)
    torch.cuda.synchronize()
    with torch.cuda.graph(attn_graph):
        plan = None if args.no_plan else pkg.decode_plan(positions, CAPACITY, HQ, HKV, out=plan_buf)
        for layer in range(LAYERS):
            pkg.decode_attention(q0, arena[layer], arena[LAYERS + layer], positions,
                                 out=out[layer], max_chunks=args.max_chunks, splits=args.splits,
                                 grid=args.grid, plan=plan)
    attn_graph.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps // 4)
    start.record(stream)
    for _ in range(reps):
        attn_graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    attn_us = start.elapsed_time(stop) * 1e3 / (reps * LAYERS)

    # the reference's own flow: SlotGraph.compute hands every layer the (B, 1, 1, ctx) additive
    # mask j <= pos[b] (continuous.py:188-197): a masked launch of the bundled grid
    allowed = torch.arange(CAPACITY, device=device)[None, :] <= positions[:, None]
    ref_mask = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).to(torch.bfloat16)[:, None, None, :]
    masked_graph = torch.cuda.CUDAGraph()

    def masked_step():
        plan = pkg.decode_plan(positions, CAPACITY, HQ, HKV, out=plan_buf)
        for q, k, v, ak, av, o in views:
            pkg.decode_step(q, k, v, ak, av, positions, cos, sin, out=o, mask=ref_mask, plan=plan)

    masked_step()
    torch.cuda.synchronize()
    with torch.cuda.graph(masked_graph):
        masked_step()
    masked_graph.replay()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        masked_graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    masked_us = start.elapsed_time(stop) * 1e3 / (reps * LAYERS)
    masked_grid = pkg.decode_grid_for(BATCH, 1, HQ, HKV, D, CAPACITY, masked=True)

    calibration_copy(pkg, device, args.calibrate_bytes, stream)

    extra = {}
    if not args.decode_only:
        extra = {"prefill": prefill_detail(pkg, device),
                 "predictor": predictor_detail(pkg, device),
                 "arena_move": arena_move_detail(pkg, arena, contexts),
                 "mixed_trace": trace_detail(pkg, device),
                 "reference_probe_shapes": reference_probe_detail(pkg, device)}
    traffic = read_traffic()
    grid_name = pkg.decode_grid_for(BATCH, 1, HQ, HKV, D, CAPACITY, splits=args.splits,
                                              grid=args.grid)
    result = {
        "metric": "decode-attn tokens/s + achieved HBM GB/s, 64-req ragged talker step, 1 GPU",
        "value": BATCH * args.steps / (gpu_ms / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V arena, QKV rows; seed-0 context lengths)",
        "config": {"workload": "talker ragged decode step: 64 requests, contexts U[64,1024] "
                               "(seed 0, sum 32718), 28 layers, 16q/8kv heads, head_dim 128, "
                               "arena capacity 1024, fused RoPE + KV write + GQA decode",
                   "global_batch": BATCH, "layers": LAYERS, "context_sum": int(contexts.sum()),
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS,
                     "traffic": traffic},
        "detail": {"kernel": KERNELS[grid_name],
                   "grid": grid_name,
                   "algorithmic_bytes_per_launch": bytes_per_launch,
                   "contexts": contexts.tolist(),
                   "us_per_layer_launch": launch_us,
                   "us_per_layer_attention_only": attn_us,
                   "attention_only_GBs": attention_bytes(contexts) / (attn_us * 1e-6) / 1e9,
                   "decode_plan": not args.no_plan,
                   "reference_masked_step": {
                       "workload": "the same step with SlotGraph.compute's (64, 1, 1, 1024) bf16 mask "
                                   "handed to every layer (the reference's flow), with the step's plan",
                       "grid": masked_grid,
                       "us_per_layer_launch": masked_us,
                       "tokens_per_s": BATCH / (masked_us * LAYERS * 1e-6)},
                   "max_chunks": args.max_chunks,
                   "splits": args.splits,
                   "wall_s_timed_region": wall,
                   **extra},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        # the reference pins torch to 4 threads (model.py:16); reported beside the all-core figure
        four = cpu_baseline(args.cpu_seconds / 2, threads=4)
        result["detail"]["cpu_baseline_4_threads"] = {"value": four["value"], "sample": four["sample"]}
        fp32 = cpu_baseline(args.cpu_seconds / 2, dtype=torch.float32)
        result["detail"]["cpu_baseline_fp32"] = {"value": fp32["value"], "sample": fp32["sample"]}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
