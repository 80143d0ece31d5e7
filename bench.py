#!/usr/bin/env python3
"""Benchmark of the MI355X paged KV-cache hot path.

Metric: decode-attention us/layer and KV HBM GB/s (% of peak) at
2K, 8x2K batch and 128K. One "step" = one decode step of the 28-layer stack at
the headline workload C4 (one session, 131072 cached tokens in 2048 pages of
64, chunk 256, two-level merge): per layer the fused append+attend decode
(phase0) over that layer's pool slice. `value` is the K+V bytes attended per
second over the whole timed region (inputs resident in HBM); the other
configurations are reported under "configs".

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c4,c3,c1,c2,c5,pf,alloc,model,mprefill,rows]
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
LAYERS = 28
P = 64
KV_BYTES_PER_TOKEN = 1024  # K+V, 2 kv heads x 128 dims x bf16, one layer
QO_BYTES = 16 * 128 * 2 * 2  # q read + out write per session


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="c4,c3,c1,c2,c5,pf,alloc,model,rows")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="no HIP graphs (eager launches)")
    ap.add_argument("--calib", action="store_true",
                    help="also run one 256 MiB device copy (PMC byte calibration)")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="attach the decode timeline hook (in-kernel clock stamps) and add "
                         "a per-layer timeline to each decode result")
    return ap.parse_args()


# Decode timeline buffer (--decode-timeline): TIMELINE_LAUNCHES regions, attached
# before any decode is captured.
TIMELINE = None
TIMELINE_LAUNCHES = 64


def timeline_of(kvm, torch, step):
    """Replays `step` once with the timeline buffer cleared and summarizes the
    decodes it ran (None without --decode-timeline)."""
    if TIMELINE is None:
        return None
    TIMELINE.zero_()
    torch.cuda.synchronize()
    step()
    torch.cuda.synchronize()
    return kvm.timeline_summary(TIMELINE.cpu().numpy())


class Timer:
    """HIP events on torch's current stream (the stream every launch uses).

    Each workload step is captured once into a HIP graph (torch.cuda.CUDAGraph)
    and replayed, so the timed region measures the GPU and not Python launch
    overhead; the kernels read positions from device memory, so replays are
    exact re-executions."""

    def __init__(self, torch, graphs=True):
        self.torch = torch
        self.graphs = graphs

    def capture(self, fns):
        """Returns a callable cycling through `fns` (one per rotation index),
        each captured into its own graph when graphs are enabled."""
        t = self.torch
        if not self.graphs:
            state = {"i": 0}

            def eager():
                fns[state["i"] % len(fns)]()
                state["i"] += 1
            return eager
        for f in fns:  # eager warm-up outside capture
            f()
        t.cuda.synchronize()
        gs = []
        for f in fns:
            g = t.cuda.CUDAGraph()
            with t.cuda.graph(g):
                f()
            gs.append(g)
        t.cuda.synchronize()
        state = {"i": 0}

        def replay():
            gs[state["i"] % len(gs)].replay()
            state["i"] += 1
        replay.graphs = gs
        return replay

    def run(self, fn, reps):
        t = self.torch
        t.cuda.synchronize()
        a, b = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        t.cuda.synchronize()
        return a.elapsed_time(b) / reps  # ms

    def median(self, fn, reps=30):
        """Median of `reps` individually timed calls (ms)."""
        t = self.torch
        ev = [(t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        t.cuda.synchronize()
        for a, b in ev:
            a.record()
            fn()
            b.record()
        t.cuda.synchronize()
        xs = sorted(a.elapsed_time(b) for a, b in ev)
        return xs[reps // 2]


def make_session_pool(torch, dev, n_pages_total, layers):
    """bf16 pool of `layers` layers, values ~N(0,1)/sqrt(128) (bf16 bits as int16)."""
    elems = n_pages_total * P * 512 * layers
    x = torch.empty(elems, dtype=torch.bfloat16, device=dev)
    x.normal_(0.0, 1.0 / 128 ** 0.5)
    return x.view(torch.int16)


def q_rows(torch, dev, n):
    x = torch.empty(n * 2560, dtype=torch.bfloat16, device=dev)
    x.normal_(0.0, 1.0 / 128 ** 0.5)
    return x.view(torch.int16)


def bench_decode_single(kvm, torch, dev, timer, ctx, steps, warmup, rot):
    """One session, `ctx` cached tokens incl. the appended one; `rot` pool copies
    rotated per step so the working set exceeds the 256 MB Infinity Cache."""
    npages = ctx // P
    maxp = npages
    lay = kvm.KvLayout(maxp, P, LAYERS)
    C = kvm.attention_decode_chunk_pos(ctx)
    NC = kvm.attention_decode_max_chunks(ctx, C)
    g = torch.Generator(device="cpu").manual_seed(1)
    pt = torch.randperm(maxp, generator=g).to(torch.int32).to(dev)
    pools = [make_session_pool(torch, dev, maxp, LAYERS) for _ in range(rot)]
    qs = q_rows(torch, dev, LAYERS)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, 5e6)
    parts = torch.empty(16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    out = torch.empty(LAYERS * 2048, dtype=torch.int16, device=dev)
    def step_on(pool):
        def f():
            for l in range(LAYERS):
                kvm.launch_attention_decode(qs[l * 2560:], pos, l, pt, pool, lay, parts,
                                            NC, out[l * 2048:], d_inv_freq=inv,
                                            chunk_pos=C, d_partials2=parts2)
        return f

    step = timer.capture([step_on(p) for p in pools])
    # The chunk kernel alone (production configuration, merge skipped): the
    # switch is read when the launches are issued, i.e. while capturing.
    prev = kvm.debug_decode_records_only(True)
    try:
        chunks_only = timer.capture([step_on(p) for p in pools])
    finally:
        kvm.debug_decode_records_only(prev)
    timer.run(step, warmup)
    ms = timer.run(step, steps)
    ms_med = timer.median(step)
    timer.run(chunks_only, max(1, warmup))
    ms_chunk = timer.run(chunks_only, steps)
    tl = timeline_of(kvm, torch, step)
    bytes_layer = ctx * KV_BYTES_PER_TOKEN + QO_BYTES
    del pools
    return {
        **({"timeline_us": tl} if tl else {}),
        "ctx": ctx, "sessions": 1, "chunk_pos": C, "pages_per_layer": npages,
        "ms_per_step": ms, "us_per_layer": ms * 1e3 / LAYERS,
        "us_per_layer_median30": ms_med * 1e3 / LAYERS,
        "kv_gbs": bytes_layer * LAYERS / (ms * 1e-3) / 1e9,
        "pct_hbm_peak": 100.0 * bytes_layer * LAYERS / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s": 1e3 / ms,
        "chunk_kernel_us": ms_chunk * 1e3 / LAYERS,
        "chunk_kernel_gbs": bytes_layer / (ms_chunk * 1e-3 / LAYERS) / 1e9,
        "merge_kernel_us": (ms - ms_chunk) * 1e3 / LAYERS,
        "algorithmic_bytes_per_layer": bytes_layer,
        "pool_copies_rotated": rot,
    }


def bench_decode_batch(kvm, torch, dev, timer, B, ctx, steps, warmup):
    """B sessions in one shared pool, pages interleaved by a seeded shuffle;
    each step appends one token per session (phase0) and attends."""
    pages_per = ctx // P
    maxp = pages_per * B
    lay = kvm.KvLayout(maxp, P, LAYERS)
    C = kvm.attention_decode_chunk_pos(ctx)
    NC = kvm.attention_decode_max_chunks(ctx, C)
    g = torch.Generator(device="cpu").manual_seed(3)
    perm = torch.randperm(maxp, generator=g).to(torch.int32)
    pts = [perm[s::B].contiguous().to(dev) for s in range(B)]
    pool = make_session_pool(torch, dev, maxp, LAYERS)
    qs = q_rows(torch, dev, LAYERS * B)
    lims = [torch.tensor([ctx - 1], dtype=torch.int32, device=dev) for _ in range(B)]
    tab = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)
    d_pos, d_pt, d_kv = tab(lims), tab(pts), tab([pool] * B)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, 5e6)
    parts = torch.empty(B * 16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(B * (16 * 32 * 130), dtype=torch.float32, device=dev)
    out = torch.empty(B * 2048, dtype=torch.int16, device=dev)

    def step_f():
        for l in range(LAYERS):
            kvm.launch_attention_decode_batch(qs[l * B * 2560:], d_pos, B, l, d_pt, d_kv, lay,
                                              parts, NC, out, d_inv_freq=inv, chunk_pos=C,
                                              d_partials2=parts2)

    step = timer.capture([step_f])
    timer.run(step, warmup)
    ms = timer.run(step, steps)
    ms_med = timer.median(step)
    tl = timeline_of(kvm, torch, step)
    bytes_layer = B * (ctx * KV_BYTES_PER_TOKEN + QO_BYTES)
    return {
        **({"timeline_us": tl} if tl else {}),
        "ctx": ctx, "sessions": B, "chunk_pos": C, "ms_per_step": ms,
        "us_per_layer": ms * 1e3 / LAYERS,
        "us_per_layer_median30": ms_med * 1e3 / LAYERS,
        "kv_gbs": bytes_layer * LAYERS / (ms * 1e-3) / 1e9,
        "pct_hbm_peak": 100.0 * bytes_layer * LAYERS / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s": B * 1e3 / ms,
        "algorithmic_bytes_per_layer": bytes_layer,
    }


def bench_churn(kvm, torch, dev, timer, steps=64, B=8, max_ctx=131072, seed=5):
    """C5: B sessions with lengths log-uniform in [16, max_ctx) in one shared
    pool; over `steps` batched decode steps sessions finish and new ones are
    admitted (pages freed and reused through the shared pool allocator), every
    step appends one token per session (phase0) and attends (ragged limits,
    chunk tier of max_ctx). The 28-layer step is one captured graph; the
    host-side churn (allocator, page-table uploads, limits) runs between
    replays and is included in the step wall time."""
    import numpy as np
    rng = np.random.default_rng(seed)
    draw = lambda: int(min(max_ctx - steps - 1,
                           round(np.exp(rng.uniform(np.log(16), np.log(max_ctx))))))
    maxp = B * (max_ctx // P + 2)
    lay = kvm.KvLayout(maxp, P, LAYERS)
    C = kvm.attention_decode_chunk_pos(max_ctx)
    NC = kvm.attention_decode_max_chunks(max_ctx, C)
    pool = make_session_pool(torch, dev, maxp, LAYERS)
    alloc = kvm.SharedPagePool(maxp, P, B)
    d_tabs = [torch.zeros(maxp, dtype=torch.int32, device=dev) for _ in range(B)]
    lens = [draw() for _ in range(B)]
    for s in range(B):
        alloc.ensure(s, lens[s], d_tabs[s])
    lims = torch.zeros(B, dtype=torch.int32, device=dev)
    h_lims = torch.zeros(B, dtype=torch.int32).pin_memory()
    tab = lambda ptrs: torch.tensor(ptrs, dtype=torch.int64, device=dev)
    d_pos = tab([lims.data_ptr() + 4 * s for s in range(B)])
    d_pt = tab([t.data_ptr() for t in d_tabs])
    d_kv = tab([pool.data_ptr()] * B)
    qs = q_rows(torch, dev, LAYERS * B)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, 5e6)
    parts = torch.empty(B * 16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.empty(B * 16 * 32 * 130, dtype=torch.float32, device=dev)
    out = torch.empty(B * 2048, dtype=torch.int16, device=dev)

    def step_f():
        for l in range(LAYERS):
            kvm.launch_attention_decode_batch(qs[l * B * 2560:], d_pos, B, l, d_pt, d_kv, lay,
                                              parts, NC, out, d_inv_freq=inv, chunk_pos=C,
                                              d_partials2=parts2)

    def host_churn(first):
        for s in range(B):
            if not first and rng.random() < 0.1:  # finish -> admit a new session
                alloc.release(s)
                lens[s] = draw()
            alloc.ensure(s, lens[s] + 1, d_tabs[s])
            h_lims[s] = lens[s]
        lims.copy_(h_lims, non_blocking=True)

    host_churn(True)
    step = timer.capture([step_f])
    torch.cuda.synchronize()
    kv_tokens = 0
    gpu_ms = 0.0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    for it in range(steps):
        if it:
            host_churn(False)
        kv_tokens += sum(l + 1 for l in lens)
        e0.record()
        step()
        e1.record()
        e1.synchronize()
        gpu_ms += e0.elapsed_time(e1)
        for s in range(B):
            lens[s] += 1
    wall = time.perf_counter() - t0
    tl = timeline_of(kvm, torch, step)
    alloc.close()
    kv_bytes = kv_tokens * KV_BYTES_PER_TOKEN * LAYERS
    return {
        **({"timeline_us": tl} if tl else {}),
        "sessions": B, "steps": steps, "max_ctx": max_ctx, "chunk_pos": C,
        "mean_ctx": kv_tokens / steps / B,
        "gpu_us_per_layer": gpu_ms * 1e3 / steps / LAYERS,
        "wall_ms_per_step": wall * 1e3 / steps,
        "kv_gbs_gpu": kv_bytes / (gpu_ms * 1e-3) / 1e9,
        "pct_hbm_peak_gpu": 100.0 * kv_bytes / (gpu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s": B * steps / wall,
    }


def bench_append(kvm, torch, dev, timer, T, steps, warmup):
    """C2: RoPE + K/V append of one 8448-token prefill chunk for 28 layers."""
    npages = T // P
    maxp = npages
    lay = kvm.KvLayout(maxp, P, LAYERS)
    g = torch.Generator(device="cpu").manual_seed(5)
    pt = torch.randperm(maxp, generator=g).to(torch.int32).to(dev)
    pool = torch.zeros(maxp * P * 512 * LAYERS, dtype=torch.int16, device=dev)
    qkv = q_rows(torch, dev, T * LAYERS)
    base = torch.zeros(1, dtype=torch.int32, device=dev)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, 1e4)

    def step_f():
        for l in range(LAYERS):
            kvm.launch_rope_kv(qkv[l * T * 2560:], T, base, l, pt, pool, lay, 1e4,
                               d_inv_freq=inv)

    step = timer.capture([step_f])
    timer.run(step, warmup)
    ms = timer.run(step, steps)
    kv_bytes = T * 512 * 2 * 2  # k,v read + page write
    q_bytes = T * 2048 * 2 * 2  # q read + write (rotated in place)
    us = ms * 1e3 / LAYERS

    # Copy ceiling: torch's in-place elementwise multiply over the same qkv
    # rows moves the same bytes (every row read once and written once).
    rows = qkv.view(torch.bfloat16)

    def ceil_f():
        for l in range(LAYERS):
            rows[l * T * 2560:(l + 1) * T * 2560].mul_(1.0)

    ceil_step = timer.capture([ceil_f])
    timer.run(ceil_step, warmup)
    ceil_us = timer.run(ceil_step, steps) * 1e3 / LAYERS
    return {
        "tokens": T, "us_per_layer": us, "ms_per_step": ms,
        "torch_inplace_mul_same_bytes_us": ceil_us,
        "kv_bytes_per_layer": kv_bytes, "all_bytes_per_layer": kv_bytes + q_bytes,
        "gbs_incl_q": (kv_bytes + q_bytes) / (us * 1e-6) / 1e9,
        "pct_hbm_peak_incl_q": 100.0 * (kv_bytes + q_bytes) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s": T / (ms * 1e-3),
    }


def bench_prefill(kvm, torch, dev, timer, T, base, steps, warmup):
    """Prefill attention (page gather + causal flash attention) of one T-token
    chunk whose rows sit at positions base..base+T-1, over the paged pool
    (positions 0..base+T-1 cached), 28 layers. Compute-bound: reported against
    the dense bf16 MFMA peak; causal flops = 4 * 16 heads * 128 * sum_t (base+t+1)."""
    ctx = base + T
    npages = -(-ctx // P)
    maxp = npages
    lay = kvm.KvLayout(maxp, P, LAYERS)
    g = torch.Generator(device="cpu").manual_seed(9)
    pt = torch.randperm(maxp, generator=g).to(torch.int32).to(dev)
    pool = make_session_pool(torch, dev, maxp, LAYERS)
    qs = q_rows(torch, dev, T * LAYERS)
    d_base = torch.tensor([base], dtype=torch.int32, device=dev)
    S = kvm.prefill_flash_split_kv(T)
    parts = torch.empty(max(1, T * 16 * S * 130) if S > 1 else 1, dtype=torch.float32,
                        device=dev)
    out = torch.empty(T * 2048, dtype=torch.int16, device=dev)

    def step_f():
        for l in range(LAYERS):
            kvm.launch_attn_prefill_flash(qs[l * T * 2560:], T, d_base, l, pt, pool, lay, out,
                                          parts, S)

    step = timer.capture([step_f])
    timer.run(step, warmup)
    ms = timer.run(step, steps)
    us = ms * 1e3 / LAYERS
    flops = 4.0 * 16 * 128 * (T * base + T * (T + 1) / 2)
    kv_bytes = ctx * KV_BYTES_PER_TOKEN + T * 2048 * 2 * 2  # KV once + q read + out write
    return {
        "tokens": T, "base": base, "split_kv": S, "us_per_layer": us, "ms_per_step": ms,
        "tflops": flops / (us * 1e-6) / 1e12,
        "pct_mfma_bf16_peak": 100.0 * flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "flops_per_layer": flops, "algorithmic_bytes_per_layer": kv_bytes,
        "tokens_per_s": T / (ms * 1e-3),
    }


def host_threads() -> int:
    """CPU threads for the host baselines: the cores this process may run on,
    capped at the 16-core share a one-GPU box gives a job."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def decode_sources_sha16() -> str:
    """Hash of the decode kernel sources (the PMC traffic file records the
    hash it was measured with)."""
    import hashlib
    h = hashlib.sha256()
    d = os.path.join(ROOT, "minicpm5-5080fast_amd", "csrc")
    for f in ("decode_kernels.h", "decode_bf16p.hip", "attention_decode.hip", "kv_common.h"):
        h.update(open(os.path.join(d, f), "rb").read())
    return h.hexdigest()[:16]


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_append_baseline(seconds: float):
    """The CPU baseline's RoPE append (oracle/cpu_baseline.c cpb_rope_append,
    -O3 -march=native, all host threads) over one 8448-token chunk of one
    layer, repeated for about `seconds`; same bytes as the GPU C2 line."""
    import numpy as np
    import oracle
    T = 8448
    maxp = T // P
    threads = host_threads()
    rng = np.random.default_rng(1)
    qkv0 = oracle.f32_to_bf16(rng.standard_normal(T * 2560, dtype=np.float32)).reshape(T, 2560)
    pt = rng.permutation(maxp).astype(np.uint32)
    pool = np.zeros(maxp * P * 512, dtype=np.uint16)
    qkv = qkv0.copy()
    _, how = oracle.cpu_baseline_lib(native=True)
    oracle.cpb_rope_append(qkv, T, 0, 0, pt, P, maxp, 1e4, pool, threads, native=True)  # warm
    n, dt = 0, 0.0
    while dt < seconds:
        np.copyto(qkv, qkv0)
        t0 = time.perf_counter()
        oracle.cpb_rope_append(qkv, T, 0, 0, pt, P, maxp, 1e4, pool, threads, native=True)
        dt += time.perf_counter() - t0
        n += 1
    per_chunk = dt / n
    all_bytes = T * 2560 * 2 * 2  # row read + q / K / V written
    return {"tokens_per_s": T / per_chunk, "gbs": all_bytes / per_chunk / 1e9,
            "cores": threads, "kind": "port", "build": how, "cpu": cpu_model(),
            "nproc": os.cpu_count(),
            "sample": f"{n} x 8448-token append of one layer, {per_chunk * 1e3:.2f} ms each"}


def cpu_baseline(seconds: float):
    """The CPU baseline's fp32 decode (oracle/cpu_baseline.c cpb_decode: K/V
    rows shared by the 8 query heads of a group, position segments on all
    host threads, -O3 -march=native for this host): one layer of the C4
    workload (131072 tokens) per call, repeated for about `seconds`."""
    import numpy as np
    import oracle
    ctx = 131072
    maxp = ctx // P
    threads = host_threads()
    rng = np.random.default_rng(0)
    pool = oracle.f32_to_bf16(rng.standard_normal(maxp * P * 512, dtype=np.float32)
                              / np.float32(128 ** 0.5))
    pt = rng.permutation(maxp).astype(np.uint32)
    q = oracle.f32_to_bf16(rng.standard_normal(2560, dtype=np.float32) / np.float32(11.3))
    _, how = oracle.cpu_baseline_lib(native=True)
    oracle.cpb_decode(q, [ctx - 1], [pt], pool, 0, P, maxp, threads, native=True)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.cpb_decode(q, [ctx - 1], [pt], pool, 0, P, maxp, threads, native=True)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    per_layer = dt / n
    return {
        "value": (ctx * KV_BYTES_PER_TOKEN + QO_BYTES) / per_layer / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "build": how,
        "cpu": cpu_model(),
        "nproc": os.cpu_count(),
        "sample": f"{n} single-layer decode steps at 131072 ctx (C4), fp32, "
                  f"{per_layer * 1e3:.2f} ms/layer",
        "us_per_layer": per_layer * 1e6,
    }


def model_long_prefill(rt, W, torch, d, reps=1):
    """Seconds of one 8448-token prefill (one full prefill chunk: 8448 rows
    per projection GEMM) on a model whose context holds it, after one
    untimed prefill that loads the GEMM kernels; the mean of `reps`."""
    m = rt.Model(d, rt.model_options(max_context_tokens=16896, max_sessions=1,
                                     enable_cuda_graph=1))
    s = rt.Session(m)
    prompt = [(i * 7919) % W.VOCAB for i in range(8448)]
    s.prefill(prompt)
    total = 0.0
    for _ in range(reps):
        s.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        s.prefill(prompt)
        total += time.perf_counter() - t0
    s.close()
    m.close()
    return total / reps


def bench_model_prefill(pkg, torch, reps):
    """Whole-model 8448-token prefill alone (random-weight model.wpk of the
    full geometry, as in bench_model)."""
    import importlib
    import shutil
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    W = importlib.import_module("wpk_util")
    rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
    d = tempfile.mkdtemp(prefix="mc_wpk_")
    try:
        W.write_wpk(os.path.join(d, "model.wpk"), W.model_sections(2), W.random_blobs(7, 2))
        sec = model_long_prefill(rt, W, torch, d, reps)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {"weights": "random bf16, full MiniCPM5-2B geometry (42 layers, vocab 130560)",
            "reps": reps, "prefill_8448_ms": sec * 1e3, "prefill_8448_tokens_per_s": 8448 / sec}


def bench_model(pkg, torch, steps):
    """Whole-model greedy decoding with weights: a full-geometry model.wpk of
    random bf16 weights (even / odd layers share one weight set, embedding
    and lm_head one table; the device holds every section separately, 5.03 GB)
    loaded through mc_model_load with HIP graphs; 2048- and 8448-token
    prefills (the latter one full prefill chunk), 8-, 16- and 32-token ones
    (best of 5), solo decode after the 2048-token prompt and 8-session batch
    steps. Each decode streams every
    layer weight and the lm_head once: 4.50 GB per step."""
    import importlib
    import shutil
    import tempfile
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    W = importlib.import_module("wpk_util")
    rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
    d = tempfile.mkdtemp(prefix="mc_wpk_")
    try:
        secs = W.model_sections(2)
        W.write_wpk(os.path.join(d, "model.wpk"), secs, W.random_blobs(7, 2))
        t0 = time.perf_counter()
        m = rt.Model(d, rt.model_options(max_context_tokens=8192, max_sessions=9,
                                         enable_cuda_graph=1))
        load_s = time.perf_counter() - t0
        weight_bytes = (W.LAYERS * (W.QKV * W.HIDDEN + W.HIDDEN * W.HIDDEN
                                    + 2 * W.INTER * W.HIDDEN + W.HIDDEN * W.INTER)
                        + W.VOCAB * W.HIDDEN) * 2
        cfg = rt.gen_config(max_new_tokens=1 << 20)
        prompt = [(i * 7919) % W.VOCAB for i in range(2048)]
        s = rt.Session(m)
        s.prefill(prompt)  # first use: rocBLAS loads its GEMM kernels
        s.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        s.prefill(prompt)
        prefill_s = time.perf_counter() - t0
        # short prompts (projections as row-group GEMVs up to 16 tokens)
        short = {}
        for n in (8, 16, 32):
            s.reset()
            s.prefill(prompt[:n])
            ts = []
            for _ in range(5):
                s.reset()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                s.prefill(prompt[:n])
                ts.append(time.perf_counter() - t0)
            short[n] = min(ts)
        s.reset()
        s.prefill(prompt)
        for _ in range(3):
            s.decode_one(cfg)
        t0 = time.perf_counter()
        for _ in range(steps):
            s.decode_one(cfg)
        solo = (time.perf_counter() - t0) / steps
        ss = [rt.Session(m) for _ in range(8)]
        for i, x in enumerate(ss):
            x.prefill(prompt[:512 + 64 * i])
        g = rt.BatchGroup(m, 8, 8192)
        slots = [g.add(x) for x in ss]
        for _ in range(3):
            g.step(slots, [cfg] * 8)
        t0 = time.perf_counter()
        for _ in range(steps):
            g.step(slots, [cfg] * 8)
        batch = (time.perf_counter() - t0) / steps
        g.close()
        for x in ss + [s]:
            x.close()
        m.close()
        prefill_long_s = model_long_prefill(rt, W, torch, d)
        # FP8 mode (precision MC_FP8): model_fp8.wpk beside model.wpk, e4m3
        # codes of normal samples (fp32 bits cut to e4m3) with row scales;
        # each decode streams the e4m3 projections and lm_head, 2.25 GB
        rng = np.random.default_rng(8)
        q8 = {}
        for key, n, k in [(f"{nm}.{i}", nn, kk) for i in range(2) for nm, nn, kk in
                          (("qkv", W.QKV, W.HIDDEN), ("o", W.HIDDEN, W.HIDDEN),
                           ("gate_up", 2 * W.INTER, W.HIDDEN), ("down", W.HIDDEN, W.INTER))] + \
                [("table", W.VOCAB, W.HIDDEN)]:
            u = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(64.0)).view(np.uint32)
            e = ((u >> 23) & 0xFF).astype(np.int32) - 120
            mag = np.where(e < 1, 0, np.minimum((e << 3) | ((u >> 20) & 7), 0x7E))
            q8[key] = ((mag | ((u >> 24) & 0x80)).astype(np.uint8),
                       np.full(n, 1.0 / (64.0 * k ** 0.5), dtype=np.float32))
            del u, e, mag
        secs8 = W.fp8_sections(2, lm_head=True)
        W.write_fp8_wpk(os.path.join(d, "model_fp8.wpk"), secs8, q8)
        del q8
        fp8_bytes = W.fp8_arena_bytes(secs8)  # codes and scales, all read per decode
        m = rt.Model(d, rt.model_options(max_context_tokens=8192, max_sessions=2,
                                         enable_cuda_graph=1, precision=2))
        s = rt.Session(m)
        s.prefill(prompt)
        for _ in range(3):
            s.decode_one(cfg)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            s.decode_one(cfg)
        solo8 = (time.perf_counter() - t0) / steps
        s.close()
        m.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {
        "weights": "random bf16, full MiniCPM5-2B geometry (42 layers, vocab 130560)",
        "load_s": load_s, "weight_bytes_per_step": weight_bytes,
        "prefill_2048_ms": prefill_s * 1e3, "prefill_tokens_per_s": 2048 / prefill_s,
        "prefill_8_ms": short[8] * 1e3, "prefill_16_ms": short[16] * 1e3,
        "prefill_32_ms": short[32] * 1e3,
        "prefill_8448_ms": prefill_long_s * 1e3,
        "prefill_8448_tokens_per_s": 8448 / prefill_long_s,
        "decode_ms_per_token": solo * 1e3, "decode_tokens_per_s": 1.0 / solo,
        "decode_weight_gbs": weight_bytes / solo / 1e9,
        "decode_pct_hbm_peak": 100.0 * weight_bytes / solo / 1e9 / HBM_PEAK_GBS,
        "batch8_ms_per_step": batch * 1e3, "batch8_tokens_per_s": 8.0 / batch,
        "fp8_decode_ms_per_token": solo8 * 1e3, "fp8_decode_tokens_per_s": 1.0 / solo8,
        "fp8_weight_bytes_per_step": fp8_bytes,
        "fp8_decode_weight_gbs": fp8_bytes / solo8 / 1e9,
    }


def bench_gemm_rows(pkg, torch, dev, reps):
    """Row GEMM (mc_model_gemm_rows) of the four projections at 9, 16 and 32
    activation rows: us per launch (HIP events over `reps` launches, weights
    rotated over copies filling 512 MB so they come from HBM) and the weight
    bytes' rate."""
    lib = pkg._native.lib()
    shapes = [("qkv", 2560, 2048, 0), ("o", 2048, 2048, 0), ("gate_up_swiglu", 6144, 2048, 1),
              ("down", 2048, 6144, 0)]
    out = {}
    for M in (9, 16, 32):
        row = {}
        for name, N, K, swi in shapes:
            rows = 2 * N if swi else N
            copies = max(2, (512 << 20) // (rows * K * 2))
            ws = [torch.randn(rows, K, device=dev).to(torch.bfloat16) for _ in range(copies)]
            x = torch.randn(M, K, device=dev).to(torch.bfloat16)
            y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
            st = torch.cuda.current_stream().cuda_stream

            def run(i):
                r = lib.mc_model_gemm_rows(ws[i % copies].data_ptr(), x.data_ptr(), K,
                                           y.data_ptr(), N, M, N, K, swi, st)
                assert r == 0, r
            for i in range(5):
                run(i)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps):
                run(i)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            row[name] = {"us": us, "weight_gbs": rows * K * 2 / us / 1e3}
            del ws
        row["total_us"] = sum(v["us"] for v in row.values())
        out[f"rows_{M}"] = row
    return out


def bench_alloc(kvm):
    """Host page allocator (reference kv_cache.cpp:8-91 semantics, shared-pool
    form): 8 sessions grown to 131072 tokens of 64-token pages in one pool,
    then released; per-page cost of the C++ allocator (one ensure call per
    session, no page-table upload) and of the oracle's Python model on a
    one-session sample (the CPU port baseline)."""
    import oracle
    P, B, ctx = 64, 8, 131072
    per = ctx // P
    maxp = B * per
    pool = kvm.SharedPagePool(maxp, P, B)
    t0 = time.perf_counter()
    for s in range(B):
        pool.ensure(s, ctx)
    t1 = time.perf_counter()
    for s in range(B):
        pool.release(s)
    t2 = time.perf_counter()
    pool.close()
    model = oracle.SharedPoolModel(maxp, P, B)
    t3 = time.perf_counter()
    model.ensure(0, ctx)
    t4 = time.perf_counter()
    return {"pages": B * per, "ns_per_page_acquire": (t1 - t0) / (B * per) * 1e9,
            "ns_per_page_release": (t2 - t1) / (B * per) * 1e9,
            "oracle_ns_per_page_acquire": (t4 - t3) / per * 1e9,
            "oracle_sample": f"1 session x {per} pages, Python model"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (the KV path has no "
              f"multi-GPU code); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    pkg = importlib.import_module("minicpm5-5080fast_amd")
    kvm = pkg.kv
    dev = torch.device("cuda:0")
    timer = Timer(torch, graphs=not args.eager)
    if args.decode_timeline:
        global TIMELINE
        TIMELINE = torch.zeros(TIMELINE_LAUNCHES * kvm.TIMELINE_WORDS, dtype=torch.int64,
                               device=dev)
        kvm.debug_decode_timeline(TIMELINE, TIMELINE_LAUNCHES)
    cfgs = [c.strip() for c in args.configs.split(",") if c.strip()]
    res = {}
    if "c4" in cfgs:
        log("C4: 128K single session ...")
        res["c4_128k"] = bench_decode_single(kvm, torch, dev, timer, 131072, args.steps,
                                             args.warmup, rot=1)
        log(res["c4_128k"])
        torch.cuda.empty_cache()
    if "c3" in cfgs:
        log("C3: 8 x 2048 batched ...")
        res["c3_8x2k"] = bench_decode_batch(kvm, torch, dev, timer, 8, 2048, args.steps * 5,
                                            args.warmup)
        log(res["c3_8x2k"])
        torch.cuda.empty_cache()
    if "c1" in cfgs:
        log("C1: 2K single session ...")
        res["c1_2k"] = bench_decode_single(kvm, torch, dev, timer, 2048, args.steps * 5,
                                           args.warmup, rot=8)
        log(res["c1_2k"])
        torch.cuda.empty_cache()
    if "c2" in cfgs:
        log("C2: append 8448 tokens ...")
        res["c2_append_8448"] = bench_append(kvm, torch, dev, timer, 8448, args.steps,
                                             args.warmup)
        log(res["c2_append_8448"])
        torch.cuda.empty_cache()

    if "c5" in cfgs:
        log("C5: churn, 8 sessions, log-uniform lengths, 64 steps ...")
        res["c5_churn"] = bench_churn(kvm, torch, dev, timer)
        log(res["c5_churn"])
        torch.cuda.empty_cache()
    if "alloc" in cfgs:
        res["alloc_host"] = bench_alloc(kvm)
        log(res["alloc_host"])
    if "model" in cfgs:
        log("whole model with weights: decode, batch 8, prefill ...")
        res["model_decode"] = bench_model(pkg, torch, max(8, args.steps))
        log(res["model_decode"])
        torch.cuda.empty_cache()
    if "rows" in cfgs:
        log("row GEMM of the projections at 9 / 16 / 32 rows ...")
        res["gemm_rows"] = bench_gemm_rows(pkg, torch, dev, 100)
        log(res["gemm_rows"])
    if "mprefill" in cfgs:
        log("whole model with weights: 8448-token prefill ...")
        res["model_prefill"] = bench_model_prefill(pkg, torch, max(1, min(args.steps, 10)))
        log(res["model_prefill"])
    if "pf" in cfgs:
        for base in (0, 8448):
            log(f"prefill attention 8448 tokens at base {base} ...")
            r = bench_prefill(kvm, torch, dev, timer, 8448, base, max(2, args.steps // 4),
                              1)
            res[f"prefill_attn_8448_base{base}"] = r
            log(r)
            torch.cuda.empty_cache()
        # the reference's published kernel-level prefill points (RTX 5080,
        # kernels.h:544-547): T=2048 0.309 ms, T=8192 3.222 ms per layer
        for T, ref_ms in ((2048, 0.309), (8192, 3.222)):
            log(f"prefill attention {T} tokens at base 0 ...")
            r = bench_prefill(kvm, torch, dev, timer, T, 0, max(2, args.steps // 4), 1)
            r["reference_rtx5080_ms_per_layer"] = ref_ms
            res[f"prefill_attn_{T}_base0"] = r
            log(r)
            torch.cuda.empty_cache()

    if args.calib:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        log("calibration copy: 268435456 bytes read + written")

    head = res.get("c4_128k")
    cpu = None if args.no_cpu or head is None else cpu_baseline(args.cpu_seconds)
    if not args.no_cpu and "c2_append_8448" in res:
        res["cpu_append_8448"] = cpu_append_baseline(min(3.0, args.cpu_seconds))
    line = {
        "metric": "decode-attn us/layer & KV HBM GB/s (% peak) at 2K, 8x2K batch, 128K",
        "value": round(head["kv_gbs"], 2) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (bf16 ~N(0,1)/sqrt(128), seeded permuted page tables)",
        "config": {"workload": "C4: 1 session x 131072 ctx, Hq16/Hkv2/D128, 64-token "
                               "pages, chunk 256, 2-level merge, phase0 append, 28 layers"},
        "roofline": None,
        "cpu_baseline": cpu,
        "configs": res,
    }
    if head:
        ach = head["chunk_kernel_gbs"]
        # HBM bytes per launch from two rocprofv3 PMC passes (FETCH_SIZE,
        # WRITE_SIZE), valid only for the kernel sources they were measured
        # on: the file records a hash of those sources.
        traffic, note = None, "no PMC measurement for these kernel sources"
        tf = os.path.join(ROOT, "profiles", "decode_chunk_c4_traffic.txt")
        if os.path.exists(tf):
            rec = json.load(open(tf))
            if rec.get("sources_sha16") == decode_sources_sha16():
                traffic, note = rec.get("traffic_bytes"), rec.get("source")
            else:
                note = "PMC file is stale (kernel sources changed since it was measured)"
        line["roofline"] = {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                            "traffic": traffic, "traffic_note": note,
                            "kernel": "decode_chunk_kernel<true,false,true,4,true,false> "
                                      "(C4 layer, merge skipped)",
                            "kernel_us": round(head["chunk_kernel_us"], 3)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
