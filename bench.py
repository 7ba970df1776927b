"""Decode-attention throughput of the tiered-KV path on one MI355X.

Workload (headline): Llama-3-8B-shaped GQA decode, bf16, batch 1, 32 query
heads / 8 KV heads, head dim 128, 32768 cached tokens in 32 chunks of 1024,
hot_ratio 0.25 (the last 8 chunks, in HBM), 24 cold chunks per layer in
pinned host memory, of which the scorer selects the top 4 per layer per step
by mean-key dot product inside the attention launch; keys carry 4 planted
high-variance channels (sigma 8); 32 layers with distinct buffers.  Each
layer's query follows a seeded drifting trajectory (AR(1) in fp32:
q_t = rho q_{t-1} + sqrt(1 - rho^2) e_t, rho 0.98), so the selection moves
from step to step.  A selected chunk is read from an HBM staging slot when
the staging cache holds it (12 slots per layer, refilled by hipMemcpyAsync on
a side stream from the returned scores) and in place over the host link
otherwise.  One step = the next query written to HBM, the commits of landed
fills, the 64 launches of the 32 layers replayed from one HIP graph, and the
score read-back with the cache's policy -- all inside the timed region;
tokens/s = 1 / step time, with the hit rate and the host-link bytes.

Beside it: the same layers with every cold chunk resident in HBM
(kernel-level roofline of the attention launch), the same workload with no
staging cache (every selected chunk read over the link), and the other
configurations (chunked prefill, ragged batch, KIVI cold tier).

Prints one JSON line.  ``--gpus N`` with N > 1 exits: this build measures
one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode attn tokens/s + achieved HBM GB/s, 8B-shape GQA @32k ctx, hot_ratio 0.25"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layers(torch, *, L, H, H_kv, D, T, chunk, n_hot, top_k, n_planted, sigma, dev, seed, split=None,
                fused=True):
    import numpy as np

    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer

    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers, qs, kvs = [], [], []
    n_chunks = T // chunk
    n_cold = n_chunks - n_hot
    for li in range(L):
        k = torch.randn((1, H_kv, T, D), generator=gen, device=dev, dtype=torch.float32)
        planted = torch.from_numpy(np.sort(rng.choice(D, size=n_planted, replace=False))).to(dev)
        k[..., planted] *= sigma
        k = k.to(torch.bfloat16)
        v = torch.randn((1, H_kv, T, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        q = torch.randn((1, H, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        refs = [ChunkRef(k[..., i * chunk:(i + 1) * chunk, :], v[..., i * chunk:(i + 1) * chunk, :], i * chunk, True)
                for i in range(n_chunks)]
        layers.append(TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16,
                                        hot=refs[n_cold:], cold=refs[:n_cold], top_k=top_k, device=dev,
                                        split=split, fused=fused))
        qs.append(q)
        kvs.append((k, v))
    return layers, qs, kvs


def cpu_baseline(torch, kvs, qs, layers, *, chunk, n_hot, top_k, L, budget_s):
    """The reference's CPU torch op sequence (the oracle's torch path) on the
    host cores over a bounded sample of layers; scaled to tokens/s."""
    from oracle import torch_path as TP

    threads = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit():
        threads = max(1, min(threads, int(share)))  # the host's CPU share for this GPU
    try:  # a cgroup CPU quota below the affinity mask: more threads than that only thrash
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            threads = max(1, min(threads, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    torch.set_num_threads(threads)
    n_sample = min(4, L)
    samples = []
    for li in range(n_sample):
        k, v = (t.cpu() for t in kvs[li])
        q = qs[li].cpu().unsqueeze(2)
        km = layers[li].kmean.cpu()
        samples.append((q, k, v, km))
    T = samples[0][1].shape[2]
    n_cold = T // chunk - n_hot
    elig = torch.arange(n_cold)

    def one_pass():
        for (q, k, v, km) in samples:
            sel = TP.select_top(q, km, elig, top_k)
            ids = list(sel.tolist()) + list(range(n_cold, T // chunk))
            TP.chunk_walk(q, [(k[..., c * chunk:(c + 1) * chunk, :], v[..., c * chunk:(c + 1) * chunk, :])
                              for c in ids], 1.0 / math.sqrt(q.shape[-1]))

    for _ in range(3):
        one_pass()
    t0 = time.perf_counter()
    one_pass()
    est = time.perf_counter() - t0
    iters = max(10, min(200, int(budget_s / max(est, 1e-6))))
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times) / n_sample
    try:
        cpu_model = [ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name")][0]
    except Exception:
        cpu_model = "unknown"
    return {
        "value": 1.0 / (per_layer * L),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_sample} of {L} layers of the same workload per pass (score top-{top_k} of {n_cold} cold "
                   f"chunks + LSE-merged attention over {n_hot}+{top_k} chunks), 3 warmup + {iters} timed "
                   f"passes, median, scaled x{L / n_sample:g} to a {L}-layer step; torch "
                   f"{torch.__version__} CPU, {threads} threads, {cpu_model}"),
    }


def host_tier(torch, layers):
    """The cold chunks of every layer as contiguous pinned host tensors (the
    cold tier), copied from their HBM originals: one pinned buffer per layer
    holding each chunk's K rows followed by its V rows, so the staging cache
    fills a chunk with one copy."""
    from halo_amd.decode import ChunkRef
    tiers = []
    for lay in layers:
        shape = tuple(lay.cold[0].k.shape)
        buf = torch.empty((len(lay.cold), 2) + shape, dtype=lay.cold[0].k.dtype, pin_memory=True)
        cold = []
        for j, c in enumerate(lay.cold):
            buf[j, 0].copy_(c.k)
            buf[j, 1].copy_(c.v)
            cold.append(ChunkRef(buf[j, 0], buf[j, 1], c.chunk_start, c.causal))
        tiers.append(cold)
    return tiers


def query_trajectory(torch, dev, *, steps, L, H, D, rho, seed, B=1):
    """Per-layer (and per-row) AR(1) query drift in fp32, rounded to bf16:
    q_0 ~ N(0, 1), q_t = rho q_{t-1} + sqrt(1 - rho^2) e_t.  (steps, L, B, H, D)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q = torch.randn((L, B, H, D), generator=gen, device=dev)
    out = torch.empty((steps, L, B, H, D), device=dev, dtype=torch.bfloat16)
    c = math.sqrt(max(0.0, 1.0 - rho * rho))
    for t in range(steps):
        q = rho * q + c * torch.randn((L, B, H, D), generator=gen, device=dev)
        out[t] = q.to(torch.bfloat16)
    return out


def refetch_run(torch, staged, staging, qtraj, *, warmup, steps, scale, label, warm_fills=None, segments=4,
                record=None, lses=None, q_pos=None):
    """Timed decode steps over the staged layers.  A step writes the next
    queries, then runs the layers as ``segments`` consecutive HIP graphs;
    before each segment the fills that landed for its layers are committed,
    after it its scores go back to the host, and while the next segment runs
    the host plans the previous segment's fills (so they have one step to
    land).  Returns the reading.

    ``record(t, lo, hi, outs)``, if given, is called right after segment
    [lo, hi) of step t is replayed, on the replay stream (to enqueue copies
    of that step's outputs: the loop itself never synchronises); ``lses``
    (one (B, H) fp32 tensor per layer) makes the graphs write the LSEs too.
    ``qtraj`` is (steps, L, B, H, D) for layers of batch B; ``q_pos`` (B,)
    int64, if given, is every launch's decode position."""
    dev = qtraj.device
    L = len(staged)
    B, H, D = staged[0].B, staged[0].H, staged[0].D
    qbuf = torch.empty((L, B, H, D), device=dev, dtype=torch.bfloat16)
    outs = [torch.empty((B, H, D), device=dev, dtype=torch.bfloat16) for _ in range(L)]
    lse_of = (lambda li: lses[li]) if lses is not None else (lambda li: None)
    bounds = [(g * L // segments, (g + 1) * L // segments) for g in range(segments)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    n_traj = qtraj.shape[0]
    graphs = []
    with torch.cuda.stream(s):
        qbuf.copy_(qtraj[0])
        for li in range(L):
            staged[li].step(qbuf[li], scale=scale, out=outs[li], lse=lse_of(li), q_pos=q_pos)
        torch.cuda.synchronize()
        for lo, hi in bounds:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for li in range(lo, hi):
                    staged[li].step(qbuf[li], scale=scale, out=outs[li], lse=lse_of(li), q_pos=q_pos)
            graphs.append(g)
        torch.cuda.synchronize()
        t0 = 0.0
        budget = staging.max_inflight
        if warm_fills is not None:
            staging.max_inflight = warm_fills   # the warm-up may fill the empty cache faster
        for t in range(warmup + steps):
            if t == warmup:
                staging.drain()
                torch.cuda.synchronize()
                staging.max_inflight = budget
                staging.reset_counters()
                t0 = time.perf_counter()
            for (lo, hi), g in zip(bounds, graphs):
                staging.before_step(lo, hi)
                if lo == 0:
                    qbuf.copy_(qtraj[t % n_traj], non_blocking=True)
                g.replay()
                if record is not None:
                    record(t, lo, hi, outs)
                staging.after_step(lo, hi)
                staging.service()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        staging.drain()      # count the last steps' selections too
    del graphs
    sel = staging.hits + staging.misses
    link = (staging.fill_bytes + staging.miss_bytes) / steps
    ns = staging.stats
    log(f"{label}: host per step: plan {ns['ns_plan'] / steps / 1e3:.0f} us (fill issue {ns['ns_issue'] / steps / 1e3:.0f} "
        f"us), feedback wait {ns['ns_wait'] / steps / 1e3:.0f} us")
    log(f"{label}: {dt * 1e3:.3f} ms/step, hit rate {staging.hit_rate():.4f} over {sel} selections "
        f"({staging.misses_predicted} of {staging.misses} misses predicted), "
        f"{staging.fills / steps:.2f} fills/step, {staging.wa_commits / steps:.2f} write-allocated/step, "
        f"link {link / 2**20:.1f} MiB/step")
    return {
        "tokens_per_s": 1.0 / dt, "ms_per_step": dt * 1e3, "hit_rate": staging.hit_rate(),
        "selections": sel, "hits": staging.hits, "misses": staging.misses,
        "misses_predicted": staging.misses_predicted,
        "fills_per_step": staging.fills / steps,
        "write_allocated_per_step": staging.wa_commits / steps,
        "prefetch_bytes_per_step": staging.fill_bytes / steps,
        "in_place_miss_bytes_per_step": staging.miss_bytes / steps,
        "link_bytes_per_step": link, "link_gbps": link / dt / 1e9, "segments": segments,
        "host_us_per_step": {"plan": ns["ns_plan"] / steps / 1e3, "fill_issue": ns["ns_issue"] / steps / 1e3,
                             "feedback_wait": ns["ns_wait"] / steps / 1e3},
    }


def kernel_level_c2(torch, layers, qs, *, scale, reps, with_scorer=True):
    """The C2 layers with every cold chunk in HBM, one HIP graph of all
    layers (attention with in-kernel selection + merge per layer), timed
    with events on the capture stream over ``reps`` replays.  Returns ms per
    layer of the attention launch and of the standalone scorer."""
    L = len(layers)
    H, D = layers[0].H, layers[0].D
    dev = qs[0].device
    outs = [torch.empty((1, H, D), device=dev, dtype=torch.bfloat16) for _ in range(L)]
    lses = [torch.empty((1, H), device=dev, dtype=torch.float32) for _ in range(L)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def capture(fn):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            fn()
            torch.cuda.synchronize()
            with torch.cuda.graph(gr, stream=s):
                fn()
        torch.cuda.synchronize()
        return gr

    def time_graph(gr, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            gr.replay()
            e0.record(s)
            for _ in range(reps):
                gr.replay()
            e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * L)

    g_attn = capture(lambda: [layers[li].step(qs[li], scale=scale, out=outs[li], lse=lses[li]) for li in range(L)])
    attn_avg = time_graph(g_attn, reps)          # ms per layer: attention kernel + merge kernel
    del g_attn
    score_avg = None
    if with_scorer:
        g_score = capture(lambda: [layers[li].select(qs[li]) for li in range(L)])
        score_avg = time_graph(g_score, reps)
        del g_score
    return attn_avg, score_avg


def bench_measured_peaks(torch, dev) -> dict:
    """What this GPU reaches on plain work, beside the published peaks the
    rooflines use: a 1 GiB device-to-device copy (bytes read + written), a
    256 MiB pinned host-to-device copy (the host link) and square bf16 GEMMs
    (torch.mm, library MFMA kernels; 8192^3 and 16384^3)."""
    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps
    n = 1 << 30
    a = torch.ones(n, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    t_copy = timed(lambda: b.copy_(a), 10)
    del a, b
    h = torch.ones(256 << 20, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    t_h2d = timed(lambda: d.copy_(h, non_blocking=True), 5)
    del h, d
    gemm = {}
    for m in (8192, 16384):
        x = torch.randn((m, m), device=dev, dtype=torch.bfloat16)
        y = torch.randn((m, m), device=dev, dtype=torch.bfloat16).contiguous()
        z = torch.empty((m, m), device=dev, dtype=torch.bfloat16)
        gemm[f"{m}^3"] = 2 * m ** 3 / timed(lambda: torch.mm(x, y, out=z), 10) / 1e12
        del x, y, z
    torch.cuda.empty_cache()
    return {"hbm_copy_gbps": 2 * n / t_copy / 1e9, "host_to_device_gbps": (256 << 20) / t_h2d / 1e9,
            "bf16_gemm_tflops": max(gemm.values()), "bf16_gemm_tflops_by_shape": gemm,
            "note": "1 GiB device copy (read + write bytes), 256 MiB pinned H2D copy, bf16 torch.mm (square, "
                    "best shape); the rooflines' peaks are the published 8 TB/s and 2.5 PFLOP/s"}


def bench_prefill_c3(torch, dev, *, reps: int):
    """Chunked causal prefill, Llama-3-8B GQA shape: a 4096-token query block
    attends 28 prior chunks of 1024 rows plus itself (causal), bf16 MFMA.
    Algorithmic work 2,061,617,856,512 FLOP (causal half of the self block)."""
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention

    H, H_kv, D, T_q, T_prior, chunk = 32, 8, 128, 4096, 28672, 1024
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    q = torch.randn((1, H, T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn((1, H_kv, T_prior + T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((1, H_kv, T_prior + T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    chunks = [ChunkRef(k[:, :, s:s + chunk], v[:, :, s:s + chunk], s, False) for s in range(0, T_prior, chunk)]
    chunks.append(ChunkRef(k[:, :, T_prior:], v[:, :, T_prior:], T_prior, True))
    for _ in range(2):
        prefill_attention(q, chunks)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        prefill_attention(q, chunks)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flops = 4 * H * D * T_q * T_prior + 2 * H * D * T_q * (T_q + 1)
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "workload": "chunked causal prefill, bf16, 32/8 heads, d128, 4096 query rows over 28x1024 prior + "
                    "4096 self (causal), one launch",
        "ms_per_call": ms, "flop_per_call": flops, "tflops": tflops,
        "roofline": {"bound": "mfma", "kernel": "prefill_attn_kernel<bf16,128>", "achieved": tflops,
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tflops / MFMA_BF16_PEAK_TFLOPS},
    }


def bench_dropin_c2(torch, dev, layers, qs, *, top_k: int, steps: int):
    """The drop-in kernel module (halo_amd.triton_chunked, the import swap of
    halo/triton_chunked.py) at the headline's layer shape: per layer one
    ``triton_chunked_attention`` call over its 8 hot chunks plus 4 cold
    chunks (the list the cache passes after its own selection), all in HBM.
    Eager calls (host planning included; repeated chunk lists hit the plan
    cache) and the same calls captured in one HIP graph per step."""
    from halo_amd.triton_chunked import triton_chunked_attention

    L = len(layers)
    lists = [[(c.k, c.v, c.chunk_start, True) for c in lay.hot + lay.cold[:top_k]] for lay in layers]
    q4 = [q.unsqueeze(2) for q in qs]
    # the decode position is the context's last row: the default (the sum of
    # the listed rows minus one) would place it inside the prefix and mask
    # the hot chunks causally
    ctx = max(c.chunk_start + c.T for c in layers[0].hot)
    q_pos = torch.full((q4[0].shape[0],), ctx - 1, dtype=torch.int64, device=dev)

    def step():
        for li in range(L):
            triton_chunked_attention(q4[li], lists[li], q_pos=q_pos)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(steps):
            step()
        e1.record(s)
        torch.cuda.synchronize()
        eager_us = e0.elapsed_time(e1) / steps / L * 1e3
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            step()
        gr.replay()
        e0.record(s)
        for _ in range(steps):
            gr.replay()
        e1.record(s)
    torch.cuda.synchronize()
    graph_us = e0.elapsed_time(e1) / steps / L * 1e3
    return {
        "workload": "halo_amd.triton_chunked.triton_chunked_attention per 32k-context decode layer: 12 chunks of 1024 rows "
                    "(8 hot + 4 cold), bf16, 32/8 heads, d128, batch 1, 32 layers",
        "eager_us_per_layer": eager_us, "graph_us_per_layer": graph_us,
        "eager_tokens_per_s": 1e6 / (eager_us * L), "graph_tokens_per_s": 1e6 / (graph_us * L),
    }


def bench_kivi_c5(torch, dev, *, steps: int, layers: int = 28):
    """KIVI 2-bit cold tier, Qwen2-7B shape: 28/4 heads, d128, 131072
    context; all but the last 128 tokens in 2-bit blocks (K per channel, V per
    token, group 32, fp16 scale/zero), dequantised inside the decode kernel;
    the 128 recent tokens fp16.  28 layers with distinct buffers, one HIP
    graph per step."""
    from halo_amd import kivi
    from halo_amd.decode import ChunkRef

    H, H_kv, D, T, resid = 28, 4, 128, 131072, 128
    T_cold = T - resid
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    lays, qs = [], []
    for _ in range(layers):
        k = torch.randn((1, H_kv, T, D), generator=gen, device=dev)
        ch = torch.randperm(D, generator=gen, device=dev)[:2]
        k[..., ch] *= 10.0
        k = k.to(torch.float16)
        v = torch.randn((1, H_kv, T, D), generator=gen, device=dev).to(torch.float16)
        blocks = kivi.quantize(k[:, :, :T_cold], v[:, :, :T_cold])
        kr, vr = k[:, :, T_cold:].clone(), v[:, :, T_cold:].clone()
        del k, v
        lays.append(kivi.KiviDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.float16, cold_blocks=blocks,
                                         recent=[ChunkRef(kr, vr, T_cold, True)], device=dev, chunk_tokens=2048))
        qs.append(torch.randn((1, H, D), generator=gen, device=dev).to(torch.float16))
    outs = [torch.empty((1, H, D), device=dev, dtype=torch.float16) for _ in range(layers)]
    scale = 1.0 / math.sqrt(D)

    def step():
        for i in range(layers):
            lays[i].step(qs[i], scale=scale, out=outs[i])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            step()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        gr.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(steps):
            gr.replay()
        e1.record(s)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    layer_us = step_ms * 1e3 / layers
    nblk = T_cold // 32
    # one launch per layer: the 2-bit blocks, the fp16 recent rows and q
    layer_bytes = nblk * H_kv * kivi.block_bytes(D) + resid * H_kv * D * 2 * 2 + 2 * H * D * 2
    achieved = layer_bytes / (layer_us * 1e-6) / 1e9
    return {
        "workload": "Qwen2-7B-shaped decode over a KIVI 2-bit cold tier: 28/4 heads, d128, 131072 ctx "
                    "(130944 quantised in 32-token blocks + 128 fp16 recent, one launch per layer), 28 layers looped",
        "tokens_per_s": 1e3 / step_ms, "ms_per_step": step_ms,
        "hbm_bytes_per_layer": layer_bytes,
        "hbm_gbps_end_to_end": layers * layer_bytes / (step_ms * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "kernel": "halo_decode_attn_kivi (decode_attn_kivi_kernel<f16,128,8,4> + merge)",
                     "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS,
                     "bytes_per_launch": layer_bytes, "avg_launch_us": layer_us},
    }


def bench_ragged_c4(torch, dev, *, steps: int):
    """Ragged batched decode: 16 sequences, 32/8 heads, d128, bf16, context
    lengths floor(U[8192, 131072] / 2048) * 2048 (seed 3), per-sequence chunk
    tables of 2048-row chunks, hot = last max(1, 0.25 n_i) chunks, every row
    selecting its top-8 cold chunks by mean-key score inside the launch."""
    import numpy as np

    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import RaggedTieredDecodeLayer

    B, H, H_kv, D, chunk, top_k = 16, 32, 8, 128, 2048, 8
    rng = np.random.default_rng(3)
    ctx = [int(x) // chunk * chunk for x in rng.uniform(8192, 131072, size=B)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    rows = []
    for b, T in enumerate(ctx):
        k = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
        n = T // chunk
        n_hot = max(1, n // 4)
        refs = [ChunkRef(k[:, i * chunk:(i + 1) * chunk], v[:, i * chunk:(i + 1) * chunk], i * chunk, True, batch=b)
                for i in range(n)]
        rows.append((refs[n - n_hot:], refs[:n - n_hot]))
    layer = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows, top_k=top_k, device=dev)
    q = torch.randn((B, H, D), generator=gen, device=dev).to(torch.bfloat16)
    q_pos = torch.tensor([T - 1 for T in ctx], device=dev, dtype=torch.int64)
    out = torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.step(q, scale=scale, out=out, q_pos=q_pos)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            layer.step(q, scale=scale, out=out, q_pos=q_pos)
        gr.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(steps):
            gr.replay()
        e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    n_cold_total = sum(len(c) for _, c in rows)
    step_bytes = layer.attended_rows() * H_kv * D * 2 * 2 + n_cold_total * H_kv * D * 2 + 2 * B * H * D * 2
    achieved = step_bytes / (ms * 1e-3) / 1e9
    return {
        "workload": "ragged batched GQA decode, bf16, 16 sequences of 8K-128K tokens (seed 3) in 2048-row chunks, "
                    "32/8 heads, d128, hot 25% per sequence + per-row top-8 of the cold chunks, one layer",
        "context_lengths": ctx, "tokens_per_s": B * 1e3 / ms, "ms_per_step": ms, "hbm_bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "kernel": "halo_decode_attn_tiered per-row selection (attention + merge)",
                     "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS},
    }


def bench_ragged_c4_host(torch, dev, *, steps: int, warmup: int = 10, layers: int = 4, slots: int = 12,
                         keep: int = 10, rho: float = 0.98):
    """The ragged batch with its cold tier in pinned host memory: ``layers``
    distinct layers of the C4 batch (16 sequences of 8K-128K tokens, seed 3,
    2048-row chunks, hot = last 25 % of each sequence's chunks in HBM), every
    row selecting its top-8 cold chunks per step inside the launch, served by
    a per-row HBM staging cache (``slots`` slots per row, the ``keep`` best
    by the last scores staged) or read in place over the host link.  Each
    row's query drifts as an AR(1) trajectory (``rho``); one step = the L
    layers as L graph segments plus the cache's commits, feedback and fills;
    tokens/s = 16 / step time."""
    import numpy as np

    from halo_amd.decode import ChunkRef
    from halo_amd.staging import ColdStaging
    from halo_amd.tiered import RaggedTieredDecodeLayer

    B, H, H_kv, D, chunk, top_k = 16, 32, 8, 128, 2048, 8
    rng = np.random.default_rng(3)
    ctx = [int(x) // chunk * chunk for x in rng.uniform(8192, 131072, size=B)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    staged = []
    hot_rows = cold_rows = 0
    for _ in range(layers):
        rows, rows_hbm = [], []
        for b, T in enumerate(ctx):
            k = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
            n = T // chunk
            n_hot = max(1, n // 4)
            refs = [ChunkRef(k[:, i * chunk:(i + 1) * chunk], v[:, i * chunk:(i + 1) * chunk], i * chunk, True,
                             batch=b) for i in range(n)]
            rows_hbm.append((refs[n - n_hot:], refs[:n - n_hot]))
            hot_rows += n_hot * chunk
            cold_rows += (n - n_hot) * chunk
        means = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows_hbm, top_k=top_k,
                                        device=dev).kmean
        for b, (hot, cold) in enumerate(rows_hbm):
            # hot chunks into HBM tensors of their own (the cold rows' HBM
            # copies are dropped), cold chunks K|V into one pinned buffer
            hk = torch.stack([c.k for c in hot], 0).contiguous()
            hv = torch.stack([c.v for c in hot], 0).contiguous()
            hot_own = [ChunkRef(hk[i], hv[i], c.chunk_start, True, batch=b) for i, c in enumerate(hot)]
            buf = torch.empty((len(cold), 2, H_kv, chunk, D), dtype=torch.bfloat16, pin_memory=True)
            host = []
            for j, c in enumerate(cold):
                buf[j, 0].copy_(c.k)
                buf[j, 1].copy_(c.v)
                host.append(ChunkRef(buf[j, 0], buf[j, 1], c.chunk_start, True, batch=b))
            rows.append((hot_own, host))
        del rows_hbm, k, v, refs
        staged.append(RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows, top_k=top_k,
                                              device=dev, cold_kmean=means))
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    staging = ColdStaging(staged, n_slots=slots, keep=keep, max_inflight=16)
    qtraj = query_trajectory(torch, dev, steps=warmup + steps, L=layers, H=H, D=D, rho=rho, seed=13, B=B)
    q_pos = torch.tensor([T - 1 for T in ctx], device=dev, dtype=torch.int64)
    rd = refetch_run(torch, staged, staging, qtraj, warmup=warmup, steps=steps, scale=1.0 / math.sqrt(D),
                     label=f"ragged batch, host tier, {layers} layers, rho {rho}", warm_fills=10 ** 6,
                     segments=layers, q_pos=q_pos)
    staged_rows = sum(min(slots, len(c)) for lay in staged for _, c in lay.rows) * chunk
    rd["tokens_per_s"] = B / (rd["ms_per_step"] * 1e-3)
    out = {
        "workload": f"ragged batched GQA decode, bf16, 16 sequences of 8K-128K tokens (seed 3) in 2048-row "
                    f"chunks, 32/8 heads, d128, {layers} layers, hot 25% per sequence in HBM, cold chunks in "
                    f"pinned host memory, per-row top-8 refetched through a per-row HBM staging cache "
                    f"({slots} slots, keep {keep}), AR(1) query drift rho {rho}",
        "context_lengths": ctx, "layers": layers, "staging_slots_per_row": slots, "staging_keep": keep,
        "hbm_resident_fraction": (hot_rows + staged_rows) / (hot_rows + cold_rows),
        "staging_bytes": staging.slot_bytes,
        **rd,
    }
    del staging, staged
    torch.cuda.empty_cache()
    return out


def bench_long_context(torch, dev, *, steps: int = 60, warmup: int = 10, L: int = 16, slots: int = 12,
                       keep: int = 6, rho: float = 0.98):
    """C2's layer shape at a 131072-token context: 128 chunks of 1024 rows,
    32 hot (25 %) in HBM, 96 cold in pinned host memory, top-4 per layer per
    step (96 x 8 = 768 (chunk, KV head) candidates: the fused selection's
    widest catalog), served by the HBM staging cache; L distinct layers,
    AR(1) query drift.  Beside it the same layers with every chunk in HBM,
    fused and on the two-launch path (standalone scorer, then the attention
    launch and its merge)."""
    H, H_kv, D, T, chunk, n_hot, top_k = 32, 8, 128, 131072, 1024, 32, 4
    from halo_amd.staging import ColdStaging
    from halo_amd.tiered import TieredDecodeLayer
    layers, qs, _ = make_layers(torch, L=L, H=H, H_kv=H_kv, D=D, T=T, chunk=chunk, n_hot=n_hot, top_k=top_k,
                                n_planted=4, sigma=8.0, dev=dev, seed=7)
    assert layers[0].fused
    scale = 1.0 / math.sqrt(D)
    attn_avg, _ = kernel_level_c2(torch, layers, qs, scale=scale, reps=20, with_scorer=False)
    two = [TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=lay.hot, cold=lay.cold,
                             top_k=top_k, device=dev, cold_kmean=lay.kmean, fused=False) for lay in layers]
    two_avg, _ = kernel_level_c2(torch, two, qs, scale=scale, reps=20, with_scorer=False)
    del two
    tiers = host_tier(torch, layers)
    staged = [TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=lay.hot, cold=tiers[li],
                                top_k=top_k, device=dev, cold_kmean=lay.kmean) for li, lay in enumerate(layers)]
    # fills dominate this layer's link traffic: two copy streams land them
    # sooner (1.06 against 1.13-1.15 ms per step, hit rate 0.948 against 0.933)
    staging = ColdStaging(staged, n_slots=slots, keep=keep, max_inflight=16, copy_streams=2)
    qtraj = query_trajectory(torch, dev, steps=warmup + steps, L=L, H=H, D=D, rho=rho, seed=17)
    rd = refetch_run(torch, staged, staging, qtraj, warmup=warmup, steps=steps, scale=scale,
                     label=f"131072-token context, 96 cold chunks, rho {rho}", warm_fills=10 ** 6, segments=4)
    rows = staged[0].attended_rows
    layer_bytes = rows * H_kv * D * 2 * 2 + 2 * H * D * 2 + H * 4 + (T // chunk - n_hot) * H_kv * D * 2
    out = {
        "workload": f"Llama-3-8B-shaped GQA decode at 131072 tokens: {L} layers, 128 chunks of 1024 rows, 32 hot in "
                    f"HBM + top-4 of 96 cold chunks in pinned host memory per layer per step (selection fused in the "
                    f"attention launch), HBM staging cache of {slots} slots (keep {keep}), AR(1) drift rho {rho}",
        "layers": L, "hbm_resident_fraction": (n_hot + slots) / (T // chunk), "copy_streams": 2,
        "all_hbm_us_per_layer": attn_avg * 1e3,
        "all_hbm_gbps": layer_bytes / (attn_avg * 1e-3) / 1e9,
        "all_hbm_two_launch_us_per_layer": two_avg * 1e3,
        "staged_us_per_layer": rd["ms_per_step"] * 1e3 / L,
        **{k: v for k, v in rd.items() if k != "tokens_per_s"},
    }
    del staging, staged, layers, tiers
    torch.cuda.empty_cache()
    return out


def bench_model_decode(torch, dev, *, new_tokens: int = 32, prompt: int = 8192):
    """Decode through a transformers model wrapped with
    ``wrap_with_halo(HALOConfig(chunked=True))``: a randomly initialised
    Qwen2-architecture model with Llama-3-8B attention shapes (hidden 4096,
    32/8 heads, head dim 128; 4 layers, MLP width 1024, bf16) prefilled with
    an 8192-token prompt in 2048-token slices, then ``new_tokens`` greedy
    steps; the cold tier (chunks of 1024 rows beyond the 512-row recent
    window) lives in pinned host memory and every decode step attends all
    of it (the lossless Path-D cache).  Beside it: the same weights
    unwrapped, decoding with SDPA over a DynamicCache in HBM."""
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config

    from halo_amd import HALOConfig, prefill_then_generate, wrap_with_halo

    def cfg():
        return Qwen2Config(vocab_size=1024, hidden_size=4096, intermediate_size=1024, num_hidden_layers=4,
                           num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=16384,
                           rope_theta=500000.0, tie_word_embeddings=False, attn_implementation="sdpa")
    torch.manual_seed(0)
    ref = AutoModelForCausalLM.from_config(cfg()).to(dev, torch.bfloat16).eval()
    halo = AutoModelForCausalLM.from_config(cfg()).to(dev, torch.bfloat16).eval()
    halo.load_state_dict(ref.state_dict())
    wrap_with_halo(halo, HALOConfig(chunked=True, chunk_size=1024, recent_window=512, use_triton=True))
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(10, 1000, (1, prompt), generator=g).to(dev)
    route_env = {"in_place": {}, "streamed": {"HALO_TRITON_STREAMED": "1"},
                 "single_launch": {"HALO_TRITON_SINGLE_LAUNCH": "1"}}

    def set_route(name):
        for k in ("HALO_TRITON_STREAMED", "HALO_TRITON_SINGLE_LAUNCH"):
            os.environ.pop(k, None)
        os.environ.update(route_env[name])

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, r

    routes = {}
    with torch.no_grad():
        prefill_then_generate(halo, ids[:, :2048], prefill_chunk_tokens=1024, max_new_tokens=2)   # warm-up
        t_pre, _ = timed(lambda: prefill_then_generate(halo, ids, prefill_chunk_tokens=2048, max_new_tokens=0))
        for name in ("streamed", "single_launch", "in_place"):   # the cache's default route last
            set_route(name)
            prefill_then_generate(halo, ids[:, :4096], prefill_chunk_tokens=2048, max_new_tokens=2)
            t_all, res = timed(lambda: prefill_then_generate(halo, ids, prefill_chunk_tokens=2048,
                                                             max_new_tokens=new_tokens))
            routes[name] = (t_all - t_pre) / new_tokens * 1e3
            log(f"model decode, route {name}: {routes[name]:.2f} ms per token")
        set_route("in_place")
        tele = res["cache_telemetry"]
        halo_ms = routes["in_place"]
        # the same weights, SDPA over a DynamicCache held in HBM
        out = ref(ids, use_cache=True, return_dict=True)
        cache, nxt = out.past_key_values, out.logits[:, -1:].argmax(-1)
        for _ in range(2):
            o = ref(nxt, past_key_values=cache, use_cache=True, return_dict=True)
            nxt = o.logits[:, -1:].argmax(-1)

        def sdpa_steps():
            nonlocal nxt
            for _ in range(new_tokens):
                o = ref(nxt, past_key_values=cache, use_cache=True, return_dict=True)
                nxt = o.logits[:, -1:].argmax(-1)
        t_ref, _ = timed(sdpa_steps)
    ref_ms = t_ref / new_tokens * 1e3
    cold_bytes = int(tele.get("cold_positions_per_layer_max", 0)) * 8 * 128 * 2 * 2 * 4   # K+V, 4 layers
    out = {
        "workload": "transformers Qwen2-architecture model (random init), Llama-3-8B attention shapes (32/8 heads, "
                    "d128), 4 layers, bf16, 8192-token prompt prefilled in 2048-token slices, then greedy decode "
                    "through wrap_with_halo(chunked=True): chunk 1024, recent window 512, cold chunks in pinned host "
                    "memory attended every step (read in place by the decode launch; the reference's streamed and "
                    "single-launch routes beside it)",
        "decode_ms_per_token": halo_ms, "decode_tokens_per_s": 1e3 / halo_ms,
        "decode_ms_per_token_by_route": routes,
        "prefill_ms": t_pre * 1e3, "sdpa_dynamic_cache_ms_per_token": ref_ms,
        "cold_bytes_per_token_over_link": cold_bytes,
        "telemetry": {k: (v if isinstance(v, (int, float, bool, str)) else str(v)) for k, v in tele.items()},
    }
    del ref, halo, cache
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode steps of the headline")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--rho", type=float, default=0.98, help="per-step correlation of the query trajectory")
    ap.add_argument("--slots", type=int, default=12, help="HBM staging slots per layer (of the 24 cold chunks)")
    ap.add_argument("--keep", type=int, default=6, help="best-scoring chunks per layer the cache stages")
    ap.add_argument("--max-inflight", type=int, default=16, help="host-to-device chunk copies in flight at once")
    ap.add_argument("--write-allocate", action="store_true",
                    help="headline cache with write-allocate (a missed chunk read in place also fills a slot)")
    ap.add_argument("--segments", type=int, default=4, help="graphs per step (layer segments) of the headline")
    ap.add_argument("--copy-streams", type=int, choices=[1, 2], default=1,
                    help="copy streams the staging fills alternate between")
    ap.add_argument("--fill-mode", choices=["kernel", "dma"], default="dma",
                    help="staging fills as copy kernels reading pinned memory in place, or hipMemcpyAsync")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the drift / no-staging comparison legs")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--split", type=int, default=None, help="rows per attention work item (default: planner)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the prefill (MFMA), ragged-batch and KIVI measurements")
    ap.add_argument("--only", choices=["c2", "c3", "c4", "c4host", "c5", "dropin", "model", "long", "peaks"], default=None,
                    help="run one leg alone (C2 kernel level, chunked prefill, ragged batch, KIVI, drop-in) and print its reading")
    ap.add_argument("--unfused", action="store_true",
                    help="kernel-level leg: select with the standalone scorer kernel instead of in the attention kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not run (how the path shards across "
              f"GPUs is designed, not measured, in this build)", file=sys.stderr)
        return 2

    import torch

    from halo_amd import _native
    from halo_amd.staging import ColdStaging
    from halo_amd.tiered import TieredDecodeLayer

    _native.lib()
    dev = torch.device("cuda:0")
    L, H, H_kv, D, T, chunk, n_hot, top_k = args.layers, 32, 8, 128, 32768, 1024, 8, 4
    if args.only is not None:
        def dropin():
            lays, q_, _ = make_layers(torch, L=L, H=H, H_kv=H_kv, D=D, T=T, chunk=chunk, n_hot=n_hot, top_k=top_k,
                                      n_planted=4, sigma=8.0, dev=dev, seed=1)
            return bench_dropin_c2(torch, dev, lays, q_, top_k=top_k, steps=max(1, args.steps))
        def c2():
            lays, q_, _ = make_layers(torch, L=L, H=H, H_kv=H_kv, D=D, T=T, chunk=chunk, n_hot=n_hot, top_k=top_k,
                                      n_planted=4, sigma=8.0, dev=dev, seed=1, split=args.split,
                                      fused=not args.unfused)
            a, _ = kernel_level_c2(torch, lays, q_, scale=1.0 / math.sqrt(D), reps=max(1, args.steps),
                                   with_scorer=False)
            return {"workload": "C2 kernel level: 32 layers, all chunks in HBM, attention with in-kernel "
                                "selection + merge per layer, one graph", "us_per_layer": a * 1e3}
        leg = {"c2": c2,
               "c4host": lambda: bench_ragged_c4_host(torch, dev, steps=max(1, args.steps)),
               "model": lambda: bench_model_decode(torch, dev),
               "long": lambda: bench_long_context(torch, dev, steps=max(1, args.steps)),
               "c3": lambda: bench_prefill_c3(torch, dev, reps=max(1, args.steps)),
               "c4": lambda: bench_ragged_c4(torch, dev, steps=max(1, args.steps)),
               "c5": lambda: bench_kivi_c5(torch, dev, steps=max(1, args.steps)),
               "dropin": dropin,
               "peaks": lambda: bench_measured_peaks(torch, dev)}[args.only]
        print(json.dumps({"leg": args.only, **leg()}), flush=True)
        return 0
    n_cold = T // chunk - n_hot
    scale = 1.0 / math.sqrt(D)
    log(f"building {L} layers of K/V ({L * 2 * H_kv * T * D * 2 / 2**30:.1f} GiB)")
    layers, qs, kvs = make_layers(torch, L=L, H=H, H_kv=H_kv, D=D, T=T, chunk=chunk, n_hot=n_hot, top_k=top_k,
                                  n_planted=4, sigma=8.0, dev=dev, seed=1, split=args.split,
                                  fused=not args.unfused)
    # algorithmic bytes of one layer's attention launch: K+V rows of hot +
    # selected chunks, q, out and lse, plus the cold chunks' mean keys it scores
    rows = layers[0].attended_rows
    score_bytes = n_cold * H_kv * D * 2
    attn_bytes = rows * H_kv * D * 2 * 2 + 2 * H * D * 2 + H * 4 + score_bytes
    step_bytes = L * attn_bytes

    # ---------------------------------------------------------------- headline
    log("cold tier: copying 24 chunks per layer to pinned host memory")
    tiers = host_tier(torch, layers)
    staged = [TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=lay.hot, cold=tiers[li],
                                top_k=top_k, device=dev, cold_kmean=lay.kmean, split=args.split)
              for li, lay in enumerate(layers)]
    staging = ColdStaging(staged, n_slots=args.slots, keep=args.keep, max_inflight=args.max_inflight,
                          write_allocate=args.write_allocate, fill_mode=args.fill_mode,
                          copy_streams=args.copy_streams)
    n_traj = args.warmup + args.steps
    qtraj = query_trajectory(torch, dev, steps=n_traj, L=L, H=H, D=D, rho=args.rho, seed=11)
    head = refetch_run(torch, staged, staging, qtraj, warmup=args.warmup, steps=args.steps, scale=scale,
                       label=f"staged, rho {args.rho}", warm_fills=10 ** 6, segments=args.segments)
    dt = head["ms_per_step"] * 1e-3

    # ------------------------------------------------- kernel-level (all HBM)
    attn_avg, score_avg = kernel_level_c2(torch, layers, qs, scale=scale, reps=50)
    achieved = attn_bytes / (attn_avg * 1e-3) / 1e9
    log(f"kernel-level (all HBM): attention launch avg {attn_avg * 1e3:.2f} us ({achieved:.0f} GB/s), "
        f"{1.0 / (attn_avg * 1e-3 * L):.0f} tokens/s; standalone scorer {score_avg * 1e3:.2f} us")

    traffic = None
    tf = os.path.join(ROOT, "profiles", "decode_attn_c2_traffic.json")
    if os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get("bytes_per_launch")
        except Exception:
            traffic = None

    result = {
        "metric": METRIC,
        "value": 1.0 / dt,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) k/v, 4 planted key channels sigma 8, AR(1) query drift rho "
                f"{args.rho}, random init)",
        "config": {
            "workload": "Llama-3-8B-shaped GQA decode, 32 layers looped, batch 1, 32/8 heads, d128, 32768 ctx in "
                        "32x1024 chunks, 8 hot chunks in HBM + top-4 of 24 cold chunks in pinned host memory "
                        "selected per layer per step by mean-key score, refetched through an HBM staging cache",
            "layers": L, "batch": 1, "q_heads": H, "kv_heads": H_kv, "head_dim": D, "ctx": T,
            "chunk": chunk, "hot_chunks": n_hot, "cold_chunks": n_cold, "top_k": top_k,
            "query_drift_rho": args.rho, "staging_slots_per_layer": args.slots, "staging_keep": staging.keep,
            "staging_bytes": staging.slot_bytes, "max_fills_in_flight": args.max_inflight,
            "write_allocate": staging.write_allocate, "segments": args.segments, "fill_mode": args.fill_mode,
            "copy_streams": args.copy_streams,
            "hbm_resident_fraction": (n_hot + args.slots) / (n_hot + n_cold),
            "launch": "per step: query copy, fill commits, hip graph of 32 x (attention kernel with in-kernel "
                      "top-k selection + merge kernel), score read-back, staging policy",
        },
        "hbm_gbps_end_to_end": step_bytes / dt / 1e9,
        "hbm_frac_end_to_end": step_bytes / dt / 1e9 / HBM_PEAK_GBPS,
        "hbm_bytes_per_step": step_bytes,
        "refetch": head,
        "roofline": {
            "bound": "hbm",
            "kernel": "halo_decode_attn_tiered (decode_attn_kernel<bf16,128,4,4> + decode_merge_kernel<128,4>), "
                      "one 32k-context decode layer with every selected chunk in HBM (kernel level)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "bytes_per_launch": attn_bytes,
            "avg_launch_us": attn_avg * 1e3,
            "kernel_level_tokens_per_s": 1.0 / (attn_avg * 1e-3 * L),
            "standalone_scorer_avg_us": score_avg * 1e3,
        },
    }
    if not args.no_sweep:
        sweep = {}
        for rho in (0.95, 0.99):
            staging.clear()   # the headline's cache and fill mode
            qt = query_trajectory(torch, dev, steps=20 + 100, L=L, H=H, D=D, rho=rho, seed=12)
            sweep[f"rho_{rho}"] = refetch_run(torch, staged, staging, qt, warmup=20, steps=100, scale=scale,
                                              label=f"staged, rho {rho}", warm_fills=10 ** 6,
                                              segments=args.segments)
        # smaller and larger caches (4, 6 and 16 slots per layer) on the headline trajectory
        for n_sl in (4, 6, 16):
            other = ColdStaging(staged, n_slots=n_sl, keep=min(args.keep, n_sl), max_inflight=args.max_inflight,
                                fill_mode=args.fill_mode)
            rd = refetch_run(torch, staged, other, qtraj, warmup=args.warmup, steps=100, scale=scale,
                             label=f"staged, {n_sl} slots, rho {args.rho}", warm_fills=10 ** 6,
                             segments=args.segments)
            rd["hbm_resident_fraction"] = (n_hot + n_sl) / (n_hot + n_cold)
            sweep[f"slots_{n_sl}"] = rd
            del other
        # the headline cache with its fills on the other number of copy streams
        n_cs = 3 - args.copy_streams
        other = ColdStaging(staged, n_slots=args.slots, keep=args.keep, max_inflight=args.max_inflight,
                            write_allocate=args.write_allocate, fill_mode=args.fill_mode, copy_streams=n_cs)
        sweep[f"copy_streams_{n_cs}"] = refetch_run(torch, staged, other, qtraj, warmup=args.warmup, steps=100,
                                                    scale=scale, label=f"staged, {n_cs} copy stream(s), rho {args.rho}",
                                                    warm_fills=10 ** 6, segments=args.segments)
        del other
        # the headline cache with the other fill mechanism
        other_mode = "dma" if args.fill_mode == "kernel" else "kernel"
        other = ColdStaging(staged, n_slots=args.slots, keep=args.keep, max_inflight=args.max_inflight,
                            write_allocate=args.write_allocate, fill_mode=other_mode)
        sweep[f"{other_mode}_fills"] = refetch_run(torch, staged, other, qtraj, warmup=args.warmup, steps=100,
                                                   scale=scale, label=f"staged, {other_mode} fills, rho {args.rho}",
                                                   warm_fills=10 ** 6, segments=args.segments)
        del other
        # the headline cache toggled between write-allocate on and off
        other = ColdStaging(staged, n_slots=args.slots, keep=args.keep, max_inflight=args.max_inflight,
                            write_allocate=not args.write_allocate, fill_mode=args.fill_mode)
        key = "no_write_allocate" if args.write_allocate else "write_allocate"
        sweep[key] = refetch_run(torch, staged, other, qtraj, warmup=args.warmup, steps=100, scale=scale,
                                 label=f"staged, {key.replace('_', ' ')}, rho {args.rho}", warm_fills=10 ** 6,
                                 segments=args.segments)
        del other
        staging = ColdStaging(staged, n_slots=args.slots, keep=args.keep, max_inflight=args.max_inflight,
                              write_allocate=False)
        staging.clear()
        budget = staging.max_inflight
        staging.max_inflight = 0                # nothing staged: every selected chunk read over the host link
        sweep["no_staging"] = refetch_run(torch, staged, staging, qtraj, warmup=3, steps=20, scale=scale,
                                          label="no staging (in-place reads)", segments=args.segments)
        staging.max_inflight = budget
        result["refetch_sweep"] = sweep
    if not args.no_extra:
        extra = {}

        def leg(key, label, fn):
            # a leg that raises is recorded with its error; the line still prints
            log(label)
            try:
                extra[key] = fn()
            except Exception as e:  # noqa: BLE001 -- reported in the JSON line
                log(f"{label} failed: {type(e).__name__}: {e}")
                extra[key] = {"error": f"{type(e).__name__}: {e}"}
                torch.cuda.synchronize()
                torch.cuda.empty_cache()

        leg("prefill_c3", "prefill leg", lambda: bench_prefill_c3(torch, dev, reps=10))
        leg("ragged_c4", "ragged leg", lambda: bench_ragged_c4(torch, dev, steps=20))
        leg("dropin_c2", "drop-in API leg", lambda: bench_dropin_c2(torch, dev, layers, qs, top_k=top_k, steps=20))
        del staging, staged
        torch.cuda.empty_cache()
        leg("kivi_c5", "kivi leg", lambda: bench_kivi_c5(torch, dev, steps=20))
        leg("ragged_c4_host_tier", "ragged host-tier leg", lambda: bench_ragged_c4_host(torch, dev, steps=40))
        leg("model_decode", "model decode leg", lambda: bench_model_decode(torch, dev))
        leg("long_context_128k", "long-context leg", lambda: bench_long_context(torch, dev))
        leg("measured_peaks", "measured peaks", lambda: bench_measured_peaks(torch, dev))
        result["extra"] = extra
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(torch, kvs, qs, layers, chunk=chunk, n_hot=n_hot, top_k=top_k, L=L,
                                              budget_s=args.cpu_seconds)
    # Copy-kernel calibration for hardware byte counters: a 64 MiB
    # device-to-device copy (reads 64 MiB, writes 64 MiB) run under the same
    # profiler pass as the kernels above scales FETCH_SIZE / WRITE_SIZE.
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
