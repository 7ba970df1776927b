"""Decode-attention throughput of the tiered-KV path on one MI355X.

Workload (default): Llama-3-8B-shaped GQA decode, bf16, batch 1, 32 query
heads / 8 KV heads, head dim 128, 32768 cached tokens in 32 chunks of 1024,
hot_ratio 0.25 (the last 8 chunks), 24 cold chunks of which the scorer
selects the top 4 per layer per step by mean-key dot product; keys carry 4
planted high-variance channels (sigma 8).  32 layers with distinct buffers
(4 GiB of K/V in HBM, far above the 256 MB last-level cache).  One step =
for every layer: the split-K attention kernel over the hot chunks and 4
selection slots (whose workgroups first score the 24 cold chunks' mean keys
and pick the top 4 in-kernel), then the split-K merge kernel; the 64
launches are replayed from one HIP graph.  Inputs are resident in HBM when the timed region starts (the
cold chunks' HBM copies stand for their refetched state); the rate with the
top-4 refetched over PCIe every step is measured separately and reported as
``pcie_inclusive``.

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


def pcie_inclusive(torch, layers, qs, *, steps, scale):
    """Every selected cold chunk refetched host->device every step: cold
    chunks live in pinned host memory, the scorer's choice is read back, the
    4 chunks are copied with hipMemcpyAsync on the copy stream into HBM
    staging slots while the hot chunks are attended, then merged."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    from halo_amd.memory_tier import copy_stream
    from halo_amd.triton_chunked import init_acc

    dev = qs[0].device
    L = len(layers)
    H, D = layers[0].H, layers[0].D
    cs = copy_stream(dev)
    compute = torch.cuda.current_stream()
    host = []
    for lay in layers:
        hk = [c.k.cpu().pin_memory() for c in lay.cold]
        hv = [c.v.cpu().pin_memory() for c in lay.cold]
        host.append((hk, hv))
    shape = tuple(layers[0].cold[0].k.shape)
    slots = [(torch.empty(shape, device=dev, dtype=torch.bfloat16), torch.empty(shape, device=dev, dtype=torch.bfloat16))
             for _ in range(layers[0].top_k)]
    hot_plans = [build_plan(B=1, H=H, H_kv=lay.H_kv, D=D, dtype=torch.bfloat16, chunks=lay.hot, device=dev)
                 for lay in layers]
    slot_plans = [build_plan(B=1, H=H, H_kv=layers[0].H_kv, D=D, dtype=torch.bfloat16,
                             chunks=[ChunkRef(sk, sv, 0, False) for (sk, sv) in slots], device=dev)]
    out = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
    ev_copy = torch.cuda.Event()
    nbytes = 0

    def step():
        nonlocal nbytes
        for li, lay in enumerate(layers):
            q = qs[li]
            lay.select(q)
            ids = lay.idx[0].cpu().tolist()
            cs.wait_stream(compute)
            with torch.cuda.stream(cs):
                for s, c in enumerate(ids):
                    slots[s][0].copy_(host[li][0][c], non_blocking=True)
                    slots[s][1].copy_(host[li][1][c], non_blocking=True)
                    nbytes += 2 * host[li][0][c].numel() * 2
                ev_copy.record(cs)
            m, l_, o = init_acc(B=1, H=H, D_v=D, device=dev)
            launch(hot_plans[li], q, scale=scale, m=m, l=l_, o=o, acc_mode=2)
            compute.wait_event(ev_copy)
            launch(slot_plans[0], q, scale=scale, m=m, l=l_, o=o, acc_mode=1, out=out)

    step()
    torch.cuda.synchronize()
    nbytes = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    # pinned H2D peak on this box: one 64 MiB copy stream-ordered, repeated
    big_h = torch.empty(64 << 20, dtype=torch.uint8).pin_memory()
    big_d = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    for _ in range(2):
        big_d.copy_(big_h, non_blocking=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(10):
        big_d.copy_(big_h, non_blocking=True)
    torch.cuda.synchronize()
    h2d_peak = 10 * (64 << 20) / (time.perf_counter() - t1) / 1e9
    res = {
        "tokens_per_s": 1.0 / dt,
        "ms_per_step": dt * 1e3,
        "refetch_bytes_per_step": nbytes // steps,
        "link_gbps": nbytes / steps / dt / 1e9,
        "h2d_pinned_peak_gbps": h2d_peak,
        "policy": "every layer's top-4 refetched from pinned host memory every step (no staging-cache hits)",
        "refetch": "host reads the selection, hipMemcpyAsync of the 4 chunks on a copy stream, hot chunks attended meanwhile",
    }
    res["in_kernel"] = zero_copy_refetch(torch, layers, qs, host, steps=steps, scale=scale)
    return res


def zero_copy_refetch(torch, layers, qs, host, *, steps, scale):
    """The same worst-case policy with the refetch inside the attention
    launch: the cold catalog points at the pinned host chunks (their
    device-visible addresses), so the selection workgroups stream the chosen
    chunks over the host link while the hot workgroups read HBM; no host
    round trip, one HIP graph for the 32-layer step."""
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer

    dev = qs[0].device
    L = len(layers)
    zl = []
    for li, lay in enumerate(layers):
        cold = [ChunkRef(host[li][0][j], host[li][1][j], c.chunk_start, c.causal) for j, c in enumerate(lay.cold)]
        zl.append(TieredDecodeLayer(B=1, H=lay.H, H_kv=lay.H_kv, D=lay.D, dtype=lay.dtype, hot=lay.hot, cold=cold,
                                    top_k=lay.top_k, device=dev, cold_kmean=lay.kmean))
    outs = [torch.empty((1, lay.H, lay.D), device=dev, dtype=lay.dtype) for lay in layers]

    def step():
        for li in range(L):
            zl[li].step(qs[li], scale=scale, out=outs[li])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(steps):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    dt = e0.elapsed_time(e1) / 1e3 / steps
    per_chunk = 2 * host[0][0][0].numel() * host[0][0][0].element_size()
    nbytes = L * layers[0].top_k * per_chunk
    return {
        "tokens_per_s": 1.0 / dt,
        "ms_per_step": dt * 1e3,
        "refetch_bytes_per_step": nbytes,
        "link_gbps": nbytes / dt / 1e9,
        "refetch": "selected cold chunks read in place from pinned host memory by the attention kernel (no host sync)",
    }


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pcie", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--split", type=int, default=None, help="rows per attention work item (default: planner)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the prefill (MFMA) and KIVI cold-tier measurements")
    ap.add_argument("--unfused", action="store_true",
                    help="select with the standalone scorer kernel instead of in the attention kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not run (how the path shards across "
              f"GPUs is designed, not measured, in this build)", file=sys.stderr)
        return 2

    import torch

    from halo_amd import _native

    _native.lib()
    dev = torch.device("cuda:0")
    L, H, H_kv, D, T, chunk, n_hot, top_k = args.layers, 32, 8, 128, 32768, 1024, 8, 4
    scale = 1.0 / math.sqrt(D)
    log(f"building {L} layers of K/V ({L * 2 * H_kv * T * D * 2 / 2**30:.1f} GiB)")
    layers, qs, kvs = make_layers(torch, L=L, H=H, H_kv=H_kv, D=D, T=T, chunk=chunk, n_hot=n_hot, top_k=top_k,
                                  n_planted=4, sigma=8.0, dev=dev, seed=1, split=args.split,
                                  fused=not args.unfused)
    outs = [torch.empty((1, H, D), device=dev, dtype=torch.bfloat16) for _ in range(L)]
    lses = [torch.empty((1, H), device=dev, dtype=torch.float32) for _ in range(L)]

    def step():
        for li in range(L):
            layers[li].step(qs[li], scale=scale, out=outs[li], lse=lses[li])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    log("graph captured; warmup")
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    log(f"timed {args.steps} steps: {dt * 1e3:.3f} ms/step")

    # Per-kernel durations with HIP events on the launch stream.  Host-side
    # launch latency would inflate per-launch event pairs, so the attention
    # launches (split-K kernel + merge kernel) and the scorer launches are each
    # captured in a graph of their own and timed over whole replays on the
    # capture stream.
    def capture(fn):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            fn()
            torch.cuda.synchronize()
            with torch.cuda.graph(gr, stream=s):
                fn()
        torch.cuda.synchronize()
        return gr

    # one layer's launch pair: attention with in-kernel selection + merge
    g_attn = capture(lambda: [layers[li].step(qs[li], scale=scale, out=outs[li], lse=lses[li]) for li in range(L)])
    # the standalone scorer kernel (plug-in API path), for reference
    g_score = capture(lambda: [layers[li].select(qs[li]) for li in range(L)])

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

    reps = max(5, min(args.steps, 50))
    attn_avg = time_graph(g_attn, reps)
    score_avg = time_graph(g_score, reps)
    rows = layers[0].attended_rows
    # algorithmic bytes of one layer's launch: K+V rows of hot + selected
    # chunks, q, out and lse, plus the cold chunks' mean keys it scores
    score_bytes = (T // chunk - n_hot) * H_kv * D * 2
    attn_bytes = rows * H_kv * D * 2 * 2 + 2 * H * D * 2 + H * 4 + (score_bytes if layers[0].fused else 0)
    achieved = attn_bytes / (attn_avg * 1e-3) / 1e9
    step_bytes = L * (attn_bytes if layers[0].fused else attn_bytes + score_bytes + H * D * 2)
    log(f"attention launch avg {attn_avg * 1e3:.2f} us ({achieved:.0f} GB/s), "
        f"standalone scorer {score_avg * 1e3:.2f} us")

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
        "data": "synthetic (N(0,1) q/k/v, 4 planted key channels sigma 8, random init)",
        "config": {
            "workload": "Llama-3-8B-shaped GQA decode, 32 layers looped, batch 1, 32/8 heads, d128, "
                        "32768 ctx in 32x1024 chunks, 8 hot + top-4 of 24 cold by mean-key score",
            "layers": L, "batch": 1, "q_heads": H, "kv_heads": H_kv, "head_dim": D, "ctx": T,
            "chunk": chunk, "hot_chunks": n_hot, "top_k": top_k,
            "launch": ("hip graph; per layer: attention kernel with in-kernel top-k selection + merge kernel"
                       if layers[0].fused else "hip graph; per layer: scorer + attention + merge kernels"),
            "split_rows": int(layers[0].plan.work_host[-1, 3] - layers[0].plan.work_host[-1, 2]),
            "selection_split_rows": int(layers[0].plan.work_host[0, 3] - layers[0].plan.work_host[0, 2]),
            "work_items": layers[0].plan.n_work,
        },
        "hbm_gbps_end_to_end": step_bytes / dt / 1e9,
        "hbm_bytes_per_step": step_bytes,
        "roofline": {
            "bound": "hbm",
            "kernel": "halo_decode_attn_tiered (decode_attn_kernel<bf16,128,4,4> + decode_merge_kernel<128,4>)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "bytes_per_launch": attn_bytes,
            "avg_launch_us": attn_avg * 1e3,
            "standalone_scorer_avg_us": score_avg * 1e3,
        },
    }
    if not args.no_extra:
        extra = {}
        log("prefill leg")
        extra["prefill_c3"] = bench_prefill_c3(torch, dev, reps=max(3, min(args.steps, 10)))
        log("ragged leg")
        extra["ragged_c4"] = bench_ragged_c4(torch, dev, steps=max(3, min(args.steps, 20)))
        log("kivi leg")
        del g, g_attn, g_score
        torch.cuda.empty_cache()
        extra["kivi_c5"] = bench_kivi_c5(torch, dev, steps=max(3, min(args.steps, 20)))
        result["extra"] = extra
    if not args.no_pcie:
        log("pcie-inclusive leg")
        result["pcie_inclusive"] = pcie_inclusive(torch, layers, qs, steps=max(3, min(args.steps, 10)), scale=scale)
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
