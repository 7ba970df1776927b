"""GPU parity of the Path-D cache (HALOCacheChunked) on the orders the
reference uses, against the float64 closed form:

* a peel immediately followed by attention, with no synchronisation and a
  busy compute stream (the reference's chunked-prefill order: update, then
  T_q > 1 attention, halo/chunked_prefill.py:99-191; decode likewise), so a
  cold-tier read that is not ordered after the peel's device-to-host copy
  reads stale host rows and fails;
* fp32 T_q > 1 (the decode kernel's fp32 path) and bf16 (MFMA prefill);
* scorer-driven placement (pages kept on the GPU out of position order,
  halo/kv_cache_chunked.py:416-457) with exact causal positions.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.inputs import round_to

pytestmark = pytest.mark.gpu

_NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _busy(dev, n: int = 24) -> None:
    """Queue a few ms of work on the current stream (no sync)."""
    a = torch.randn(4096, 4096, device=dev)
    for _ in range(n):
        a = a @ a
        a = a / a.abs().max()


def _rows(rng, shape, dtype):
    return round_to(rng.standard_normal(shape).astype(np.float32), _NAME[dtype])


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-5)])
def test_peel_then_attention_without_sync(dev, dtype, tol):
    """Warm-up rows, the transition peel, then a 512-row slice whose update
    peels again and whose T_q = 512 attention is issued right away; then one
    decode token, again with a peel and no synchronisation in between."""
    from halo_amd import HALOCacheChunked
    rng = np.random.default_rng(11)
    B, H, H_kv, D = 1, 8, 2, 128
    T0, S = 600, 512
    T = T0 + 1 + S + 1
    ks, vs = _rows(rng, (B, H_kv, T, D), dtype), _rows(rng, (B, H_kv, T, D), dtype)
    kg = torch.from_numpy(ks).to(dev).to(dtype)
    vg = torch.from_numpy(vs).to(dev).to(dtype)
    cache = HALOCacheChunked(chunk_size=256, recent_window=64)
    cache.update(kg[:, :, :T0], vg[:, :, :T0], 0)
    cache.update(kg[:, :, T0:T0 + 1], vg[:, :, T0:T0 + 1], 0)          # transition: peel to cold
    assert cache._mode == "chunked" and cache._cold[0].rows == T0 + 1 - 64
    torch.cuda.synchronize()
    # chunked-prefill order: busy stream, update (peels the slice), attention at once
    _busy(dev)
    cache.update(kg[:, :, T0 + 1:T0 + 1 + S], vg[:, :, T0 + 1:T0 + 1 + S], 0)
    qs = _rows(rng, (B, H, S, D), dtype)
    out = cache.compute_attention(torch.from_numpy(qs).to(dev).to(dtype), layer_idx=0)
    assert cache._cold[0].rows == T0 + 1 + S - 64
    want, _ = A.prefill_f64(qs, ks[:, :, :T0 + 1 + S], vs[:, :, :T0 + 1 + S], scale=1 / math.sqrt(D), q_start=T0 + 1)
    got = out.float().cpu().numpy()
    assert np.abs(got - want).max() <= tol
    # decode right after a peel on a busy stream
    cache2 = HALOCacheChunked(chunk_size=256, recent_window=64)
    cache2.update(kg[:, :, :T - 1], vg[:, :, :T - 1], 0)
    torch.cuda.synchronize()
    _busy(dev)
    cache2.update(kg[:, :, T - 1:], vg[:, :, T - 1:], 0)
    q1 = _rows(rng, (B, H, 1, D), dtype)
    out1, lse1 = cache2.compute_attention(torch.from_numpy(q1).to(dev).to(dtype), layer_idx=0, return_lse=True)
    w1, wl = A.attention_f64(q1[:, :, 0], ks, vs, scale=1 / math.sqrt(D))
    assert np.abs(out1[:, :, 0].float().cpu().numpy() - w1).max() <= tol
    assert np.abs(lse1[:, :, 0].cpu().numpy() - wl).max() <= (1e-5 if dtype == torch.float32 else 1e-2)


def test_prefill_rows_ragged_batch_fp32(dev):
    """fp32 T_q > 1 for B = 2 with per-row query starts through
    prefill_attention (decode-kernel fp32 path), LSE included."""
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention
    rng = np.random.default_rng(3)
    B, H, H_kv, D, T, T_q = 2, 4, 2, 64, 300, 37
    ks, vs = _rows(rng, (B, H_kv, T, D), torch.float32), _rows(rng, (B, H_kv, T, D), torch.float32)
    qs = _rows(rng, (B, H, T_q, D), torch.float32)
    k = torch.from_numpy(ks).to(dev)
    v = torch.from_numpy(vs).to(dev)
    chunks = [ChunkRef(k[:, :, a:a + 128], v[:, :, a:a + 128], a, True) for a in range(0, T, 128)]
    starts = torch.tensor([T - T_q, 100], dtype=torch.int64)
    out, lse = prefill_attention(torch.from_numpy(qs).to(dev), chunks, q_start=starts, return_lse=True)
    for b, s0 in enumerate(starts.tolist()):
        w, wl = A.prefill_f64(qs[b:b + 1], ks[b:b + 1], vs[b:b + 1], scale=1 / math.sqrt(D), q_start=s0)
        assert np.abs(out[b:b + 1].cpu().numpy() - w).max() <= 1e-5
        assert np.abs(lse[b:b + 1].cpu().numpy() - wl).max() <= 1e-5


def test_scorer_driven_placement_keeps_exact_positions(dev):
    """A ChunkScorer attached as the placement plug-in keeps its hot pages of
    the GPU rows on the GPU at each peel; the GPU and cold rows are then out
    of position order, and decode and T_q > 1 attention still equal full
    causal attention over every row."""
    from halo_amd import HALOCacheChunked
    from halo_amd.chunk_scorer import ChunkScorer, ChunkScorerConfig
    rng = np.random.default_rng(5)
    dtype = torch.bfloat16
    B, H, H_kv, D = 1, 8, 2, 128
    T0, steps = 700, 300
    T = T0 + steps
    ks, vs = _rows(rng, (B, H_kv, T, D), dtype), _rows(rng, (B, H_kv, T, D), dtype)
    kg = torch.from_numpy(ks).to(dev).to(dtype)
    vg = torch.from_numpy(vs).to(dev).to(dtype)
    cache = HALOCacheChunked(chunk_size=128, recent_window=32)
    cache._quest_scorer = ChunkScorer(ChunkScorerConfig(page_size=16, memory_ratio=4, min_pages_selected=2))
    cache.update(kg[:, :, :T0], vg[:, :, :T0], 0)
    qd = None
    for t in range(T0, T):
        cache.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
        qd = _rows(rng, (B, H, 1, D), dtype)
        out = cache.compute_attention(torch.from_numpy(qd).to(dev).to(dtype), layer_idx=0)
    pos = cache._gpu_pos[0]
    assert len(pos) > cache.recent_window and (np.diff(pos) != 1).any(), "placement kept no non-recent page"
    allpos = np.sort(np.concatenate([pos] + [c.pos[:c.n] for c in cache._cold[0].chunks]))
    assert np.array_equal(allpos, np.arange(T))
    w, _ = A.attention_f64(qd[:, :, 0], ks, vs, scale=1 / math.sqrt(D))
    assert np.abs(out[:, :, 0].float().cpu().numpy() - w).max() <= 2e-2
    # causal prefill over the shuffled tiers: the last 40 rows as queries
    qp = _rows(rng, (B, H, 40, D), dtype)
    outp = cache.compute_attention(torch.from_numpy(qp).to(dev).to(dtype), layer_idx=0, query_pos_offset=T - 40)
    wp, _ = A.prefill_f64(qp, ks, vs, scale=1 / math.sqrt(D), q_start=T - 40)
    assert np.abs(outp.float().cpu().numpy() - wp).max() <= 2e-2
    tel = cache.telemetry()
    assert tel["mode"] == "chunked" and tel["cold_layers"] == 1 and tel["chunked_used_lse_merge_any"]


def test_cold_chunk_means_on_device(dev):
    """Per-chunk mean keys accumulated at peel time equal the chunk's row
    means within one bf16 rounding."""
    from halo_amd import HALOCacheChunked
    rng = np.random.default_rng(9)
    ks = _rows(rng, (1, 2, 700, 64), torch.bfloat16)
    kg = torch.from_numpy(ks).to(dev).to(torch.bfloat16)
    cache = HALOCacheChunked(chunk_size=128, recent_window=32)
    cache.update(kg[:, :, :699], kg[:, :, :699], 0)
    cache.update(kg[:, :, 699:], kg[:, :, 699:], 0)
    got = cache.cold_chunk_means(0).float().cpu().numpy()
    n = cache._cold[0].rows
    for j, a in enumerate(range(0, n, 128)):
        want = ks[:, :, a:min(a + 128, n)].astype(np.float64).mean(axis=-2)
        assert np.abs(got[:, :, j] - want).max() <= 2.0 ** -7 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("route", ["in_place", "streamed", "single_launch"])
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-5)])
def test_decode_routes(dev, monkeypatch, route, dtype, tol):
    """The three decode routes (halo/kv_cache_chunked.py:610-700): cold
    chunks read in place by one launch (default), streamed through HBM
    staging buffers (use_triton + HALO_TRITON_STREAMED=1), staged whole then
    one launch (use_triton + HALO_TRITON_SINGLE_LAUNCH=1); each right after a
    peel on a busy stream, against the float64 closed form, with the
    route's telemetry."""
    from halo_amd import HALOCacheChunked
    monkeypatch.delenv("HALO_TRITON_STREAMED", raising=False)
    monkeypatch.delenv("HALO_TRITON_SINGLE_LAUNCH", raising=False)
    if route == "streamed":
        monkeypatch.setenv("HALO_TRITON_STREAMED", "1")
    if route == "single_launch":
        monkeypatch.setenv("HALO_TRITON_SINGLE_LAUNCH", "1")
        monkeypatch.setenv("HALO_TRITON_STREAMED", "1")   # single launch is checked first
    rng = np.random.default_rng(17)
    B, H, H_kv, D = 2, 8, 2, 128
    T = 1400
    ks, vs = _rows(rng, (B, H_kv, T, D), dtype), _rows(rng, (B, H_kv, T, D), dtype)
    kg = torch.from_numpy(ks).to(dev).to(dtype)
    vg = torch.from_numpy(vs).to(dev).to(dtype)
    cache = HALOCacheChunked(chunk_size=256, recent_window=64, use_triton=True)
    assert cache.decode_route() == route
    cache.update(kg[:, :, :T - 2], vg[:, :, :T - 2], 0)
    torch.cuda.synchronize()
    _busy(dev)
    esz = torch.tensor([], dtype=dtype).element_size()
    for t in (T - 2, T - 1):       # the transition peel, then a plain decode step
        cache.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
        q1 = _rows(rng, (B, H, 1, D), dtype)
        out, lse = cache.compute_attention(torch.from_numpy(q1).to(dev).to(dtype), layer_idx=0, return_lse=True)
        w, wl = A.attention_f64(q1[:, :, 0], ks[:, :, :t + 1], vs[:, :, :t + 1], scale=1 / math.sqrt(D))
        assert np.abs(out[:, :, 0].float().cpu().numpy() - w).max() <= tol, (route, t)
        assert np.abs(lse[:, :, 0].cpu().numpy() - wl).max() <= (1e-5 if dtype == torch.float32 else 1e-2)
        st = cache.last_stats
        cold_rows = cache._cold[0].rows
        assert st.cold_positions == cold_rows and st.hot_positions == t + 1 - cold_rows
        if route == "in_place":
            assert st.dma_bytes == 2 * cold_rows * B * H_kv * D * esz and st.peak_staging_bytes == 0
        elif route == "single_launch":
            assert st.n_chunks == 1 and not st.used_lse_merge
            assert st.dma_bytes >= 2 * cold_rows * B * H_kv * D * esz and st.peak_staging_bytes == st.dma_bytes
        else:
            assert st.dma_bytes >= 2 * cold_rows * B * H_kv * D * esz and st.peak_staging_bytes > 0
