"""GPU parity of the HALOScorer kernels (closed-form score, sorted top-k
with the lower-index tie rule) and of the Path-D cache's attention against
the float64 closed form."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import scoring as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K,step", [(64, 10), (1000, 999), (40000, 100)])
def test_halo_score_matches_closed_form(dev, small_config, fake_attention, K, step):
    from halo_amd import HALOScorer
    attn = fake_attention(K)
    got = HALOScorer(small_config).score(attn.to(dev), step=step).cpu().numpy()
    c = small_config
    want = S.halo_score(attn.numpy(), step=step, alpha=c.score_alpha, beta=c.score_beta, gamma=c.score_gamma,
                        sink_tokens=c.sink_tokens, refresh_window=c.refresh_window)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-7)
    assert np.isfinite(got).all() and got.min() >= 0 and got.max() <= 1


def test_scorer_reference_expectations(dev, small_config, fake_attention):
    """tests/test_scorer.py:9-69 of the reference: shape/range, hot-set size,
    sinks always hot, recency monotone."""
    from halo_amd import HALOScorer
    sc = HALOScorer(small_config)
    s = sc.score(fake_attention(128).to(dev), step=0)
    assert sc.topk_hot(s).numel() == int(small_config.hot_ratio * 128)
    s64 = sc.score(fake_attention(64).to(dev), step=0)
    hot = set(sc.topk_hot(s64, ratio=0.5).tolist())
    assert all(p in hot for p in range(small_config.sink_tokens))
    assert torch.equal(sc.topk_hot(s64, ratio=1.0).cpu(), torch.arange(64))
    from halo_amd import HALOConfig
    rc = HALOScorer(HALOConfig(score_alpha=0.0, score_gamma=0.0, score_beta=1.0, refresh_window=8))
    r = rc.score(torch.zeros(32, device=dev), step=31)
    assert ((r[1:] - r[:-1]) >= -1e-6).all()


@pytest.mark.parametrize("K,k,kind", [(64, 16, "rand"), (5000, 700, "rand"), (70000, 17, "rand"),
                                      (1000, 100, "ties"), (4096, 4096, "rand"), (333, 1, "nan")])
def test_topk_sorted_bitexact(dev, K, k, kind):
    from halo_amd.scorer import topk_sorted
    rng = np.random.default_rng(K + k)
    x = rng.standard_normal(K).astype(np.float32)
    if kind == "ties":
        x = np.round(x * 2).astype(np.float32)          # heavy ties at the boundary
    if kind == "nan":
        x[::7] = np.nan                                  # NaN ranks as -inf
    got = topk_sorted(torch.from_numpy(x).to(dev), k).cpu().numpy()
    want = S.topk_indices(np.where(np.isnan(x), -np.inf, x), k)
    assert got.tolist() == want.tolist()


def test_predict_hot_size_and_order(dev, small_config, fake_attention):
    from halo_amd import HALORefetcher
    r = HALORefetcher(small_config, storage=None)
    score = fake_attention(64).to(dev)
    pred = r.predict_hot(layer=0, last_hot_indices=None, last_score=score)
    assert pred.numel() == int(small_config.hot_ratio * 64) + small_config.lookahead
    want = S.predict_hot(score.cpu().numpy(), hot_ratio=small_config.hot_ratio, lookahead=small_config.lookahead)
    assert pred.cpu().tolist() == want.tolist()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunked_cache_decode_and_prefill(dev, dtype):
    """Prefill rows through the warm-up, peel on the first decode step, then
    compute_attention over cold host chunks + recent GPU rows equals full
    attention over every cached row (decode: T_q = 1; chunked prefill of a
    new block of rows in bf16)."""
    from halo_amd import HALOCacheChunked
    rng = np.random.default_rng(5)
    B, H, H_kv, D, T0 = 1, 8, 2, 64, 700
    cache = HALOCacheChunked(chunk_size=128, recent_window=32)
    ks = rng.standard_normal((B, H_kv, T0 + 3, D)).astype(np.float32)
    vs = rng.standard_normal((B, H_kv, T0 + 3, D)).astype(np.float32)
    from oracle.inputs import round_to
    nm = "bfloat16" if dtype == torch.bfloat16 else "float32"
    ks, vs = round_to(ks, nm), round_to(vs, nm)
    kg = torch.from_numpy(ks).to(dev).to(dtype)
    vg = torch.from_numpy(vs).to(dev).to(dtype)
    cache.update(kg[:, :, :T0], vg[:, :, :T0], 0)
    for t in range(T0, T0 + 3):
        cache.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
    assert cache._mode == "chunked" and cache.get_seq_length(0) == T0 + 3
    q = round_to(rng.standard_normal((B, H, 1, D)).astype(np.float32), nm)
    out = cache.compute_attention(torch.from_numpy(q).to(dev).to(dtype), layer_idx=0)
    torch.cuda.synchronize()
    ro, _ = A.attention_f64(q[:, :, 0], ks, vs, scale=1 / math.sqrt(D))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert np.abs(out[:, :, 0].float().cpu().numpy() - ro).max() <= tol
    st = cache.last_stats
    assert st.cold_positions + st.hot_positions == T0 + 3 and st.used_lse_merge
    tel = cache.telemetry()
    assert tel["mode"] == "chunked" and tel["cold_positions_per_layer_max"] == st.cold_positions
    qp = round_to(rng.standard_normal((B, H, 20, D)).astype(np.float32), nm)
    outp = cache.compute_attention(torch.from_numpy(qp).to(dev).to(dtype), layer_idx=0)
    rp, _ = A.prefill_f64(qp, ks, vs, scale=1 / math.sqrt(D), q_start=T0 + 3 - 20)
    assert np.abs(outp.float().cpu().numpy() - rp).max() <= tol
