"""GPU parity of the Quest bounding-box scorer against the oracle:
page minima / maxima bit-exact (NaN channels included), bounds bit-exact in
the fixed summation order, page scores and top-k order exact; the scorer
adapter's counters as the reference test drives them
(tests/test_quest_path_d.py:147-188) and the scorer driving placement in the
Path-D cache."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import scoring as S
from oracle.inputs import round_to

pytestmark = pytest.mark.gpu

_NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _t(x: np.ndarray, dev, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(dtype)


def _rows(rng, shape, dtype):
    return round_to(rng.standard_normal(shape).astype(np.float32), _NAME[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_page_minmax_bit_exact(dev, dtype):
    from halo_amd.quest_scorer import page_minmax
    rng = np.random.default_rng(1)
    B, H_kv, T, D = 2, 3, 16 * 9 + 5, 128
    K = _rows(rng, (B, H_kv, T, D), dtype)
    K[1, 2, 37, 100] = np.nan
    kt = _t(K, dev, dtype)
    kmin, kmax = page_minmax(kt, 16)
    omin, omax = S.page_minmax(K, 16)
    assert np.array_equal(kmin.float().cpu().numpy(), omin, equal_nan=True)
    assert np.array_equal(kmax.float().cpu().numpy(), omax, equal_nan=True)
    assert torch.isnan(kmin[1, 2, 2, 100]) and torch.isnan(kmax[1, 2, 2, 100])
    # appending pages from row0 into an existing buffer, from a strided view
    wide = torch.zeros((B, H_kv, T, 2 * D), device=dev, dtype=dtype)
    wide[..., :D] = kt
    view = wide[..., :D]
    a_min = torch.full((B, H_kv, 9, D), 7.0, device=dev, dtype=dtype)
    a_max = torch.full_like(a_min, 7.0)
    page_minmax(view, 16, row0=48, n_pages=5, kmin=a_min, kmax=a_max, page_offset=3)
    assert torch.equal(a_min[:, :, :3], torch.full_like(a_min[:, :, :3], 7.0))
    assert np.array_equal(a_min[:, :, 3:8].float().cpu().numpy(), omin[:, :, 3:8], equal_nan=True)
    assert np.array_equal(a_max[:, :, 3:8].float().cpu().numpy(), omax[:, :, 3:8], equal_nan=True)


@pytest.mark.parametrize("dtype,H,H_kv,T_q,D,per_row", [
    (torch.bfloat16, 32, 8, 1, 128, False),
    (torch.float16, 8, 2, 3, 64, False),
    (torch.float32, 4, 4, 2, 64, False),
    (torch.bfloat16, 28, 4, 5, 128, True),
])
def test_bounds_and_topk_bit_exact(dev, dtype, H, H_kv, T_q, D, per_row):
    from halo_amd.quest_scorer import page_minmax, quest_score_topk
    rng = np.random.default_rng(2)
    B, P, page = 2, 150, 16
    K = _rows(rng, (B, H_kv, P * page, D), dtype)
    q = _rows(rng, (B, H, T_q, D), dtype)
    kmin, kmax = page_minmax(_t(K, dev, dtype), page)
    k = 37
    idx, dots, scores = quest_score_topk(_t(q, dev, dtype), kmin, kmax, k, per_row=per_row,
                                         want_dots=True, want_scores=True)
    omin, omax = S.page_minmax(K, page)
    want = S.quest_scores(q, omin, omax, _NAME[dtype])
    assert np.array_equal(dots.cpu().numpy(), want)
    rows = [np.s_[b:b + 1] for b in range(B)] if per_row else [np.s_[:]]
    for s, r in enumerate(rows):
        ps = S.quest_page_scores(q[r], omin[r], omax[r], _NAME[dtype])
        assert np.array_equal(scores[s].cpu().numpy(), ps)
        order = sorted(range(P), key=lambda p: (-float(ps[p]), p))[:k]
        assert idx[s].cpu().tolist() == order


def test_topk_ties_nan_and_large_page_counts(dev):
    """Equal bounds rank by lower page index, NaN bounds rank last, and the
    full 8192-page table ranks in descending order."""
    from halo_amd.quest_scorer import page_minmax, quest_score_topk
    rng = np.random.default_rng(3)
    dtype = torch.bfloat16
    K = _rows(rng, (1, 2, 64 * 16, 64), dtype)
    K[:, :, 5 * 16:6 * 16] = K[:, :, 9 * 16:10 * 16]   # pages 5 and 9 tie
    K[:, :, 3 * 16, 0] = np.nan                          # page 3 is NaN
    q = _rows(rng, (1, 4, 1, 64), dtype)
    kmin, kmax = page_minmax(_t(K, dev, dtype), 16)
    idx, _, scores = quest_score_topk(_t(q, dev, dtype), kmin, kmax, 64, want_scores=True)
    got = idx[0].cpu().tolist()
    assert got[-1] == 3 and scores[0, 3].item() == -math.inf
    assert got.index(5) + 1 == got.index(9)
    omin, omax = S.page_minmax(K, 16)
    assert got == S.quest_select(q, omin, omax, memory_ratio=1.0, min_pages_selected=1, dtype="bfloat16").tolist()
    # 8192 pages of 16 rows: rank order against the oracle's page scores
    P = 8192
    K = _rows(rng, (1, 1, P * 16, 64), dtype)
    q = _rows(rng, (1, 1, 1, 64), dtype)
    kmin, kmax = page_minmax(_t(K, dev, dtype), 16)
    idx, _, scores = quest_score_topk(_t(q, dev, dtype), kmin, kmax, 2048, want_scores=True)
    omin, omax = S.page_minmax(K, 16)
    ps = S.quest_page_scores(q, omin, omax, "bfloat16")
    assert np.array_equal(scores[0].cpu().numpy(), ps)
    order = np.lexsort((np.arange(P), -ps.astype(np.float64)))[:2048]
    assert idx[0].cpu().numpy().tolist() == order.tolist()


def test_adapter_counters_as_the_reference_test(dev):
    """tests/test_quest_path_d.py:147-188 at D = 16 (the kernels need
    D % 16 == 0): counters, shapes, bounds within 1e-5 of the torch
    recipe, and the K_total budget."""
    from halo_amd.quest_scorer import QuestPathDConfig, QuestScorer
    cfg = QuestPathDConfig(page_size=4, memory_ratio=2.0, min_pages_selected=1)
    adapter = QuestScorer(cfg)
    torch.manual_seed(7)
    B, H_kv, T, D = 1, 2, 16, 16
    K = torch.randn(B, H_kv, T, D)
    adapter.observe_keys(layer_idx=0, K_full=K.to(dev))
    assert adapter.observe_calls == 1
    assert adapter._num_full_pages[0] == 4
    q = torch.randn(B, H_kv, 1, D)
    scores = adapter.score_pages(0, q.to(dev))
    assert scores is not None and scores.shape == (B, H_kv, 1, 4)
    assert adapter.score_calls == 1
    kp = K.view(B, H_kv, 4, 4, D)
    expected = torch.maximum(q.unsqueeze(-2) * kp.amin(dim=-2).unsqueeze(-3),
                             q.unsqueeze(-2) * kp.amax(dim=-2).unsqueeze(-3)).sum(dim=-1)
    assert torch.allclose(scores.cpu(), expected, atol=1e-5)
    topk = adapter.select_hot_pages(0, q.to(dev))
    K_total = max(cfg.min_pages_selected, int((4 + cfg.memory_ratio - 1) // cfg.memory_ratio))
    assert topk.shape == (K_total,) and topk.device.type == "cpu"
    assert adapter.cumulative_hot_pages == K_total
    assert topk.tolist() == torch.topk(expected.amax(dim=(0, 1, 2)), K_total).indices.tolist()
    # incremental: only the new pages are computed, earlier ones kept
    adapter.observe_keys(0, torch.cat([K, torch.randn(B, H_kv, 9, D)], dim=2).to(dev))
    assert adapter._num_full_pages[0] == 6 and adapter.observe_calls == 2
    kmin, kmax = adapter.bounds(0)
    assert torch.equal(kmin[:, :, :4].cpu(), kp.amin(dim=-2))


def test_quest_scorer_drives_placement_in_the_cache(dev):
    """The reference's integration order (tests/test_quest_path_d.py:191-260):
    update calls observe_keys, compute_attention records the query, the next
    update's peel consults select_hot_pages; the kept pages leave the GPU
    rows out of position order and attention still equals full causal
    attention."""
    from halo_amd import HALOCacheChunked
    from halo_amd.quest_scorer import QuestPathDConfig, QuestScorer
    rng = np.random.default_rng(4)
    dtype = torch.bfloat16
    B, H, H_kv, D = 1, 8, 2, 128
    T0, steps = 600, 200
    T = T0 + steps
    ks, vs = _rows(rng, (B, H_kv, T, D), dtype), _rows(rng, (B, H_kv, T, D), dtype)
    kg, vg = _t(ks, dev, dtype), _t(vs, dev, dtype)
    cache = HALOCacheChunked(chunk_size=128, recent_window=32)
    adapter = QuestScorer(QuestPathDConfig(page_size=16, memory_ratio=4.0, min_pages_selected=2))
    cache._quest_scorer = adapter
    cache.update(kg[:, :, :T0], vg[:, :, :T0], 0)
    assert adapter.observe_calls >= 1
    out = qd = None
    for t in range(T0, T):
        cache.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
        qd = _rows(rng, (B, H, 1, D), dtype)
        out = cache.compute_attention(_t(qd, dev, dtype), layer_idx=0)
    assert 0 in cache._last_query
    assert adapter.score_calls >= 1 and adapter.cumulative_hot_pages >= 1
    pos = cache._gpu_pos[0]
    assert len(pos) > cache.recent_window and (np.diff(pos) != 1).any(), "placement kept no non-recent page"
    allpos = np.sort(np.concatenate([pos] + [c.pos[:c.n] for c in cache._cold[0].chunks]))
    assert np.array_equal(allpos, np.arange(T))
    w, _ = A.attention_f64(qd[:, :, 0], ks, vs, scale=1 / math.sqrt(D))
    assert np.abs(out[:, :, 0].float().cpu().numpy() - w).max() <= 2e-2
