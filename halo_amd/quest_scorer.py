"""Quest bounding-box page scorer on the GPU.

Reference: ``_QuestScorerAdapter`` and ``QuestPathDConfig``
(baselines/quest_path_d.py:40-205) and ``wrap_with_quest_path_d``
(:208-258).  The adapter keeps per-page channel-wise key minima and maxima,
bounds each page's attention score by
``sum_d max(q_d * K_min_d, q_d * K_max_d)`` and keeps the top
``max(min_pages_selected, ceil(P / memory_ratio))`` pages on the GPU when
the cache peels (the placement plug-in protocol ``observe_keys`` /
``select_hot_pages``, halo/kv_cache_chunked.py:306-311, :416-457).
Differences:
  * the minima and maxima of a page are computed once, when it fills, by
    ``halo_page_minmax``, into a buffer that grows by doubling (the
    reference concatenates per call);
  * bounds, the max over (b, h_kv, t_q) and the top-k are one
    ``halo_quest_score_topk`` call; the bounds are summed in the library's
    fixed order (the reference's order is torch's);
  * ties are broken by lower page index and NaN bounds rank last (torch.topk
    leaves ties undefined and ranks NaN first).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as nat


def page_minmax(K: torch.Tensor, page: int, *, row0: int = 0, n_pages: Optional[int] = None,
                kmin: Optional[torch.Tensor] = None, kmax: Optional[torch.Tensor] = None,
                page_offset: int = 0):
    """Channel-wise minima and maxima of the pages of K (B, H_kv, T, D)
    starting at ``row0``, into ``kmin/kmax[..., page_offset:page_offset+n_pages, :]``
    (allocated when None).  Returns (kmin, kmax)."""
    L = nat.lib()
    B, H_kv, T, D = K.shape
    if K.stride(-1) != 1:
        K = K.contiguous()
    if n_pages is None:
        n_pages = (T - row0) // page
    if row0 + n_pages * page > T:
        raise AssertionError(f"pages [{row0}, {row0 + n_pages * page}) exceed T={T}")
    shape = (B, H_kv, page_offset + n_pages, D)
    if kmin is None:
        kmin = torch.empty(shape, device=K.device, dtype=K.dtype)
    if kmax is None:
        kmax = torch.empty(shape, device=K.device, dtype=K.dtype)
    for t in (kmin, kmax):
        if t.dtype != K.dtype or t.stride(-1) != 1 or t.shape[-2] < page_offset + n_pages:
            raise AssertionError("kmin/kmax must have K's dtype, unit last stride and room for the pages")
    if kmin.stride() != kmax.stride():
        raise AssertionError("kmin and kmax must share strides")
    nat.check(L.halo_page_minmax(K.data_ptr(), K.stride(0), K.stride(1), K.stride(2),
                                 nat.dtype_code(K.dtype), B, H_kv, D, row0, page, n_pages,
                                 kmin[..., page_offset:, :].data_ptr(), kmax[..., page_offset:, :].data_ptr(),
                                 kmin.stride(0), kmin.stride(1), kmin.stride(2), nat.stream_ptr()),
              "halo_page_minmax")
    return kmin, kmax


def quest_score_topk(query: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *,
                     per_row: bool = False, want_dots: bool = False, want_scores: bool = False):
    """Bound scores and top-k pages.  query (B, H, T_q, D) in the pages'
    dtype; kmin/kmax (B, H_kv, P, D).  Returns (idx int32 (n_sel, k) in
    descending score order, dots (B, H_kv, T_q, P) fp32 or None, page scores
    fp32 (n_sel, P) or None)."""
    L = nat.lib()
    if query.dim() != 4:
        raise AssertionError(f"query must be (B, H, T_q, D), got {tuple(query.shape)}")
    B, H, T_q, D = query.shape
    H_kv, P = kmin.shape[1], kmin.shape[2]
    if kmin.dtype != query.dtype or kmax.dtype != query.dtype:
        raise AssertionError(f"kmin/kmax dtype {kmin.dtype} != query dtype {query.dtype}")
    if kmin.shape != kmax.shape or kmin.stride() != kmax.stride() or kmin.stride(-1) != 1:
        raise AssertionError("kmin and kmax must share shape and strides with a unit last stride")
    if query.stride(-1) != 1:
        query = query.contiguous()
    n_sel = B if per_row else 1
    dev = query.device
    work = torch.empty((n_sel, P), device=dev, dtype=torch.int32)
    idx = torch.empty((n_sel, max(k, 1)), device=dev, dtype=torch.int32)
    dots = torch.empty((B, H_kv, T_q, P), device=dev, dtype=torch.float32) if want_dots else None
    scores = torch.empty((n_sel, P), device=dev, dtype=torch.float32) if want_scores else None
    nat.check(L.halo_quest_score_topk(
        query.data_ptr(), query.stride(0), query.stride(1), query.stride(2), nat.dtype_code(query.dtype),
        B, H, H_kv, T_q, D, kmin.data_ptr(), kmax.data_ptr(), kmin.stride(0), kmin.stride(1), kmin.stride(2),
        P, int(k), int(per_row), work.data_ptr(), nat.ptr(dots), nat.ptr(scores), idx.data_ptr(),
        nat.stream_ptr()), "halo_quest_score_topk")
    return idx[:, :k], dots, scores


def num_hot_pages(P: int, memory_ratio: float, min_pages_selected: int) -> int:
    """K = min(P, max(min_pages_selected, ceil(P / memory_ratio))) computed
    as the reference does, with a float ratio
    (baselines/quest_path_d.py:197-200)."""
    K = max(int(min_pages_selected), int((P + memory_ratio - 1) // memory_ratio))
    return min(K, P)


@dataclass
class QuestPathDConfig:
    """Quest selection knobs plus the Path-D knobs they are combined with
    (baselines/quest_path_d.py:40-84; same fields and defaults)."""

    page_size: int = 16
    memory_ratio: float = 4.0
    min_pages_selected: int = 4
    chunk_size: int = 512
    recent_window: int = 64
    use_triton: bool = True


class QuestScorer:
    """GPU Quest scorer implementing the placement plug-in protocol, with the
    reference adapter's attributes and telemetry counters."""

    def __init__(self, cfg: Optional[QuestPathDConfig] = None) -> None:
        self.cfg = cfg or QuestPathDConfig()
        self.page_size = int(self.cfg.page_size)
        self.memory_ratio = self.cfg.memory_ratio
        self.min_pages_selected = int(self.cfg.min_pages_selected)
        self._k_min: dict = {}
        self._k_max: dict = {}
        self._num_full_pages: dict = {}
        self.observe_calls = 0
        self.score_calls = 0
        self.last_hot_pages_per_layer: dict = {}
        self.cumulative_hot_pages = 0

    def observe_keys(self, layer_idx: int, K_full: torch.Tensor) -> None:
        """Minima and maxima of the pages that filled since the last call
        (O(new rows x D)); a K with fewer full pages than seen before means
        the rows were replaced, and every page is recomputed."""
        if K_full is None or K_full.numel() == 0:
            return
        B, H_kv, T, D = K_full.shape
        p = self.page_size
        n_full = T // p
        prev = int(self._num_full_pages.get(layer_idx, 0))
        if n_full < prev:
            prev = 0
        elif n_full == prev:
            return
        kmin, kmax = self._k_min.get(layer_idx), self._k_max.get(layer_idx)
        if kmin is None or kmin.shape[-2] < n_full or kmin.dtype != K_full.dtype or kmin.shape[:2] != (B, H_kv):
            cap = max(n_full, 2 * (kmin.shape[-2] if kmin is not None else 0), 64)
            nmin = torch.empty((B, H_kv, cap, D), device=K_full.device, dtype=K_full.dtype)
            nmax = torch.empty_like(nmin)
            if kmin is not None and prev > 0:
                nmin[..., :prev, :] = kmin[..., :prev, :]
                nmax[..., :prev, :] = kmax[..., :prev, :]
            kmin, kmax = nmin, nmax
        page_minmax(K_full, p, row0=prev * p, n_pages=n_full - prev, kmin=kmin, kmax=kmax, page_offset=prev)
        self._k_min[layer_idx], self._k_max[layer_idx] = kmin, kmax
        self._num_full_pages[layer_idx] = n_full
        self.observe_calls += 1

    def forget(self, layer_idx: int) -> None:
        """Drop the metadata of ``layer_idx`` (its GPU rows were replaced)."""
        self._k_min.pop(layer_idx, None)
        self._k_max.pop(layer_idx, None)
        self._num_full_pages.pop(layer_idx, None)

    def bounds(self, layer_idx: int):
        """(K_min, K_max) (B, H_kv, P, D) of the full pages, or None."""
        if layer_idx not in self._k_min:
            return None
        n = self._num_full_pages[layer_idx]
        return self._k_min[layer_idx][..., :n, :], self._k_max[layer_idx][..., :n, :]

    def score_pages(self, layer_idx: int, query: torch.Tensor) -> Optional[torch.Tensor]:
        """Quest's per-page upper bounds (B, H_kv, T_q, P) fp32, or None when
        the layer has no metadata yet."""
        bb = self.bounds(layer_idx)
        if bb is None:
            return None
        kmin, kmax = bb
        q = query if query.dim() == 4 else query.unsqueeze(2)
        _, dots, _ = quest_score_topk(q.to(kmin.dtype), kmin, kmax, 0, want_dots=True)
        self.score_calls += 1
        return dots

    def select_hot_pages(self, layer_idx: int, query: torch.Tensor) -> Optional[torch.Tensor]:
        """Indices (CPU int64, descending score) of the Quest-top-K pages."""
        bb = self.bounds(layer_idx)
        if bb is None:
            return None
        kmin, kmax = bb
        P = kmin.shape[-2]
        K = num_hot_pages(P, self.memory_ratio, self.min_pages_selected)
        q = query if query.dim() == 4 else query.unsqueeze(2)
        if q.shape[0] != kmin.shape[0]:
            raise AssertionError("query batch != key batch")
        idx, _, _ = quest_score_topk(q.to(kmin.dtype), kmin, kmax, K)
        self.score_calls += 1
        topk = idx[0].to(torch.int64).cpu()
        self.last_hot_pages_per_layer[layer_idx] = topk
        self.cumulative_hot_pages += K
        return topk


def wrap_with_quest_path_d(model, config: Optional[QuestPathDConfig] = None):
    """Path D (``wrap_with_halo`` with chunked=True) with the Quest scorer
    driving GPU placement (baselines/quest_path_d.py:208-258)."""
    import os

    from .policy import HALOConfig, wrap_with_halo
    config = config or QuestPathDConfig()
    use_triton = config.use_triton and os.environ.get("HALO_DISABLE_TRITON", "0") != "1"
    wrap_with_halo(model, HALOConfig(chunked=True, chunk_size=config.chunk_size,
                                     recent_window=config.recent_window,
                                     hot_ratio=1.0 / max(1.0, config.memory_ratio), use_triton=use_triton))
    model._quest_path_d_config = config
    model._halo_cache._quest_scorer = QuestScorer(config)
    return model
