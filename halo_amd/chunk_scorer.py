"""Chunk-relevance scoring on the GPU: page-mean keys and top-k selection.

Reference: ``HALOPressScorerAdapter`` (baselines/scorer_ablations.py:185-268)
and the placement-scorer plug-in protocol ``observe_keys`` /
``select_hot_pages`` consulted by the cache (halo/kv_cache_chunked.py:306-311,
416-424).  Differences:
  * page means are computed once per page when it fills (the reference
    recomputes every page on every update, :215);
  * scoring, the min-max/recency/sink combination and the top-k run in one
    HIP kernel; ``select_into_table`` writes the chosen chunks straight into
    a device chunk table so attention can follow with no host sync (the
    reference syncs with ``.cpu()`` at :266);
  * ties are broken by lower chunk index (torch.topk leaves them undefined).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as nat


def chunk_means(K: torch.Tensor, page: int, *, row0: int = 0, n_pages: Optional[int] = None,
                out: Optional[torch.Tensor] = None, page_offset: int = 0) -> torch.Tensor:
    """Page means of K (B, H_kv, T, D) for pages starting at ``row0``, into
    ``out[..., page_offset:page_offset+n_pages, :]`` (allocated when None)."""
    L = nat.lib()
    B, H_kv, T, D = K.shape
    if K.stride(-1) != 1:
        K = K.contiguous()
    if n_pages is None:
        n_pages = (T - row0) // page
    if row0 + n_pages * page > T:
        raise AssertionError(f"pages [{row0}, {row0 + n_pages * page}) exceed T={T}")
    if out is None:
        out = torch.empty((B, H_kv, page_offset + n_pages, D), device=K.device, dtype=K.dtype)
    if out.dtype != K.dtype or out.stride(-1) != 1 or out.shape[-2] < page_offset + n_pages:
        raise AssertionError("out must have K's dtype, unit last stride and room for the pages")
    base = out[..., page_offset:, :]
    nat.check(L.halo_chunk_means(K.data_ptr(), K.stride(0), K.stride(1), K.stride(2),
                                 nat.dtype_code(K.dtype), B, H_kv, D, row0, page, n_pages,
                                 base.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                                 nat.stream_ptr()), "halo_chunk_means")
    return out


def score_topk(q: torch.Tensor, kmean: torch.Tensor, eligible: torch.Tensor, k: int, *,
               per_row: bool = False, n_elig_per_sel: Optional[torch.Tensor] = None,
               alpha: float = 1.0, beta: float = 0.0, gamma: float = 0.0,
               normalize: bool = False, refresh_window: int = 64, sink_pages: int = 0,
               P_total: Optional[int] = None,
               catalog: Optional[torch.Tensor] = None, table: Optional[torch.Tensor] = None,
               table_stride: int = 0, table_slot0: int = 0, catalog_stride: int = 0,
               idx_out: Optional[torch.Tensor] = None, score_out: Optional[torch.Tensor] = None,
               staging: Optional[tuple] = None):
    """Score eligible chunks and pick the top ``k``.

    q (B, H, D) or (B, H, 1, D); kmean (B, H_kv, P, D) in q's dtype;
    eligible int32 (n_sel, n_elig) or (n_elig,).  Returns (idx int32
    (n_sel, k) ascending with -1 padding, scores fp32 (n_sel, n_elig)).
    With ``table``/``catalog`` (uint8 views of halo_chunk_desc arrays) the
    chosen descriptors are copied into the table on the device.
    ``staging`` = (residency int32 tensor, slot catalog uint8 tensor,
    n_slots, res_out int32 tensor): chosen chunks held by an HBM staging
    slot are written to the table with the slot's addresses
    (``halo_chunk_score_topk_staged``; raw scores only)."""
    L = nat.lib()
    q3 = q.squeeze(2) if q.dim() == 4 else q
    B, H, D = q3.shape
    H_kv, P = kmean.shape[1], kmean.shape[2]
    if kmean.dtype != q3.dtype:
        raise AssertionError(f"kmean dtype {kmean.dtype} != q dtype {q3.dtype}")
    if kmean.stride(-1) != 1:
        kmean = kmean.contiguous()
    eligible = eligible.to(device=q3.device, dtype=torch.int32)
    if eligible.dim() == 1:
        eligible = eligible.unsqueeze(0)
    n_sel = B if per_row else 1
    n_elig = eligible.shape[-1]
    if eligible.shape[0] not in (1, n_sel):
        raise AssertionError(f"eligible rows {eligible.shape[0]} != selections {n_sel}")
    elig_stride = n_elig if eligible.shape[0] == n_sel and n_sel > 1 else 0
    eligible = eligible.contiguous()
    if idx_out is None:
        idx_out = torch.empty((n_sel, k), device=q3.device, dtype=torch.int32)
    if score_out is None:
        score_out = torch.empty((n_sel, max(n_elig, 1)), device=q3.device, dtype=torch.float32)
    if catalog is not None and catalog_stride == 0 and per_row:
        catalog_stride = catalog.numel() // 88 // n_sel
    if staging is not None:
        if normalize or table is None:
            raise AssertionError("the staged selection writes a table and uses raw scores")
        res, scat, n_slots, res_out = staging
        nat.check(L.halo_chunk_score_topk_staged(
            q3.data_ptr(), q3.stride(0), q3.stride(1), nat.dtype_code(q3.dtype),
            B, H, H_kv, D,
            kmean.data_ptr(), kmean.stride(0), kmean.stride(1), kmean.stride(2),
            eligible.data_ptr(), elig_stride, nat.ptr(n_elig_per_sel), n_elig, int(k), int(per_row),
            idx_out.data_ptr(), score_out.data_ptr(),
            nat.ptr(catalog), catalog_stride or n_elig, nat.ptr(table), table_stride, table_slot0,
            res.data_ptr(), scat.data_ptr(), int(n_slots), res_out.data_ptr(), nat.stream_ptr()),
            "halo_chunk_score_topk_staged")
        return idx_out, score_out
    nat.check(L.halo_chunk_score_topk(
        q3.data_ptr(), q3.stride(0), q3.stride(1), nat.dtype_code(q3.dtype),
        B, H, H_kv, D,
        kmean.data_ptr(), kmean.stride(0), kmean.stride(1), kmean.stride(2),
        eligible.data_ptr(), elig_stride, nat.ptr(n_elig_per_sel), n_elig, int(k), int(per_row),
        idx_out.data_ptr(), score_out.data_ptr(),
        nat.ptr(catalog), catalog_stride, nat.ptr(table), table_stride, table_slot0,
        int(normalize), float(alpha), float(beta), float(gamma), int(refresh_window), int(sink_pages),
        int(P_total if P_total is not None else P), nat.stream_ptr()), "halo_chunk_score_topk")
    return idx_out, score_out


def num_hot_pages(P: int, memory_ratio: int, min_pages_selected: int) -> int:
    """Hot-page budget (baselines/scorer_ablations.py:133-139)."""
    K = max(min_pages_selected, int((P + memory_ratio - 1) // memory_ratio))
    return min(K, P)


@dataclass
class ChunkScorerConfig:
    """Knobs of the page scorer (baselines/scorer_ablations.py AblationScorerConfig)."""

    page_size: int = 16
    memory_ratio: int = 4
    min_pages_selected: int = 4
    halopress_alpha: float = 1.0
    halopress_beta: float = 0.0
    halopress_gamma: float = 0.0
    halopress_refresh_window: int = 64
    halopress_sink_tokens: int = 4


class ChunkScorer:
    """GPU page scorer implementing the placement plug-in protocol."""

    def __init__(self, cfg: Optional[ChunkScorerConfig] = None) -> None:
        self.cfg = cfg or ChunkScorerConfig()
        self.page_size = self.cfg.page_size
        self._k_mean: dict = {}
        self._num_full_pages: dict = {}
        self.observe_calls = 0
        self.score_calls = 0
        self.last_hot_pages_per_layer: dict = {}
        self.cumulative_hot_pages = 0

    def observe_keys(self, layer_idx: int, K_full: torch.Tensor) -> None:
        """Page means for pages that filled since the last call."""
        if K_full is None or K_full.numel() == 0:
            return
        B, H_kv, T, D = K_full.shape
        p = self.page_size
        n_full = T // p
        prev = int(self._num_full_pages.get(layer_idx, 0))
        self.observe_calls += 1
        if n_full < prev:  # the rows were replaced (a peel): recompute every page
            prev = 0
        elif n_full == prev:
            return
        km = self._k_mean.get(layer_idx)
        if km is None or km.shape[-2] < n_full or km.dtype != K_full.dtype:
            cap = max(n_full, 2 * (km.shape[-2] if km is not None else 0), 64)
            new = torch.empty((B, H_kv, cap, D), device=K_full.device, dtype=K_full.dtype)
            if km is not None and prev > 0:
                new[..., :prev, :] = km[..., :prev, :]
            km = new
        chunk_means(K_full, p, row0=prev * p, n_pages=n_full - prev, out=km, page_offset=prev)
        self._k_mean[layer_idx] = km
        self._num_full_pages[layer_idx] = n_full

    def forget(self, layer_idx: int) -> None:
        """Drop the page means of ``layer_idx`` (its GPU rows were replaced)."""
        self._k_mean.pop(layer_idx, None)
        self._num_full_pages.pop(layer_idx, None)

    def page_means(self, layer_idx: int) -> Optional[torch.Tensor]:
        km = self._k_mean.get(layer_idx)
        if km is None:
            return None
        return km[..., : self._num_full_pages[layer_idx], :]

    def select_hot_pages(self, layer_idx: int, query: torch.Tensor) -> Optional[torch.Tensor]:
        """Indices (CPU int64, ascending) of the hot pages for ``query``."""
        km = self.page_means(layer_idx)
        if km is None:
            return None
        P = km.shape[-2]
        K = num_hot_pages(P, self.cfg.memory_ratio, self.cfg.min_pages_selected)
        q = query[:, :, -1, :] if query.dim() == 4 else query
        if q.shape[0] != km.shape[0]:
            raise AssertionError("query batch != key batch")
        elig = torch.arange(P, device=q.device, dtype=torch.int32)
        c = self.cfg
        idx, _ = score_topk(q.to(km.dtype).contiguous(), km, elig, K, normalize=True,
                            alpha=c.halopress_alpha, beta=c.halopress_beta, gamma=c.halopress_gamma,
                            refresh_window=c.halopress_refresh_window,
                            sink_pages=min(c.halopress_sink_tokens // max(self.page_size, 1) + 1, P),
                            P_total=P)
        topk = idx[0].to(torch.int64).cpu()
        self.last_hot_pages_per_layer[layer_idx] = topk
        self.cumulative_hot_pages += int(topk.numel())
        self.score_calls += 1
        return topk
