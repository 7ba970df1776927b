"""HALO-Refetcher: prefetch blocks predicted to become hot.

Reference: halo/refetcher.py:38-114.  ``predict_hot`` runs the GPU sorted
top-k (``halo_topk_sorted``); ``schedule`` keeps the reference's block
bookkeeping (position -> block, dedupe, GPU-resident blocks are hits, others
misses unless already in flight) and issues ``TieredStorage.move_block`` on
a side stream (its copies are hipMemcpyAsync from pinned host memory).
"""
from __future__ import annotations

from typing import Iterable

import torch

from .scorer import topk_sorted


class HALORefetcher:
    """Predictive, asynchronous refetcher of cold blocks."""

    def __init__(self, config, *, storage) -> None:
        self.cfg = config
        self.storage = storage
        self._stream = None
        self._inflight: set[tuple[int, int]] = set()
        self.hits = 0
        self.misses = 0

    def predict_hot(self, *, layer: int, last_hot_indices: torch.Tensor, last_score: torch.Tensor) -> torch.Tensor:
        """Top-(clamp(int(hot_ratio*K), 1) + lookahead) positions, sorted."""
        K = last_score.shape[-1]
        if self.cfg.hot_ratio >= 1.0:
            return torch.arange(K, device=last_score.device, dtype=torch.long)
        k = min(max(int(self.cfg.hot_ratio * K), 1) + self.cfg.lookahead, K)
        return topk_sorted(last_score, k)

    def schedule(self, *, layer: int, predicted_indices: "Iterable[int] | torch.Tensor") -> None:
        """Issue refetches for predicted blocks that are not on the GPU tier."""
        if isinstance(predicted_indices, torch.Tensor):
            predicted_indices = predicted_indices.tolist()
        block_size = self.cfg.block_size
        seen: set[int] = set()
        for pos in predicted_indices:
            blk = int(pos) // block_size
            if blk in seen:
                continue
            seen.add(blk)
            tier = self.storage.locate_block(layer=layer, block=blk)
            key = (layer, blk)
            if tier == "gpu":
                self.hits += 1
                continue
            if key in self._inflight:
                continue
            self.misses += 1
            self._inflight.add(key)
            self._issue(layer=layer, block=blk, src=tier)

    def wait(self) -> None:
        """Order the current stream after the outstanding refetches."""
        if self._stream is not None and torch.cuda.is_available():
            torch.cuda.current_stream().wait_stream(self._stream)
        self._inflight.clear()

    def _issue(self, *, layer: int, block: int, src: str) -> None:
        def _do() -> None:
            self.storage.move_block(layer=layer, block=block, src=src, dst="gpu")

        if self.cfg.async_refetch and torch.cuda.is_available() and self.storage.gpu_device.type == "cuda":
            if self._stream is None:
                self._stream = torch.cuda.Stream()  # default priority
            self._stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(self._stream):
                _do()
        else:
            _do()

    def __repr__(self) -> str:  # pragma: no cover
        total = self.hits + self.misses
        rate = (self.hits / total) if total else 0.0
        return f"HALORefetcher(hit_rate={rate:.3f}, inflight={len(self._inflight)})"
