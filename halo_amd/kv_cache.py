"""Tier-aware HuggingFace cache: the base of the Path-D cache.

Reference: HALOCache (halo/kv_cache.py:69-209).  It derives from
transformers' ``DynamicCache`` when transformers is importable, so a wrapped
model sees the ``Cache`` protocol it expects (``update``,
``get_seq_length``, ``get_mask_sizes``, ``layers[i].keys/values``), and
adds HALO's hot-set bookkeeping: ``update_hotness`` scores a head-mean
attention snapshot, demotes the blocks that left the hot set and schedules
the predicted ones for refetch (halo/kv_cache.py:120-170).  All scoring and
block moves run on the GPU (HALOScorer / HALODemoter / HALORefetcher of this
package); the hot-set difference is a device-side mask, not a Python set.
"""
from __future__ import annotations

from typing import Optional

import torch

try:  # transformers is optional for the kernel path; the cache protocol needs it
    from transformers.cache_utils import DynamicCache as _BaseCache
    HAS_TRANSFORMERS = True
except Exception:  # pragma: no cover - exercised only without transformers

    class _Layer:
        def __init__(self) -> None:
            self.keys: Optional[torch.Tensor] = None
            self.values: Optional[torch.Tensor] = None

        def get_seq_length(self) -> int:
            return 0 if self.keys is None else int(self.keys.shape[-2])

    class _BaseCache:  # type: ignore[no-redef]
        """Stand-in with DynamicCache's per-layer ``keys`` / ``values``."""

        def __init__(self, *args, **kwargs) -> None:
            self.layers: list = []

        def update(self, key_states, value_states, layer_idx, *args, **kwargs):
            while len(self.layers) <= layer_idx:
                self.layers.append(_Layer())
            lay = self.layers[layer_idx]
            if lay.keys is None:
                lay.keys, lay.values = key_states, value_states
            else:
                lay.keys = torch.cat([lay.keys, key_states], dim=-2)
                lay.values = torch.cat([lay.values, value_states], dim=-2)
            return lay.keys, lay.values

        def get_seq_length(self, layer_idx: int = 0) -> int:
            return self.layers[layer_idx].get_seq_length() if layer_idx < len(self.layers) else 0

    HAS_TRANSFORMERS = False


class HALOCache(_BaseCache):
    """DynamicCache plus hot-set tracking, demotion and predictive refetch."""

    def __init__(self, *, config, storage, scorer, demoter, refetcher) -> None:
        super().__init__()
        self.cfg = config
        self.storage = storage
        self.scorer = scorer
        self.demoter = demoter
        self.refetcher = refetcher
        self._step = 0
        self._last_hot: dict = {}
        self._last_score: dict = {}
        self.demoted_blocks_total = 0
        self.refetched_blocks_total = 0

    # ----------------------------------------------------------------- lifecycle
    def reset(self) -> None:
        """Clear the cached rows and HALO's bookkeeping (one generate call)."""
        try:
            _BaseCache.__init__(self)
        except Exception:  # pragma: no cover
            self.layers = []
        self._step = 0
        self._last_hot.clear()
        self._last_score.clear()
        self.demoted_blocks_total = 0
        self.refetched_blocks_total = 0

    def step(self) -> None:
        self._step += 1

    @property
    def step_index(self) -> int:
        return self._step

    # ----------------------------------------------------------------- hot set
    def update_hotness(self, layer_idx: int, attn_weights: torch.Tensor) -> None:
        """Score ``attn_weights`` (K,), demote the blocks of positions that
        left the hot set and schedule the predicted hot blocks for refetch
        (halo/kv_cache.py:120-170).  At hot_ratio 1.0 nothing is demoted."""
        score = self.scorer.score(attn_weights, step=self._step)
        hot = self.scorer.topk_hot(score)
        K = score.shape[-1]
        prev = self._last_hot.get(layer_idx)
        if prev is not None:
            was = torch.zeros(K, dtype=torch.bool, device=score.device)
            now = torch.zeros(K, dtype=torch.bool, device=score.device)
            was[prev.clamp(0, K - 1)] = True
            now[hot] = True
            cooled = was & ~now
            # blocks of cooled positions, one entry per block (first position of
            # each block that has a cooled position); others are -1
            bs = self.cfg.block_size
            pos = torch.arange(K, device=score.device)
            blk = torch.div(pos, bs, rounding_mode="floor")
            n_blk = int((K + bs - 1) // bs)
            per_blk = torch.zeros(n_blk, dtype=torch.int32, device=score.device)
            any_cooled = per_blk.index_add_(0, blk, cooled.to(torch.int32)) > 0
            ids = torch.arange(n_blk, device=score.device)
            blocks = torch.where(any_cooled, ids, torch.full_like(ids, -1))
            n = int(any_cooled.sum().item())
            if n:
                self.demoter.demote(layer=layer_idx, block_indices=blocks, src="gpu",
                                    dst=self._next_tier_after("gpu"))
                self.demoted_blocks_total += n
        predicted = self.refetcher.predict_hot(layer=layer_idx, last_hot_indices=hot, last_score=score)
        before = self.refetcher.misses
        self.refetcher.schedule(layer=layer_idx, predicted_indices=predicted)
        self.refetched_blocks_total += self.refetcher.misses - before
        self._last_hot[layer_idx] = hot
        self._last_score[layer_idx] = score

    def telemetry(self) -> dict:
        r = self.refetcher
        hits, misses = (r.hits, r.misses) if r is not None else (0, 0)
        total = hits + misses
        return {
            "step": self._step,
            "demoted_blocks": self.demoted_blocks_total,
            "refetched_blocks": self.refetched_blocks_total,
            "refetch_hits": hits,
            "refetch_misses": misses,
            "refetch_hit_rate": (hits / total) if total else 0.0,
        }

    def _next_tier_after(self, current: str) -> str:
        names = [str(getattr(t, "value", t)) for t in self.cfg.tiers]
        try:
            i = names.index(current)
        except ValueError:
            return current
        return names[min(i + 1, len(names) - 1)]
