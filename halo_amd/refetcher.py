"""Predictive refetch of cold KV blocks, scheduled on the device.

Reference: HALORefetcher (halo/refetcher.py:24-114): predict the next hot
positions from the last score (top-(hot_ratio*K) + lookahead), map them to
blocks, count GPU-resident blocks as hits and the others as misses, and move
the misses to the GPU tier on a side stream.

This implementation keeps that contract but never brings the prediction to
the host: positions become blocks with a sort and a first-of-run mask (fixed
shapes, no ``unique``), hit and miss counts accumulate in a device counter,
an in-flight bitmap on the device skips blocks already being fetched, and
every miss of one call moves in a single ``halo_copy_blocks`` launch on the
refetch stream.  The directory entry of a moved block flips to the GPU tier
after its copy, in that stream's order, so no reader sees a block as
resident before its rows have landed.  ``hits`` / ``misses`` read the
counter (one host sync, only when asked).
"""
from __future__ import annotations

from typing import Iterable, Optional

import torch

from .memory_tier import MemoryTier
from .scorer import topk_sorted


class HALORefetcher:
    """Predictive, asynchronous refetcher of cold blocks."""

    def __init__(self, config, *, storage) -> None:
        self.cfg = config
        self.storage = storage
        self._stream: Optional[torch.cuda.Stream] = None
        self._counts: Optional[torch.Tensor] = None   # int64 [hits, misses] on the storage device
        self._offset = [0, 0]                          # host-side adjustments (cache telemetry)
        self._inflight: Optional[torch.Tensor] = None  # uint8 (L, max_blocks): fetch issued

    # ----------------------------------------------------------------- counters
    def _counter(self) -> torch.Tensor:
        if self._counts is None:
            self._counts = torch.zeros(2, dtype=torch.int64, device=self.storage.gpu_device)
        return self._counts

    @property
    def hits(self) -> int:
        return self._offset[0] + (int(self._counts[0].item()) if self._counts is not None else 0)

    @hits.setter
    def hits(self, value: int) -> None:
        self._offset[0] += int(value) - self.hits

    @property
    def misses(self) -> int:
        return self._offset[1] + (int(self._counts[1].item()) if self._counts is not None else 0)

    @misses.setter
    def misses(self, value: int) -> None:
        self._offset[1] += int(value) - self.misses

    def count_hits(self, n: int) -> None:
        """Add ``n`` hits without reading the device counter."""
        self._offset[0] += int(n)

    # ----------------------------------------------------------------- prediction
    def predict_hot(self, *, layer: int, last_hot_indices: torch.Tensor, last_score: torch.Tensor) -> torch.Tensor:
        """Top-(clamp(int(hot_ratio*K), 1) + lookahead) positions, ascending
        (halo/refetcher.py:38-57); ties go to the lower position."""
        K = last_score.shape[-1]
        if self.cfg.hot_ratio >= 1.0:
            return torch.arange(K, device=last_score.device, dtype=torch.long)
        k = min(max(int(self.cfg.hot_ratio * K), 1) + self.cfg.lookahead, K)
        return topk_sorted(last_score, k)

    # ----------------------------------------------------------------- schedule
    def _blocks(self, predicted) -> tuple[torch.Tensor, torch.Tensor]:
        """(sorted block ids, first-of-run mask) of the predicted positions."""
        dev = self.storage.directory().device
        pos = torch.as_tensor(predicted).to(device=dev, dtype=torch.int64).reshape(-1)
        blk = torch.div(pos, self.cfg.block_size, rounding_mode="floor").sort().values
        first = torch.ones_like(blk, dtype=torch.bool)
        if blk.numel() > 1:
            first[1:] = blk[1:] != blk[:-1]
        return blk, first & (blk >= 0) & (blk < self.storage.max_blocks)

    def schedule(self, *, layer: int, predicted_indices: "Iterable[int] | torch.Tensor") -> None:
        """Count hits and misses of the predicted blocks and fetch the misses
        to the GPU tier (asynchronously when ``async_refetch``)."""
        st = self.storage
        blk, valid = self._blocks(predicted_indices)
        if blk.numel() == 0:
            return
        if self._inflight is None:
            self._inflight = torch.zeros((st.num_layers, st.max_blocks), dtype=torch.uint8, device=blk.device)
        idx = blk.clamp(0, st.max_blocks - 1)
        tiers = st.directory()[layer].index_select(0, idx)
        busy = self._inflight[layer].index_select(0, idx).bool()
        hit = valid & (tiers == st.tier_code("gpu"))
        miss = valid & ~hit & ~busy
        self._counter().add_(torch.stack([hit.sum(), miss.sum()]))
        # mark the misses in flight (max-reduction: duplicate entries never
        # clear a mark another entry sets)
        self._inflight[layer].scatter_reduce_(0, idx, miss.to(torch.uint8), reduce="amax")
        todo = torch.where(miss, blk, torch.full_like(blk, -1)).to(torch.int32)
        self._issue(layer, todo)

    def _issue(self, layer: int, blocks: torch.Tensor) -> None:
        st = self.storage
        sources = [t for t in st.tiers if t is not MemoryTier.GPU]
        use_side = bool(self.cfg.async_refetch) and st.on_device
        if use_side:
            if self._stream is None:
                self._stream = torch.cuda.Stream(device=st.gpu_device)  # default priority
            self._stream.wait_stream(torch.cuda.current_stream(st.gpu_device))
        for src in sources:
            st.move_blocks(layer=layer, blocks=blocks, src=src, dst=MemoryTier.GPU, only_if_in_src=True,
                           stream=self._stream if use_side else None)

    def wait(self) -> None:
        """Order the current stream after the outstanding refetches and clear
        the in-flight marks."""
        if self._stream is not None:
            torch.cuda.current_stream(self.storage.gpu_device).wait_stream(self._stream)
        if self._inflight is not None:
            self._inflight.zero_()

    def __repr__(self) -> str:  # pragma: no cover
        return f"HALORefetcher(block_size={self.cfg.block_size}, lookahead={self.cfg.lookahead})"
