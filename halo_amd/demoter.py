"""HALO-Demoter: stream cold KV blocks down the tier ladder.

Reference: halo/demoter.py:31-77.  Demotions are queued and drained on a side
stream that first waits for the compute stream (the source blocks must be
final), so the decode path never blocks on them.
"""
from __future__ import annotations

from collections import deque
from typing import Deque, Iterable

import torch


class HALODemoter:
    """Move cold KV blocks from a faster tier to a slower one."""

    def __init__(self, config, *, storage) -> None:
        self.cfg = config
        self.storage = storage
        self._pending: Deque[tuple[int, int, str, str]] = deque()
        self._stream = None

    def demote(self, *, layer: int, block_indices: "Iterable[int] | torch.Tensor", src: str = "gpu",
               dst: str = "dram") -> None:
        if isinstance(block_indices, torch.Tensor):
            block_indices = block_indices.tolist()
        for blk in block_indices:
            self._pending.append((layer, int(blk), src, dst))
        if self.cfg.async_refetch:
            self._kick_async()
        else:
            self.flush()

    def flush(self) -> None:
        """Drain the pending queue on the current stream."""
        while self._pending:
            layer, blk, src, dst = self._pending.popleft()
            self.storage.move_block(layer=layer, block=blk, src=src, dst=dst)

    def _kick_async(self) -> None:
        if not (torch.cuda.is_available() and self.storage.gpu_device.type == "cuda"):
            self.flush()
            return
        if self._stream is None:
            self._stream = torch.cuda.Stream()  # default priority
        self._stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self._stream):
            self.flush()

    def wait(self) -> None:
        """Order the current stream after the issued demotions."""
        if self._stream is not None:
            torch.cuda.current_stream().wait_stream(self._stream)

    def __repr__(self) -> str:  # pragma: no cover
        return f"HALODemoter(pending={len(self._pending)}, async={self.cfg.async_refetch})"
