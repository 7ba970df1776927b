"""Demotion of cooled KV blocks down the tier ladder, as batched moves.

Reference: HALODemoter (halo/demoter.py:20-77) queues (layer, block, src,
dst) entries and drains them with one ``move_block`` per block, on a side
stream that first waits for the compute stream.

Here a demotion request is one (layer, block tensor, src, dst) entry: the
blocks stay a device tensor (never a Python list), and draining an entry is
one ``TieredStorage.move_blocks`` launch that moves every listed block still
in the source tier.  Asynchronous drains run on the demotion stream after
the compute stream's pending work (the source rows must be final); ``wait``
orders the compute stream after them.
"""
from __future__ import annotations

from collections import deque
from typing import Deque, Iterable, Optional

import torch


class HALODemoter:
    """Move cold KV blocks from a faster tier to a slower one."""

    def __init__(self, config, *, storage) -> None:
        self.cfg = config
        self.storage = storage
        self._queue: Deque[tuple[int, torch.Tensor, str, str]] = deque()
        self._stream: Optional[torch.cuda.Stream] = None
        self.demoted_requests = 0

    def demote(self, *, layer: int, block_indices: "Iterable[int] | torch.Tensor", src: str = "gpu",
               dst: str = "dram") -> None:
        dev = self.storage.directory().device
        blocks = torch.as_tensor(block_indices).to(device=dev, dtype=torch.int32).reshape(-1)
        if blocks.numel() == 0:
            return
        self._queue.append((layer, blocks, src, dst))
        self.demoted_requests += 1
        if self.cfg.async_refetch and self.storage.on_device:
            self._drain_async()
        else:
            self.flush()

    def flush(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Apply every queued demotion (on ``stream``, default current)."""
        while self._queue:
            layer, blocks, src, dst = self._queue.popleft()
            self.storage.move_blocks(layer=layer, blocks=blocks, src=src, dst=dst, only_if_in_src=True,
                                     stream=stream)

    def _drain_async(self) -> None:
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self.storage.gpu_device)  # default priority
        self._stream.wait_stream(torch.cuda.current_stream(self.storage.gpu_device))
        self.flush(stream=self._stream)

    def wait(self) -> None:
        """Order the current stream after the issued demotions."""
        if self._stream is not None:
            torch.cuda.current_stream(self.storage.gpu_device).wait_stream(self._stream)

    def __repr__(self) -> str:  # pragma: no cover
        return f"HALODemoter(queued={len(self._queue)}, async={self.cfg.async_refetch})"
