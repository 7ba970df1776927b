"""Cold tier in pinned host DRAM and its refetch path (MI355X).

Reference: halo/memory_tier.py:31-258 (TieredStorage / _BlockBuffer /
MemoryTier) and the DMA-overlap driver of halo/triton_chunked.py:270-362.

What changes on MI355X:
  * the DRAM tier is pinned (page-locked) host memory, so every refetch is an
    asynchronous ``hipMemcpyAsync`` issued on a dedicated copy stream, gated
    by HIP events, never a synchronous pageable copy;
  * refetch targets are a fixed ring of HBM staging slots reused call after
    call (the reference allocates a fresh device tensor per chunk,
    halo/triton_chunked.py:340-341);
  * attention over GPU-resident chunks runs while copies are in flight; a
    copied chunk is merged as soon as its event fires (the LSE merge is
    order-free, tests/test_triton_chunked.py:263-275 in the reference).
All streams are created at the default priority.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Optional, Sequence

import torch

from .decode import ChunkRef, build_plan, launch


class MemoryTier(str, Enum):
    """Symbolic tier names, fast to slow (halo/memory_tier.py:31-42)."""

    GPU = "gpu"
    DRAM = "dram"
    NVME = "nvme"

    @classmethod
    def from_name(cls, name) -> "MemoryTier":
        if isinstance(name, cls):
            return name
        return cls(str(name).lower())


_COPY_STREAMS: dict = {}


def copy_stream(device) -> torch.cuda.Stream:
    """The per-device side stream used for host<->device tier traffic."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    s = _COPY_STREAMS.get(idx)
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _COPY_STREAMS[idx] = s
    return s


def stream_cold_chunks(q3: torch.Tensor, cold_chunks_host: Sequence, *, scale: float,
                       q_pos: torch.Tensor, m: torch.Tensor, l: torch.Tensor, o: torch.Tensor,
                       n_buffers: int = 2) -> int:
    """Copy each ``(k_host, v_host, chunk_start)`` chunk into one of
    ``n_buffers`` HBM staging slots on the copy stream and merge it into the
    (m, l, o) accumulators on the current stream as soon as it lands.
    Returns the number of bytes copied."""
    compute = torch.cuda.current_stream()
    cs = copy_stream(q3.device)
    B, H, D = q3.shape
    n_buffers = max(1, int(n_buffers))
    shapes = [tuple(k.shape) for (k, _, _) in cold_chunks_host]
    numel = max(int(torch.Size(s).numel()) for s in shapes)
    dtype = cold_chunks_host[0][0].dtype
    slots = [(torch.empty(numel, dtype=dtype, device=q3.device),
              torch.empty(numel, dtype=dtype, device=q3.device)) for _ in range(n_buffers)]
    slot_free = [torch.cuda.Event() for _ in range(n_buffers)]
    copied = [torch.cuda.Event() for _ in range(n_buffers)]
    for ev in slot_free:
        ev.record(compute)
    nbytes = 0
    for i, (k_h, v_h, c0) in enumerate(cold_chunks_host):
        s = i % n_buffers
        kb = slots[s][0][: k_h.numel()].view(k_h.shape)
        vb = slots[s][1][: v_h.numel()].view(v_h.shape)
        with torch.cuda.stream(cs):
            cs.wait_event(slot_free[s])
            kb.copy_(k_h, non_blocking=True)
            vb.copy_(v_h, non_blocking=True)
            copied[s].record(cs)
        nbytes += k_h.numel() * k_h.element_size() + v_h.numel() * v_h.element_size()
        compute.wait_event(copied[s])
        plan = build_plan(B=B, H=H, H_kv=k_h.shape[1], D=D, dtype=dtype,
                          chunks=[ChunkRef(kb, vb, int(c0), True)], device=q3.device)
        launch(plan, q3, scale=scale, q_pos=q_pos, m=m, l=l, o=o, acc_mode=3)
        slot_free[s].record(compute)
    for kb, vb in slots:
        kb.record_stream(cs)
        vb.record_stream(cs)
    return nbytes
