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


@dataclass
class _BlockBuffer:
    """One tier's block store: keys/values (L, max_blocks, H_kv, block_size, D)."""

    keys: torch.Tensor
    values: torch.Tensor

    def block(self, layer: int, block: int):
        return self.keys[layer, block], self.values[layer, block]

    def write(self, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        # pinned host <-> device copies are hipMemcpyAsync on the current stream
        self.keys[layer, block].copy_(keys, non_blocking=True)
        self.values[layer, block].copy_(values, non_blocking=True)


class _FileBuffer:
    """NVMe tier: one byte-addressed numpy memmap per K and V; blocks are
    read into host memory and written from it (halo/memory_tier.py:61-102)."""

    def __init__(self, shape, dtype: torch.dtype, path: str) -> None:
        import os

        import numpy as np
        self.shape = tuple(shape)
        self.dtype = dtype
        self.itemsize = torch.tensor([], dtype=dtype).element_size()
        per_block = int(np.prod(self.shape[2:])) * self.itemsize
        self.per_block = per_block
        total = self.shape[0] * self.shape[1] * per_block
        os.makedirs(path, exist_ok=True)
        self._k = np.memmap(os.path.join(path, "keys.bin"), dtype=np.uint8, mode="w+", shape=(total,))
        self._v = np.memmap(os.path.join(path, "values.bin"), dtype=np.uint8, mode="w+", shape=(total,))

    def _span(self, layer: int, block: int):
        s = (layer * self.shape[1] + block) * self.per_block
        return s, s + self.per_block

    def block(self, layer: int, block: int):
        s, e = self._span(layer, block)
        out = []
        for mm in (self._k, self._v):
            buf = torch.frombuffer(bytearray(mm[s:e].tobytes()), dtype=self.dtype)
            out.append(buf.view(*self.shape[2:]))
        return out[0], out[1]

    def write(self, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        s, e = self._span(layer, block)
        for mm, src in ((self._k, keys), (self._v, values)):
            host = src.detach().contiguous().cpu()
            mm[s:e] = host.view(torch.uint8).numpy().reshape(-1)
        self._k.flush()
        self._v.flush()


class TieredStorage:
    """Per-tier block stores and a per-(layer, block) tier directory
    (halo/memory_tier.py:105-226).  Tier buffers are allocated on first use;
    the DRAM tier is pinned when the GPU tier is a device, so block moves are
    asynchronous copies on the caller's stream.  The default tier of an
    unknown block is GPU."""

    def __init__(self, *, tiers, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int,
                 dtype: torch.dtype, device, nvme_path: Optional[str] = None, max_blocks: int = 4096) -> None:
        self.tiers = [MemoryTier.from_name(t) for t in tiers]
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.gpu_device = torch.device(device)
        self.max_blocks = max_blocks
        self._shape = (num_layers, max_blocks, num_kv_heads, block_size, head_dim)
        self._nvme_path = nvme_path
        self._directory: dict = {}
        self._buffers: dict = {}

    def move_block(self, *, layer: int, block: int, src, dst) -> None:
        s, d = MemoryTier.from_name(src), MemoryTier.from_name(dst)
        if s == d:
            return
        k, v = self._buffer(s).block(layer, block)
        self._buffer(d).write(layer, block, k, v)
        self._directory[(layer, block)] = d

    def locate_block(self, *, layer: int, block: int) -> str:
        return self._directory.get((layer, block), MemoryTier.GPU).value

    def write_new_block(self, *, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor,
                        tier: str = "gpu") -> None:
        t = MemoryTier.from_name(tier)
        self._buffer(t).write(layer, block, keys, values)
        self._directory[(layer, block)] = t

    def read_block(self, *, layer: int, block: int):
        t = self._directory.get((layer, block), MemoryTier.GPU)
        return self._buffer(t).block(layer, block)

    def _buffer(self, tier: MemoryTier):
        buf = self._buffers.get(tier)
        if buf is not None:
            return buf
        if tier not in self.tiers:
            raise ValueError(f"Tier {tier} not requested at construction time.")
        if tier is MemoryTier.GPU:
            buf = _BlockBuffer(torch.empty(self._shape, dtype=self.dtype, device=self.gpu_device),
                               torch.empty(self._shape, dtype=self.dtype, device=self.gpu_device))
        elif tier is MemoryTier.DRAM:
            pin = self.gpu_device.type == "cuda" and torch.cuda.is_available()
            buf = _BlockBuffer(torch.empty(self._shape, dtype=self.dtype, pin_memory=pin),
                               torch.empty(self._shape, dtype=self.dtype, pin_memory=pin))
        else:
            import os
            path = self._nvme_path or os.environ.get("HALO_NVME_PATH") or "/tmp/halo_nvme"
            buf = _FileBuffer(self._shape, self.dtype, path)
        self._buffers[tier] = buf
        return buf

    def __repr__(self) -> str:  # pragma: no cover
        return f"TieredStorage(tiers=[{','.join(t.value for t in self.tiers)}], blocks={self.max_blocks})"


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
