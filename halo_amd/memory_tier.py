"""Cold tier in pinned host DRAM, the block store behind it, and the
host-to-device staging of cold chunks (MI355X).

Reference: halo/memory_tier.py:31-258 (MemoryTier / _BlockBuffer /
_MemmapBuffer / TieredStorage) and the DMA-overlap driver of
halo/triton_chunked.py:270-362.

What changes on MI355X:
  * the tier directory is a device tensor (int8 tier code per (layer,
    block)), so a refetch or demotion schedule computed on the GPU is applied
    with no host round trip: one ``halo_copy_blocks`` launch moves every
    listed block whose directory entry names the source tier, and the
    directory entries flip afterwards on the same stream, i.e. a block reads
    as resident only once its copy has run;
  * the DRAM tier is pinned (page-locked) host memory; the copy kernel reads
    or writes it in place through its device-visible mapping;
  * a strided view of pinned memory is moved as the contiguous byte span that
    covers it (``span_to_device``) and re-viewed on the device, so the host
    never reads pinned rows itself (a host-side ``.contiguous()`` of a view
    whose device-to-host copy is still in flight reads stale rows);
  * refetch targets are a ring of HBM staging slots reused chunk after chunk
    (the reference allocates a fresh device tensor per chunk,
    halo/triton_chunked.py:340-341); attention over GPU-resident chunks runs
    while copies are in flight, a copied chunk is merged as soon as its event
    fires (the LSE merge is order-free, tests/test_triton_chunked.py:263-275
    in the reference).
All streams are created at the default priority.
"""
from __future__ import annotations

from enum import Enum
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native as nat


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


_TIER_CODE = {MemoryTier.GPU: 0, MemoryTier.DRAM: 1, MemoryTier.NVME: 2}
_CODE_TIER = {v: k for k, v in _TIER_CODE.items()}


# ---------------------------------------------------------------------------
# Streams and span copies
# ---------------------------------------------------------------------------
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


def _span(t: torch.Tensor) -> tuple[int, int]:
    """[lo, hi) element offsets in t's storage that cover every element of t."""
    if any(st < 0 for st in t.stride()):
        raise AssertionError("negative strides are not supported")
    lo = t.storage_offset()
    hi = lo + 1 + sum((n - 1) * st for n, st in zip(t.shape, t.stride()) if n > 0)
    return lo, (hi if t.numel() else lo)


def span_elems(t: torch.Tensor) -> int:
    lo, hi = _span(t)
    return hi - lo


def span_to_device(t: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """Enqueue a copy of the contiguous storage span covering ``t`` (pinned
    host memory) into the flat device buffer ``dst`` on the current stream,
    and return ``t``'s view of it on the device.  The copy is one DMA of
    plain bytes: the host touches no row of ``t``."""
    lo, hi = _span(t)
    n = hi - lo
    if dst.dim() != 1 or dst.dtype != t.dtype or dst.numel() < n:
        raise AssertionError(f"staging buffer must be 1-D {t.dtype} with >= {n} elements")
    if n == 0:
        return dst[:0].as_strided(t.shape, t.stride())
    src = torch.empty(0, dtype=t.dtype).set_(t.untyped_storage(), lo, (n,), (1,))
    dst[:n].copy_(src, non_blocking=True)
    return dst.as_strided(t.shape, t.stride(), dst.storage_offset())


def stream_cold_chunks(q3: torch.Tensor, cold_chunks_host: Sequence, *, scale: float,
                       q_pos: torch.Tensor, m: torch.Tensor, l: torch.Tensor, o: torch.Tensor,
                       n_buffers: int = 2, after: Optional[torch.cuda.Event] = None) -> int:
    """Copy each host chunk into one of ``n_buffers`` HBM staging slots on
    the copy stream and merge it into the (m, l, o) accumulators on the
    current stream as soon as it lands.

    An entry is ``(k_host, v_host, chunk_start)`` (every row, causal at
    chunk_start + t) or ``(k_host, v_host, pieces)`` with pieces a list of
    ``(row_lo, row_hi, chunk_start, causal)``: rows of the staged chunk
    attended as separate table entries.  ``after`` (an event) orders the
    first copy after work that fills the host chunks (e.g. the cold tier's
    device-to-host peel).  Returns the number of bytes copied."""
    from .decode import ChunkRef, cached_plan, launch
    compute = torch.cuda.current_stream()
    cs = copy_stream(q3.device)
    B, H, D = q3.shape
    n_buffers = max(1, int(n_buffers))
    numel = max(max(span_elems(k), span_elems(v)) for (k, v, _) in cold_chunks_host)
    dtype = cold_chunks_host[0][0].dtype
    slots = [(torch.empty(numel, dtype=dtype, device=q3.device),
              torch.empty(numel, dtype=dtype, device=q3.device)) for _ in range(n_buffers)]
    slot_free = [torch.cuda.Event() for _ in range(n_buffers)]
    copied = [torch.cuda.Event() for _ in range(n_buffers)]
    for ev in slot_free:
        ev.record(compute)
    if after is not None:
        cs.wait_event(after)
    nbytes = 0
    for i, (k_h, v_h, spec) in enumerate(cold_chunks_host):
        pieces = [(0, k_h.shape[-2], int(spec), True)] if isinstance(spec, (int, np.integer)) else list(spec)
        if not pieces:
            continue
        s = i % n_buffers
        with torch.cuda.stream(cs):
            cs.wait_event(slot_free[s])
            kb = span_to_device(k_h, slots[s][0])
            vb = span_to_device(v_h, slots[s][1])
            copied[s].record(cs)
        nbytes += (span_elems(k_h) + span_elems(v_h)) * k_h.element_size()
        compute.wait_event(copied[s])
        refs = [ChunkRef(kb[..., lo:hi, :], vb[..., lo:hi, :], int(c0), bool(causal))
                for lo, hi, c0, causal in pieces]
        plan = cached_plan(B=B, H=H, H_kv=k_h.shape[1], D=D, dtype=dtype, chunks=refs, device=q3.device)
        launch(plan, q3, scale=scale, q_pos=q_pos, m=m, l=l, o=o, acc_mode=3)
        slot_free[s].record(compute)
    for kb, vb in slots:
        kb.record_stream(cs)
        vb.record_stream(cs)
    return nbytes


# ---------------------------------------------------------------------------
# Block store
# ---------------------------------------------------------------------------
class _BlockBuffer:
    """One tier's block store: keys/values (L, max_blocks, H_kv, block_size, D)
    in device memory or pinned host memory."""

    def __init__(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        self.keys, self.values = keys, values
        self._dev_addr = None

    def block(self, layer: int, block: int):
        return self.keys[layer, block], self.values[layer, block]

    def write(self, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        self.keys[layer, block].copy_(keys, non_blocking=True)
        self.values[layer, block].copy_(values, non_blocking=True)

    def layer_addr(self, layer: int) -> tuple[int, int]:
        """Device-visible addresses of this layer's K and V blocks."""
        if self._dev_addr is None:
            if self.keys.is_cuda:
                self._dev_addr = (self.keys.data_ptr(), self.values.data_ptr())
            else:
                self._dev_addr = (nat.host_device_pointer(self.keys.data_ptr()),
                                  nat.host_device_pointer(self.values.data_ptr()))
        stride = self.keys.stride(0) * self.keys.element_size()
        return self._dev_addr[0] + layer * stride, self._dev_addr[1] + layer * stride


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

    def _range(self, layer: int, block: int):
        s = (layer * self.shape[1] + block) * self.per_block
        return s, s + self.per_block

    def block(self, layer: int, block: int):
        s, e = self._range(layer, block)
        out = []
        for mm in (self._k, self._v):
            buf = torch.frombuffer(bytearray(mm[s:e].tobytes()), dtype=self.dtype)
            out.append(buf.view(*self.shape[2:]))
        return out[0], out[1]

    def write(self, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        s, e = self._range(layer, block)
        for mm, src in ((self._k, keys), (self._v, values)):
            host = src.detach().contiguous().cpu()
            mm[s:e] = host.view(torch.uint8).numpy().reshape(-1)
        self._k.flush()
        self._v.flush()

    def read_runs(self, layer: int, ids, out_k, out_v) -> None:
        """Blocks ``ids`` (sorted, unique) of ``layer`` into the uint8 arrays
        out_k / out_v (len(ids), per_block): one slice copy per run of
        consecutive block indices."""
        for i0, i1 in _runs_of(ids):
            s, _ = self._range(layer, int(ids[i0]))
            e = s + (i1 - i0) * self.per_block
            out_k[i0:i1] = self._k[s:e].reshape(i1 - i0, self.per_block)
            out_v[i0:i1] = self._v[s:e].reshape(i1 - i0, self.per_block)

    def write_runs(self, layer: int, ids, src_k, src_v) -> None:
        """The inverse of ``read_runs``; flushes once."""
        for i0, i1 in _runs_of(ids):
            s, _ = self._range(layer, int(ids[i0]))
            e = s + (i1 - i0) * self.per_block
            self._k[s:e] = src_k[i0:i1].reshape(-1)
            self._v[s:e] = src_v[i0:i1].reshape(-1)
        self._k.flush()
        self._v.flush()


def _runs_of(ids):
    """(start, end) index ranges of runs of consecutive values in sorted ids."""
    n = len(ids)
    i = 0
    while i < n:
        j = i + 1
        while j < n and int(ids[j]) == int(ids[j - 1]) + 1:
            j += 1
        yield i, j
        i = j


class TieredStorage:
    """Per-tier block stores and a per-(layer, block) tier directory
    (halo/memory_tier.py:105-226).

    Tier buffers are allocated on first use; the DRAM tier is pinned when
    the GPU tier is a device.  The directory is an int8 tensor on the GPU
    tier's device (0 = gpu, 1 = dram, 2 = nvme; an unknown block reads as
    gpu, the reference's default).  ``move_blocks`` applies a device-side
    block list in one launch; ``move_block`` / ``locate_block`` are the
    reference's per-block calls on top of it."""

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
        self._buffers: dict = {}
        self._dir: Optional[torch.Tensor] = None

    # ----------------------------------------------------------- directory
    @property
    def on_device(self) -> bool:
        return self.gpu_device.type == "cuda"

    def directory(self) -> torch.Tensor:
        """The (L, max_blocks) int8 tier codes (device tensor on a GPU tier)."""
        if self._dir is None:
            self._dir = torch.zeros((self.num_layers, self.max_blocks), dtype=torch.int8, device=self.gpu_device)
        return self._dir

    @staticmethod
    def tier_code(tier) -> int:
        return _TIER_CODE[MemoryTier.from_name(tier)]

    def locate_block(self, *, layer: int, block: int) -> str:
        """Tier of one block (reads the directory: a host sync on a device)."""
        return _CODE_TIER[int(self.directory()[layer, block].item())].value

    @property
    def block_bytes(self) -> int:
        return self.num_kv_heads * self.block_size * self.head_dim * torch.tensor([], dtype=self.dtype).element_size()

    # ----------------------------------------------------------- single blocks
    def move_block(self, *, layer: int, block: int, src, dst) -> None:
        s, d = MemoryTier.from_name(src), MemoryTier.from_name(dst)
        if s == d:
            return
        if not self.on_device:
            k, v = self._buffer(s).block(layer, block)
            self._buffer(d).write(layer, block, k, v)
            self.directory()[layer, block] = _TIER_CODE[d]
            return
        blocks = torch.tensor([block], dtype=torch.int32).to(self.gpu_device, non_blocking=True)
        self.move_blocks(layer=layer, blocks=blocks, src=s, dst=d, only_if_in_src=False)

    def write_new_block(self, *, layer: int, block: int, keys: torch.Tensor, values: torch.Tensor,
                        tier: str = "gpu") -> None:
        t = MemoryTier.from_name(tier)
        self._buffer(t).write(layer, block, keys, values)
        self.directory()[layer, block] = _TIER_CODE[t]

    def read_block(self, *, layer: int, block: int):
        t = MemoryTier.from_name(self.locate_block(layer=layer, block=block))
        return self._buffer(t).block(layer, block)

    # ----------------------------------------------------------- batched moves
    def move_blocks(self, *, layer: int, blocks: torch.Tensor, src, dst, only_if_in_src: bool = True,
                    stream: Optional[torch.cuda.Stream] = None) -> None:
        """Move every block of ``blocks`` (int32 tensor on the GPU tier's
        device; entries < 0 are skipped) from tier ``src`` to ``dst`` in one
        launch on ``stream`` (default: current).  With ``only_if_in_src`` a
        block moves only when the directory says it is in ``src``; the
        directory entries of moved blocks become ``dst`` after the copy, in
        stream order."""
        s, d = MemoryTier.from_name(src), MemoryTier.from_name(dst)
        if s == d:
            return
        if blocks.numel() == 0:
            return
        if not self.on_device:
            self._move_blocks_host(layer, blocks, s, d, only_if_in_src)
            return
        if MemoryTier.NVME in (s, d):
            self._move_blocks_nvme(layer, blocks, s, d, only_if_in_src, stream)
            return
        L = nat.lib()
        blocks = blocks.to(device=self.gpu_device, dtype=torch.int32).contiguous()
        dirl = self.directory()[layer]
        sb, db = self._buffer(s), self._buffer(d)
        src_k, src_v = sb.layer_addr(layer)
        dst_k, dst_v = db.layer_addr(layer)
        strm = stream if stream is not None else torch.cuda.current_stream(self.gpu_device)
        with torch.cuda.stream(strm):
            code_s, code_d = _TIER_CODE[s], _TIER_CODE[d]
            nat.check(L.halo_copy_blocks(dst_k, src_k, dst_v, src_v, self.block_bytes, blocks.data_ptr(),
                                         blocks.numel(), self.max_blocks,
                                         dirl.data_ptr() if only_if_in_src else None, code_s,
                                         nat.stream_ptr(strm)), "halo_copy_blocks")
            # the moved blocks' entries only (a whole-row rewrite would undo a
            # concurrent move of other blocks on another stream)
            nat.check(L.halo_set_tier(dirl.data_ptr(), blocks.data_ptr(), blocks.numel(), self.max_blocks,
                                      code_s if only_if_in_src else -1, code_d, nat.stream_ptr(strm)),
                      "halo_set_tier")
        blocks.record_stream(strm)

    def _move_blocks_nvme(self, layer: int, blocks: torch.Tensor, s: MemoryTier, d: MemoryTier,
                          only_if_in_src: bool, stream: Optional[torch.cuda.Stream]) -> None:
        """Moves to or from the NVMe tier of a device-backed store, batched:
        one host read of the block list and of the layer's directory row, the
        file touched once per run of consecutive blocks, one pinned staging
        buffer, one host<->device copy and one gather (or scatter) kernel for
        the GPU side, and the directory entries updated on the device.  File
        I/O needs the bytes on the host, so a move out of the GPU waits for
        its device-to-host copy (the reference's per-block ``.cpu()``,
        halo/memory_tier.py:86-102, does the same once per block)."""
        import numpy as np
        strm = stream if stream is not None else torch.cuda.current_stream(self.gpu_device)
        dirl = self.directory()[layer]
        with torch.cuda.stream(strm):
            ids = np.unique(blocks.reshape(-1).to("cpu").numpy().astype(np.int64))
            ids = ids[(ids >= 0) & (ids < self.max_blocks)]
            if only_if_in_src and ids.size:
                codes = dirl.to("cpu").numpy()
                ids = ids[codes[ids] == _TIER_CODE[s]]
            if ids.size == 0:
                return
            n = int(ids.size)
            ids_dev = torch.from_numpy(ids).to(self.gpu_device, non_blocking=True)
            item = (self.num_kv_heads, self.block_size, self.head_dim)
            sb, db = self._buffer(s), self._buffer(d)

            def as_bytes(t: torch.Tensor):
                return t.view(torch.uint8).numpy().reshape(t.shape[0], -1)

            if s is MemoryTier.NVME:
                stg_k = torch.empty((n,) + item, dtype=self.dtype, pin_memory=True)
                stg_v = torch.empty_like(stg_k, pin_memory=True)
                sb.read_runs(layer, ids, as_bytes(stg_k), as_bytes(stg_v))
                if d is MemoryTier.GPU:
                    db.keys[layer].index_copy_(0, ids_dev, stg_k.to(self.gpu_device, non_blocking=True))
                    db.values[layer].index_copy_(0, ids_dev, stg_v.to(self.gpu_device, non_blocking=True))
                else:  # DRAM: host memory, written in place after queued device work on it
                    strm.synchronize()
                    db.keys[layer][torch.from_numpy(ids)] = stg_k
                    db.values[layer][torch.from_numpy(ids)] = stg_v
            else:
                if s is MemoryTier.GPU:
                    stg_k = torch.empty((n,) + item, dtype=self.dtype, pin_memory=True)
                    stg_v = torch.empty_like(stg_k, pin_memory=True)
                    stg_k.copy_(sb.keys[layer].index_select(0, ids_dev), non_blocking=True)
                    stg_v.copy_(sb.values[layer].index_select(0, ids_dev), non_blocking=True)
                    strm.synchronize()
                else:  # DRAM: read on the host once queued device writes to it landed
                    strm.synchronize()
                    idx = torch.from_numpy(ids)
                    stg_k, stg_v = sb.keys[layer][idx], sb.values[layer][idx]
                db.write_runs(layer, ids, as_bytes(stg_k), as_bytes(stg_v))
            dirl.index_fill_(0, ids_dev, _TIER_CODE[d])

    def _move_blocks_host(self, layer: int, blocks: torch.Tensor, s: MemoryTier, d: MemoryTier,
                          only_if_in_src: bool) -> None:
        dirl = self.directory()[layer]
        for b in blocks.reshape(-1).tolist():
            if b < 0 or b >= self.max_blocks:
                continue
            if only_if_in_src and int(dirl[b].item()) != _TIER_CODE[s]:
                continue
            k, v = self._buffer(s).block(layer, b)
            self._buffer(d).write(layer, b, k, v)
            dirl[b] = _TIER_CODE[d]

    # ----------------------------------------------------------- buffers
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
            pin = self.on_device and torch.cuda.is_available()
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
