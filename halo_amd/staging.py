"""HBM staging cache for cold chunks kept in pinned host memory.

A stack of tiered decode layers (``TieredDecodeLayer`` whose cold chunks
live in pinned host DRAM) selects its top-k cold chunks inside the attention
launch every step.  Without staging, every selected chunk is read in place
over the host link.  This cache keeps up to ``n_slots`` cold chunks per layer
in HBM slots and points the in-kernel selection at them through a per-chunk
residency entry (``halo_select_cfg.residency``): a chosen chunk whose entry
names a slot is read from HBM (a hit), otherwise in place from host memory
(a miss, still exact: the rows are the same).

The host side (feedback ring, accounting, policy, fill issue, commits) is
the library's native runtime (``halo_staging_*`` in include/halo_hip.h), one
C call per segment of layers; this class owns the device buffers, points the
layers' selections at them and wraps the runtime.

Policy (reference: HALORefetcher.predict_hot / schedule,
halo/refetcher.py:38-114 -- predict the next hot set as the top
(hot + lookahead) by the last score and fetch what is missing on a side
stream): the layers' chunk scores, written by the selection itself, come
back to the host through a small pinned ring; the ``keep`` best-scoring
chunks of each layer are the predicted set, and those not staged are copied
host-to-device into free slots with ``hipMemcpyAsync`` on the copy stream,
best ranks first across layers, at most ``max_inflight`` copies in flight.

Ordering (no kernel observes a change while it runs):
  * a fill copies the chunk's rows into a slot that no residency entry
    names, on the copy stream, and records an event (slot descriptors never
    change: the kernel takes a staged chunk's rows, start and flags from its
    own catalog entry and only the addresses from the slot);
  * a fill whose event has completed is committed before the next launches
    of its layer: one batched store of residency entries on the compute
    stream; every launch after it reads the slot, every launch before it read
    host memory.  A fill still in flight is committed later, except an urgent
    one (a chunk among its layer's current top-k, which the next launch would
    otherwise read over the link): the compute stream waits for its copy;
  * evictions are decided only for layers whose feedback just came back:
    every launch of such a layer has finished (the kernel that published its
    feedback ran behind it) and its next launch is not enqueued yet.  So the slot can take a
    fill at once, and the eviction's -1 store goes out with the layer's next
    ``before_step`` batch, ahead of that batch's commits: it runs before any
    later launch of the layer, and the new chunk's entry is committed only
    after it (``drain`` flushes the stores still held).
A step may run as consecutive segments of layers (one graph each): a
segment's scores are planned while the later segments execute, so the
scores of step t can decide that segment's residency from step t + 1 on.
Hit and miss counts come from ``res_out``: the entry the kernel actually
used for each chosen chunk.

Write-allocate (16-bit layers, one selection per launch): each layer keeps
two reserved free slots and names one of them in ``halo_select_cfg.
alloc_slot`` for each launch, alternating between launches.  The launch's
first chosen chunk that is not staged is read in place (a miss, as before)
and its rows are also written into that slot by the kernel; ``res_out``
reports it, and the host commits the slot as the chunk's residency when it
processes that feedback, so a missed chunk crosses the host link once
instead of being fetched again by a fill.  The two reservations alternate
because feedback lags the launches: a reservation is named again only once
the feedback of the launch that last named it has been processed (else the
launch gets none), so a slot the host commits still holds what that launch
wrote.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native as nat
from .decode import ChunkRef, descs_to_device, pack_descs
from .memory_tier import copy_stream

_FREE, _FILLING, _READY, _RESERVED = 0, 1, 2, 4
_FILL_MODE = {"dma": 0, "kernel": 1}


class ColdStaging:
    """HBM staging slots + residency for the cold chunks of ``layers``.

    ``layers``: ``TieredDecodeLayer`` objects with the fused in-kernel
    selection over cold chunks held as contiguous pinned host tensors, the
    same number of cold chunks each -- or ``RaggedTieredDecodeLayer``
    objects (per-row selection), where every batch row is a unit of its own:
    its own cold chunks (ragged counts), slots and policy.  ``n_slots`` HBM
    slots per unit (each the size of the unit's widest cold chunk); ``keep``
    best-scoring chunks per unit are staged (default n_slots - 2); ``spare``
    slots per unit are kept free (staged chunks outside the kept set are
    evicted worst rank first to keep them); ``max_inflight`` bounds the copies in flight on the
    link; ``write_allocate`` reserves two slots per layer for missed chunks
    the kernel writes while reading them (16-bit layers with one selection
    per launch; ignored otherwise).  It pays when the selection moves fast
    (fewer bytes over the link) and costs hits when it moves slowly (the
    reserved slots are missing from the cache).  ``fill_mode`` "dma" copies
    with hipMemcpyAsync, "kernel" with copy kernels that read the pinned
    chunk in place; ``urgent_stream`` gives fills the next launch waits for
    a copy stream of their own; ``copy_streams`` 2 alternates the other DMA
    fills between two copy streams (two DMA engines overlap each copy's
    start-up: 4 MiB pieces move at ~56 GB/s instead of ~46 on one stream).
    Fills then land sooner, but leave chunks read in place over the link
    (misses, on their layer's critical path) less of it: a 131072-token
    layer with 96 cold chunks gains (1.06 against 1.13 ms per 16-layer
    step), a 32768-token one loses (0.91-0.96 against 0.87 ms per 32-layer
    step), so the default is 1.  ``track_busy`` counts operations issued
    while the compute stream still had work queued (a test aid)."""

    def __init__(self, layers: Sequence, *, n_slots: int = 12, keep: Optional[int] = None,
                 max_inflight: int = 8, spare: int = 0, ring: int = 16, write_allocate: bool = False,
                 fill_mode: str = "dma", urgent_stream: bool = True, copy_streams: int = 1,
                 track_busy: bool = False) -> None:
        if not layers:
            raise AssertionError("no layers")
        self.layers = list(layers)
        lay0 = self.layers[0]
        self.device = lay0.plan.descs.device
        self.top_k = lay0.top_k
        # fused layers select in the attention launch (halo_select_cfg);
        # unfused ones (beyond the fused selection's limits) run the staged
        # scorer (halo_chunk_score_topk_staged) before the attention launch
        for li, lay in enumerate(self.layers):
            fused = getattr(lay, "select_cfg", None) is not None and getattr(lay, "fused", True)
            if not fused and not hasattr(lay, "staging"):
                raise AssertionError(f"layer {li}: no selection that staging can drive")
        per_row_of = [bool(lay.select_cfg.per_row) if getattr(lay, "select_cfg", None) is not None else False
                      for lay in self.layers]
        self.all_fused = all(getattr(lay, "select_cfg", None) is not None for lay in self.layers)
        # the cache's unit is a selection: the layer's one selection, or one
        # per batch row of a layer with per-row selection (ragged batches)
        self.per_row = per_row_of[0]
        self.sels = lay0.B if self.per_row else 1
        units = []                          # cold chunks of each unit, unit = layer * sels + row
        for li, lay in enumerate(self.layers):
            if per_row_of[li] != self.per_row or (lay.B if self.per_row else 1) != self.sels \
                    or lay.top_k != self.top_k:
                raise AssertionError("every layer must have the same selections per layer and top_k")
            units += [list(cold) for _, cold in lay.rows] if self.per_row else [list(lay.cold)]
        self.n_cold = int(lay0.select_cfg.catalog_stride) if self.per_row else len(lay0.cold)
        if any(len(u) > self.n_cold for u in units) or any(
                int(lay.select_cfg.catalog_stride if self.per_row else len(lay.cold)) != self.n_cold
                for lay in self.layers):
            raise AssertionError("every layer must have the same number of cold chunks (catalog stride)")
        if not 1 <= n_slots <= 64:
            raise AssertionError("n_slots must be in [1, 64]")
        self.n_slots = int(n_slots)
        self.keep = int(keep if keep is not None else max(self.top_k, n_slots - 2))
        if not self.top_k <= self.keep <= self.n_slots:
            raise AssertionError(f"keep={self.keep} must be in [top_k={self.top_k}, n_slots={self.n_slots}]")
        if fill_mode not in _FILL_MODE:
            raise AssertionError("fill_mode must be 'kernel' or 'dma'")
        if copy_streams not in (1, 2):
            raise AssertionError(f"copy_streams must be 1 or 2, got {copy_streams}")
        self.fill_mode = fill_mode
        self.spare = int(spare)
        self._max_inflight = int(max_inflight)
        for ui, cold in enumerate(units):
            for c in cold:
                if c.k.device.type != "cpu" or not c.k.is_pinned() or not c.k.is_contiguous() \
                        or not c.v.is_contiguous():
                    raise AssertionError(f"layer {ui // self.sels}: cold chunks must be contiguous pinned host "
                                         f"tensors")
        L, n, k, Bs = len(self.layers), self.n_cold, self.top_k, self.sels
        U = L * Bs
        dev = self.device
        # residency (U, n) and the per-layer write-allocate slot (L) in one
        # device buffer, so one store kernel updates both
        self._dev_i32 = torch.full((U * n + L,), -1, dtype=torch.int32, device=dev)
        self.residency = self._dev_i32[:U * n].view(L, Bs * n)
        self.alloc = self._dev_i32[U * n:]
        self.write_allocate = bool(write_allocate) and self.all_fused and not self.per_row \
            and self.n_slots >= self.top_k + 2 and all(lay.dtype != torch.float32 for lay in self.layers)
        # one feedback row per layer, as the selection writes it:
        # scores (sels, n) fp32 | picks (sels, k) int32 | residency used (sels, k) int32
        W = Bs * (n + 2 * k)
        self.feedback = torch.zeros((L, W), dtype=torch.float32, device=dev)
        scores = self.feedback[:, :Bs * n]
        idx = self.feedback[:, Bs * n:Bs * (n + k)].view(torch.int32)
        res = self.feedback[:, Bs * (n + k):].view(torch.int32)
        idx.fill_(-1)
        res.fill_(-1)
        if self.per_row:
            self.scores, self.idx, self.res_out = scores.view(L, Bs, n), idx.view(L, Bs, k), res.view(L, Bs, k)
        else:
            self.scores, self.idx, self.res_out = scores, idx, res
        self.chunk_bytes = np.zeros((U, n), dtype=np.int64)
        self._slot_k, self._slot_v, self._slot_cat = [], [], []
        # slot (unit, s) K/V addresses, cold chunk (unit, c) K/V addresses, bytes per tensor
        dst = np.zeros((U, self.n_slots, 2), dtype=np.uint64)
        src = np.zeros((U, n, 2), dtype=np.uint64)
        nbytes = np.zeros((U, n), dtype=np.int64)
        ncold = np.asarray([len(u) for u in units], dtype=np.int32)
        for li, lay in enumerate(self.layers):
            sdescs = []
            for r in range(Bs):
                ui = li * Bs + r
                cold = units[ui]
                if cold:
                    shape = max((tuple(c.k.shape) for c in cold), key=lambda sh: sh[-2])
                elif self.per_row:
                    shape = (lay.H_kv, 1, lay.D)
                else:
                    raise AssertionError(f"layer {li} has no cold chunks")
                # a slot's K rows and V rows are adjacent, so a cold chunk laid
                # out the same way on the host is filled by one copy
                skv = torch.empty((self.n_slots, 2) + shape, dtype=lay.dtype, device=dev)
                sk, sv = skv[:, 0], skv[:, 1]
                # slot descriptors never change: they give the addresses and
                # strides a staged chunk is read through; its rows, start, flags
                # and batch come from the chunk's own catalog entry
                d, _ = pack_descs([ChunkRef(sk[s], sv[s], 0, False, r if self.per_row else -1)
                                   for s in range(self.n_slots)], B=lay.B, H_kv=lay.H_kv, D=lay.D, dtype=lay.dtype)
                sdescs.append(d)
                self._slot_k.append(sk)
                self._slot_v.append(sv)
                for j in range(self.n_slots):
                    dst[ui, j] = (sk[j].data_ptr(), sv[j].data_ptr())
                for j, c in enumerate(cold):
                    if tuple(c.k.shape) != tuple(sk.shape[1:]):
                        raise AssertionError(f"layer {li} cold chunk {j}: shape {tuple(c.k.shape)} differs from the "
                                             f"unit's other cold chunks {tuple(sk.shape[1:])}")
                    if fill_mode == "kernel":   # the copy kernel reads the pinned chunk in place
                        src[ui, j] = (nat.host_device_pointer(c.k.data_ptr()),
                                      nat.host_device_pointer(c.v.data_ptr()))
                    else:
                        src[ui, j] = (c.k.data_ptr(), c.v.data_ptr())
                    nbytes[ui, j] = c.k.numel() * c.k.element_size()
                self.chunk_bytes[ui] = 2 * nbytes[ui]
            self._slot_cat.append(descs_to_device(np.concatenate(sdescs), dev))
            cfg = lay.select_cfg
            if cfg is None:
                # the staged scorer writes the feedback row and the table
                lay.idx, lay.scores = idx[li:li + 1], scores[li:li + 1]
                lay.staging = (self.residency[li], self._slot_cat[li], self.n_slots, res[li])
                continue
            cfg.n_slots = self.n_slots
            cfg.slot_catalog = self._slot_cat[li].data_ptr()
            cfg.residency = self.residency[li].data_ptr()
            cfg.res_out = res[li].data_ptr()
            cfg.score_out = scores[li].data_ptr()
            cfg.idx_out = idx[li].data_ptr()
            cfg.alloc_slot = self.alloc[li].data_ptr() if self.write_allocate else None
        # the copy streams outlive the runtime (it holds their handles)
        self._copy = copy_stream(dev)
        # urgent fills (chunks the next launch of their layer selects) go on a
        # stream of their own, so they share the link with the prefetches
        # queued before them instead of waiting behind them
        self._urgent = torch.cuda.Stream(device=dev) if urgent_stream else None
        self._copy2 = torch.cuda.Stream(device=dev) if copy_streams == 2 else None
        self._addr = (dst, src, nbytes, ncold)    # read at creation; kept for inspection
        d = nat.StagingDesc(n_layers=L, n_cold=n, n_slots=self.n_slots, top_k=k, keep=self.keep,
                            max_inflight=self._max_inflight, spare=self.spare, ring=max(2, int(ring)),
                            write_allocate=int(self.write_allocate), fill_mode=_FILL_MODE[fill_mode],
                            track_busy=int(track_busy), sels_per_layer=Bs, residency=self._dev_i32.data_ptr(),
                            feedback=self.feedback.data_ptr(), slot_addr=dst.ctypes.data,
                            chunk_addr=src.ctypes.data, chunk_nbytes=nbytes.ctypes.data,
                            n_cold_per_unit=ncold.ctypes.data, copy_stream=self._copy.cuda_stream,
                            urgent_stream=self._urgent.cuda_stream if self._urgent is not None else None,
                            copy_stream2=self._copy2.cuda_stream if self._copy2 is not None else None)
        self._L = nat.lib()
        h = ctypes.c_void_p()
        nat.check(self._L.halo_staging_create(ctypes.byref(d), ctypes.byref(h)), "halo_staging_create")
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._L.halo_staging_destroy(h)
            self._h = None

    # ----------------------------------------------------------------- per step
    # ``lo``/``hi`` name a segment of layers [lo, hi) run as one graph; the
    # defaults cover every layer.
    def before_step(self, lo: int = 0, hi: Optional[int] = None) -> None:
        """Commit the fills of layers [lo, hi) that have landed, and the
        urgent ones (chunks among the layer's current top-k, which the next
        launch would otherwise read over the link) after a device-side wait
        for their copy, with one batched store of residency entries on the
        compute stream.  Call before enqueueing those layers' launches."""
        hi = len(self.layers) if hi is None else hi
        nat.check(self._L.halo_staging_before(self._h, lo, hi, nat.stream_ptr()), "halo_staging_before")

    def after_step(self, lo: int = 0, hi: Optional[int] = None) -> None:
        """Mark the feedback rows of layers [lo, hi) (scores, picks,
        residency used) for the host.  The next ``before_step`` on the same
        stream enqueues one small kernel that writes the rows into a pinned
        ring entry and stores that call's residency entries (``service`` and
        ``drain`` publish a marked entry themselves when they must wait for
        it)."""
        hi = len(self.layers) if hi is None else hi
        rc = self._L.halo_staging_after(self._h, lo, hi, nat.stream_ptr())
        if rc == nat.HALO_E_INVALID and b"overrun" in self._L.halo_last_error():
            raise RuntimeError("feedback ring overrun: call service() after every after_step()")
        nat.check(rc, "halo_staging_after")

    def drain(self) -> None:
        """Process every queued segment's feedback now (waits for it)."""
        self.service(lag=0)

    def service(self, *, lag: int = 1) -> None:
        """Process returned feedback -- waiting for every queued segment but
        the ``lag`` newest, and taking those too when they are done -- count
        hits and misses, and plan evictions and fills for the processed
        segments' layers."""
        nat.check(self._L.halo_staging_service(self._h, int(lag), nat.stream_ptr()), "halo_staging_service")

    # ----------------------------------------------------------------- control
    def clear(self) -> None:
        """Empty every slot (synchronises the device first)."""
        torch.cuda.synchronize(self.device)
        nat.check(self._L.halo_staging_reset(self._h), "halo_staging_reset")
        self._dev_i32.fill_(-1)
        torch.cuda.synchronize(self.device)

    @property
    def max_inflight(self) -> int:
        return self._max_inflight

    @max_inflight.setter
    def max_inflight(self, v: int) -> None:
        self._max_inflight = int(v)
        nat.check(self._L.halo_staging_set(self._h, self._max_inflight, 0), "halo_staging_set")

    def reset_counters(self) -> None:
        nat.check(self._L.halo_staging_set(self._h, self._max_inflight, 1), "halo_staging_set")

    def _snapshot(self):
        L = len(self.layers)
        U = L * self.sels
        stats = nat.StagingStats()
        state = np.empty((U, self.n_slots), dtype=np.int8)
        holds = np.empty((U, self.n_slots), dtype=np.int64)
        wa = np.empty((L, 2), dtype=np.int64)
        nat.check(self._L.halo_staging_get(self._h, ctypes.byref(stats), state.ctypes.data, holds.ctypes.data,
                                           wa.ctypes.data), "halo_staging_get")
        return stats, state, holds, wa

    @property
    def stats(self) -> dict:
        s = self._snapshot()[0]
        return {name: int(getattr(s, name)) for name, _ in nat.StagingStats._fields_}

    def __getattr__(self, name):
        # counters of the native runtime: hits, misses, misses_predicted,
        # fills, fill_bytes, miss_bytes, wa_commits, wa_dups, *_while_busy
        if name in {f for f, _ in nat.StagingStats._fields_}:
            return int(getattr(self._snapshot()[0], name))
        raise AttributeError(name)

    @property
    def state(self) -> np.ndarray:
        """Slot states (units, n_slots): 0 free, 1 filling, 2 ready, 4
        reserved; unit = layer * selections per layer + row."""
        return self._snapshot()[1]

    @property
    def holds(self) -> np.ndarray:
        """Chunk each slot holds (units, n_slots), -1 for none."""
        return self._snapshot()[2]

    @property
    def wa(self) -> np.ndarray:
        """Write-allocate slots (layers, 2), -1 for none."""
        return self._snapshot()[3]

    def resident(self, layer: int, row: int = 0) -> list:
        """Chunks of ``layer`` (batch ``row`` of a per-row layer) whose
        residency entry has been committed."""
        _, state, holds, _ = self._snapshot()
        u = layer * self.sels + row
        return sorted(int(holds[u, s]) for s in np.flatnonzero(state[u] == _READY))

    def hit_rate(self) -> float:
        s = self._snapshot()[0]
        n = s.hits + s.misses
        return s.hits / n if n else 0.0

    @property
    def slot_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._slot_k + self._slot_v)
