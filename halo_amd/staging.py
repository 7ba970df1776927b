"""HBM staging cache for cold chunks kept in pinned host memory.

A stack of tiered decode layers (``TieredDecodeLayer`` whose cold chunks
live in pinned host DRAM) selects its top-k cold chunks inside the attention
launch every step.  Without staging, every selected chunk is read in place
over the host link.  This cache keeps up to ``n_slots`` cold chunks per layer
in HBM slots and points the in-kernel selection at them through a per-chunk
residency entry (``halo_select_cfg.residency``): a chosen chunk whose entry
names a slot is read from HBM (a hit), otherwise in place from host memory
(a miss, still exact: the rows are the same).

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
  * an eviction stores -1 on the compute stream after the launches already
    queued; the slot becomes free for a new fill only once an event
    recorded after that store has completed, i.e. once every launch that
    could have read the old entry has finished.
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

_FREE, _FILLING, _READY, _RELEASING, _RESERVED = 0, 1, 2, 3, 4


class ColdStaging:
    """HBM staging slots + residency for the cold chunks of ``layers``.

    ``layers``: ``TieredDecodeLayer`` objects with the fused in-kernel
    selection over cold chunks held as contiguous pinned host tensors, the
    same number of cold chunks each.  ``n_slots`` HBM slots per layer (each
    the size of the layer's widest cold chunk); ``keep`` best-scoring chunks
    per layer are staged (default n_slots - 2); ``spare`` slots per layer are
    kept free or releasing (staged chunks outside the kept set are released
    worst rank first to keep them); ``max_inflight`` bounds the copies in
    flight on the link; ``write_allocate`` reserves two slots per layer for
    missed chunks the kernel writes while reading them (16-bit layers with
    one selection per launch; ignored otherwise).  It pays when the
    selection moves fast (fewer bytes over the link) and costs hits when it
    moves slowly (the reserved slots are missing from the cache)."""

    def __init__(self, layers: Sequence, *, n_slots: int = 12, keep: Optional[int] = None,
                 max_inflight: int = 8, spare: int = 0, ring: int = 16, write_allocate: bool = False) -> None:
        if not layers:
            raise AssertionError("no layers")
        self.layers = list(layers)
        lay0 = self.layers[0]
        self.device = lay0.plan.descs.device
        self.n_cold = len(lay0.cold)
        self.top_k = lay0.top_k
        if not 1 <= n_slots <= 64:
            raise AssertionError("n_slots must be in [1, 64]")
        self.n_slots = int(n_slots)
        self.keep = int(keep if keep is not None else max(self.top_k, n_slots - 2))
        if not self.top_k <= self.keep <= self.n_slots:
            raise AssertionError(f"keep={self.keep} must be in [top_k={self.top_k}, n_slots={self.n_slots}]")
        self.max_inflight = int(max_inflight)
        self.spare = int(spare)
        L, n, k = len(self.layers), self.n_cold, self.top_k
        for li, lay in enumerate(self.layers):
            if not lay.fused or lay.select_cfg is None:
                raise AssertionError(f"layer {li}: staging needs the fused in-kernel selection")
            if len(lay.cold) != n or lay.top_k != k:
                raise AssertionError("every layer must have the same number of cold chunks and top_k")
            for c in lay.cold:
                if c.k.device.type != "cpu" or not c.k.is_pinned() or not c.k.is_contiguous() \
                        or not c.v.is_contiguous():
                    raise AssertionError(f"layer {li}: cold chunks must be contiguous pinned host tensors")
        dev = self.device
        # residency (L, n) and the per-layer write-allocate slot (L) in one
        # device buffer, so one store kernel updates both
        self._dev_i32 = torch.full((L * n + L,), -1, dtype=torch.int32, device=dev)
        self.residency = self._dev_i32[:L * n].view(L, n)
        self.alloc = self._dev_i32[L * n:]
        self.write_allocate = bool(write_allocate) and self.n_slots >= self.top_k + 2 and all(
            lay.dtype != torch.float32 and not lay.select_cfg.per_row for lay in self.layers)
        # one feedback row per layer: scores (fp32) | picks (int32) | residency used (int32)
        self._W = n + 2 * k
        self.feedback = torch.zeros((L, self._W), dtype=torch.float32, device=dev)
        self.scores = self.feedback[:, :n]
        self.idx = self.feedback[:, n:n + k].view(torch.int32)
        self.res_out = self.feedback[:, n + k:].view(torch.int32)
        self.idx.fill_(-1)
        self.res_out.fill_(-1)
        self._ring = [torch.empty((L, self._W), dtype=torch.float32, pin_memory=True) for _ in range(max(2, ring))]
        self._ring_ev = [torch.cuda.Event() for _ in self._ring]
        self._ring_rows = [(0, L)] * len(self._ring)
        self._queued = 0           # segments whose feedback was queued for the host
        self._seen = 0             # segments the host has processed
        # host mirror of the cache
        self.slot_of = np.full((L, n), -1, dtype=np.int64)        # FILLING / READY slot of a chunk
        self.state = np.full((L, self.n_slots), _FREE, dtype=np.int8)
        self.holds = np.full((L, self.n_slots), -1, dtype=np.int64)
        self._pending: list = []   # (layer, chunk, slot, event, urgent): fills not committed yet
        self._last_rank = np.full((L, n), n, dtype=np.int64)     # rank at the last planning pass
        self._releasing: list = []
        self._release_ev: Optional[torch.cuda.Event] = None
        self.chunk_bytes = np.zeros((L, n), dtype=np.int64)
        self._slot_k, self._slot_v, self._slot_cat = [], [], []
        # addresses for the batched copies: slot (layer, s) K/V, cold chunk (layer, c) K/V, bytes per tensor
        self._dst = np.zeros((L, self.n_slots, 2), dtype=np.uint64)
        self._src = np.zeros((L, n, 2), dtype=np.uint64)
        self._nbytes = np.zeros((L, n), dtype=np.int64)
        for li, lay in enumerate(self.layers):
            shape = max((tuple(c.k.shape) for c in lay.cold), key=lambda s: s[-2])
            sk = torch.empty((self.n_slots,) + shape, dtype=lay.dtype, device=dev)
            sv = torch.empty_like(sk)
            # slot descriptors never change: they give the addresses and strides
            # a staged chunk is read through; its rows, start and flags come
            # from the chunk's own catalog entry
            sdesc, _ = pack_descs([ChunkRef(sk[s], sv[s], 0, False) for s in range(self.n_slots)],
                                  B=lay.B, H_kv=lay.H_kv, D=lay.D, dtype=lay.dtype)
            self._slot_k.append(sk)
            self._slot_v.append(sv)
            self._slot_cat.append(descs_to_device(sdesc, dev))
            for j in range(self.n_slots):
                self._dst[li, j] = (sk[j].data_ptr(), sv[j].data_ptr())
            for j, c in enumerate(lay.cold):
                if tuple(c.k.shape) != tuple(sk.shape[1:]):
                    raise AssertionError(f"layer {li} cold chunk {j}: shape {tuple(c.k.shape)} differs from the "
                                         f"layer's other cold chunks {tuple(sk.shape[1:])}")
                self._src[li, j] = (c.k.data_ptr(), c.v.data_ptr())
                self._nbytes[li, j] = c.k.numel() * c.k.element_size()
            self.chunk_bytes[li] = 2 * self._nbytes[li]
            cfg = lay.select_cfg
            cfg.n_slots = self.n_slots
            cfg.slot_catalog = self._slot_cat[li].data_ptr()
            cfg.residency = self.residency[li].data_ptr()
            cfg.res_out = self.res_out[li].data_ptr()
            cfg.score_out = self.scores[li].data_ptr()
            cfg.idx_out = self.idx[li].data_ptr()
            cfg.alloc_slot = self.alloc[li].data_ptr() if self.write_allocate else None
        # write-allocate reservations (two per layer), launches queued and
        # feedback rows processed per layer
        self.wa = np.full((L, 2), -1, dtype=np.int64)
        self._launches = np.zeros(L, dtype=np.int64)
        self._processed = np.zeros(L, dtype=np.int64)
        self._reserve_wa()
        self.reset_counters()

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
        compute = torch.cuda.current_stream(self.device)
        done, rest, waited = [], [], set()
        for p in self._pending:
            li, c, s, ev, urgent = p
            if lo <= li < hi and (urgent or ev.query()):
                if urgent and id(ev) not in waited:
                    compute.wait_event(ev)
                    waited.add(id(ev))
                done.append(p)
            else:
                rest.append(p)
        self._pending = rest
        idx = [li * self.n_cold + c for li, c, _, _, _ in done]
        val = [s for _, _, s, _, _ in done]
        for li, c, s, _, _ in done:
            self.state[li, s] = _READY
        if self.write_allocate:
            base = len(self.layers) * self.n_cold
            for li in range(lo, hi):
                # a reservation is named again only after the feedback of the
                # launch that last named it (two launches back) was processed
                par = int(self._launches[li] & 1)
                ok = self._launches[li] - self._processed[li] < 2
                idx.append(base + li)
                val.append(int(self.wa[li, par]) if ok else -1)
        self._launches[lo:hi] += 1
        if idx:
            self._store(idx, val)

    def after_step(self, lo: int = 0, hi: Optional[int] = None) -> None:
        """Queue the feedback rows of layers [lo, hi) (scores, picks,
        residency used) for the host: one copy after those layers' launches."""
        hi = len(self.layers) if hi is None else hi
        if self._queued - self._seen >= len(self._ring):
            raise RuntimeError("feedback ring overrun: call service() after every after_step()")
        r = self._queued % len(self._ring)
        self._ring[r][lo:hi].copy_(self.feedback[lo:hi], non_blocking=True)
        self._ring_ev[r].record(torch.cuda.current_stream(self.device))
        self._ring_rows[r] = (lo, hi)
        self._queued += 1

    def drain(self) -> None:
        """Process every queued segment's feedback now (waits for it)."""
        self.service(lag=0)

    def service(self, *, lag: int = 1) -> None:
        """Process returned feedback -- waiting for every queued segment but
        the ``lag`` newest, and taking those too when they are done -- count
        hits and misses, free released slots, and plan evictions and fills
        for the processed segments' layers."""
        target = self._queued - lag
        rows, scores = [], []
        while self._seen < self._queued:
            r = self._seen % len(self._ring)
            if self._seen < target:
                self._ring_ev[r].synchronize()
            elif not self._ring_ev[r].query():
                break
            lo, hi = self._ring_rows[r]
            fb = self._ring[r].numpy()[lo:hi]
            self._account(fb, lo)
            rows.append(np.arange(lo, hi))
            scores.append(fb[:, :self.n_cold].copy())
            self._seen += 1
        if self._release_ev is not None and self._release_ev.query():
            for li, s in self._releasing:
                self.state[li, s] = _FREE
                self.holds[li, s] = -1
            self._releasing = []
            self._release_ev = None
            self._reserve_wa()
        if rows:
            self._plan(np.concatenate(rows), np.concatenate(scores))

    # ----------------------------------------------------------------- internals
    def _store(self, flat_idx: list, values: list) -> None:
        """residency.view(-1)[flat_idx] = values on the compute stream (the
        pairs travel in the kernel arguments)."""
        idx = np.ascontiguousarray(flat_idx, dtype=np.int64)
        val = np.ascontiguousarray(values, dtype=np.int32)
        nat.check(nat.lib().halo_store_i32(self._dev_i32.data_ptr(), self._dev_i32.numel(), idx.ctypes.data,
                                           val.ctypes.data, len(idx), nat.stream_ptr()), "halo_store_i32")

    def _account(self, fb: np.ndarray, lo: int) -> None:
        n, k = self.n_cold, self.top_k
        idx = np.ascontiguousarray(fb[:, n:n + k]).view(np.int32)
        res = np.ascontiguousarray(fb[:, n + k:]).view(np.int32)
        valid = idx >= 0
        miss = valid & (res < 0)
        self.hits += int((valid & (res >= 0)).sum())
        self.misses += int(miss.sum())
        self._processed[lo:lo + fb.shape[0]] += 1
        if self.write_allocate:
            wr, wj = np.nonzero(valid & (res <= -2))
            commits_i, commits_v = [], []
            for r, j in zip(wr.tolist(), wj.tolist()):
                li, c, w = lo + r, int(idx[r, j]), -2 - int(res[r, j])
                q = np.flatnonzero(self.wa[li] == w)
                if q.size == 0:
                    continue  # not a current reservation: nothing to commit
                if self.slot_of[li, c] >= 0:
                    self.wa_dups += 1  # staged or filling elsewhere meanwhile: keep the reservation
                    continue
                self.state[li, w] = _READY
                self.holds[li, w] = c
                self.slot_of[li, c] = w
                commits_i.append(li * self.n_cold + c)
                commits_v.append(w)
                self.wa[li, q[0]] = -1
                self.wa_commits += 1
            if commits_i:
                self._store(commits_i, commits_v)
                self._reserve_wa()
        if miss.any():
            r, j = np.nonzero(miss)
            self.miss_bytes += int(self.chunk_bytes[lo + r, idx[r, j]].sum())
            # a miss the policy had predicted (in the kept set at the last plan:
            # its fill had not landed or been committed) or one it had not
            predicted = self._last_rank[lo + r, idx[r, j]] < self.keep
            self.misses_predicted += int(predicted.sum())

    def _plan(self, layers: np.ndarray, scores: np.ndarray) -> None:
        sc = np.where(np.isnan(scores), -np.inf, scores)
        order = np.argsort(-sc, axis=1, kind="stable")      # score desc, index asc
        rank = np.empty_like(order)
        np.put_along_axis(rank, order, np.arange(sc.shape[1])[None, :], axis=1)
        self._last_rank[layers] = rank
        missing = (rank < self.keep) & (self.slot_of[layers] < 0)
        evicted, fills = [], []
        # keep `spare` slots per layer free or on their way to free, releasing
        # the worst-ranked staged chunks outside the kept set, so a newly
        # predicted chunk finds a slot without waiting for a release
        for i, li in enumerate(layers):
            st = self.state[li]
            short = self.spare - int(((st == _FREE) | (st == _RELEASING)).sum())
            if short <= 0:
                continue
            ready = np.flatnonzero(st == _READY)
            if ready.size == 0:
                continue
            rk = rank[i][self.holds[li, ready]]
            for j in np.argsort(-rk, kind="stable")[:short]:
                if rk[j] < self.keep:
                    break
                s = int(ready[j])
                evicted.append((int(li), int(self.holds[li, s]), s))
                self.slot_of[li, self.holds[li, s]] = -1
                self.state[li, s] = _RELEASING
        r, c = np.nonzero(missing)
        pri = np.lexsort((layers[r], rank[r, c]))           # best ranks first, then layer order
        budget = self.max_inflight - len(self._pending)
        for i in pri:
            if budget <= 0:
                break
            li, ch, rk = int(layers[r[i]]), int(c[i]), rank[r[i]]
            free = np.flatnonzero(self.state[li] == _FREE)
            if free.size == 0:
                ready = np.flatnonzero(self.state[li] == _READY)
                if ready.size:
                    worst = ready[np.argmax(rk[self.holds[li, ready]])]
                    if rk[self.holds[li, worst]] >= self.keep:
                        evicted.append((li, int(self.holds[li, worst]), int(worst)))
                        self.slot_of[li, self.holds[li, worst]] = -1
                        self.state[li, worst] = _RELEASING
                continue
            fills.append(self._reserve(li, ch, int(free[0]), bool(rk[ch] < self.top_k)))
            budget -= 1
        if fills:
            self._issue(fills)
        if evicted:
            self._store([li * self.n_cold + ch for li, ch, _ in evicted], [-1] * len(evicted))
            self._releasing += [(li, s) for li, _, s in evicted]
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            self._release_ev = ev

    def _reserve_wa(self) -> None:
        """Give every empty write-allocate reservation a free slot (highest
        index first, away from the fills, which take the lowest)."""
        if not self.write_allocate:
            return
        for li, q in zip(*np.nonzero(self.wa < 0)):
            free = np.flatnonzero(self.state[li] == _FREE)
            if free.size:
                s = int(free[-1])
                self.state[li, s] = _RESERVED
                self.wa[li, q] = s

    def _reserve(self, li: int, c: int, s: int, urgent: bool) -> tuple:
        self.state[li, s] = _FILLING
        self.holds[li, s] = c
        self.slot_of[li, c] = s
        self.fills += 1
        self.fill_bytes += int(self.chunk_bytes[li, c])
        return li, c, s, urgent

    def _issue(self, fills: list) -> None:
        """hipMemcpyAsync copies on the copy stream in the given order (best
        ranks first), each fill followed by its own event so it commits as
        soon as it lands."""
        cs = copy_stream(self.device)
        L = nat.lib()
        arr = nat.Fill()
        for li, c, s, urgent in fills:
            arr.dst_k, arr.dst_v = int(self._dst[li, s, 0]), int(self._dst[li, s, 1])
            arr.src_k, arr.src_v = int(self._src[li, c, 0]), int(self._src[li, c, 1])
            arr.bytes = int(self._nbytes[li, c])
            nat.check(L.halo_stage_fills(ctypes.byref(arr), 1, nat.stream_ptr(cs)), "halo_stage_fills")
            ev = torch.cuda.Event()
            ev.record(cs)
            self._pending.append((li, c, s, ev, urgent))

    # ----------------------------------------------------------------- control
    def clear(self) -> None:
        """Empty every slot (synchronises the device first)."""
        torch.cuda.synchronize(self.device)
        self._pending, self._releasing, self._release_ev = [], [], None
        self._seen = self._queued
        self._dev_i32.fill_(-1)
        self.slot_of.fill(-1)
        self._last_rank.fill(self.n_cold)
        self.state.fill(_FREE)
        self.holds.fill(-1)
        self.wa.fill(-1)
        self._launches.fill(0)
        self._processed.fill(0)
        self._reserve_wa()
        torch.cuda.synchronize(self.device)
        self.reset_counters()

    def resident(self, layer: int) -> list:
        """Chunks of ``layer`` whose residency entry has been committed."""
        return sorted(int(self.holds[layer, s]) for s in np.flatnonzero(self.state[layer] == _READY))

    def reset_counters(self) -> None:
        self.hits = self.misses = self.fills = self.fill_bytes = self.miss_bytes = 0
        self.wa_commits = self.wa_dups = 0
        self.misses_predicted = 0

    def hit_rate(self) -> float:
        n = self.hits + self.misses
        return self.hits / n if n else 0.0

    @property
    def slot_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._slot_k + self._slot_v)
