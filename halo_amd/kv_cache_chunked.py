"""Path-D KV cache: recent rows on the GPU, older rows in a pinned-host cold
tier, attention as an LSE-merged walk over both.

Reference: HALOCacheChunked (halo/kv_cache_chunked.py:140-993): ``update``
with the warm-up -> chunked transition and the peel of cold rows to host
memory (:279-336, :384-548), the optional placement scorer that keeps
query-relevant pages on the GPU (:306-311, :416-457, ``_last_query`` :800),
the chunk walk of ``compute_attention`` (:765-964) and the telemetry
(:72-82, :966-985).

What changes on MI355X:
  * the cold tier is a list of pinned host chunks of ``chunk_size`` rows that
    peels append to (the reference re-concatenates the whole cold tensor on
    every peel, :481-521); every cold row keeps its global position, so a
    scorer-driven peel (non-contiguous rows) still attends with exact causal
    positions;
  * peels are device-to-host copies on the tier copy stream; an event
    recorded after each peel orders every later use of that layer's cold
    tier: staging copies run on the same stream behind it, and the compute
    stream waits on the staging event, never on the host (the reference's
    async variant had to block the host, :86-100, :833-848);
  * pinned chunks are staged as whole byte spans (``span_to_device``), so the
    host never reads a pinned row;
  * decode (T_q == 1) is one ``halo_decode_attn`` launch over the GPU rows
    and the cold chunks read in place over the host link (no staging
    memory, no copy); with ``use_triton`` the reference's route switches
    pick the other two shapes of its fast path (:610-700):
    ``HALO_TRITON_STREAMED=1`` streams the cold chunks through two HBM
    staging buffers merged into fp32 accumulators, and
    ``HALO_TRITON_SINGLE_LAUNCH=1`` stages the whole cold tier in HBM first
    and attends it with the GPU rows in one launch.  T_q > 1 stages the cold
    chunks and runs one ``halo_prefill_attn`` (bf16/fp16 MFMA; fp32 on the
    decode kernel's fp32 path) over them and the GPU rows;
  * per-chunk fp32 key sums are accumulated at peel time, so every filled
    cold chunk has its mean key on the GPU (the page-mean metadata a chunk
    scorer reads) without touching host memory.
The cache is lossless: every cold row is attended (Path D).
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from .kv_cache import HALOCache
from .memory_tier import copy_stream, span_elems, span_to_device


@dataclass
class ChunkedAttentionStats:
    """Per-call telemetry (halo/kv_cache_chunked.py:72-82)."""

    hot_positions: int = 0
    cold_positions: int = 0
    n_chunks: int = 0
    chunk_size: int = 0
    peak_staging_bytes: int = 0
    used_lse_merge: bool = False
    dma_bytes: int = 0


_ChunkedAttentionStats = ChunkedAttentionStats


@dataclass
class _ColdChunk:
    k: torch.Tensor            # pinned (B, H_kv, chunk_size, D)
    v: torch.Tensor
    pos: np.ndarray            # int64 [chunk_size] global positions of the filled rows
    n: int = 0                 # filled rows
    ksum: Optional[torch.Tensor] = None  # fp32 (B, H_kv, D) sum of the filled rows' keys (GPU)


@dataclass
class _ColdTier:
    chunk_size: int
    chunks: list = field(default_factory=list)
    rows: int = 0
    ready: Optional[torch.cuda.Event] = None  # recorded on the copy stream after the last peel


def _runs(pos: np.ndarray):
    """Maximal runs of consecutive positions: [(row_lo, row_hi, first_pos)]."""
    n = len(pos)
    if n == 0:
        return []
    cut = np.flatnonzero(np.diff(pos) != 1) + 1
    lo = np.concatenate([[0], cut])
    hi = np.concatenate([cut, [n]])
    return [(int(a), int(b), int(pos[a])) for a, b in zip(lo, hi)]


class HALOCacheChunked(HALOCache):
    """Recent-window GPU cache plus pinned-host cold tier (Path D)."""

    def __init__(self, *, config=None, storage=None, scorer=None, demoter=None, refetcher=None,
                 chunk_size: int = 512, recent_window: int = 64, use_triton: bool = False) -> None:
        super().__init__(config=config, storage=storage, scorer=scorer, demoter=demoter, refetcher=refetcher)
        self.chunk_size = int(chunk_size)
        self.recent_window = int(recent_window)
        # Every route of this cache runs the HIP kernels; as in the reference
        # (halo/kv_cache_chunked.py:152-167, :610-660) the flag enables the
        # route switches HALO_TRITON_SINGLE_LAUNCH / HALO_TRITON_STREAMED.
        self.use_triton = bool(use_triton)
        self._mode = "warmup"
        self._cold: dict = {}
        self._gpu_pos: dict = {}
        self._stats: dict = {}
        self._dma_bytes_cumulative = 0
        self._quest_scorer = None
        self._last_query: dict = {}

    # ------------------------------------------------------------- layer access
    def _iter_layer_kv(self):
        """(layer_idx, layer object, K, V) of every GPU layer."""
        for i, lay in enumerate(getattr(self, "layers", [])):
            yield i, lay, getattr(lay, "keys", None), getattr(lay, "values", None)

    def _get_layer_kv(self, layer_idx: int):
        layers = getattr(self, "layers", [])
        if layer_idx >= len(layers):
            return None, None
        lay = layers[layer_idx]
        return getattr(lay, "keys", None), getattr(lay, "values", None)

    def _replace_layer_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> None:
        lay = self.layers[layer_idx]
        lay.keys, lay.values = k, v

    @staticmethod
    def _rows(t: Optional[torch.Tensor]) -> int:
        return 0 if t is None or t.numel() == 0 else int(t.shape[-2])

    # ------------------------------------------------------------- cache API
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        """Append new rows and peel when the mode asks for it; returns this
        layer's GPU rows (all rows in warm-up, the kept rows in chunked mode)."""
        T_new = key_states.shape[-2]
        before = self.get_seq_length(layer_idx)
        k_full, v_full = super().update(key_states, value_states, layer_idx, *args, **kwargs)
        old = self._gpu_pos.get(layer_idx)
        new = np.arange(before, before + T_new, dtype=np.int64)
        self._gpu_pos[layer_idx] = new if old is None else np.concatenate([old, new])
        if self._quest_scorer is not None and k_full is not None and k_full.numel() > 0:
            self._quest_scorer.observe_keys(layer_idx, k_full)
        T = self._rows(k_full)
        if self._mode == "warmup":
            if T_new == 1 and T > 2 * self.chunk_size:
                self._mode = "chunked"
                self._peel_to_cold(layer_idx)
        elif T > self.recent_window + self.chunk_size:
            self._peel_to_cold(layer_idx)
        elif layer_idx not in self._cold and T_new == 1 and T > 2 * self.chunk_size:
            self._peel_to_cold(layer_idx)  # a layer that reaches the transition after the first
        return self._get_layer_kv(layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Cold rows + GPU rows (the true length, so positions roll forward)."""
        cold = self._cold.get(layer_idx)
        k, _ = self._get_layer_kv(layer_idx)
        return (cold.rows if cold is not None else 0) + self._rows(k)

    def get_max_cache_shape(self, layer_idx: int = 0):
        """No static upper bound (halo/kv_cache_chunked.py:566-568)."""
        return None

    def reset(self) -> None:
        if self._cold and torch.cuda.is_available():
            # decode launches read the pinned chunks in place: they must be
            # done before the chunks go back to the host allocator
            torch.cuda.synchronize()
        super().reset()
        self._cold.clear()
        self._gpu_pos.clear()
        self._stats.clear()
        self._last_query.clear()
        self._mode = "warmup"
        self._dma_bytes_cumulative = 0

    def telemetry(self) -> dict:
        base = super().telemetry()
        base["mode"] = self._mode
        base["dma_bytes_cumulative"] = int(self._dma_bytes_cumulative)
        if self._stats:
            st = list(self._stats.values())
            base["chunked_n_layers_called"] = len(st)
            base["chunked_total_chunks"] = sum(s.n_chunks for s in st)
            base["chunked_peak_staging_bytes_max"] = max(s.peak_staging_bytes for s in st)
            base["chunked_used_lse_merge_any"] = any(s.used_lse_merge for s in st)
            base["chunked_total_dma_bytes"] = sum(s.dma_bytes for s in st)
        if self._cold:
            base["cold_positions_per_layer_max"] = max(c.rows for c in self._cold.values())
            base["cold_layers"] = len(self._cold)
        return base

    @property
    def last_stats(self) -> ChunkedAttentionStats:
        return self._stats[max(self._stats)] if self._stats else ChunkedAttentionStats()

    # ------------------------------------------------------------- helpers
    @staticmethod
    def _lse_merge(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor):
        """Two partial attention results over disjoint key sets merged into
        one (halo/kv_cache_chunked.py:194-239): lse = logaddexp(lse_a,
        lse_b), out = exp(lse_a - lse) out_a + exp(lse_b - lse) out_b, a side
        whose lse is -inf adding nothing; fp32, on the GPU
        (``halo_lse_merge``)."""
        from .triton_chunked import lse_merge
        return lse_merge(out_a, lse_a, out_b, lse_b)

    @staticmethod
    def _chunk_attention(q: torch.Tensor, k_chunk: torch.Tensor, v_chunk: torch.Tensor, *,
                         scaling: Optional[float] = None, causal_mask: Optional[torch.Tensor] = None):
        """Attention of q (B, H, T_q, D) over one chunk (B, H_kv, T_c, D),
        query heads grouped over the KV heads, returning the fp32 partial
        (out (B, H, T_q, D), lse (B, H, T_q)) (halo/kv_cache_chunked.py:
        241-276): one prefill launch (``halo_prefill_attn``; fp32 through the
        decode kernel).  The kernels mask by position, so ``causal_mask``
        (T_q, T_c, additive) is taken in the form the reference's chunk walk
        builds -- 0 where key j <= q_start + i, -inf elsewhere, for some
        offset q_start -- and any other mask raises."""
        from .decode import ChunkRef
        from .prefill import prefill_attention

        if q.dim() != 4 or k_chunk.dim() != 4 or v_chunk.shape != k_chunk.shape:
            raise AssertionError(f"shapes: q {tuple(q.shape)}, k {tuple(k_chunk.shape)}, v {tuple(v_chunk.shape)}")
        B, H, T_q, D = q.shape
        H_kv, T_c = k_chunk.shape[1], k_chunk.shape[2]
        if H % H_kv:
            raise AssertionError(f"head count mismatch: q has {H}, kv has {H_kv}")
        causal, q_start = False, T_c - T_q
        if causal_mask is not None:
            if tuple(causal_mask.shape) != (T_q, T_c):
                raise AssertionError(f"causal_mask must be (T_q, T_c) = {(T_q, T_c)}")
            visible = causal_mask == 0
            q_start = int(visible[0].sum().item()) - 1
            i = torch.arange(T_q, device=causal_mask.device).unsqueeze(1)
            j = torch.arange(T_c, device=causal_mask.device).unsqueeze(0)
            want = j <= q_start + i
            if not (torch.equal(visible, want) and bool(torch.isneginf(causal_mask[~want]).all())):
                raise NotImplementedError("only the causal mask of a position offset is supported: the kernels "
                                          "mask by key and query positions")
            causal = True
        chunk = ChunkRef(k_chunk.to(q.dtype), v_chunk.to(q.dtype), 0, causal)
        return prefill_attention(q, [chunk], scale=scaling, q_start=q_start, out_dtype=torch.float32,
                                 return_lse=True)

    # ------------------------------------------------------------- peel
    def _keep_mask(self, layer_idx: int, T: int) -> Optional[np.ndarray]:
        """Rows the placement scorer keeps on the GPU (None: no scorer or no
        query yet, so the oldest rows go): its hot pages of the GPU rows plus
        the recent window (halo/kv_cache_chunked.py:416-457)."""
        sc = self._quest_scorer
        q = self._last_query.get(layer_idx)
        if sc is None or q is None:
            return None
        pages = sc.select_hot_pages(layer_idx, q)
        if pages is None or pages.numel() == 0:
            return None
        keep = np.zeros(T, dtype=bool)
        p = int(sc.page_size)
        for pg in pages.reshape(-1).tolist():
            keep[pg * p: min(pg * p + p, T)] = True
        keep[max(0, T - self.recent_window):] = True
        if keep.all() or not keep.any():
            return None
        return keep

    def _peel_to_cold(self, layer_idx: int) -> None:
        """Move the GPU rows that leave the recent window to the cold tier:
        device-to-host copies on the tier copy stream, appended to pinned
        chunks; an event after them orders every later read of the tier."""
        k, v = self._get_layer_kv(layer_idx)
        T = self._rows(k)
        peel_n = T - min(self.recent_window, T)
        if peel_n <= 0:
            return
        pos = self._gpu_pos[layer_idx]
        keep = self._keep_mask(layer_idx, T)
        if keep is None:
            peel_rows = None
            peel_pos = pos[:peel_n]
            kp, vp = k[..., :peel_n, :], v[..., :peel_n, :]
            k_keep, v_keep, pos_keep = k[..., peel_n:, :], v[..., peel_n:, :], pos[peel_n:]
        else:
            peel_rows = np.flatnonzero(~keep)
            keep_rows = np.flatnonzero(keep)
            idx_p = torch.from_numpy(peel_rows).to(k.device, non_blocking=True)
            idx_k = torch.from_numpy(keep_rows).to(k.device, non_blocking=True)
            kp, vp = k.index_select(-2, idx_p), v.index_select(-2, idx_p)
            k_keep, v_keep = k.index_select(-2, idx_k), v.index_select(-2, idx_k)
            peel_pos, pos_keep = pos[peel_rows], pos[keep_rows]
        n = kp.shape[-2]
        cold = self._cold.setdefault(layer_idx, _ColdTier(self.chunk_size))
        on_gpu = k.is_cuda
        cs = copy_stream(k.device) if on_gpu else None
        if cs is not None:
            cs.wait_stream(torch.cuda.current_stream(k.device))
        done = 0
        while done < n:
            if not cold.chunks or cold.chunks[-1].n == self.chunk_size:
                shape = (k.shape[0], k.shape[1], self.chunk_size, k.shape[3])
                cold.chunks.append(_ColdChunk(torch.empty(shape, dtype=k.dtype, pin_memory=on_gpu),
                                              torch.empty(shape, dtype=v.dtype, pin_memory=on_gpu),
                                              np.zeros(self.chunk_size, dtype=np.int64)))
            ch = cold.chunks[-1]
            m = min(self.chunk_size - ch.n, n - done)
            src_k, src_v = kp[..., done:done + m, :], vp[..., done:done + m, :]
            part = src_k.float().sum(dim=-2)
            ch.ksum = part if ch.ksum is None else ch.ksum + part
            if cs is not None:
                with torch.cuda.stream(cs):
                    ch.k[..., ch.n:ch.n + m, :].copy_(src_k, non_blocking=True)
                    ch.v[..., ch.n:ch.n + m, :].copy_(src_v, non_blocking=True)
            else:
                ch.k[..., ch.n:ch.n + m, :].copy_(src_k)
                ch.v[..., ch.n:ch.n + m, :].copy_(src_v)
            ch.pos[ch.n:ch.n + m] = peel_pos[done:done + m]
            ch.n += m
            cold.rows += m
            done += m
        if cs is not None:
            ev = torch.cuda.Event()
            ev.record(cs)
            cold.ready = ev
            for t in (k, v, kp, vp):
                t.record_stream(cs)
        self._replace_layer_kv(layer_idx, k_keep.contiguous(), v_keep.contiguous())
        self._gpu_pos[layer_idx] = np.ascontiguousarray(pos_keep)
        self._dma_bytes_cumulative += 2 * n * k.shape[0] * k.shape[1] * k.shape[3] * k.element_size()
        bs = max(1, int(getattr(self.cfg, "block_size", 32) if self.cfg is not None else 32))
        self.demoted_blocks_total += (n + bs - 1) // bs
        if self._quest_scorer is not None and hasattr(self._quest_scorer, "forget"):
            self._quest_scorer.forget(layer_idx)
            self._quest_scorer.observe_keys(layer_idx, k_keep)

    def cold_chunk_means(self, layer_idx: int) -> Optional[torch.Tensor]:
        """Mean key of every cold chunk (B, H_kv, n_chunks, D) in the key
        dtype: the fp32 row sums kept at peel time divided by the row count,
        rounded once.  None before the first peel."""
        cold = self._cold.get(layer_idx)
        if cold is None or not cold.chunks:
            return None
        dt = cold.chunks[0].k.dtype
        return torch.stack([(c.ksum / c.n).to(dt) for c in cold.chunks], dim=2)

    # ------------------------------------------------------------- attention
    def compute_attention(self, q: torch.Tensor, *, layer_idx: int, scaling: Optional[float] = None,
                          query_pos_offset: Optional[int] = None, return_lse: bool = False):
        """Attention of ``q`` (B, H, T_q, D) over every cached row of the
        layer (cold chunks + GPU rows), causal by global position; the query
        rows sit at ``query_pos_offset`` (default T_total - T_q)."""
        from .decode import ChunkRef
        from .prefill import prefill_attention
        from .triton_chunked import finalize, init_acc
        from .decode import build_plan, launch
        from .memory_tier import stream_cold_chunks

        B, H, T_q, D = q.shape
        if self._quest_scorer is not None:
            self._last_query[layer_idx] = q.detach()
        gpu_k, gpu_v = self._get_layer_kv(layer_idx)
        cold = self._cold.get(layer_idx)
        T_cold = cold.rows if cold is not None else 0
        T_gpu = self._rows(gpu_k)
        T_total = T_cold + T_gpu
        if T_total == 0:
            out = torch.zeros(B, H, T_q, D, dtype=q.dtype, device=q.device)
            return (out, torch.full((B, H, T_q), float("-inf"), device=q.device)) if return_lse else out
        q0 = T_total - T_q if query_pos_offset is None else int(query_pos_offset)
        scale = 1.0 / math.sqrt(D) if scaling is None else float(scaling)
        last_q = q0 + T_q - 1

        def refs(kt, vt, pos, n):
            """ChunkRefs of rows [0, n) of (kt, vt) with positions pos: one
            non-causal ref when every row precedes the first query, else one
            causal ref per run of consecutive positions."""
            if n == 0:
                return []
            if int(pos[:n].max()) <= q0:
                return [ChunkRef(kt[..., :n, :], vt[..., :n, :], 0, False)]
            return [ChunkRef(kt[..., lo:hi, :], vt[..., lo:hi, :], start, True)
                    for lo, hi, start in _runs(pos[:n]) if start <= last_q]

        hot = refs(gpu_k, gpu_v, self._gpu_pos[layer_idx], T_gpu) if T_gpu else []
        chunks = [c for c in (cold.chunks if cold is not None else []) if c.n > 0]
        stats = ChunkedAttentionStats(hot_positions=T_gpu, cold_positions=T_cold, chunk_size=self.chunk_size,
                                      n_chunks=len(chunks) + (1 if T_gpu else 0))
        stats.used_lse_merge = stats.n_chunks > 1
        route = self.decode_route(T_q) if chunks else "in_place"
        if T_q == 1 and route == "streamed":
            q3 = q[:, :, 0, :]
            qp = torch.full((B,), q0, dtype=torch.int64).to(q.device, non_blocking=True)
            m, l, o = init_acc(B=B, H=H, D_v=D, device=q.device)
            if hot:
                plan = build_plan(B=B, H=H, H_kv=hot[0].k.shape[1], D=D, dtype=hot[0].k.dtype, chunks=hot,
                                  device=q.device)
                launch(plan, q3, scale=scale, q_pos=qp, m=m, l=l, o=o, acc_mode=2)
            entries = [(c.k, c.v, self._cold_runs(c, q0, last_q)) for c in chunks]
            stats.dma_bytes = stream_cold_chunks(q3, entries, scale=scale, q_pos=qp, m=m, l=l, o=o,
                                                 after=cold.ready)
            stats.peak_staging_bytes = 2 * max(2 * span_elems(c.k) * c.k.element_size() for c in chunks)
            res = finalize(m=m, l=l, o=o, out_dtype=q.dtype, return_lse=return_lse)
            res = (res[0].unsqueeze(2), res[1].unsqueeze(2)) if return_lse else res.unsqueeze(2)
        elif T_q == 1:
            # one launch over the GPU rows and the cold chunks: read in place
            # over the host link, or (single_launch) staged in HBM first
            compute = torch.cuda.current_stream(q.device)
            if route == "single_launch":
                cold_refs = self._stage_cold(chunks, cold, q, q0, last_q, stats)
                stats.peak_staging_bytes = stats.dma_bytes
                stats.n_chunks = 1
                stats.used_lse_merge = False
            else:
                if cold is not None and cold.ready is not None:
                    compute.wait_event(cold.ready)   # the peel's copies into the pinned chunks
                cold_refs = [ChunkRef(c.k[..., lo:hi, :], c.v[..., lo:hi, :], start, causal)
                             for c in chunks for lo, hi, start, causal in self._cold_runs(c, q0, last_q)]
                stats.dma_bytes = sum(2 * (hi - lo) * c.k.shape[0] * c.k.shape[1] * c.k.shape[-1] *
                                      c.k.element_size()
                                      for c in chunks for lo, hi, _, _ in self._cold_runs(c, q0, last_q))
            q3 = q[:, :, 0, :]
            qp = torch.full((B,), q0, dtype=torch.int64).to(q.device, non_blocking=True)
            all_chunks = cold_refs + hot
            out = torch.empty((B, H, D), dtype=q.dtype, device=q.device)
            lse = torch.empty((B, H), dtype=torch.float32, device=q.device) if return_lse else None
            if all_chunks:
                ref = all_chunks[0]
                plan = build_plan(B=B, H=H, H_kv=ref.k.shape[1], D=D, dtype=ref.k.dtype, chunks=all_chunks,
                                  device=q.device)
                launch(plan, q3, scale=scale, q_pos=qp, out=out, lse=lse)
            else:
                out.zero_()
                if lse is not None:
                    lse.fill_(float("-inf"))
            res = (out.unsqueeze(2), lse.unsqueeze(2)) if return_lse else out.unsqueeze(2)
        else:
            staged = self._stage_cold(chunks, cold, q, q0, last_q, stats) if chunks else []
            stats.peak_staging_bytes = stats.dma_bytes
            all_chunks = staged + hot
            if not all_chunks:
                out = torch.zeros(B, H, T_q, D, dtype=q.dtype, device=q.device)
                res = (out, torch.full((B, H, T_q), float("-inf"), device=q.device)) if return_lse else out
            else:
                res = prefill_attention(q, all_chunks, scale=scale, q_start=q0, return_lse=return_lse)
        self._stats[layer_idx] = stats
        self._dma_bytes_cumulative += stats.dma_bytes
        bs = max(1, int(getattr(self.cfg, "block_size", 32) if self.cfg is not None else 32))
        blocks = sum((c.n + bs - 1) // bs for c in chunks)
        self.refetched_blocks_total += blocks
        if self.refetcher is not None and hasattr(self.refetcher, "count_hits"):
            self.refetcher.count_hits(blocks)
        return res

    def decode_route(self, T_q: int = 1) -> str:
        """Shape of a decode call's cold-tier traffic, read per call as the
        reference reads its switches (halo/kv_cache_chunked.py:610-660,
        851-862): "single_launch" (``use_triton`` and
        HALO_TRITON_SINGLE_LAUNCH=1, checked first), "streamed"
        (``use_triton`` and HALO_TRITON_STREAMED=1), else "in_place"."""
        if T_q != 1 or not self.use_triton:
            return "in_place"
        if os.environ.get("HALO_TRITON_SINGLE_LAUNCH", "0") == "1":
            return "single_launch"
        if os.environ.get("HALO_TRITON_STREAMED", "0") == "1":
            return "streamed"
        return "in_place"

    def _stage_cold(self, chunks, cold, q: torch.Tensor, q0: int, last_q: int, stats) -> list:
        """Copy every cold chunk's byte span to HBM on the tier copy stream
        (behind the peel's event) and make the compute stream wait for the
        copies; returns the staged rows as chunk refs and adds the copied
        bytes to ``stats.dma_bytes``."""
        from .decode import ChunkRef

        cs = copy_stream(q.device)
        compute = torch.cuda.current_stream(q.device)
        if cold.ready is not None:
            cs.wait_event(cold.ready)
        cs.wait_stream(compute)
        bufs = []
        for c in chunks:  # allocated on the compute stream, which reads them
            kb = torch.empty(span_elems(c.k), dtype=c.k.dtype, device=q.device)
            vb = torch.empty(span_elems(c.v), dtype=c.v.dtype, device=q.device)
            bufs.append((c, kb, vb))
        with torch.cuda.stream(cs):
            bufs = [(c, span_to_device(c.k, kb), span_to_device(c.v, vb), kb, vb) for c, kb, vb in bufs]
            ev = torch.cuda.Event()
            ev.record(cs)
        compute.wait_event(ev)
        staged = []
        for c, kd, vd, kb, vb in bufs:
            kb.record_stream(cs)
            vb.record_stream(cs)
            for lo, hi, start, causal in self._cold_runs(c, q0, last_q):
                staged.append(ChunkRef(kd[..., lo:hi, :], vd[..., lo:hi, :], start, causal))
            stats.dma_bytes += 2 * kb.numel() * kb.element_size()
        return staged

    @staticmethod
    def _cold_runs(c: _ColdChunk, q0: int, last_q: int):
        """(row_lo, row_hi, chunk_start, causal) pieces of one cold chunk."""
        if c.n == 0:
            return []
        if int(c.pos[:c.n].max()) <= q0:
            return [(0, c.n, 0, False)]
        return [(lo, hi, start, True) for lo, hi, start in _runs(c.pos[:c.n]) if start <= last_q]
