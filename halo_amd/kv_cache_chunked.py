"""Path-D KV cache: recent rows on the GPU, older rows in a pinned-host cold
tier, attention as an LSE-merged chunk walk over both.

Reference: HALOCacheChunked (halo/kv_cache_chunked.py:140-993): update with
the warm-up -> chunked transition and the peel of cold rows to host memory
(:279-336, :384-548), the chunk walk of compute_attention (:765-964) and the
telemetry record (:72-82, :966-985).

What changes on MI355X:
  * the cold tier is a list of pinned host chunks of ``chunk_size`` rows that
    peels append to (the reference re-concatenates the whole cold tensor on
    every peel, :481-521); peel copies run on the tier copy stream;
  * decode (T_q == 1) streams the cold chunks through HBM staging slots while
    the recent rows are attended (``halo_decode_attn`` with fp32
    accumulators), prefill (T_q > 1) is one ``halo_prefill_attn`` launch over
    the staged cold chunks and the recent rows.
The cache is lossless: every cold row is attended (Path D).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch

from .memory_tier import copy_stream


@dataclass
class ChunkedAttentionStats:
    """Per-call telemetry (halo/kv_cache_chunked.py:72-82)."""

    hot_positions: int = 0
    cold_positions: int = 0
    n_chunks: int = 0
    peak_staging_bytes: int = 0
    dma_bytes: int = 0
    used_lse_merge: bool = False


@dataclass
class _ColdTier:
    """Pinned host chunks (B, H_kv, chunk_size, D) of one layer's K and V."""

    chunk_size: int
    k: list = field(default_factory=list)
    v: list = field(default_factory=list)
    rows: int = 0

    def chunks(self):
        """(k, v, start) views of the filled part of every chunk."""
        out = []
        for i, (k, v) in enumerate(zip(self.k, self.v)):
            n = min(self.chunk_size, self.rows - i * self.chunk_size)
            if n > 0:
                out.append((k[..., :n, :], v[..., :n, :], i * self.chunk_size))
        return out


class HALOCacheChunked:
    """Recent-window GPU cache plus pinned-host cold tier (Path D)."""

    def __init__(self, *, config=None, storage=None, scorer=None, demoter=None, refetcher=None,
                 chunk_size: int = 512, recent_window: int = 64, use_triton: bool = True) -> None:
        self.cfg = config
        self.storage, self.scorer, self.demoter, self.refetcher = storage, scorer, demoter, refetcher
        self.chunk_size = int(chunk_size)
        self.recent_window = int(recent_window)
        self.use_triton = use_triton
        self._k: dict = {}
        self._v: dict = {}
        self._cold: dict = {}
        self._mode = "warmup"
        self.last_stats = ChunkedAttentionStats()
        self.demoted_blocks_total = 0
        self._dma_bytes_cumulative = 0

    # ------------------------------------------------------------- cache API
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        """Append new rows; returns this layer's GPU rows (all rows in warm-up,
        the recent window in chunked mode)."""
        T_new = key_states.shape[-2]
        if layer_idx in self._k:
            self._k[layer_idx] = torch.cat([self._k[layer_idx], key_states], dim=-2)
            self._v[layer_idx] = torch.cat([self._v[layer_idx], value_states], dim=-2)
        else:
            self._k[layer_idx], self._v[layer_idx] = key_states, value_states
        T = self._k[layer_idx].shape[-2]
        if self._mode == "warmup":
            if T_new == 1 and T > 2 * self.chunk_size:
                self._mode = "chunked"
                self._peel(layer_idx)
        elif T > self.recent_window + self.chunk_size:
            self._peel(layer_idx)
        elif layer_idx not in self._cold and T > 2 * self.chunk_size:
            self._peel(layer_idx)  # a layer that reaches the transition after the first
        return self._k[layer_idx], self._v[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        cold = self._cold.get(layer_idx)
        rec = self._k.get(layer_idx)
        return (cold.rows if cold is not None else 0) + (rec.shape[-2] if rec is not None else 0)

    def reset(self) -> None:
        self._k.clear()
        self._v.clear()
        self._cold.clear()
        self._mode = "warmup"
        self.demoted_blocks_total = 0
        self._dma_bytes_cumulative = 0

    def telemetry(self) -> dict:
        s = self.last_stats
        return {"mode": self._mode, "hot_positions": s.hot_positions, "cold_positions": s.cold_positions,
                "n_chunks": s.n_chunks, "peak_staging_bytes": s.peak_staging_bytes, "dma_bytes": s.dma_bytes,
                "used_lse_merge": s.used_lse_merge, "demoted_blocks_total": self.demoted_blocks_total,
                "dma_bytes_cumulative": self._dma_bytes_cumulative}

    # ------------------------------------------------------------- peel
    def _peel(self, layer_idx: int) -> None:
        """Move all but the last ``recent_window`` rows to the cold tier."""
        k, v = self._k[layer_idx], self._v[layer_idx]
        T = k.shape[-2]
        peel = T - self.recent_window
        if peel <= 0:
            return
        cold = self._cold.setdefault(layer_idx, _ColdTier(self.chunk_size))
        on_gpu = k.is_cuda
        cs = copy_stream(k.device) if on_gpu else None
        if cs is not None:
            cs.wait_stream(torch.cuda.current_stream(k.device))
        done = 0
        while done < peel:
            ci, off = divmod(cold.rows, self.chunk_size)
            if ci == len(cold.k):
                shape = (k.shape[0], k.shape[1], self.chunk_size, k.shape[3])
                cold.k.append(torch.empty(shape, dtype=k.dtype, pin_memory=on_gpu))
                cold.v.append(torch.empty(shape, dtype=v.dtype, pin_memory=on_gpu))
            n = min(self.chunk_size - off, peel - done)
            if cs is not None:
                with torch.cuda.stream(cs):
                    cold.k[ci][..., off:off + n, :].copy_(k[..., done:done + n, :], non_blocking=True)
                    cold.v[ci][..., off:off + n, :].copy_(v[..., done:done + n, :], non_blocking=True)
            else:
                cold.k[ci][..., off:off + n, :].copy_(k[..., done:done + n, :])
                cold.v[ci][..., off:off + n, :].copy_(v[..., done:done + n, :])
            cold.rows += n
            done += n
        if cs is not None:
            k.record_stream(cs)
            v.record_stream(cs)
        self._k[layer_idx] = k[..., peel:, :].contiguous()
        self._v[layer_idx] = v[..., peel:, :].contiguous()
        self._dma_bytes_cumulative += 2 * peel * k.shape[0] * k.shape[1] * k.shape[3] * k.element_size()
        bs = max(1, getattr(self.cfg, "block_size", 32) if self.cfg is not None else 32)
        self.demoted_blocks_total += (peel + bs - 1) // bs

    # ------------------------------------------------------------- attention
    def compute_attention(self, query: torch.Tensor, layer_idx: int, *, scaling: Optional[float] = None,
                          query_pos_offset: Optional[int] = None, return_lse: bool = False):
        """Attention of ``query`` (B, H, T_q, D) over every cached row of the
        layer (cold chunks + recent rows), causal by global position; the
        query rows sit at ``query_pos_offset`` (default T_total - T_q)."""
        from .decode import ChunkRef
        from .prefill import prefill_attention
        from .triton_chunked import triton_chunked_attention_streamed
        B, H, T_q, D = query.shape
        scale = 1.0 / math.sqrt(D) if scaling is None else float(scaling)
        rec_k, rec_v = self._k[layer_idx], self._v[layer_idx]
        cold = self._cold.get(layer_idx)
        cold_chunks = cold.chunks() if cold is not None else []
        T_cold = cold.rows if cold is not None else 0
        T_total = T_cold + rec_k.shape[-2]
        q0 = T_total - T_q if query_pos_offset is None else int(query_pos_offset)
        stats = ChunkedAttentionStats(hot_positions=rec_k.shape[-2], cold_positions=T_cold,
                                      n_chunks=len(cold_chunks) + 1, used_lse_merge=bool(cold_chunks))
        if T_q == 1:
            q_pos = torch.full((B,), q0, dtype=torch.int64, device=query.device)
            res = triton_chunked_attention_streamed(
                query, [(k, v, c0) for (k, v, c0) in cold_chunks], [(rec_k, rec_v, T_cold)],
                scale=scale, q_pos=q_pos, return_lse=return_lse)
            per = max((k.numel() * k.element_size() for (k, _, _) in cold_chunks), default=0)
            stats.peak_staging_bytes = 2 * 2 * per
            stats.dma_bytes = sum(2 * k.numel() * k.element_size() for (k, _, _) in cold_chunks)
        else:
            staged = [ChunkRef(k.to(query.device, non_blocking=True), v.to(query.device, non_blocking=True),
                               c0, True) for (k, v, c0) in cold_chunks]
            chunks = staged + [ChunkRef(rec_k, rec_v, T_cold, True)]
            res = prefill_attention(query, chunks, scale=scale, q_start=q0, return_lse=return_lse)
            stats.peak_staging_bytes = sum(2 * c.k.numel() * c.k.element_size() for c in staged)
            stats.dma_bytes = stats.peak_staging_bytes
        self.last_stats = stats
        return res
