"""KIVI cache with quantise-on-demote on the GPU.

Reference: ``KIVICache`` (baselines/kivi_cache.py:80-195).  Each layer keeps
a recent window of unquantised rows and a quantised buffer for everything
older: when the recent window exceeds ``residual_length``, its oldest whole
groups of 32 tokens are quantised (K per channel over the 32 tokens, V per
token over 32 channels, the arithmetic of ``_quantize_per_group``, :44-69)
and leave the window.  Differences:
  * the quantised rows are packed into 32-token blocks by
    ``halo_kivi_quantize`` written straight into a per-layer block buffer
    that grows by doubling (the reference concatenates (codes, scale, zero)
    tensors on every demotion, :162-178);
  * ``update`` returns the dequantised cache as the reference does
    (:187-195), but blocks never change once written, so each block is
    dequantised once, into a per-layer buffer, instead of the whole
    quantised buffer on every call; with ``materialize=False`` nothing is
    dequantised and ``update`` returns None;
  * ``compute_attention`` attends the blocks and the recent rows directly:
    decode (T_q = 1) is one ``halo_decode_attn_kivi`` launch plus its merge,
    dequantising in registers; T_q > 1 runs the MFMA prefill over the
    dequantised blocks and the recent rows.
As in the reference the class is a transformers ``DynamicCache`` when
transformers is importable: ``update`` also leaves the dequantised cache in
the layer's ``keys`` / ``values``, so the model's own attention and mask
sizes see it, and ``wrap_with_kivi`` installs a fresh cache per
``generate`` call (:205-226).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import kivi
from .decode import ChunkRef

try:  # the HF cache protocol when transformers is importable (baselines/kivi_cache.py:27-34)
    from transformers.cache_utils import DynamicCache as _BaseCache
    from transformers.cache_utils import DynamicLayer as _Layer
    HAS_TRANSFORMERS = True
except Exception:  # pragma: no cover - exercised only without transformers
    _BaseCache, _Layer = object, None
    HAS_TRANSFORMERS = False

GROUP = kivi.GROUP


class KIVICache(_BaseCache):
    """Per-layer recent window + packed KIVI blocks (B, H_kv, n, block_bytes)."""

    def __init__(self, *, bits: int = 2, group_size: int = 32, residual_length: int = 32,
                 materialize: bool = True, chunk_tokens: int = 2048) -> None:
        if HAS_TRANSFORMERS:
            super().__init__()
        if group_size != GROUP:
            raise AssertionError(f"KIVI blocks hold {GROUP} tokens; group_size={group_size} is not supported")
        if bits not in (2, 4, 8):
            raise AssertionError(f"bits must be 2, 4 or 8, got {bits}")
        if residual_length < 0:
            raise AssertionError("residual_length must be >= 0")
        self.bits = bits
        self.group_size = group_size
        self.residual_length = residual_length
        self.materialize = materialize
        self.chunk_tokens = chunk_tokens
        self._k_recent: list = []
        self._v_recent: list = []
        self._blocks: list = []      # uint8 (B, H_kv, capacity, block_bytes) per layer
        self._n_seen: list = []      # tokens absorbed into blocks per layer
        self._deq: list = []         # (k, v) dequantised buffers per layer (materialize)
        self._n_deq: list = []       # blocks already dequantised into them

    @classmethod
    def from_memory_ratio(cls, *, memory_ratio: int, **kw) -> "KIVICache":
        """bits = max(16 // memory_ratio, 2) (baselines/kivi_cache.py:106-109)."""
        return cls(bits=max(16 // memory_ratio, 2), **kw)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self._n_seen):
            return 0
        rec = self._k_recent[layer_idx]
        return self._n_seen[layer_idx] + (rec.shape[-2] if rec is not None else 0)

    def reset(self) -> None:
        for lst in (self._k_recent, self._v_recent, self._blocks, self._n_seen, self._deq, self._n_deq):
            lst.clear()
        if HAS_TRANSFORMERS:
            self.layers = []

    def blocks(self, layer_idx: int) -> Optional[torch.Tensor]:
        """The layer's packed blocks (B, H_kv, n_seen / 32, block_bytes)."""
        buf = self._blocks[layer_idx] if layer_idx < len(self._blocks) else None
        if buf is None:
            return None
        return buf[:, :, : self._n_seen[layer_idx] // GROUP]

    def recent(self, layer_idx: int):
        return self._k_recent[layer_idx], self._v_recent[layer_idx]

    # ------------------------------------------------------------ update
    def _ensure_layer(self, layer_idx: int) -> None:
        while len(self._k_recent) <= layer_idx:
            for lst in (self._k_recent, self._v_recent, self._blocks, self._deq):
                lst.append(None)
            self._n_seen.append(0)
            self._n_deq.append(0)

    def _demote(self, layer_idx: int, k_rows: torch.Tensor, v_rows: torch.Tensor) -> None:
        """Quantise whole groups of rows into the layer's block buffer."""
        B, H_kv, T, D = k_rows.shape
        nb = kivi.block_bytes(D, self.bits)
        n0 = self._n_seen[layer_idx] // GROUP
        n_new = T // GROUP
        buf = self._blocks[layer_idx]
        if buf is None or buf.shape[2] < n0 + n_new:
            cap = max(n0 + n_new, 2 * (buf.shape[2] if buf is not None else 0), 64)
            grown = torch.empty((B, H_kv, cap, nb), device=k_rows.device, dtype=torch.uint8)
            if buf is not None and n0 > 0:
                grown[:, :, :n0] = buf[:, :, :n0]
            buf = grown
            self._blocks[layer_idx] = buf
        kivi.quantize(k_rows, v_rows, bits=self.bits, out=buf[:, :, n0:n0 + n_new])
        self._n_seen[layer_idx] += T

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        """Append the new rows, demote the recent window's overflow in whole
        groups (baselines/kivi_cache.py:121-185) and return the dequantised
        cache (K, V) (B, H_kv, T, D) when ``materialize`` (:187-195)."""
        self._ensure_layer(layer_idx)
        k_rec, v_rec = self._k_recent[layer_idx], self._v_recent[layer_idx]
        if k_rec is None:
            new_k, new_v = key_states, value_states
        else:
            new_k = torch.cat([k_rec, key_states], dim=-2)
            new_v = torch.cat([v_rec, value_states], dim=-2)
        T_rec = new_k.shape[-2]
        if T_rec > self.residual_length:
            overflow_q = ((T_rec - self.residual_length) // GROUP) * GROUP
            if overflow_q > 0:
                self._demote(layer_idx, new_k[..., :overflow_q, :].contiguous(),
                             new_v[..., :overflow_q, :].contiguous())
                new_k = new_k[..., overflow_q:, :]
                new_v = new_v[..., overflow_q:, :]
        self._k_recent[layer_idx] = new_k.contiguous()
        self._v_recent[layer_idx] = new_v.contiguous()
        if not self.materialize:
            return None
        k_full, v_full = self._materialized(layer_idx)
        if HAS_TRANSFORMERS:
            # the HF layer holds what attention reads: its length gives the mask sizes
            while len(self.layers) <= layer_idx:
                self.layers.append(_Layer())
            lay = self.layers[layer_idx]
            if not lay.is_initialized:
                lay.lazy_initialization(key_states, value_states)
            lay.keys, lay.values = k_full, v_full
        return k_full, v_full

    def _materialized(self, layer_idx: int):
        """Dequantise the blocks not yet dequantised and place the recent
        rows after them; returns views of the layer's buffers."""
        k_rec, v_rec = self._k_recent[layer_idx], self._v_recent[layer_idx]
        n_blk = self._n_seen[layer_idx] // GROUP
        T = self._n_seen[layer_idx] + k_rec.shape[-2]
        if n_blk == 0:
            return k_rec, v_rec
        B, H_kv, _, D = k_rec.shape
        deq = self._deq[layer_idx]
        if deq is None or deq[0].shape[2] < T or deq[0].dtype != k_rec.dtype:
            cap = max(T, 2 * (deq[0].shape[2] if deq is not None else 0), 256)
            nk = torch.empty((B, H_kv, cap, D), device=k_rec.device, dtype=k_rec.dtype)
            nv = torch.empty_like(nk)
            done = self._n_deq[layer_idx] if deq is not None and deq[0].dtype == k_rec.dtype else 0
            if done:
                nk[:, :, : done * GROUP] = deq[0][:, :, : done * GROUP]
                nv[:, :, : done * GROUP] = deq[1][:, :, : done * GROUP]
            deq = (nk, nv)
            self._deq[layer_idx] = deq
            self._n_deq[layer_idx] = done
        done = self._n_deq[layer_idx]
        if done < n_blk:
            kd, vd = kivi.dequantize(self._blocks[layer_idx][:, :, done:n_blk], D=D, dtype=k_rec.dtype,
                                     bits=self.bits)
            deq[0][:, :, done * GROUP: n_blk * GROUP] = kd
            deq[1][:, :, done * GROUP: n_blk * GROUP] = vd
            self._n_deq[layer_idx] = n_blk
        t0 = n_blk * GROUP
        deq[0][:, :, t0:T] = k_rec
        deq[1][:, :, t0:T] = v_rec
        return deq[0][:, :, :T], deq[1][:, :, :T]

    # --------------------------------------------------------- attention
    def compute_attention(self, q: torch.Tensor, *, layer_idx: int, scaling: Optional[float] = None,
                          query_pos_offset: Optional[int] = None, return_lse: bool = False):
        """Attention of q (B, H, T_q, D) over the layer's cache, causal with
        query row i at position query_pos_offset + i (default T - T_q).
        Decode reads 2-bit blocks directly; 4- and 8-bit decode and T_q > 1
        attend the dequantised blocks and the recent rows (the decode kernel,
        or the MFMA prefill)."""
        from .decode import build_plan, launch
        from .prefill import prefill_attention
        if layer_idx >= len(self._n_seen) or self._k_recent[layer_idx] is None:
            raise AssertionError(f"layer {layer_idx} has no cache")
        B, H, T_q, D = q.shape
        k_rec, v_rec = self._k_recent[layer_idx], self._v_recent[layer_idx]
        H_kv = k_rec.shape[1]
        n_seen = self._n_seen[layer_idx]
        T = n_seen + k_rec.shape[-2]
        q0 = T - T_q if query_pos_offset is None else int(query_pos_offset)
        scale = 1.0 / math.sqrt(D) if scaling is None else float(scaling)
        if q.dtype != k_rec.dtype:
            raise AssertionError(f"q dtype {q.dtype} != cache dtype {k_rec.dtype}")
        recent = [ChunkRef(k_rec, v_rec, n_seen, True)] if k_rec.shape[-2] > 0 else []
        if T_q == 1 and self.bits == 2:
            blocks = self.blocks(layer_idx)
            n = 0 if blocks is None else blocks.shape[2]
            per = self.chunk_tokens // GROUP
            cold = [kivi.KiviChunkRef(blocks[:, :, j:min(j + per, n)], j * GROUP, True, bits=self.bits)
                    for j in range(0, n, per)]
            plan = kivi.plan_kivi(B=B, H=H, H_kv=H_kv, D=D, dtype=q.dtype, cold=cold, recent=recent, device=q.device)
            out = torch.empty((B, H, D), device=q.device, dtype=q.dtype)
            lse = torch.empty((B, H), device=q.device, dtype=torch.float32) if return_lse else None
            q_pos = torch.full((B,), q0, dtype=torch.int64, device=q.device)
            launch(plan, q[:, :, 0], scale=scale, q_pos=q_pos, out=out, lse=lse)
            out = out.unsqueeze(2)
            return (out, lse.unsqueeze(2)) if return_lse else out
        chunks = []
        if n_seen:
            if self.materialize and self._deq[layer_idx] is not None and self._n_deq[layer_idx] * GROUP == n_seen:
                kd, vd = self._deq[layer_idx][0][:, :, :n_seen], self._deq[layer_idx][1][:, :, :n_seen]
            else:
                kd, vd = kivi.dequantize(self.blocks(layer_idx), D=D, dtype=q.dtype, bits=self.bits)
            chunks.append(ChunkRef(kd, vd, 0, True))
        if T_q == 1:
            out = torch.empty((B, H, D), device=q.device, dtype=q.dtype)
            lse = torch.empty((B, H), device=q.device, dtype=torch.float32) if return_lse else None
            if chunks + recent:
                plan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=q.dtype, chunks=chunks + recent, device=q.device)
                q_pos = torch.full((B,), q0, dtype=torch.int64, device=q.device)
                launch(plan, q[:, :, 0], scale=scale, q_pos=q_pos, out=out, lse=lse)
            else:
                out.zero_()
                if lse is not None:
                    lse.fill_(float("-inf"))
            out = out.unsqueeze(2)
            return (out, lse.unsqueeze(2)) if return_lse else out
        return prefill_attention(q, chunks + recent, scale=scale, q_start=q0, return_lse=return_lse)


def wrap_with_kivi(model, *, memory_ratio: int = 4, **kw):
    """Install the KIVI cache on a HF model (baselines/kivi_cache.py:205-226):
    ``generate`` resets one ``KIVICache`` (bits = max(16 // memory_ratio, 2);
    ``kw`` are its other arguments) and passes it as ``past_key_values``
    unless the caller passes a cache of its own.  Returns the model."""
    cache = KIVICache.from_memory_ratio(memory_ratio=memory_ratio, **kw)
    if getattr(model, "_kivi_patched", False):
        return model
    original_generate = model.generate

    def kivi_generate(*args, **kwargs):
        cache.reset()
        kwargs.setdefault("past_key_values", cache)
        kwargs.setdefault("use_cache", True)
        return original_generate(*args, **kwargs)

    model.generate = kivi_generate
    model._kivi_patched = True
    model._kivi_cache = cache
    return model
