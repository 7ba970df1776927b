"""Chunked causal prefill attention on bf16/fp16 MFMA.

``prefill_attention(q, chunks)`` attends a block of query rows to a list of
KV chunks (prior context chunks plus the query block's own K/V, the latter
causal) and returns the output, optionally with the log-sum-exp, in one
launch of ``halo_prefill_attn``.

Reference: the chunked prefill path of HALOCacheChunked.compute_attention
(halo/kv_cache_chunked.py:864-964), which runs _chunk_attention per chunk and
folds the partials with _lse_merge (:194-276); the causal rule is
chunk_start + t <= q_start + i (halo/triton_chunked.py:114-119) and the
default query offset is T_total - T_q (halo/kv_cache_chunked.py:839-840).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _native as nat
from .decode import ChunkRef, descs_to_device, pack_descs


def prefill_attention(q: torch.Tensor, chunks: Sequence[ChunkRef], *, scale: Optional[float] = None,
                      q_start=None, out_dtype: Optional[torch.dtype] = None, return_lse: bool = False,
                      stream=None):
    """q (B, H, T_q, D) bf16/fp16; chunks (B, H_kv, T_c, D) of the same dtype.
    Returns out (B, H, T_q, D) in ``out_dtype`` (default q.dtype) and, with
    ``return_lse``, lse (B, H, T_q) fp32."""
    L = nat.lib()
    if q.dim() != 4:
        raise AssertionError(f"q must be (B, H, T_q, D), got {tuple(q.shape)}")
    B, H, T_q, D = q.shape
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise AssertionError(f"prefill runs on bf16/fp16 MFMA; got {q.dtype}")
    if not chunks:
        raise AssertionError("no chunks to attend")
    H_kv = chunks[0].k.shape[-3]
    if H % H_kv:
        raise AssertionError(f"head count mismatch: q has {H}, kv has {H_kv}")
    if q.stride(-1) != 1 or (q.stride(-2) * 2) % 16 or q.data_ptr() % 16:
        q = q.contiguous()
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if q_start is None:
        q_start = sum(c.T for c in chunks) - T_q
    if not torch.is_tensor(q_start):
        q_start = torch.full((B,), int(q_start), dtype=torch.int64)
    q_start = q_start.to(device=q.device, dtype=torch.int64).reshape(B).contiguous()
    descs, keep = pack_descs(chunks, B=B, H_kv=H_kv, D=D, dtype=q.dtype)
    d_descs = descs_to_device(descs, q.device)
    out = torch.empty((B, H, T_q, D), device=q.device, dtype=out_dtype or q.dtype)
    lse = torch.empty((B, H, T_q), device=q.device, dtype=torch.float32) if return_lse else None
    nat.check(L.halo_prefill_attn(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), nat.dtype_code(q.dtype), B, H, H_kv, T_q, D,
        q_start.data_ptr(), d_descs.data_ptr(), len(chunks), scale,
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), nat.dtype_code(out.dtype),
        nat.ptr(lse), nat.stream_ptr(stream)), "halo_prefill_attn")
    # The descriptor buffer is freed into torch's stream-ordered caching
    # allocator, so later work on the launch stream cannot reuse it early;
    # on another stream it is recorded.  The caller owns the K/V tensors.
    if stream is not None:
        d_descs.record_stream(stream)
    del keep
    return (out, lse) if return_lse else out
