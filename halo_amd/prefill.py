"""Chunked causal prefill attention on bf16/fp16 MFMA.

``prefill_attention(q, chunks)`` attends a block of query rows to a list of
KV chunks (prior context chunks plus the query block's own K/V, the latter
causal) and returns the output, optionally with the log-sum-exp, in one
launch of ``halo_prefill_attn``.  fp32 queries run on the decode kernel's
fp32 path instead: the query rows of each batch row are laid out as the
batch of one ``halo_decode_attn`` launch whose chunk descriptors repeat the
same K/V for every such row (batch stride 0), with the causal position of
row i at q_start + i.  That path reads K/V once per query row; it exists
for fp32 models (the reference computes every T_q in fp32,
halo/kv_cache_chunked.py:241-276), not for throughput.

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
from .decode import ChunkRef, _to_device, descs_to_device, pack_descs


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
    if not chunks:
        raise AssertionError("no chunks to attend")
    if q.dtype == torch.float32:
        return _prefill_fp32_rows(q, chunks, scale=scale, q_start=q_start, out_dtype=out_dtype,
                                  return_lse=return_lse, stream=stream)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise AssertionError(f"prefill runs on bf16/fp16 MFMA or the fp32 decode path; got {q.dtype}")
    H_kv = chunks[0].k.shape[-3]
    if H % H_kv:
        raise AssertionError(f"head count mismatch: q has {H}, kv has {H_kv}")
    if q.stride(-1) != 1 or (q.stride(-2) * 2) % 16 or q.data_ptr() % 16:
        q = q.contiguous()
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if q_start is None:
        q_start = sum(c.T for c in chunks) - T_q
    descs, keep = pack_descs(chunks, B=B, H_kv=H_kv, D=D, dtype=q.dtype)
    # The uploads and the launch share one stream (the caller's, or the
    # current one), so the kernel sees the tables; the tables are freed into
    # torch's stream-ordered caching allocator on that stream.  q_start gets
    # there without a blocking copy (a pageable host-to-device copy would
    # hold the host until the stream drains).  The caller owns the K/V.
    with torch.cuda.stream(stream) if stream is not None else _nullctx():
        if not torch.is_tensor(q_start):
            q_start = torch.full((B,), int(q_start), dtype=torch.int64, device=q.device)
        elif q_start.device.type != "cuda":
            q_start = _to_device(q_start.to(torch.int64).reshape(-1).expand(B).numpy(), q.device)
        q_start = q_start.to(device=q.device, dtype=torch.int64).reshape(B).contiguous()
        d_descs = descs_to_device(descs, q.device)
        out = torch.empty((B, H, T_q, D), device=q.device, dtype=out_dtype or q.dtype)
        lse = torch.empty((B, H, T_q), device=q.device, dtype=torch.float32) if return_lse else None
        nat.check(L.halo_prefill_attn(
            q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), nat.dtype_code(q.dtype), B, H, H_kv, T_q, D,
            q_start.data_ptr(), d_descs.data_ptr(), len(chunks), scale,
            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), nat.dtype_code(out.dtype),
            nat.ptr(lse), nat.stream_ptr(stream)), "halo_prefill_attn")
    del keep
    return (out, lse) if return_lse else out


def _prefill_fp32_rows(q: torch.Tensor, chunks: Sequence[ChunkRef], *, scale, q_start, out_dtype,
                       return_lse: bool, stream):
    """fp32 prefill as one decode launch per batch row: pseudo-batch row i is
    query row i, every chunk is read through a batch stride of 0, and the
    causal cut of row i is q_start + i."""
    from .decode import build_plan, launch
    B, H, T_q, D = q.shape
    H_kv = chunks[0].k.shape[-3]
    if H % H_kv:
        raise AssertionError(f"head count mismatch: q has {H}, kv has {H_kv}")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if q_start is None:
        q_start = sum(c.T for c in chunks) - T_q
    if torch.is_tensor(q_start):
        starts = [int(x) for x in q_start.reshape(-1).tolist()]
        if len(starts) == 1:
            starts = starts * B
    else:
        starts = [int(q_start)] * B
    if len(starts) != B:
        raise AssertionError(f"q_start must have B={B} entries")
    out = torch.empty((B, H, T_q, D), device=q.device, dtype=out_dtype or q.dtype)
    lse = torch.empty((B, H, T_q), device=q.device, dtype=torch.float32) if return_lse else None
    ctx = torch.cuda.stream(stream) if stream is not None else _nullctx()
    with ctx:
        for b in range(B):
            rows = []
            for c in chunks:
                if c.k.dtype != torch.float32 or c.v.dtype != torch.float32:
                    raise AssertionError(f"fp32 query needs fp32 chunks, got {c.k.dtype}/{c.v.dtype}")
                kb, vb = c.k[b:b + 1], c.v[b:b + 1]
                rows.append(ChunkRef(kb.expand(T_q, *kb.shape[1:]), vb.expand(T_q, *vb.shape[1:]),
                                     int(c.chunk_start), bool(c.causal)))
            q_pos_host = [starts[b] + i for i in range(T_q)]
            plan = build_plan(B=T_q, H=H, H_kv=H_kv, D=D, dtype=torch.float32, chunks=rows, device=q.device,
                              q_pos_host=q_pos_host)
            q_pos = torch.arange(starts[b], starts[b] + T_q, dtype=torch.int64).to(q.device, non_blocking=True)
            o_b = torch.empty((T_q, H, D), device=q.device, dtype=out.dtype)
            l_b = torch.empty((T_q, H), device=q.device, dtype=torch.float32) if return_lse else None
            launch(plan, q[b].transpose(0, 1), scale=scale, q_pos=q_pos, out=o_b, lse=l_b)
            out[b].copy_(o_b.transpose(0, 1))
            if return_lse:
                lse[b].copy_(l_b.transpose(0, 1))
    return (out, lse) if return_lse else out


class _nullctx:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False
