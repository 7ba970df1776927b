"""Drop-in replacement for ``halo/triton_chunked.py`` on MI355X.

The module keeps the reference's name and its public call signatures
(halo/triton_chunked.py:141-501) so that ``from halo.triton_chunked import
...`` can be rewritten to ``from halo_amd.triton_chunked import ...`` with no
other change.  There is no Triton here: every entry point enqueues the
hand-written HIP kernel of ``halo_amd/csrc/decode_attn.hip`` through the
C-ABI.  ``HAS_TRITON`` keeps its role as the availability flag the cache
reads (halo/kv_cache_chunked.py:156-163): it is True when the HIP library is
loaded and a GPU is visible.

Differences that are deliberate:
  * one launch covers a whole chunk list (the reference launches once per
    chunk, halo/triton_chunked.py:259-264), with chunk starts as runtime
    table entries instead of a JIT constant (:52);
  * a chunk whose rows are all causally masked contributes zero weight
    (the PyTorch route's rule, halo/kv_cache_chunked.py:221-238) instead of
    the NaN the Triton kernel produces when that chunk comes first (:122-128);
  * every function accepts ``return_lse=True`` to also return the
    log-sum-exp of the attended scores (the reference computes and drops it);
  * ``_single_launch`` attends the hot tensors in place instead of copying
    them device-to-device into the staging buffer (:474-477);
  * launch plans (descriptor and work tables on the device) are cached by
    chunk addresses and layout (``decode.cached_plan``), so a call that
    repeats a chunk list uploads nothing and can be captured in a HIP graph;
    ``triton_chunked_attention`` keeps, per chunk-list layout and stream, the
    plan, its default query positions and the fixed launch arguments, so a
    repeated call does one key build, two allocations and one library call.
"""
from __future__ import annotations

import collections
import math
from typing import Optional

import torch

from . import _native as nat
from .decode import ChunkRef, cached_plan, keep_for_capture, launch

HAS_TRITON = nat.available()
HAS_HIP = HAS_TRITON


def _require() -> None:
    nat.lib()  # raises RuntimeError when the library or the GPU is missing


def init_acc(
    *, B: int, H: int, D_v: int, device, dtype=torch.float32,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Initialise the (m, l, o) accumulators (halo/triton_chunked.py:141-148)."""
    m = torch.full((B, H), float("-inf"), device=device, dtype=dtype)
    l = torch.zeros((B, H), device=device, dtype=dtype)
    o = torch.zeros((B, H, D_v), device=device, dtype=dtype)
    return m, l, o


def update_chunk(
    *, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    m: torch.Tensor, l: torch.Tensor, o: torch.Tensor,
    scale: float, chunk_start: int, q_pos: torch.Tensor,
    apply_causal: bool, block_n: int = 64,
) -> None:
    """Merge one chunk into the running (m, l, o) in place
    (halo/triton_chunked.py:151-192).  ``block_n`` is accepted for signature
    compatibility; the HIP kernel tiles by 64-row wavefront tiles."""
    _require()
    assert q.dim() == 3, f"expected q (B, H, D), got {q.shape}"
    B, H, D = q.shape
    H_KV = k.shape[1]
    T_c = k.shape[2]
    D_V = v.shape[-1]
    assert k.shape == (B, H_KV, T_c, D), f"k shape {k.shape}"
    assert v.shape == (B, H_KV, T_c, D_V), f"v shape {v.shape}"
    assert D_V == D, "the HIP kernel requires D_v == D"
    if T_c == 0:
        return
    dtype = k.dtype
    plan = cached_plan(B=B, H=H, H_kv=H_KV, D=D, dtype=dtype,
                       chunks=[ChunkRef(_al(k), _al(v), int(chunk_start), bool(apply_causal))],
                       device=q.device)
    launch(plan, q, scale=float(scale), q_pos=q_pos, m=m, l=l, o=o, acc_mode=3)


def finalize(
    *, m: torch.Tensor, l: torch.Tensor, o: torch.Tensor,
    out_dtype: torch.dtype, return_lse: bool = False,
):
    """out = o / (l > 0 ? l : 1) in ``out_dtype`` (halo/triton_chunked.py:195-207);
    with ``return_lse`` also lse = m + log(l) (-inf where l == 0)."""
    L = nat.lib()
    B, H, D = o.shape
    m_, l_, o_ = m.contiguous().float(), l.contiguous().float(), o.contiguous().float()
    out = torch.empty((B, H, D), device=o.device, dtype=out_dtype)
    lse = torch.empty((B, H), device=o.device, dtype=torch.float32) if return_lse else None
    nat.check(L.halo_finalize(m_.data_ptr(), l_.data_ptr(), o_.data_ptr(), B, H, D,
                              out.data_ptr(), nat.dtype_code(out_dtype), nat.ptr(lse),
                              nat.stream_ptr()), "halo_finalize")
    return (out, lse) if return_lse else out


def lse_merge(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor):
    """Combine two partial attention results over disjoint key sets
    (``halo_lse_merge``; HALOCacheChunked._lse_merge,
    halo/kv_cache_chunked.py:194-239): lse = logaddexp(lse_a, lse_b), out =
    exp(lse_a - lse) out_a + exp(lse_b - lse) out_b, where a side whose lse
    is -inf contributes nothing.  out_* (..., D) and lse_* (...) any float
    dtype; returns fp32 (out, lse)."""
    L = nat.lib()
    if out_a.shape != out_b.shape or lse_a.shape != lse_b.shape or tuple(out_a.shape[:-1]) != tuple(lse_a.shape):
        raise AssertionError(f"shapes: out {tuple(out_a.shape)}/{tuple(out_b.shape)}, "
                             f"lse {tuple(lse_a.shape)}/{tuple(lse_b.shape)}")
    D = out_a.shape[-1]
    oa, ob = out_a.float().contiguous(), out_b.float().contiguous()
    la, lb = lse_a.float().contiguous(), lse_b.float().contiguous()
    out = torch.empty_like(oa)
    lse = torch.empty_like(la)
    n = la.numel()
    if n:
        nat.check(L.halo_lse_merge(oa.data_ptr(), la.data_ptr(), ob.data_ptr(), lb.data_ptr(), n, D,
                                   out.data_ptr(), lse.data_ptr(), nat.stream_ptr()), "halo_lse_merge")
    return out, lse


def _al(t: torch.Tensor) -> torch.Tensor:
    esz = t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16 or (t.stride(-2) * esz) % 16:
        return t.contiguous()
    return t


def _q3(q: torch.Tensor) -> torch.Tensor:
    if q.dim() == 4:
        assert q.shape[2] == 1, f"decode path supports T_q=1 only; got {q.shape}"
        return q.squeeze(2)
    return q


def _qpos(q_pos, B: int, total_T: int, device) -> torch.Tensor:
    if q_pos is None:
        return torch.full((B,), total_T - 1, device=device, dtype=torch.int64)
    if not torch.is_tensor(q_pos):
        q_pos = torch.as_tensor(q_pos)
    return q_pos.to(device=device, dtype=torch.int64)


def _run(q3: torch.Tensor, chunks: list, scale: float, q_pos: torch.Tensor,
         out_dtype, return_lse: bool, q_pos_host=None, want_plan: bool = False):
    B, H, D = q3.shape
    H_kv = chunks[0].k.shape[1]
    opts = {} if q_pos_host is None else {"q_pos_host": tuple(int(x) for x in q_pos_host)}
    plan = cached_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=chunks[0].k.dtype, chunks=chunks,
                       device=q3.device, **opts)
    out = torch.empty((B, H, D), device=q3.device, dtype=out_dtype)
    lse = torch.empty((B, H), device=q3.device, dtype=torch.float32) if return_lse else None
    launch(plan, q3, scale=scale, q_pos=q_pos, out=out, lse=lse)
    return (out, lse, plan) if want_plan else (out, lse)


# Repeated calls of triton_chunked_attention: key = the query's shape, dtype
# and device, the stream, whether q_pos was given, and each chunk's K/V
# addresses, shapes, strides, dtype, start and causal flag.  A chunk list
# that needed a contiguous copy (misaligned rows) is never entered, so a hit
# implies the checks the full path makes.  Least recently used entries go
# beyond FAST_CACHE_SIZE.
FAST_CACHE_SIZE = 256
_fast: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()


def clear_fast_cache() -> None:
    """Drop the per-layout entries.  Entries replayed under graph capture
    stay alive (``decode.captured_plans``)."""
    _fast.clear()


def _load_layout_key(path=None):
    """The prebuilt host extension (halo_amd/_lib/fastkey_build, made by
    build()) that reads the chunk list's layout in C++, or None when it is
    missing or cannot be loaded."""
    import importlib.util
    import os
    if path is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "fastkey_build",
                            "_halo_fastkey.so")
    if not os.path.exists(path):
        return None
    try:
        spec = importlib.util.spec_from_file_location("_halo_fastkey", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod.chunk_layout_key
    except (ImportError, OSError, AttributeError):
        # built against another torch, or not a loadable module: the key is
        # then built in Python (same fields, slower)
        return None


_layout_key = _load_layout_key()


def _fast_key_py(q3: torch.Tensor, chunks, stream, default_pos: bool) -> tuple:
    return (q3.shape, q3.dtype, q3.device, stream, default_pos,
            *[(k.data_ptr(), k.shape, k.stride(), k.dtype, v.data_ptr(), v.shape, v.stride(), v.dtype,
               int(c0), bool(causal)) for (k, v, c0, causal) in chunks])


def _fast_key(q3: torch.Tensor, chunks, stream, default_pos: bool) -> tuple:
    """Key of the per-layout fast path: the query's shape, dtype and device,
    the stream, whether q_pos was defaulted, and every chunk's K/V address,
    dtype, sizes and strides with its start and causal flag (read in C++ when
    the host extension is built: ~4 us instead of ~15 us for 12 chunks)."""
    if _layout_key is not None:
        try:
            return (q3.shape, q3.dtype, q3.device, stream, default_pos, _layout_key(chunks))
        except (TypeError, RuntimeError):
            pass
    return _fast_key_py(q3, chunks, stream, default_pos)


def _fast_entry(plan, q3: torch.Tensor, qp_default) -> tuple:
    from .decode import plan_workspace
    nbytes = int(nat.lib().halo_decode_workspace_size(plan.n_work, plan.rep_t, plan.D))
    ws = plan_workspace(plan, q3.device)
    if ws.numel() < nbytes:
        raise AssertionError("plan workspace smaller than the launch needs")
    mid = (plan.B, plan.H, plan.H_kv, plan.D, plan.rep_t, plan.descs.data_ptr(), plan.n_desc,
           plan.work.data_ptr(), plan.n_work, None if plan.uniform_groups else plan.offsets.data_ptr(),
           plan.n_groups)
    return (plan, qp_default, mid, nat.dtype_code(plan.dtype), ws.data_ptr(), ws.numel())


def triton_chunked_attention(
    q: torch.Tensor,
    chunks: list[tuple[torch.Tensor, torch.Tensor, int, bool]],
    *,
    scale: Optional[float] = None,
    q_pos: Optional[torch.Tensor] = None,
    block_n: int = 64,
    return_lse: bool = False,
):
    """LSE-merged attention of one query token over a list of
    ``(k, v, chunk_start, apply_causal)`` chunks, one launch for the whole list
    (halo/triton_chunked.py:210-267).  Returns (B, H, 1, D_v) in ``q.dtype``
    (and the (B, H) fp32 LSE when ``return_lse``)."""
    q3 = _q3(q)
    B, H, D = q3.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if not chunks:
        out = torch.zeros(B, H, 1, D, device=q.device, dtype=q.dtype)
        if return_lse:
            return out, torch.full((B, H), float("-inf"), device=q.device)
        return out
    L = nat.lib()  # raises RuntimeError when the library or the GPU is missing
    stream = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else 0
    key = _fast_key(q3, chunks, stream, q_pos is None)
    ent = _fast.get(key)
    if ent is not None and q3.stride(-1) == 1:
        _fast.move_to_end(key)
        keep_for_capture(ent)
        plan, qp_default, mid, dt, ws_ptr, ws_n = ent
        qp = qp_default if q_pos is None else _qpos(q_pos, B, 0, q.device).contiguous()
        if qp.numel() != B:
            raise AssertionError(f"q_pos must have B={B} entries, got {qp.numel()}")
        out = torch.empty((B, H, D), device=q.device, dtype=q.dtype)
        lse = torch.empty((B, H), device=q.device, dtype=torch.float32) if return_lse else None
        nat.check(L.halo_decode_attn(q3.data_ptr(), q3.stride(0), q3.stride(1), dt, *mid, qp.data_ptr(),
                                     float(scale), None, None, None, H, 0, out.data_ptr(), dt, nat.ptr(lse),
                                     ws_ptr, ws_n, stream), "halo_decode_attn")
        out = out.unsqueeze(2)
        return (out, lse) if return_lse else out
    total_T = sum(k.shape[-2] for (k, _, _, _) in chunks)
    qp = _qpos(q_pos, B, total_T, q.device)
    refs = [ChunkRef(_al(k), _al(v), int(c0), bool(causal)) for (k, v, c0, causal) in chunks]
    out, lse, plan = _run(q3, refs, float(scale), qp, q.dtype, return_lse, want_plan=True)
    copied = any(r.k is not k or r.v is not v for r, (k, v, _, _) in zip(refs, chunks))
    if not copied and q3.dtype == plan.dtype and q3.is_cuda and not torch.cuda.is_current_stream_capturing():
        _fast[key] = _fast_entry(plan, q3, qp if q_pos is None else None)
        while len(_fast) > FAST_CACHE_SIZE:
            _fast.popitem(last=False)
    out = out.unsqueeze(2)
    return (out, lse) if return_lse else out


def triton_chunked_attention_streamed(
    q: torch.Tensor,
    cold_chunks_host: list[tuple[torch.Tensor, torch.Tensor, int]],
    hot_chunks_gpu: list[tuple[torch.Tensor, torch.Tensor, int]],
    *,
    scale: Optional[float] = None,
    q_pos: torch.Tensor,
    block_n: int = 64,
    n_buffers: int = 2,
    return_lse: bool = False,
):
    """Cold chunks are copied host->device on a side stream through
    ``n_buffers`` staging slots while the hot chunks are attended on the
    compute stream; each cold chunk is merged as soon as its copy lands
    (halo/triton_chunked.py:270-362).  The merge is order-free, so attending
    hot first gives the same result as the reference's cold-first order."""
    from .memory_tier import stream_cold_chunks
    q3 = _q3(q).contiguous()
    B, H, D = q3.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    first = (cold_chunks_host[0] if cold_chunks_host else
             (hot_chunks_gpu[0] if hot_chunks_gpu else None))
    if first is None:
        out = torch.zeros(B, H, 1, D, device=q.device, dtype=q.dtype)
        return (out, torch.full((B, H), float("-inf"), device=q.device)) if return_lse else out
    _require()
    qp = _qpos(q_pos, B, 0, q.device)
    m, l, o = init_acc(B=B, H=H, D_v=D, device=q.device)
    if hot_chunks_gpu:
        refs = [ChunkRef(_al(k), _al(v), int(c0), True) for (k, v, c0) in hot_chunks_gpu]
        plan = cached_plan(B=B, H=H, H_kv=refs[0].k.shape[1], D=D, dtype=refs[0].k.dtype,
                           chunks=refs, device=q.device)
        launch(plan, q3, scale=float(scale), q_pos=qp, m=m, l=l, o=o, acc_mode=2)
    if cold_chunks_host:
        stream_cold_chunks(q3, cold_chunks_host, scale=float(scale), q_pos=qp,
                           m=m, l=l, o=o, n_buffers=n_buffers)
    res = finalize(m=m, l=l, o=o, out_dtype=q.dtype, return_lse=return_lse)
    if return_lse:
        return res[0].unsqueeze(2), res[1]
    return res.unsqueeze(2)


def triton_chunked_attention_single_launch(
    q: torch.Tensor,
    cold_k_host: Optional[torch.Tensor],
    cold_v_host: Optional[torch.Tensor],
    hot_k_gpu: Optional[torch.Tensor],
    hot_v_gpu: Optional[torch.Tensor],
    *,
    scale: Optional[float] = None,
    q_pos: torch.Tensor,
    block_n: int = 64,
    apply_causal: bool = True,
    return_lse: bool = False,
):
    """One H2D copy per cold tensor on a side stream, then one kernel over
    the cold staging buffer and the hot tensors in place
    (halo/triton_chunked.py:365-490).  Cold rows sit at positions
    [0, T_cold), hot rows at [T_cold, T_cold + T_hot)."""
    q3 = _q3(q).contiguous()
    B, H, D = q3.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ref = None
    for cand in (cold_v_host, hot_v_gpu):
        if cand is not None and cand.shape[-2] > 0:
            ref = cand
            break
    if ref is None:
        out = torch.zeros(B, H, 1, D, device=q.device, dtype=q.dtype)
        return (out, torch.full((B, H), float("-inf"), device=q.device)) if return_lse else out
    _require()
    T_cold = cold_k_host.shape[-2] if cold_k_host is not None else 0
    T_hot = hot_k_gpu.shape[-2] if hot_k_gpu is not None else 0
    qp = _qpos(q_pos, B, T_cold + T_hot, q.device)
    chunks = []
    compute = torch.cuda.current_stream()
    if T_cold > 0:
        copy_stream = torch.cuda.Stream(device=q.device)
        k_buf = torch.empty(cold_k_host.shape, device=q.device, dtype=cold_k_host.dtype)
        v_buf = torch.empty(cold_v_host.shape, device=q.device, dtype=cold_v_host.dtype)
        copy_stream.wait_stream(compute)
        with torch.cuda.stream(copy_stream):
            k_buf.copy_(cold_k_host, non_blocking=True)
            v_buf.copy_(cold_v_host, non_blocking=True)
        compute.wait_stream(copy_stream)
        k_buf.record_stream(copy_stream)
        v_buf.record_stream(copy_stream)
        chunks.append(ChunkRef(k_buf, v_buf, 0, bool(apply_causal)))
    if T_hot > 0:
        chunks.append(ChunkRef(_al(hot_k_gpu), _al(hot_v_gpu), T_cold, bool(apply_causal)))
    out, lse = _run(q3, chunks, float(scale), qp, q.dtype, return_lse)
    out = out.unsqueeze(2)
    return (out, lse) if return_lse else out


__all__ = [
    "HAS_TRITON",
    "HAS_HIP",
    "init_acc",
    "update_chunk",
    "finalize",
    "lse_merge",
    "triton_chunked_attention",
    "triton_chunked_attention_streamed",
    "triton_chunked_attention_single_launch",
]
