"""Planning and launching of the split-K decode-attention kernel.

A *plan* is the device-resident chunk table (``halo_chunk_desc`` records) and
work list (``{desc, group, t0, t1, partial slot}`` int32 records) of one
``halo_decode_attn`` launch.  Building it costs a few host microseconds per
chunk; a plan can be replayed for as long as the K/V tensors it points at
stay alive (the plan keeps references to them), which is how the benchmark
and graph-captured decode loops use it.

Reference behaviour mirrored here: the chunk list of
``triton_chunked_attention`` (halo/triton_chunked.py:210-267) and the
per-launch arguments of ``update_chunk`` (halo/triton_chunked.py:151-192).
"""
from __future__ import annotations

import collections
import ctypes
import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native as nat

WORK_INTS = 8  # int32 per work record (kWorkInts in the kernels)

DESC_DTYPE = np.dtype([
    ("k", "<u8"), ("v", "<u8"),
    ("ksb", "<i8"), ("ksh", "<i8"), ("kst", "<i8"),
    ("vsb", "<i8"), ("vsh", "<i8"), ("vst", "<i8"),
    ("start", "<i8"), ("T", "<i4"), ("flags", "<i4"), ("batch", "<i4"), ("res", "<i4"),
])
assert DESC_DTYPE.itemsize == 88

_WAVES_PER_GROUP = 4
_TILE_ROWS = 64


@dataclass
class ChunkRef:
    """One KV chunk: k, v are (B, H_kv, T_c, D) -- or (H_kv, T_c, D) when
    ``batch`` >= 0 names the single batch row the chunk belongs to."""

    k: torch.Tensor
    v: torch.Tensor
    chunk_start: int
    causal: bool = True
    batch: int = -1

    @property
    def T(self) -> int:
        return int(self.k.shape[-2])


@dataclass
class SlotRef:
    """A chunk-table slot whose chunk is chosen on the device (by the
    in-kernel selection or by ``halo_chunk_score_topk`` writing the table):
    it holds no tensor until then; ``T`` is the largest chunk it may receive,
    so the planner covers that many rows."""

    T: int
    chunk_start: int = 0
    causal: bool = False
    batch: int = -1


@dataclass
class DecodePlan:
    B: int
    H: int
    H_kv: int
    D: int
    rep_t: int
    dtype: torch.dtype
    descs: torch.Tensor          # uint8 [n_desc*88] on device
    work: torch.Tensor           # int32 [n_work*4] on device
    offsets: torch.Tensor        # int32 [n_groups+1] on device
    n_desc: int
    n_work: int
    n_groups: int
    rows: int                    # attended K/V rows summed over (b, h_kv)
    keep: list = field(default_factory=list)  # tensors the descriptors point at
    uniform_groups: bool = False  # group g owns slots [g*per, (g+1)*per): the merge needs no offsets
    work_host: Optional[np.ndarray] = None
    kivi: bool = False           # the table holds KIVI block runs (plain chunks may join them)
    kivi_rows: int = 0           # rows of ``rows`` that are KIVI-quantised
    ws: Optional[torch.Tensor] = None  # this plan's partial buffer (halo_decode_workspace_size bytes)

    @property
    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes one launch streams (every row read once)."""
        from .kivi import GROUP, block_bytes
        esz = torch.tensor([], dtype=self.dtype).element_size()
        return (self.kivi_rows // GROUP * block_bytes(self.D)
                + (self.rows - self.kivi_rows) * 2 * self.D * esz)


def choose_rep_t(rep: int) -> int:
    for r in (1, 2, 4, 8):
        if rep <= r:
            return r
    return 8


def _check_kv(t: torch.Tensor, name: str) -> None:
    if t.stride(-1) != 1:
        raise AssertionError(f"{name}: head dim must be contiguous (stride {t.stride()})")
    esz = t.element_size()
    if t.data_ptr() % 16 or (t.stride(-2) * esz) % 16:
        raise AssertionError(f"{name}: rows must be 16-byte aligned")


def _kernel_address(t: torch.Tensor, name: str) -> int:
    """Address a kernel reads ``t`` at: device memory as is; a chunk kept in
    pinned host memory (the cold tier) through its device-visible mapping,
    so the kernel streams it over the host link in place."""
    if t.device.type != "cpu":
        return t.data_ptr()
    if not t.is_pinned():
        raise AssertionError(f"{name}: a host-resident chunk must be in pinned memory (pin_memory())")
    base = t.untyped_storage().data_ptr()
    return nat.host_device_pointer(base) + (t.data_ptr() - base)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    esz = t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16 or (t.stride(-2) * esz) % 16:
        return t.contiguous()
    return t


def _to_device(a: np.ndarray, device) -> torch.Tensor:
    """Host array -> device tensor through pinned memory, without a host sync
    (torch's pinned allocator keeps the staging block alive until the copy
    has run)."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t


def choose_split(total_rows: int, n_cu: int, *, kivi: bool = False) -> int:
    """Rows per work item: aim for about 4 workgroups per CU, in whole
    4-wave x 64-row tiles, between 256 and 4096 rows.  KIVI items: about 2
    per CU (2 resident workgroups per CU), in whole 4-wave x 64-token block
    pairs."""
    if kivi:
        unit = _WAVES_PER_GROUP * 64
        target = max(1, total_rows // max(1, 2 * n_cu))
        split = unit * max(1, math.ceil(target / unit))
        return int(min(max(split, unit), 16 * unit))
    unit = _WAVES_PER_GROUP * _TILE_ROWS
    target = max(1, total_rows // max(1, 4 * n_cu))
    split = unit * max(1, math.ceil(target / unit))
    return int(min(max(split, unit), 16 * unit))


def _num_cus(device) -> int:
    try:
        return int(torch.cuda.get_device_properties(device).multi_processor_count)
    except Exception:  # pragma: no cover
        return 256


def pack_descs(chunks: Sequence[ChunkRef], *, B: int, H_kv: int, D: int, dtype: torch.dtype):
    """halo_chunk_desc records for ``chunks`` (validated); returns
    (numpy structured array, list of tensors to keep alive)."""
    descs = np.zeros(len(chunks), dtype=DESC_DTYPE)
    keep = []
    for i, c in enumerate(chunks):
        if hasattr(c, "blocks"):
            keep.append(_pack_kivi(descs[i], c, i, B=B, H_kv=H_kv, D=D, dtype=dtype))
            continue
        if isinstance(c, SlotRef):
            d = descs[i]
            d["start"], d["T"] = int(c.chunk_start), int(c.T)
            d["flags"] = nat.CHUNK_CAUSAL if c.causal else 0
            d["batch"] = int(c.batch)
            continue
        k, v = c.k, c.v
        if k.dtype != dtype or v.dtype != dtype:
            raise AssertionError(f"chunk {i}: dtype {k.dtype}/{v.dtype} != {dtype}")
        if k.shape[-1] != D or v.shape[-1] != D:
            raise AssertionError(f"chunk {i}: head dim {k.shape[-1]}/{v.shape[-1]} != {D}")
        if c.batch < 0:
            if k.dim() != 4 or k.shape[0] != B or k.shape[1] != H_kv:
                raise AssertionError(f"k shape {tuple(k.shape)} != ({B}, {H_kv}, T_c, {D})")
            if tuple(v.shape) != tuple(k.shape):
                raise AssertionError(f"v shape {tuple(v.shape)} != k shape {tuple(k.shape)}")
        else:
            if k.dim() != 3 or k.shape[0] != H_kv or tuple(v.shape) != tuple(k.shape):
                raise AssertionError(f"ragged chunk {i}: expected (H_kv, T_c, D), got {tuple(k.shape)}")
            if not 0 <= c.batch < B:
                raise AssertionError(f"ragged chunk {i}: batch {c.batch} outside [0, {B})")
        _check_kv(k, f"chunk {i} k")
        _check_kv(v, f"chunk {i} v")
        keep += [k, v]
        d = descs[i]
        d["k"], d["v"] = _kernel_address(k, f"chunk {i} k"), _kernel_address(v, f"chunk {i} v")
        if c.batch < 0:
            d["ksb"], d["ksh"], d["kst"] = k.stride(0), k.stride(1), k.stride(2)
            d["vsb"], d["vsh"], d["vst"] = v.stride(0), v.stride(1), v.stride(2)
        else:
            d["ksb"], d["ksh"], d["kst"] = 0, k.stride(0), k.stride(1)
            d["vsb"], d["vsh"], d["vst"] = 0, v.stride(0), v.stride(1)
        d["start"] = int(c.chunk_start)
        d["T"] = c.T
        d["flags"] = nat.CHUNK_CAUSAL if c.causal else 0
        d["batch"] = int(c.batch)
    return descs, keep


def _pack_kivi(d, c, i: int, *, B: int, H_kv: int, D: int, dtype: torch.dtype) -> torch.Tensor:
    """Descriptor of a run of KIVI blocks (kivi.KiviChunkRef): ``k`` is the
    first block, strides are in bytes, the v fields are unused."""
    from .kivi import GROUP, block_bytes
    blk = c.blocks
    bb = block_bytes(D, c.bits)
    if c.bits != 2:
        raise AssertionError(f"chunk {i}: decode attention reads 2-bit KIVI blocks, got bits={c.bits}")
    if dtype not in (torch.float16, torch.bfloat16):
        raise AssertionError(f"chunk {i}: KIVI chunks need an fp16 or bf16 query, got {dtype}")
    if blk.dtype != torch.uint8 or blk.shape[-1] != bb or blk.stride(-1) != 1 or blk.stride(-2) != bb:
        raise AssertionError(f"chunk {i}: blocks must be uint8 (..., n, {bb}) with contiguous blocks")
    if c.batch < 0:
        if blk.dim() != 4 or blk.shape[0] != B or blk.shape[1] != H_kv:
            raise AssertionError(f"chunk {i}: blocks shape {tuple(blk.shape)} != ({B}, {H_kv}, n, {bb})")
        ssb, ssh = blk.stride(0), blk.stride(1)
    else:
        if blk.dim() != 3 or blk.shape[0] != H_kv or not 0 <= c.batch < B:
            raise AssertionError(f"ragged chunk {i}: expected blocks (H_kv, n, {bb}) of a row in [0, {B})")
        ssb, ssh = 0, blk.stride(0)
    if blk.data_ptr() % 16 or ssb % 16 or ssh % 16:
        raise AssertionError(f"chunk {i}: KIVI blocks must be 16-byte aligned")
    d["k"], d["v"] = blk.data_ptr(), 0
    d["ksb"], d["ksh"], d["kst"] = ssb, ssh, bb
    d["vsb"], d["vsh"], d["vst"] = 0, 0, 0
    d["start"] = int(c.chunk_start)
    d["T"] = int(blk.shape[-2]) * GROUP
    d["flags"] = (nat.CHUNK_CAUSAL if c.causal else 0) | nat.CHUNK_KIVI2
    d["batch"] = int(c.batch)
    return blk


def descs_to_device(descs: np.ndarray, device) -> torch.Tensor:
    return _to_device(descs.view(np.uint8).copy(), device)


def build_plan(*, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype,
               chunks: Sequence[ChunkRef], device, rep_t: Optional[int] = None,
               split: Optional[int] = None, q_pos_host: Optional[Sequence[int]] = None,
               first: Optional[Sequence[int]] = None, split_first: Optional[int] = None,
               first_half_split: bool = False) -> DecodePlan:
    """Lay out descriptors and work items for a chunk list.

    ``q_pos_host`` (per batch row) lets the planner drop causal chunks that
    lie entirely after the query, as the reference's chunk walk does with
    ``c0 > q_pos`` (halo/kv_cache_chunked.py:658,714); the kernel applies the
    row-level causal cut itself either way.

    Work records are ``WORK_INTS`` int32: (chunk, group, t0, t1, partial
    slot, 0, 0, 0).  Partial slots are numbered group by group, which is the
    order the merge reads them; the records themselves are in dispatch
    order, where the items of the chunks listed in ``first`` come before
    all others (the tiered layer puts its selection slots there, so their
    longer dependency chain starts first); ``split_first`` (rows per item of
    those chunks, default ``split``) cuts them finer, and
    ``first_half_split`` sets it to half the split (at least 128 rows).
    """
    if H % H_kv:
        raise AssertionError(f"head count mismatch: q has {H}, kv has {H_kv}")
    rep = H // H_kv
    rep_t = rep_t or choose_rep_t(rep)
    n_sub = -(-rep // rep_t)
    n_groups = B * H_kv * n_sub

    descs, keep = pack_descs(chunks, B=B, H_kv=H_kv, D=D, dtype=dtype)
    kinds = {hasattr(c, "blocks") for c in chunks if not isinstance(c, SlotRef)}
    kivi = True in kinds  # KIVI block runs, possibly with plain chunks (one KIVI launch)
    if kivi and split is not None and split % 32:
        raise AssertionError(f"split={split} must be a multiple of the 32-token KIVI block")

    def live(c: ChunkRef, b: int) -> bool:
        if c.batch >= 0 and c.batch != b:
            return False
        if c.T == 0:
            return False
        if c.causal and q_pos_host is not None and c.chunk_start > int(q_pos_host[b]):
            return False
        return True

    total_rows = 0
    for b in range(B):
        for c in chunks:
            if live(c, b):
                rows = c.T
                if c.causal and q_pos_host is not None:
                    rows = min(rows, int(q_pos_host[b]) - c.chunk_start + 1)
                total_rows += rows * H_kv * n_sub
    if split is None:
        split = choose_split(total_rows, _num_cus(device), kivi=kivi)
    if first_half_split and split_first is None:
        split_first = max(128, split // 2)

    work = []
    offsets = [0]
    rows_attended = 0
    kivi_rows = 0
    for b in range(B):
        live_idx = [i for i, c in enumerate(chunks) if live(c, b)]
        for h in range(H_kv):
            for s in range(n_sub):
                g = (b * H_kv + h) * n_sub + s
                n0 = len(work)
                for i in live_idx:
                    T = chunks[i].T
                    hi = T
                    if chunks[i].causal and q_pos_host is not None:
                        hi = min(T, int(q_pos_host[b]) - chunks[i].chunk_start + 1)
                    sp = split_first if (split_first and first is not None and i in first) else split
                    for t0 in range(0, hi, sp):
                        work.append((i, g, t0, min(t0 + sp, hi), len(work), 0, 0, 0))
                    if s == 0:
                        rows_attended += hi
                        if hasattr(chunks[i], "blocks"):
                            kivi_rows += hi
                if len(work) == n0:
                    work.append((0, g, 0, 0, len(work), 0, 0, 0))
                offsets.append(len(work))
    if first:
        early = set(int(i) for i in first)
        work = [w for w in work if w[0] in early] + [w for w in work if w[0] not in early]
    work_np = np.asarray(work, dtype=np.int32).reshape(-1, WORK_INTS)
    dev_descs = _to_device(descs.view(np.uint8).copy(), device)
    per = len(work) // n_groups
    uniform = len(work) % n_groups == 0 and offsets == [g * per for g in range(n_groups + 1)]
    return DecodePlan(
        B=B, H=H, H_kv=H_kv, D=D, rep_t=rep_t, dtype=dtype,
        descs=dev_descs, work=_to_device(work_np.reshape(-1), device),
        offsets=_to_device(np.asarray(offsets, dtype=np.int32), device),
        n_desc=len(chunks), n_work=len(work), n_groups=n_groups,
        rows=rows_attended, keep=keep, work_host=work_np, kivi=kivi, kivi_rows=kivi_rows,
        uniform_groups=uniform,
    )


# ---------------------------------------------------------------------------
# Workspace: every plan owns its partial buffer, sized when the plan is built
# and alive as long as the plan.  A HIP graph that captured a launch of the
# plan therefore keeps replaying into memory that nobody else can be handed
# (a buffer shared per stream and regrown for a larger plan would be returned
# to the caching allocator while a captured graph still writes through it).
# Launches of one plan are ordered when they share a stream; launching the
# same plan on two streams at once needs a ``workspace=`` of its own for one.
# ---------------------------------------------------------------------------
# Plans of repeated calls: a plan's tables hold only addresses, strides,
# chunk starts, flags and the work split, so a call whose chunk list has the
# same addresses and layout (and the same planner options) can launch the
# same plan again -- also when a tensor was freed and its memory reused with
# that layout.  The launch stream is part of the key, so calls on different
# streams never share a plan's workspace.  Least recently used plans are
# dropped beyond PLAN_CACHE_SIZE.
PLAN_CACHE_SIZE = 256
_plan_cache: "collections.OrderedDict[tuple, DecodePlan]" = collections.OrderedDict()


def _chunk_key(c) -> tuple:
    if isinstance(c, SlotRef):
        return ("slot", int(c.chunk_start), int(c.T), bool(c.causal), int(c.batch))
    if hasattr(c, "blocks"):
        b = c.blocks
        return ("kivi", b.data_ptr(), tuple(b.shape), tuple(b.stride()), int(c.chunk_start), bool(c.causal),
                int(c.bits), int(c.batch))
    k, v = c.k, c.v
    return (k.data_ptr(), tuple(k.shape), tuple(k.stride()), k.dtype, k.device,
            v.data_ptr(), tuple(v.shape), tuple(v.stride()), v.dtype, v.device,
            int(c.chunk_start), bool(c.causal), int(c.batch))


def cached_plan(*, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype, chunks: Sequence,
                device, **opts) -> DecodePlan:
    """``build_plan`` through the plan cache (same arguments).  The returned
    plan does not keep the chunk tensors alive: the caller owns them, as for
    a plan used once."""
    dev = torch.device(device)
    stream = torch.cuda.current_stream(dev).cuda_stream if dev.type == "cuda" else 0
    key = (B, H, H_kv, D, dtype, str(dev), stream, tuple(_chunk_key(c) for c in chunks),
           tuple(sorted((k, tuple(v) if isinstance(v, (list, tuple)) else v) for k, v in opts.items())))
    plan = _plan_cache.get(key)
    if plan is not None:
        _plan_cache.move_to_end(key)
        return plan
    plan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype, chunks=chunks, device=device, **opts)
    plan.keep = []
    _plan_cache[key] = plan
    while len(_plan_cache) > PLAN_CACHE_SIZE:
        _plan_cache.popitem(last=False)
    return plan


def clear_plan_cache() -> None:
    """Drop the cache of repeated plans.  Plans launched under graph capture
    stay alive (``captured_plans``)."""
    _plan_cache.clear()


# Plans (and launch arguments that hold device tensors) used by a launch
# recorded into a HIP graph.  A captured launch holds raw addresses of the
# plan's tables, workspace and default query positions, so these objects must
# outlive every graph that recorded them.  Neither the plan cache's LRU nor
# clear_plan_cache() drops them; a caller that has destroyed all of its graphs
# may call release_captured_plans().
_captured: dict = {}


def keep_for_capture(obj, stream=None) -> None:
    """Keep ``obj`` alive for the process (or until
    ``release_captured_plans``) when ``stream`` (default: the current stream)
    is capturing a graph; otherwise do nothing."""
    if _capturing(stream):
        _captured.setdefault(id(obj), obj)


def _capturing(stream=None) -> bool:
    if torch.cuda.is_current_stream_capturing():
        return True
    if stream is None or stream == torch.cuda.current_stream(stream.device):
        return False
    with torch.cuda.stream(stream):
        return bool(torch.cuda.is_current_stream_capturing())


def captured_plans() -> list:
    """The objects kept alive for captured graphs (plans and launch entries)."""
    return list(_captured.values())


def release_captured_plans() -> None:
    """Forget the objects kept for captured graphs.  Call only once every
    graph that recorded a launch of them has been destroyed: a replay after
    this may read freed tables and workspaces."""
    _captured.clear()


def workspace_bytes(n_work: int, rep_t: int, D: int) -> int:
    """Bytes of partials a launch with ``n_work`` items writes
    (``halo_decode_workspace_size``: n_work x rep_t x (D + 2) fp32)."""
    return int(n_work) * int(rep_t) * (int(D) + 2) * 4


def plan_workspace(plan: "DecodePlan", device) -> torch.Tensor:
    """The plan's own workspace, allocated on first use."""
    if plan.ws is None:
        nbytes = workspace_bytes(plan.n_work, plan.rep_t, plan.D)
        plan.ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    return plan.ws


def launch(plan: DecodePlan, q: torch.Tensor, *, scale: float,
           q_pos: Optional[torch.Tensor] = None,
           m: Optional[torch.Tensor] = None, l: Optional[torch.Tensor] = None,
           o: Optional[torch.Tensor] = None, acc_mode: int = 0,
           out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
           stream: Optional[torch.cuda.Stream] = None, select=None,
           workspace: Optional[torch.Tensor] = None, noalloc: bool = False) -> None:
    """Enqueue one ``halo_decode_attn`` on ``stream`` (default: current).

    ``select`` (a ``_native.SelectCfg``) enqueues ``halo_decode_attn_tiered``
    instead: the table's selection slots choose their chunks in-kernel.
    ``workspace`` (a uint8 device tensor) replaces the plan's own partial
    buffer, for a second concurrent launch of the same plan.  ``noalloc``
    enqueues ``halo_decode_attn_noalloc`` instead: the partials go to the
    library's static device scratch (no workspace at all; launches that
    overlap on one GPU must not use it)."""
    L = nat.lib()
    if q.dim() != 3 or tuple(q.shape) != (plan.B, plan.H, plan.D):
        raise AssertionError(f"expected q (B, H, D) = {(plan.B, plan.H, plan.D)}, got {tuple(q.shape)}")
    if q.stride(-1) != 1:
        q = q.contiguous()
    if q.dtype != plan.dtype:
        q = q.to(plan.dtype)
    if q_pos is not None:
        if q_pos.dtype != torch.int64 or q_pos.device != q.device:
            q_pos = q_pos.to(device=q.device, dtype=torch.int64)
        q_pos = q_pos.contiguous()
        if q_pos.numel() != plan.B:
            raise AssertionError(f"q_pos must have B={plan.B} entries, got {q_pos.numel()}")
    BH, BHD = (plan.B, plan.H), (plan.B, plan.H, plan.D)
    for t, name, shape in ((m, "m", BH), (l, "l", BH), (o, "o", BHD)):
        if t is None:
            continue
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape:
            raise AssertionError(f"accumulator {name} must be contiguous float32 {shape}, got "
                                 f"{t.dtype} {tuple(t.shape)}")
    if (m is None) != (l is None) or (m is None) != (o is None):
        raise AssertionError("m, l, o must be passed together")
    if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                            or tuple(lse.shape) != BH):
        raise AssertionError(f"lse must be contiguous float32 {BH}")
    if out is not None and (not out.is_contiguous() or tuple(out.shape) != BHD):
        raise AssertionError(f"out must be contiguous {BHD}")
    for t in (m, l, o, out, lse, q_pos):
        if t is not None and t.device != q.device:
            raise AssertionError("all tensors must be on the query's device")
    sp = nat.stream_ptr(stream)
    keep_for_capture(plan, stream)
    if noalloc:
        if plan.kivi:
            raise AssertionError("the allocation-free entry point covers plain and tiered tables, not KIVI")
        head = (q.data_ptr(), q.stride(0), q.stride(1), nat.dtype_code(plan.dtype),
                plan.B, plan.H, plan.H_kv, plan.D, plan.rep_t, plan.descs.data_ptr(), plan.n_desc,
                plan.work.data_ptr(), plan.n_work, None if plan.uniform_groups else plan.offsets.data_ptr(),
                plan.n_groups, nat.ptr(q_pos), float(scale), nat.ptr(m), nat.ptr(l), nat.ptr(o), plan.H, acc_mode,
                nat.ptr(out), nat.dtype_code(out.dtype) if out is not None else 0, nat.ptr(lse))
        nat.check(L.halo_decode_attn_noalloc(*head, ctypes.byref(select) if select is not None else None, sp),
                  "halo_decode_attn_noalloc")
        return
    nbytes = int(L.halo_decode_workspace_size(plan.n_work, plan.rep_t, plan.D))
    ws = plan_workspace(plan, q.device) if workspace is None else workspace
    if ws.dtype != torch.uint8 or ws.device != q.device or ws.numel() < nbytes:
        raise AssertionError(f"workspace must be a uint8 tensor of >= {nbytes} bytes on {q.device}")
    args = (
        q.data_ptr(), q.stride(0), q.stride(1), nat.dtype_code(plan.dtype),
        plan.B, plan.H, plan.H_kv, plan.D, plan.rep_t,
        plan.descs.data_ptr(), plan.n_desc,
        plan.work.data_ptr(), plan.n_work,
        None if plan.uniform_groups else plan.offsets.data_ptr(), plan.n_groups,
        nat.ptr(q_pos), float(scale),
        nat.ptr(m), nat.ptr(l), nat.ptr(o), plan.H, acc_mode,
        nat.ptr(out), nat.dtype_code(out.dtype) if out is not None else 0, nat.ptr(lse),
        ws.data_ptr(), ws.numel(),
    )
    if plan.kivi:
        if select is not None:
            raise AssertionError("in-kernel selection is not available for KIVI chunk tables")
        nat.check(L.halo_decode_attn_kivi(*args, sp), "halo_decode_attn_kivi")
    elif select is None:
        nat.check(L.halo_decode_attn(*args, sp), "halo_decode_attn")
    else:
        nat.check(L.halo_decode_attn_tiered(*args, ctypes.byref(select), sp), "halo_decode_attn_tiered")
