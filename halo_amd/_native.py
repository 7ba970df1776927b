"""ctypes binding of libhalo_hip.so, the C-ABI declared in include/halo_hip.h.

The library is built in-tree (``halo_amd/_lib/libhalo_hip.so``) by
``__graft_entry__.build()`` or ``make -C halo_amd/csrc``.  It links the HIP
runtime by soname (``libamdhip64.so.7``); torch is imported first so that the
library binds to the runtime torch already loaded and both share one device
context.

There is no CPU fallback: every product entry point calls :func:`lib`, which
raises ``RuntimeError`` when the library is missing or no GPU is visible.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch  # noqa: F401  -- must load torch's HIP runtime before the library

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libhalo_hip.so")

HALO_OK = 0
HALO_E_INVALID = -1
HALO_E_UNSUPPORTED = -2
HALO_E_HIP = -3
HALO_E_WORKSPACE = -4

F32, BF16, F16 = 0, 1, 2
CHUNK_CAUSAL = 1
CHUNK_KIVI2 = 2

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_size_t = ctypes.c_size_t



class SelectCfg(ctypes.Structure):
    """halo_select_cfg (include/halo_hip.h)."""
    _fields_ = [
        ("kmean", _c_void_p),
        ("km_stride_b", _i64), ("km_stride_h", _i64), ("km_stride_p", _i64),
        ("catalog", _c_void_p),
        ("catalog_stride", _i64),
        ("n_cold_per_sel", _c_void_p),
        ("n_cold", _i32), ("top_k", _i32), ("slot0", _i32), ("per_row", _i32),
        ("idx_out", _c_void_p),
        ("score_out", _c_void_p),
        ("lead_items", _i32), ("n_slots", _i32),
        ("slot_catalog", _c_void_p), ("residency", _c_void_p), ("res_out", _c_void_p),
        ("alloc_slot", _c_void_p),
    ]


class Fill(ctypes.Structure):
    """halo_fill (include/halo_hip.h)."""
    _fields_ = [("dst_k", _c_void_p), ("src_k", _c_void_p), ("dst_v", _c_void_p), ("src_v", _c_void_p),
                ("bytes", _i64)]


class StagingDesc(ctypes.Structure):
    """halo_staging_desc (include/halo_hip.h)."""
    _fields_ = [
        ("n_layers", _i32), ("n_cold", _i32), ("n_slots", _i32), ("top_k", _i32), ("keep", _i32),
        ("max_inflight", _i32), ("spare", _i32), ("ring", _i32),
        ("write_allocate", _i32), ("fill_mode", _i32), ("track_busy", _i32), ("sels_per_layer", _i32),
        ("residency", _c_void_p), ("feedback", _c_void_p), ("slot_addr", _c_void_p), ("chunk_addr", _c_void_p),
        ("chunk_nbytes", _c_void_p), ("n_cold_per_unit", _c_void_p), ("copy_stream", _c_void_p),
        ("urgent_stream", _c_void_p), ("copy_stream2", _c_void_p),
    ]


class StagingStats(ctypes.Structure):
    """halo_staging_stats (include/halo_hip.h)."""
    _fields_ = [(name, _i64) for name in (
        "hits", "misses", "misses_predicted", "fills", "fill_bytes", "miss_bytes", "wa_commits", "wa_dups",
        "fills_while_busy", "commits_while_busy", "evictions_while_busy", "ns_plan", "ns_issue", "ns_wait")]


_DECODE_ARGS = [
    _c_void_p, _i64, _i64, _i32,             # q, q_stride_b, q_stride_h, dtype
    _i32, _i32, _i32, _i32, _i32,            # B, H, H_kv, D, rep_t
    _c_void_p, _i32,                         # descs, n_desc
    _c_void_p, _i32,                         # work, n_work
    _c_void_p, _i32,                         # group_offsets, n_groups
    _c_void_p, _f32,                         # q_pos, scale
    _c_void_p, _c_void_p, _c_void_p, _i64, _i32,  # m, l, o, acc_stride_b, acc_mode
    _c_void_p, _i32, _c_void_p,              # out, out_dtype, lse
    _c_void_p, _size_t,                      # workspace, bytes
]

# name -> (restype, argtypes); mirrors include/halo_hip.h one to one.
_SIGNATURES = {
    "halo_decode_workspace_size": (_size_t, [_i32, _i32, _i32]),
    "halo_decode_attn": (_i32, _DECODE_ARGS + [_c_void_p]),                      # + stream
    "halo_decode_attn_tiered": (_i32, _DECODE_ARGS + [ctypes.POINTER(SelectCfg), _c_void_p]),  # + sel, stream
    "halo_decode_attn_kivi": (_i32, _DECODE_ARGS + [_c_void_p]),                 # + stream
    "halo_decode_static_scratch_bytes": (_size_t, []),
    "halo_decode_attn_noalloc": (_i32, _DECODE_ARGS[:-2] + [ctypes.POINTER(SelectCfg), _c_void_p]),  # sel, stream
    "halo_finalize": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32,
                             _c_void_p, _i32, _c_void_p, _c_void_p]),
    "halo_lse_merge": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
                              _c_void_p, _c_void_p, _c_void_p]),
    "halo_prefill_attn": (_i32, [_c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _c_void_p,
                                 _c_void_p, _i32, _f32, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "halo_halo_score": (_i32, [_c_void_p, _i32, _i32, _f32, _f32, _f32, _i32, _i32, _c_void_p, _c_void_p]),
    "halo_topk_sorted": (_i32, [_c_void_p, _i32, _i32, _c_void_p, _c_void_p]),
    "halo_kivi_block_bytes": (_size_t, [_i32, _i32]),
    "halo_kivi_quantize": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64,
                                  _i32, _i32, _i32, _i32, _i32, _i32, _c_void_p, _i64, _i64, _c_void_p]),
    "halo_kivi_dequantize": (_i32, [_c_void_p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
                                    _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "halo_chunk_means": (_i32, [_c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _i32, _i32,
                                _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "halo_chunk_score_topk": (_i32, [
        _c_void_p, _i64, _i64, _i32,             # q, strides, dtype
        _i32, _i32, _i32, _i32,                  # B, H, H_kv, D
        _c_void_p, _i64, _i64, _i64,             # kmean + strides
        _c_void_p, _i64, _c_void_p, _i32, _i32, _i32,  # eligible, stride, n_elig_per_sel, n_elig, k, per_row
        _c_void_p, _c_void_p,                    # idx_out, score_out
        _c_void_p, _i64, _c_void_p, _i64, _i32,  # catalog, stride, table, stride, slot0
        _i32, _f32, _f32, _f32, _i32, _i32, _i32,  # normalize, alpha, beta, gamma, refresh, sink_pages, P_total
        _c_void_p,
    ]),
    "halo_chunk_score_topk_staged": (_i32, [
        _c_void_p, _i64, _i64, _i32,             # q, strides, dtype
        _i32, _i32, _i32, _i32,                  # B, H, H_kv, D
        _c_void_p, _i64, _i64, _i64,             # kmean + strides
        _c_void_p, _i64, _c_void_p, _i32, _i32, _i32,  # eligible, stride, n_elig_per_sel, n_elig, k, per_row
        _c_void_p, _c_void_p,                    # idx_out, score_out
        _c_void_p, _i64, _c_void_p, _i64, _i32,  # catalog, stride, table, stride, slot0
        _c_void_p, _c_void_p, _i32, _c_void_p,   # residency, slot_catalog, n_slots, res_out
        _c_void_p,
    ]),
    "halo_page_minmax": (_i32, [_c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _i32, _i32,
                                _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "halo_quest_score_topk": (_i32, [
        _c_void_p, _i64, _i64, _i64, _i32,       # q, strides (b, h, t), dtype
        _i32, _i32, _i32, _i32, _i32,            # B, H, H_kv, T_q, D
        _c_void_p, _c_void_p, _i64, _i64, _i64,  # kmin, kmax, strides
        _i32, _i32, _i32, _c_void_p,             # P, k, per_row, workspace
        _c_void_p, _c_void_p, _c_void_p,         # dots_out, score_out, idx_out
        _c_void_p,
    ]),
    "halo_copy_blocks": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i32, _i64,
                                _c_void_p, _i32, _c_void_p]),
    "halo_set_tier": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _c_void_p]),
    "halo_stage_fills": (_i32, [ctypes.POINTER(Fill), _i32, _c_void_p]),
    "halo_stage_fills_read": (_i32, [ctypes.POINTER(Fill), _i32, _c_void_p]),
    "halo_store_i32": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i32, _c_void_p]),
    "halo_staging_create": (_i32, [ctypes.POINTER(StagingDesc), ctypes.POINTER(_c_void_p)]),
    "halo_staging_destroy": (_i32, [_c_void_p]),
    "halo_staging_before": (_i32, [_c_void_p, _i32, _i32, _c_void_p]),
    "halo_staging_after": (_i32, [_c_void_p, _i32, _i32, _c_void_p]),
    "halo_staging_service": (_i32, [_c_void_p, _i32, _c_void_p]),
    "halo_staging_reset": (_i32, [_c_void_p]),
    "halo_staging_set": (_i32, [_c_void_p, _i32, _i32]),
    "halo_staging_get": (_i32, [_c_void_p, ctypes.POINTER(StagingStats), _c_void_p, _c_void_p, _c_void_p]),
    "halo_host_device_pointer": (_i32, [_c_void_p, ctypes.POINTER(_c_void_p)]),
    "halo_last_error": (ctypes.c_char_p, []),
    "halo_build_info": (ctypes.c_char_p, []),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def library_path() -> str:
    return _LIB_PATH


def _load() -> Optional[ctypes.CDLL]:
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        _load_error = (f"{_LIB_PATH} is not built; run __graft_entry__.build() "
                       f"or `make -C halo_amd/csrc`")
        return None
    try:
        handle = ctypes.CDLL(_LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the host
        _load_error = f"cannot load {_LIB_PATH}: {exc}"
        return None
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return _lib


def loadable() -> bool:
    """True when the shared library loads (no GPU needed)."""
    return _load() is not None


def available() -> bool:
    """True when the library loads and a GPU is visible."""
    return loadable() and torch.cuda.is_available()


_gpu_seen = False


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it or the GPU is missing."""
    global _gpu_seen
    handle = _load()
    if handle is None:
        raise RuntimeError(f"HALO HIP library unavailable: {_load_error}")
    if not _gpu_seen:  # a GPU, once visible, stays visible for the process
        if not torch.cuda.is_available():
            raise RuntimeError("HALO HIP kernels need a GPU (torch.cuda.is_available() is False)")
        _gpu_seen = True
    return handle


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the exception the reference raises."""
    if status == HALO_OK:
        return
    msg = (_load().halo_last_error() or b"").decode(errors="replace")
    if status == HALO_E_INVALID:
        raise AssertionError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({status}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def stream_ptr(stream: Optional[torch.cuda.Stream] = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


def host_device_pointer(ptr: int) -> int:
    """Device-visible address of pinned host memory at ``ptr``
    (``halo_host_device_pointer``)."""
    out = _c_void_p()
    check(lib().halo_host_device_pointer(ptr, ctypes.byref(out)), "halo_host_device_pointer")
    return int(out.value)
