"""The C-ABI library: every function declared in include/halo_hip.h is bound
by the ctypes layer and exported by the built library (loading needs no GPU;
nothing is called)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "halo_hip.h")


def _declared() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(halo_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_entry_points():
    names = _declared()
    for must in ("halo_decode_attn", "halo_decode_attn_tiered", "halo_decode_attn_kivi", "halo_finalize",
                 "halo_lse_merge", "halo_chunk_means", "halo_chunk_score_topk", "halo_prefill_attn",
                 "halo_kivi_quantize", "halo_kivi_dequantize", "halo_kivi_block_bytes",
                 "halo_decode_workspace_size", "halo_last_error", "halo_build_info"):
        assert must in names


def test_ctypes_layer_binds_every_declaration():
    from halo_amd import _native as nat
    assert set(nat._SIGNATURES) == _declared()


def test_library_exports_every_declared_symbol():
    from halo_amd import _native as nat
    if not os.path.exists(nat.library_path()):
        pytest.skip("library not built (run __graft_entry__.build())")
    handle = ctypes.CDLL(nat.library_path())
    missing = [n for n in sorted(_declared()) if not hasattr(handle, n)]
    assert not missing, f"not exported: {missing}"


def test_select_cfg_layout_matches_header():
    """halo_select_cfg: 9 pointers + 4 int64 + 6 int32 = 128 bytes, field order as declared."""
    from halo_amd import _native as nat
    assert ctypes.sizeof(nat.SelectCfg) == 128
    assert nat.SelectCfg.alloc_slot.offset == 120
    assert nat.SelectCfg.n_cold.offset == 56 and nat.SelectCfg.idx_out.offset == 72
    assert nat.SelectCfg.lead_items.offset == 88 and nat.SelectCfg.n_slots.offset == 92
    assert nat.SelectCfg.slot_catalog.offset == 96 and nat.SelectCfg.res_out.offset == 112


def test_staging_structs_match_header():
    """halo_staging_desc: 12 int32 then 9 pointers (120 bytes);
    halo_staging_stats: 14 int64."""
    from halo_amd import _native as nat
    assert ctypes.sizeof(nat.StagingDesc) == 120
    assert nat.StagingDesc.residency.offset == 48 and nat.StagingDesc.urgent_stream.offset == 104
    assert nat.StagingDesc.copy_stream2.offset == 112
    assert ctypes.sizeof(nat.StagingStats) == 112 and nat.StagingStats.evictions_while_busy.offset == 80


def test_descriptor_record_size():
    from halo_amd.decode import DESC_DTYPE, WORK_INTS
    assert DESC_DTYPE.itemsize == 88 and WORK_INTS == 8


def test_entry_points_fail_loudly_without_gpu():
    """The product path has no CPU fallback."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from halo_amd import _native as nat
    with pytest.raises(RuntimeError):
        nat.lib()
