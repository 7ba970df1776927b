"""The drop-in's per-layout fast-path key (host only).  The C++ key (the
built extension) must separate exactly the chunk lists the Python key
separates: a different tensor, view, stride, dtype, chunk start or causal
flag gives a different key; the same list of the same views gives the same
key."""
from __future__ import annotations

import itertools

import pytest
import torch


def _variants():
    base = torch.zeros(1, 8, 3072, 128, dtype=torch.bfloat16)
    other = torch.zeros(1, 8, 3072, 128, dtype=torch.bfloat16)
    k0, v0 = base[..., :1024, :], other[..., :1024, :]
    return {
        "same": [(k0, v0, 0, True), (base[..., 1024:2048, :], other[..., 1024:2048, :], 1024, True)],
        "same_views_again": [(base[..., :1024, :], other[..., :1024, :], 0, True),
                             (base[..., 1024:2048, :], other[..., 1024:2048, :], 1024, True)],
        "other_rows": [(k0, v0, 0, True), (base[..., 2048:3072, :], other[..., 1024:2048, :], 1024, True)],
        "transposed_v": [(k0, v0.transpose(2, 3), 0, True),
                         (base[..., 1024:2048, :], other[..., 1024:2048, :], 1024, True)],
        "dtype": [(k0.view(torch.float16), v0, 0, True),
                  (base[..., 1024:2048, :], other[..., 1024:2048, :], 1024, True)],
        "start": [(k0, v0, 0, True), (base[..., 1024:2048, :], other[..., 1024:2048, :], 1025, True)],
        "causal": [(k0, v0, 0, False), (base[..., 1024:2048, :], other[..., 1024:2048, :], 1024, True)],
        "shorter": [(k0, v0, 0, True)],
    }


def test_cpp_key_separates_what_the_python_key_separates():
    from halo_amd import triton_chunked as tc
    if tc._layout_key is None:
        pytest.skip("layout-key extension not built (run __graft_entry__.build())")
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    v = _variants()
    cpp = {n: tc._fast_key(q, c, 0, True) for n, c in v.items()}
    py = {n: tc._fast_key_py(q, c, 0, True) for n, c in v.items()}
    assert isinstance(cpp["same"][-1], bytes)
    for a, b in itertools.combinations(v, 2):
        assert (cpp[a] == cpp[b]) == (py[a] == py[b]), (a, b)
    assert cpp["same"] == cpp["same_views_again"]
    assert tc._fast_key(q, v["same"], 0, False) != cpp["same"]          # q_pos defaulted or not
    assert tc._fast_key(q, v["same"], 1, True) != cpp["same"]           # stream


def test_malformed_chunk_lists_fall_back_to_the_python_key():
    from halo_amd import triton_chunked as tc
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        tc._fast_key(q, [(k, k, 0)], 0, True)    # the Python key's own error for a 3-tuple


def test_corrupt_extension_falls_back_to_the_python_key(tmp_path):
    """A layout-key extension that cannot be loaded (another torch's build,
    a truncated file) leaves the drop-in importable with the Python key."""
    from halo_amd import triton_chunked as tc
    bad = tmp_path / "_halo_fastkey.so"
    bad.write_bytes(b"\x7fELF not really a shared object")
    assert tc._load_layout_key(str(bad)) is None
    assert tc._load_layout_key(str(tmp_path / "missing.so")) is None
