"""The allocation-free decode entry point (``halo_decode_attn_noalloc``):
its partials live in the library's static device scratch, so a caller that
cannot allocate (graph capture, serving loops) passes only inputs and
outputs.  Checked through the C-ABI against the workspace entry points on
the same plans, bit for bit, on two calls in a row with the second one
smaller, with and without the fused selection; a plan whose partials exceed
the scratch is refused before anything is launched."""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _fn():
    from halo_amd import _native as nat
    L = nat.lib()
    return L.halo_decode_attn_noalloc, int(L.halo_decode_static_scratch_bytes())


def _args(plan, q, scale, out, lse):
    from halo_amd import _native as nat
    return (q.data_ptr(), q.stride(0), q.stride(1), nat.dtype_code(plan.dtype),
            plan.B, plan.H, plan.H_kv, plan.D, plan.rep_t,
            plan.descs.data_ptr(), plan.n_desc, plan.work.data_ptr(), plan.n_work,
            None if plan.uniform_groups else plan.offsets.data_ptr(), plan.n_groups,
            None, float(scale), None, None, None, plan.H, 0,
            out.data_ptr(), nat.dtype_code(out.dtype), lse.data_ptr())


def _layer(dev, n_chunks, chunk, seed):
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer
    g = torch.Generator(device=dev).manual_seed(seed)
    H, H_kv, D = 32, 8, 128
    k = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev).to(torch.bfloat16)
    refs = [ChunkRef(k[..., i * chunk:(i + 1) * chunk, :], v[..., i * chunk:(i + 1) * chunk, :], i * chunk, True)
            for i in range(n_chunks)]
    n_hot = max(1, n_chunks // 4)
    lay = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[-n_hot:],
                            cold=refs[:-n_hot], top_k=min(4, n_chunks - n_hot), device=dev)
    q = torch.randn((1, H, D), generator=g, device=dev).to(torch.bfloat16)
    return lay, q


def test_noalloc_matches_workspace_entry_points(dev):
    from halo_amd import _native as nat
    from halo_amd.decode import launch
    f, cap = _fn()
    assert cap == 8 << 20
    scale = 1 / math.sqrt(128)
    stream = nat.stream_ptr()
    # two calls in a row: the larger layer first, then a smaller one (the
    # scratch keeps the first call's partials; nothing must depend on them)
    for n_chunks, chunk, seed in ((32, 1024, 1), (8, 256, 2)):
        lay, q = _layer(dev, n_chunks, chunk, seed)
        out_ref = torch.empty((1, 32, 128), device=dev, dtype=torch.bfloat16)
        lse_ref = torch.empty((1, 32), device=dev, dtype=torch.float32)
        lay.step(q, scale=scale, out=out_ref, lse=lse_ref)          # halo_decode_attn_tiered + workspace
        out = torch.full_like(out_ref, float("nan"))
        lse = torch.full_like(lse_ref, float("nan"))
        nat.check(f(*_args(lay.plan, q, scale, out, lse), ctypes.byref(lay.select_cfg), stream),
                  "halo_decode_attn_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, out_ref) and torch.equal(lse, lse_ref), (n_chunks, chunk)
        # through the Python launcher as well
        out4 = torch.full_like(out_ref, float("nan"))
        launch(lay.plan, q, scale=scale, out=out4, select=lay.select_cfg, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(out4, out_ref)
        # sel = NULL: the plain halo_decode_attn over the table as it stands
        out2 = torch.empty_like(out_ref)
        lse2 = torch.empty_like(lse_ref)
        launch(lay.plan, q, scale=scale, out=out2, lse=lse2)
        out3 = torch.full_like(out_ref, float("nan"))
        lse3 = torch.full_like(lse_ref, float("nan"))
        nat.check(f(*_args(lay.plan, q, scale, out3, lse3), None, stream), "halo_decode_attn_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out3, out2) and torch.equal(lse3, lse2)


def test_noalloc_refuses_plans_beyond_the_scratch(dev):
    """A table whose partials exceed the static scratch is refused on the
    host with HALO_E_WORKSPACE before any launch."""
    from halo_amd import _native as nat
    f, cap = _fn()
    lay, q = _layer(dev, 8, 256, 3)
    per_item = lay.plan.rep_t * (lay.plan.D + 2) * 4
    too_many = cap // per_item + 1
    out = torch.empty((1, 32, 128), device=dev, dtype=torch.bfloat16)
    lse = torch.empty((1, 32), device=dev, dtype=torch.float32)
    args = list(_args(lay.plan, q, 0.1, out, lse))
    args[12] = too_many                               # n_work
    rc = f(*args, None, nat.stream_ptr())
    assert rc == nat.HALO_E_WORKSPACE
    assert b"static scratch" in nat.lib().halo_last_error()


def _first_call_in_capture() -> None:
    """Run in a fresh process: the first halo_decode_attn_noalloc call of the
    process -- the one that looks up the scratch address -- is made while a
    HIP graph is being captured; three replays (with eager work and a new
    query between them) equal the workspace entry point bit for bit."""
    from halo_amd import _native as nat
    dev = torch.device("cuda:0")
    f, _ = _fn()
    lay, q0 = _layer(dev, 8, 1024, 4)
    scale = 1 / math.sqrt(128)
    q = q0.clone()
    out = torch.full((1, 32, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    lse = torch.full((1, 32), float("nan"), device=dev, dtype=torch.float32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = f(*_args(lay.plan, q, scale, out, lse), ctypes.byref(lay.select_cfg), nat.stream_ptr(s))
    nat.check(rc, "halo_decode_attn_noalloc (first call, under capture)")
    out_ref = torch.empty_like(out)
    lse_ref = torch.empty_like(lse)
    for i in range(3):
        q.copy_(q0 * (1 + 0.5 * i))
        lay.step(q, scale=scale, out=out_ref, lse=lse_ref)      # workspace entry point, eager
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, out_ref) and torch.equal(lse, lse_ref), i
    print("first-call-in-capture: 3 replays equal", flush=True)


def test_noalloc_first_call_inside_graph_capture(dev):
    """The documented use: a caller whose very first allocation-free call is
    recorded into a graph (a fresh process, so the scratch address has not
    been looked up yet)."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = ("import sys; sys.path[:0] = [%r, %r]; import test_zz_no_alloc as t; t._first_call_in_capture()"
            % (here, os.path.dirname(here)))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=150)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "3 replays equal" in r.stdout
