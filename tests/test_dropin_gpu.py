"""The drop-in kernel module's plan cache: a repeated chunk list launches the
cached plan (no new tables), results equal the first call's bit for bit and
the float64 closed form; a changed chunk start or stream plans again; calls
captured in a HIP graph replay to the eager result (several replays with
eager work in between)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu


def _chunks(dev, *, n=5, T=192, H_kv=2, D=128, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((1, H_kv, n * T, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, H_kv, n * T, D), generator=g, device=dev).to(torch.bfloat16)
    return k, v, [(k[:, :, i * T:(i + 1) * T], v[:, :, i * T:(i + 1) * T], i * T, True) for i in range(n)]


def test_repeated_calls_reuse_the_cached_plan(dev):
    from halo_amd import decode
    from halo_amd.triton_chunked import triton_chunked_attention
    decode.clear_plan_cache()
    k, v, chunks = _chunks(dev)
    q = torch.randn((1, 8, 1, 128), device=dev).to(torch.bfloat16)
    o1, l1 = triton_chunked_attention(q, chunks, return_lse=True)
    n_plans = len(decode._plan_cache)
    for _ in range(3):
        o2, l2 = triton_chunked_attention(q, chunks, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert len(decode._plan_cache) == n_plans == 1
    want, want_lse = A.attention_f64(q[:, :, 0].float().cpu().numpy(), k.float().cpu().numpy(),
                                     v.float().cpu().numpy(), scale=1 / math.sqrt(128))
    assert np.abs(o1[:, :, 0].float().cpu().numpy() - want).max() <= 2e-2
    assert np.abs(l1.cpu().numpy() - want_lse).max() <= 2e-2
    # another chunk start is another plan; so is another stream
    moved = [(kk, vv, c0 + 1, causal) for (kk, vv, c0, causal) in chunks]
    triton_chunked_attention(q, moved)
    assert len(decode._plan_cache) == 2
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        o3 = triton_chunked_attention(q, chunks)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert len(decode._plan_cache) == 3
    assert torch.equal(o3, o1)


def test_graph_capture_replays_the_eager_result(dev):
    from halo_amd import decode
    from halo_amd.triton_chunked import triton_chunked_attention
    decode.clear_plan_cache()
    _, _, chunks = _chunks(dev, seed=2)
    q = torch.randn((1, 8, 1, 128), device=dev).to(torch.bfloat16)
    qbuf = q.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ref = triton_chunked_attention(qbuf, chunks)        # plans (outside the capture)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = triton_chunked_attention(qbuf, chunks)
        for i in range(4):
            qbuf.copy_(q * (1 + i % 2))
            eager = triton_chunked_attention(qbuf, chunks)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), i
    torch.cuda.synchronize()
    assert torch.equal(triton_chunked_attention(q, chunks), ref)


def test_repeated_calls_take_the_fast_path(dev):
    """The second call with the same chunk layout and stream launches from
    the fast cache: bit-identical results, with and without q_pos and LSE; a
    misaligned chunk (copied to an aligned one) never enters the cache."""
    from halo_amd import triton_chunked as tc
    tc.clear_fast_cache()
    k, v, chunks = _chunks(dev, seed=4)
    q = torch.randn((1, 8, 1, 128), device=dev).to(torch.bfloat16)
    o1, l1 = tc.triton_chunked_attention(q, chunks, return_lse=True)
    assert len(tc._fast) == 1
    for _ in range(3):
        o2, l2 = tc.triton_chunked_attention(q, chunks, return_lse=True)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
    o3 = tc.triton_chunked_attention(q, chunks)
    assert torch.equal(o3, o1) and len(tc._fast) == 1
    qp = torch.tensor([700], device=dev)
    o4 = tc.triton_chunked_attention(q, chunks, q_pos=qp)
    o5 = tc.triton_chunked_attention(q, chunks, q_pos=qp)
    assert len(tc._fast) == 2 and torch.equal(o4, o5)
    torch.cuda.synchronize()
    want, _ = A.attention_f64(q[:, :, 0].float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                              scale=1 / math.sqrt(128), q_pos=np.array([700]))
    assert np.abs(o4[:, :, 0].float().cpu().numpy() - want).max() <= 2e-2
    # a chunk whose rows are not 16-byte aligned goes through a copy each call
    wide = torch.zeros((1, 2, 192, 129), device=dev, dtype=torch.bfloat16)
    wide[..., :128] = k[:, :, :192]
    odd = [(wide[..., :128], v[:, :, :192], 0, True)]
    tc.triton_chunked_attention(q, odd)
    tc.triton_chunked_attention(q, odd)
    assert len(tc._fast) == 2


def test_captured_plan_outlives_cache_eviction(dev):
    """A launch recorded into a graph keeps its plan (tables, workspace,
    default query positions) alive: after 300 calls with other layouts
    (beyond both caches' 256 entries), clear_plan_cache(),
    clear_fast_cache() and junk allocations that reuse freed memory, every
    replay still equals the eager result bit for bit."""
    from halo_amd import decode
    from halo_amd import triton_chunked as tc
    decode.clear_plan_cache()
    tc.clear_fast_cache()
    decode.release_captured_plans()
    k, v, chunks = _chunks(dev, n=4, T=256, seed=9)
    q = torch.randn((1, 8, 1, 128), device=dev).to(torch.bfloat16)
    qbuf = q.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        tc.triton_chunked_attention(qbuf, chunks)             # plans and enters the fast cache
        tc.triton_chunked_attention(qbuf, chunks)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = tc.triton_chunked_attention(qbuf, chunks)
    torch.cuda.synchronize()
    assert len(decode.captured_plans()) >= 1
    for i in range(300):  # other layouts: each moved start is a new plan and a new fast entry
        moved = [(kk, vv, c0 + 1 + i, causal) for (kk, vv, c0, causal) in chunks[:2]]
        tc.triton_chunked_attention(q, moved)
    decode.clear_plan_cache()
    tc.clear_fast_cache()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 20,), 0x7f7f, device=dev, dtype=torch.int32) for _ in range(16)]
    for i in range(3):
        qbuf.copy_(q * (1 + i))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        eager = tc.triton_chunked_attention(qbuf, chunks)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
    del junk
    decode.release_captured_plans()
    assert decode.captured_plans() == []
