"""Workspace lifetime under HIP graph capture, and the standalone LSE merge.

* A captured ``TieredDecodeLayer`` step keeps replaying into its own plan's
  partial buffer after a 4x larger plan has been launched on the same
  stream (a workspace shared per stream and regrown for the larger plan
  would have been freed under the graph); every replay equals the eager
  step bit for bit.
* ``halo_lse_merge`` against the oracle's ``lse_merge``
  (halo/kv_cache_chunked.py:194-239), including rows where one or both
  sides are -inf.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu


def _layer(dev, n_chunks: int, chunk: int, seed: int):
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer
    g = torch.Generator(device=dev).manual_seed(seed)
    H, H_kv, D = 32, 8, 128
    k = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev).to(torch.bfloat16)
    refs = [ChunkRef(k[..., i * chunk:(i + 1) * chunk, :], v[..., i * chunk:(i + 1) * chunk, :], i * chunk, True)
            for i in range(n_chunks)]
    n_hot = n_chunks // 4
    lay = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[-n_hot:],
                            cold=refs[:-n_hot], top_k=2, device=dev)
    q = torch.randn((1, H, D), generator=g, device=dev).to(torch.bfloat16)
    return lay, q, (k, v)


def test_graph_replay_survives_a_larger_plan(dev):
    small, q_s, _ = _layer(dev, 8, 512, 1)
    big, q_b, _ = _layer(dev, 32, 1024, 2)   # 4x the work items of the small plan, and more
    assert big.plan.n_work >= 4 * small.plan.n_work
    scale = 1 / math.sqrt(128)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out_e = torch.empty((1, 32, 128), device=dev, dtype=torch.bfloat16)
    out_g = torch.empty_like(out_e)
    out_b = torch.empty_like(out_e)
    with torch.cuda.stream(s):
        small.step(q_s, scale=scale, out=out_e)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            small.step(q_s, scale=scale, out=out_g)
        for rep in range(3):
            big.step(q_b, scale=scale, out=out_b)       # larger plan on the capture stream
            junk = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(0xA5)  # reuse freed memory
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_e), f"replay {rep} differs from the eager step"
            del junk
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,D", [(7, 64), (300, 128)])
def test_lse_merge_matches_oracle(dev, n, D):
    from halo_amd.triton_chunked import lse_merge
    rng = np.random.default_rng(n)
    oa = rng.standard_normal((n, D)).astype(np.float32)
    ob = rng.standard_normal((n, D)).astype(np.float32)
    la = (rng.standard_normal(n) * 5).astype(np.float32)
    lb = (rng.standard_normal(n) * 5).astype(np.float32)
    la[::5] = -np.inf             # side a empty
    lb[1::5] = -np.inf            # side b empty
    la[2::5] = lb[2::5] = -np.inf  # both empty: lse -inf, out 0
    oa[::5] = np.nan              # an empty side's output never contributes
    out, lse = lse_merge(*(torch.from_numpy(x).to(dev) for x in (oa, la, ob, lb)))
    wo, wl = A.lse_merge(oa, la, ob, lb)
    got_o, got_l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.array_equal(np.isneginf(got_l), np.isneginf(wl))
    fin = np.isfinite(wl)
    np.testing.assert_allclose(got_l[fin], wl[fin], rtol=0, atol=1e-5)
    np.testing.assert_allclose(got_o, wo, rtol=0, atol=1e-5)
    assert not np.isnan(got_o).any()


def test_lse_merge_composes_partials(dev):
    """Merging the (out, lse) of two disjoint key sets equals attention over
    their union (the associativity the chunk walk relies on)."""
    from halo_amd.triton_chunked import lse_merge, triton_chunked_attention
    rng = np.random.default_rng(2)
    B, H, H_kv, D, T = 1, 8, 2, 64, 640
    q = rng.standard_normal((B, H, 1, D)).astype(np.float32)
    k = rng.standard_normal((B, H_kv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, H_kv, T, D)).astype(np.float32)
    qg, kg, vg = (torch.from_numpy(x).to(dev) for x in (q, k, v))
    oa, la = triton_chunked_attention(qg, [(kg[:, :, :200], vg[:, :, :200], 0, False)], return_lse=True)
    ob, lb = triton_chunked_attention(qg, [(kg[:, :, 200:], vg[:, :, 200:], 200, False)], return_lse=True)
    out, lse = lse_merge(oa[:, :, 0], la, ob[:, :, 0], lb)
    w, wl = A.attention_f64(q[:, :, 0], k, v, scale=1 / math.sqrt(D))
    assert np.abs(out.cpu().numpy() - w).max() <= 1e-5
    assert np.abs(lse.cpu().numpy() - wl).max() <= 1e-5
