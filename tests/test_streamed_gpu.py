"""The public ``triton_chunked_attention_streamed`` (the import-swap entry of
halo/triton_chunked.py:270-362): cold chunks given as pinned host tensors
``(k, v, chunk_start)`` are copied through ``n_buffers`` HBM slots on the
copy stream while hot chunks are attended in place; every chunk is causal at
its start.  Checked against the float64 closed form over the union of the
listed rows at their global positions: mixed, hot-only and cold-only lists,
1, 2 and 3 buffers, a causal cut inside a chunk, non-contiguous selected
chunk starts, a cold chunk that is a strided view of a larger pinned tensor,
with and without the LSE."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu

B, H, H_kv, D = 2, 16, 4, 128


def _pinned(t: torch.Tensor) -> torch.Tensor:
    h = torch.empty(tuple(t.shape), dtype=t.dtype, pin_memory=True)
    h.copy_(t)
    return h


def _lists(dev, dtype, case, seed):
    """Cold chunks at starts 0, 512 (a strided view of a larger pinned tensor)
    and 1280; hot chunks at 2048 and 2560 (a short one).  Chunks 256-511 and
    768-1279 are not listed (not selected)."""
    g = torch.Generator().manual_seed(seed)

    def kv(T):
        k = torch.randn((B, H_kv, T, D), generator=g)
        k[..., :2] *= 4
        return k.to(dtype), torch.randn((B, H_kv, T, D), generator=g).to(dtype)

    cold, hot, rows = [], [], []
    if case in ("mixed", "cold_only"):
        k0, v0 = kv(256)
        cold.append((_pinned(k0), _pinned(v0), 0))
        big_k, big_v = kv(768)                       # pinned (B, H_kv, 768, D); the chunk is rows 256:512
        bk, bv = _pinned(big_k), _pinned(big_v)
        cold.append((bk[:, :, 256:512], bv[:, :, 256:512], 512))
        k2, v2 = kv(384)
        cold.append((_pinned(k2), _pinned(v2), 1280))
        rows += [(k0, v0, 0), (big_k[:, :, 256:512], big_v[:, :, 256:512], 512), (k2, v2, 1280)]
    if case in ("mixed", "hot_only"):
        k3, v3 = kv(512)
        k4, v4 = kv(100)
        hot += [(k3.to(dev), v3.to(dev), 2048), (k4.to(dev), v4.to(dev), 2560)]
        rows += [(k3, v3, 2048), (k4, v4, 2560)]
    return cold, hot, rows


def _reference(q, rows, q_pos, scale):
    k = np.concatenate([r[0].float().numpy() for r in rows], axis=2)
    v = np.concatenate([r[1].float().numpy() for r in rows], axis=2)
    pos = np.concatenate([np.arange(r[0].shape[2]) + r[2] for r in rows])
    return A.attention_f64(q, k, v, scale=scale, q_pos=q_pos, positions=pos)


@pytest.mark.parametrize("n_buffers", [1, 2, 3])
@pytest.mark.parametrize("case", ["mixed", "hot_only", "cold_only"])
def test_streamed_matches_closed_form(dev, case, n_buffers):
    from halo_amd.triton_chunked import triton_chunked_attention_streamed as streamed
    dtype = torch.bfloat16
    cold, hot, rows = _lists(dev, dtype, case, seed=n_buffers + 10 * len(case))
    q = torch.randn((B, H, 1, D), generator=torch.Generator().manual_seed(5)).to(dtype)
    last = max(r[2] + r[0].shape[2] for r in rows) - 1
    # row 0 decodes at the last listed position; row 1 is cut inside the
    # second cold chunk (mixed / cold-only) or inside the first hot chunk
    cut = 600 if cold else 2300
    qp = torch.tensor([last, cut], dtype=torch.int64)
    scale = 1 / math.sqrt(D)
    out, lse = streamed(q.to(dev), cold, hot, scale=scale, q_pos=qp.to(dev), n_buffers=n_buffers,
                        return_lse=True)
    out_only = streamed(q.to(dev), cold, hot, scale=scale, q_pos=qp.to(dev), n_buffers=n_buffers)
    torch.cuda.synchronize()
    assert out.shape == (B, H, 1, D) and out.dtype == dtype and lse.shape == (B, H)
    assert torch.equal(out, out_only)
    want, want_lse = _reference(q[:, :, 0].float().numpy(), rows, qp.numpy(), scale)
    assert np.abs(out[:, :, 0].float().cpu().numpy() - want).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - want_lse).max() <= 1e-2


def test_streamed_fp32_and_empty(dev):
    from halo_amd.triton_chunked import triton_chunked_attention_streamed as streamed
    cold, hot, rows = _lists(dev, torch.float32, "mixed", seed=3)
    q = torch.randn((B, H, 1, D), generator=torch.Generator().manual_seed(6))
    qp = torch.tensor([2659, 1400], dtype=torch.int64)
    out, lse = streamed(q.to(dev), cold, hot, q_pos=qp.to(dev), return_lse=True)
    torch.cuda.synchronize()
    want, want_lse = _reference(q[:, :, 0].numpy(), rows, qp.numpy(), 1 / math.sqrt(D))
    assert np.abs(out[:, :, 0].cpu().numpy() - want).max() <= 1e-5
    assert np.abs(lse.cpu().numpy() - want_lse).max() <= 1e-5
    # nothing listed: zeros and an LSE of -inf
    z, zl = streamed(q.to(dev), [], [], q_pos=qp.to(dev), return_lse=True)
    assert z.shape == (B, H, 1, D) and not z.any() and torch.isneginf(zl).all()
