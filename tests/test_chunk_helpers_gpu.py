"""GPU parity of HALOCacheChunked's chunk helpers ``_chunk_attention`` and
``_lse_merge`` on the reference's own checks (tests/test_kv_cache_chunked.py:
65-135): a chunk walk merged by LSE equals full attention for every chunk
size, bf16 within its rounding, GQA head groups, against the float64 closed
form; plus the causal mask of a position offset, and a mask of any other form
refused.  Head dim 64 (the kernels take 64, 128 and 256; the reference's
tests use 32)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu


def _qkv(dev, B=1, H=4, H_kv=4, T=128, D=64, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=g)
    k = torch.randn(B, H_kv, T, D, generator=g)
    v = torch.randn(B, H_kv, T, D, generator=g)
    return tuple(t.to(dtype) for t in (q, k, v)), tuple(t.to(dev).to(dtype) for t in (q, k, v))


def _walk(q, k, v, chunk):
    from halo_amd import HALOCacheChunked
    out = lse = None
    for c0 in range(0, k.shape[2], chunk):
        oc, lc = HALOCacheChunked._chunk_attention(q, k[..., c0:c0 + chunk, :], v[..., c0:c0 + chunk, :])
        out, lse = (oc, lc) if out is None else HALOCacheChunked._lse_merge(out, lse, oc, lc)
    return out, lse


@pytest.mark.parametrize("T", [1, 16, 128, 1024])
@pytest.mark.parametrize("chunk", [1, 16, 64, 256, 1024])
def test_chunk_walk_matches_full_attention(dev, T, chunk):
    (qc, kc, vc), (q, k, v) = _qkv(dev, T=T)
    out, lse = _walk(q, k, v, chunk)
    want, wl = A.attention_f64(qc.numpy()[:, :, 0], kc.numpy(), vc.numpy(), scale=1 / math.sqrt(64))
    assert out.dtype == torch.float32 and out.shape == (1, 4, 1, 64)
    assert np.abs(out[:, :, 0].cpu().numpy() - want).max() <= 1e-5
    assert np.abs(lse[:, :, 0].cpu().numpy() - wl).max() <= 1e-5


def test_chunk_walk_bf16(dev):
    (qc, kc, vc), (q, k, v) = _qkv(dev, T=512, dtype=torch.bfloat16)
    out, _ = _walk(q, k, v, 64)
    want, _ = A.attention_f64(qc.float().numpy()[:, :, 0], kc.float().numpy(), vc.float().numpy(),
                              scale=1 / math.sqrt(64))
    assert np.abs(out[:, :, 0].cpu().numpy() - want).max() <= 2e-2


@pytest.mark.parametrize("H,H_kv", [(8, 1), (8, 2), (8, 4), (8, 8), (16, 2)])
def test_chunk_attention_head_groups(dev, H, H_kv):
    from halo_amd import HALOCacheChunked
    (qc, kc, vc), (q, k, v) = _qkv(dev, H=H, H_kv=H_kv, T=64)
    out, _ = HALOCacheChunked._chunk_attention(q, k, v)
    want, _ = A.attention_f64(qc.numpy()[:, :, 0], kc.numpy(), vc.numpy(), scale=1 / math.sqrt(64))
    assert np.abs(out[:, :, 0].cpu().numpy() - want).max() <= 1e-5


def test_chunk_attention_causal_mask(dev):
    """Queries at positions q_start + i over one chunk at 0: the additive
    mask with -inf where j > q_start + i is taken as a causal cut; a mask of
    any other form raises."""
    from halo_amd import HALOCacheChunked
    g = torch.Generator().manual_seed(3)
    T_q, T_c, D, q_start = 5, 40, 64, 30
    qc = torch.randn(1, 4, T_q, D, generator=g)
    kc = torch.randn(1, 2, T_c, D, generator=g)
    vc = torch.randn(1, 2, T_c, D, generator=g)
    i = torch.arange(T_q).unsqueeze(1)
    j = torch.arange(T_c).unsqueeze(0)
    mask = torch.where(j > q_start + i, float("-inf"), 0.0)
    out, lse = HALOCacheChunked._chunk_attention(qc.to(dev), kc.to(dev), vc.to(dev), causal_mask=mask.to(dev))
    want, wl = A.prefill_f64(qc.numpy(), kc.numpy(), vc.numpy(), scale=1 / math.sqrt(D), q_start=q_start)
    assert np.abs(out.cpu().numpy() - want).max() <= 1e-5
    assert np.abs(lse.cpu().numpy() - wl).max() <= 1e-5
    bad = mask.clone()
    bad[0, 3] = float("-inf")
    with pytest.raises(NotImplementedError):
        HALOCacheChunked._chunk_attention(qc.to(dev), kc.to(dev), vc.to(dev), causal_mask=bad.to(dev))
