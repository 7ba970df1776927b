"""Parity at the full benchmark shapes (the sizes bench.py times), checked
on seeded samples against the float64 closed form:

* chunked causal prefill, 32/8 heads, d128: 4096 query rows over 28 x 1024
  prior rows plus the causal self block -- 64 query rows (0, 127, 128, 4095,
  the 64/128-row tile and 1024-row chunk boundaries, the rest seeded) for
  all 32 heads, output and LSE;
* ragged batched decode, 16 sequences of 8K-128K tokens (seed 3) in
  2048-row chunks, per-row top-8 selection: every row's selected chunk
  indices against the oracle's ranking where the top-8 boundary has a
  margin, and sampled rows' outputs against attention over hot + selected
  chunks;
* KIVI decode over 131072 tokens (4092 2-bit blocks + 128 fp16 rows, the
  129-partial merge): output and LSE against attention over the
  dequantised cache.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import scoring as S

pytestmark = pytest.mark.gpu


def _rows_f64(q, k, v, scale, rows, q_start):
    """Causal attention of the given query rows: q (H, T_q, D) f32, k/v
    (H_kv, T, D); row i attends keys <= q_start + i.  Returns out (H, n, D),
    lse (H, n)."""
    H, H_kv = q.shape[0], k.shape[0]
    rep = H // H_kv
    out = np.zeros((H, len(rows), q.shape[-1]))
    lse = np.zeros((H, len(rows)))
    for hk in range(H_kv):
        kk = k[hk].astype(np.float64)
        vv = v[hk].astype(np.float64)
        for j, i in enumerate(rows):
            n = q_start + i + 1
            qs = q[hk * rep:(hk + 1) * rep, i].astype(np.float64)      # (rep, D)
            s = qs @ kk[:n].T * scale
            mx = s.max(-1, keepdims=True)
            w = np.exp(s - mx)
            den = w.sum(-1, keepdims=True)
            out[hk * rep:(hk + 1) * rep, j] = (w @ vv[:n]) / den
            lse[hk * rep:(hk + 1) * rep, j] = (mx + np.log(den))[:, 0]
    return out, lse


def test_prefill_full_shape(dev):
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention
    H, H_kv, D, T_q, T_prior, chunk = 32, 8, 128, 4096, 28672, 1024
    gen = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn((1, H, T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn((1, H_kv, T_prior + T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((1, H_kv, T_prior + T_q, D), generator=gen, device=dev).to(torch.bfloat16)
    chunks = [ChunkRef(k[:, :, s:s + chunk], v[:, :, s:s + chunk], s, False) for s in range(0, T_prior, chunk)]
    chunks.append(ChunkRef(k[:, :, T_prior:], v[:, :, T_prior:], T_prior, True))
    out, lse = prefill_attention(q, chunks, return_lse=True)
    torch.cuda.synchronize()
    fixed = [0, 1, 63, 64, 127, 128, 129, 255, 256, 511, 1023, 1024, 2047, 2048, 3071, 3072, 4094, 4095]
    rng = np.random.default_rng(2)
    extra = rng.choice(np.setdiff1d(np.arange(T_q), fixed), size=64 - len(fixed), replace=False)
    rows = sorted(fixed + extra.tolist())
    qn = q[0].float().cpu().numpy()
    kn = k[0].float().cpu().numpy()
    vn = v[0].float().cpu().numpy()
    want, want_lse = _rows_f64(qn, kn, vn, 1 / math.sqrt(D), rows, T_prior)
    got = out[0][:, rows].float().cpu().numpy()
    got_lse = lse[0][:, rows].cpu().numpy()
    assert np.abs(got - want).max() <= 2e-2
    assert np.abs(got_lse - want_lse).max() <= 2e-2


def test_ragged_decode_full_shape(dev):
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import RaggedTieredDecodeLayer
    B, H, H_kv, D, chunk, top_k = 16, 32, 8, 128, 2048, 8
    rng = np.random.default_rng(3)
    ctx = [int(x) // chunk * chunk for x in rng.uniform(8192, 131072, size=B)]
    gen = torch.Generator(device=dev).manual_seed(3)
    rows, kv = [], []
    for b, T in enumerate(ctx):
        k = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((H_kv, T, D), generator=gen, device=dev).to(torch.bfloat16)
        n = T // chunk
        n_hot = max(1, n // 4)
        refs = [ChunkRef(k[:, i * chunk:(i + 1) * chunk], v[:, i * chunk:(i + 1) * chunk], i * chunk, True, batch=b)
                for i in range(n)]
        rows.append((refs[n - n_hot:], refs[:n - n_hot]))
        kv.append((k, v, n_hot))
    layer = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows, top_k=top_k, device=dev)
    q = torch.randn((B, H, D), generator=gen, device=dev).to(torch.bfloat16)
    q_pos = torch.tensor([T - 1 for T in ctx], device=dev, dtype=torch.int64)
    out = torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)
    lse = torch.empty((B, H), device=dev, dtype=torch.float32)
    layer.step(q, scale=1 / math.sqrt(D), out=out, lse=lse, q_pos=q_pos)
    torch.cuda.synchronize()
    idx = layer.idx.cpu().numpy()
    km = layer.kmean.float().cpu().numpy()
    qn = q.float().cpu().numpy()
    checked = 0
    for b in range(B):
        n_cold = len(rows[b][1])
        sc = S.mean_key_scores(qn[b:b + 1, :, None, :], km[b:b + 1, :, :n_cold], "bfloat16").astype(np.float64)
        order = np.lexsort((np.arange(n_cold), -sc))
        kk = min(top_k, n_cold)
        want = np.sort(order[:kk])
        margin = sc[order[kk - 1]] - sc[order[kk]] if kk < n_cold else np.inf
        if margin > 1e-4 * max(1.0, np.abs(sc).max()):
            assert idx[b, :kk].tolist() == want.tolist(), b
            checked += 1
        assert (idx[b, kk:] == -1).all()
    assert checked >= B - 2
    for b in (0, 5, 11, 15):
        k, v, n_hot = kv[b]
        n = ctx[b] // chunk
        sel = [int(c) for c in idx[b] if c >= 0] + list(range(n - n_hot, n))
        rows_k = torch.cat([k[:, c * chunk:(c + 1) * chunk] for c in sel], dim=1).float().cpu().numpy()
        rows_v = torch.cat([v[:, c * chunk:(c + 1) * chunk] for c in sel], dim=1).float().cpu().numpy()
        w, wl = A.attention_f64(qn[b:b + 1], rows_k[None], rows_v[None], scale=1 / math.sqrt(D))
        assert np.abs(out[b:b + 1].float().cpu().numpy() - w).max() <= 2e-2, b
        assert np.abs(lse[b:b + 1].cpu().numpy() - wl).max() <= 2e-2, b


def test_kivi_decode_full_shape(dev):
    from halo_amd import kivi
    from halo_amd.decode import ChunkRef
    H, H_kv, D, T, resid = 28, 4, 128, 131072, 128
    T_cold = T - resid
    gen = torch.Generator(device=dev).manual_seed(4)
    k = torch.randn((1, H_kv, T, D), generator=gen, device=dev)
    ch = torch.randperm(D, generator=gen, device=dev)[:2]
    k[..., ch] *= 10.0
    k = k.to(torch.float16)
    v = torch.randn((1, H_kv, T, D), generator=gen, device=dev).to(torch.float16)
    blocks = kivi.quantize(k[:, :, :T_cold], v[:, :, :T_cold])
    kr, vr = k[:, :, T_cold:].clone(), v[:, :, T_cold:].clone()
    lay = kivi.KiviDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.float16, cold_blocks=blocks,
                               recent=[ChunkRef(kr, vr, T_cold, True)], device=dev, chunk_tokens=2048)
    per_group = lay.plan.n_work // lay.plan.n_groups
    assert per_group > 64        # the wide merge (more than 64 partials per group) is exercised
    q = torch.randn((1, H, D), generator=gen, device=dev).to(torch.float16)
    out = torch.empty((1, H, D), device=dev, dtype=torch.float16)
    lse = torch.empty((1, H), device=dev, dtype=torch.float32)
    lay.step(q, scale=1 / math.sqrt(D), out=out, lse=lse)
    kd, vd = kivi.dequantize(blocks, D=D, dtype=torch.float16)
    kk = torch.cat([kd, kr], dim=2).float().cpu().numpy()
    vv = torch.cat([vd, vr], dim=2).float().cpu().numpy()
    w, wl = A.attention_f64(q.float().cpu().numpy(), kk, vv, scale=1 / math.sqrt(D))
    assert np.abs(out.float().cpu().numpy() - w).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - wl).max() <= 1e-3
