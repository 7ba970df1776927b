"""Oracle: chunked attention, LSE merge and the chunk walk (numpy).

Test infrastructure only (see oracle/__init__.py).  Every function cites the
reference lines it restates.  Arrays use the reference's shapes:
q (B, H, T_q, D), k/v (B, H_kv, T, D).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

NEG_INF = np.float32(-np.inf)


def _repeat_kv(k: np.ndarray, rep: int) -> np.ndarray:
    # GQA broadcast, torch.repeat_interleave(rep, dim=1)
    # (halo/kv_cache_chunked.py:260-265)
    return np.repeat(k, rep, axis=1) if rep > 1 else k


def logsumexp(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """torch.logsumexp semantics: all -inf row -> -inf, no NaN."""
    m = np.max(x, axis=axis, keepdims=True)
    m_safe = np.where(np.isneginf(m), 0.0, m).astype(x.dtype)
    with np.errstate(under="ignore"):
        s = np.sum(np.exp(x - m_safe), axis=axis, keepdims=True)
    with np.errstate(divide="ignore"):
        out = np.log(s) + m_safe
    return np.squeeze(out, axis=axis)


def chunk_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, *,
                    scaling: Optional[float] = None,
                    causal_mask: Optional[np.ndarray] = None):
    """HALOCacheChunked._chunk_attention (halo/kv_cache_chunked.py:241-276).

    fp32 upcast, GQA repeat, qk = q k^T * scale (+ additive mask),
    lse = logsumexp(qk), out = exp(qk - lse) v.  Returns fp32 (out, lse).
    A fully masked row gives lse = -inf and out = NaN, exactly as torch does;
    the merge below discards it.
    """
    H, H_kv = q.shape[1], k.shape[1]
    if H != H_kv:
        assert H % H_kv == 0
        rep = H // H_kv
        k = _repeat_kv(k, rep)
        v = _repeat_kv(v, rep)
    if scaling is None:
        scaling = 1.0 / math.sqrt(q.shape[-1])
    q32 = q.astype(np.float32)
    k32 = k.astype(np.float32)
    v32 = v.astype(np.float32)
    qk = np.matmul(q32, np.swapaxes(k32, -1, -2)) * np.float32(scaling)
    if causal_mask is not None:
        qk = qk + causal_mask.astype(np.float32)
    lse = logsumexp(qk, axis=-1)
    with np.errstate(invalid="ignore"):
        weights = np.exp(qk - lse[..., None])
    out = np.matmul(weights, v32)
    return out.astype(np.float32), lse.astype(np.float32)


def lse_merge(out_a, lse_a, out_b, lse_b):
    """HALOCacheChunked._lse_merge (halo/kv_cache_chunked.py:194-239).

    lse = logaddexp(la, lb); weights exp(l - lse); a side whose lse is -inf
    gets zero weight and its (possibly NaN) output is replaced by zeros.
    """
    oa = out_a.astype(np.float32)
    ob = out_b.astype(np.float32)
    la = lse_a.astype(np.float32)
    lb = lse_b.astype(np.float32)
    lse = np.logaddexp(la, lb)
    a_inf = np.isneginf(la)
    b_inf = np.isneginf(lb)
    with np.errstate(invalid="ignore"):
        wa = np.exp(la - lse)
        wb = np.exp(lb - lse)
    wa = np.where(a_inf, 0.0, wa).astype(np.float32)[..., None]
    wb = np.where(b_inf, 0.0, wb).astype(np.float32)[..., None]
    a_safe = np.where(a_inf[..., None], 0.0, oa)
    b_safe = np.where(b_inf[..., None], 0.0, ob)
    return (wa * a_safe + wb * b_safe).astype(np.float32), lse.astype(np.float32)


def compute_attention(q: np.ndarray, cold_k: Optional[np.ndarray], cold_v: Optional[np.ndarray],
                      gpu_k: Optional[np.ndarray], gpu_v: Optional[np.ndarray], *,
                      chunk_size: int, scaling: Optional[float] = None,
                      query_pos_offset: Optional[int] = None):
    """The PyTorch chunk walk of HALOCacheChunked.compute_attention
    (halo/kv_cache_chunked.py:765-964): cold rows [0, T_cold) in chunk_size
    steps, then recent rows at global offset T_cold; for T_q > 1 an additive
    causal mask per chunk and skipping of chunks with no allowed key.
    Returns (out fp32, lse fp32, n_chunks).  (The reference returns only
    ``out`` cast to q.dtype; the LSE is what it computes and drops.)
    """
    B, H, T_q, D = q.shape
    T_cold = cold_k.shape[-2] if cold_k is not None else 0
    T_gpu = gpu_k.shape[-2] if gpu_k is not None else 0
    T_total = T_cold + T_gpu
    if T_total == 0:
        return np.zeros((B, H, T_q, D), np.float32), np.full((B, H, T_q), -np.inf, np.float32), 0
    if query_pos_offset is None:
        query_pos_offset = T_total - T_q
    running_out = running_lse = None
    n_chunks = 0

    def mask_for(c0: int, n: int, skip_all_masked: bool):
        if T_q == 1:
            return None, False
        i = np.arange(T_q)[:, None]
        j = np.arange(n)[None, :]
        allowed = (c0 + j) <= (query_pos_offset + i)
        if allowed.all():
            return None, False
        if skip_all_masked and not allowed.any():
            return None, True
        return np.where(allowed, 0.0, -np.inf).astype(np.float32), False

    segments = []
    if cold_k is not None and T_cold > 0:
        for c0 in range(0, T_cold, chunk_size):
            c1 = min(c0 + chunk_size, T_cold)
            segments.append((cold_k[..., c0:c1, :], cold_v[..., c0:c1, :], c0))
    if gpu_k is not None and T_gpu > 0:
        for c0 in range(0, T_gpu, chunk_size):
            c1 = min(c0 + chunk_size, T_gpu)
            segments.append((gpu_k[..., c0:c1, :], gpu_v[..., c0:c1, :], T_cold + c0))
    for kc, vc, g0 in segments:
        mask, skip = mask_for(g0, kc.shape[-2], True)
        if skip:
            continue
        out_c, lse_c = chunk_attention(q, kc, vc, scaling=scaling, causal_mask=mask)
        if running_out is None:
            running_out, running_lse = out_c, lse_c
        else:
            running_out, running_lse = lse_merge(running_out, running_lse, out_c, lse_c)
        n_chunks += 1
    return running_out, running_lse, n_chunks


def chunked_decode(q: np.ndarray, chunks: Sequence, *, scale: Optional[float] = None,
                   q_pos: Optional[np.ndarray] = None):
    """triton_chunked_attention semantics (halo/triton_chunked.py:210-267)
    restated with the PyTorch route's arithmetic: each ``(k, v, chunk_start,
    apply_causal)`` chunk is attended with mask ``chunk_start + j <= q_pos[b]``
    and the partials are LSE-merged in list order.  Default q_pos is
    total_T - 1 (:250-253).  q is (B, H, D) or (B, H, 1, D).  Returns fp32
    (out (B, H, D), lse (B, H)); a query with every key masked gets out 0 and
    lse -inf (finalize's l == 0 rule, :205-207).
    """
    q3 = q[:, :, 0, :] if q.ndim == 4 else q
    B, H, D = q3.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if q_pos is None:
        total = sum(c[0].shape[-2] for c in chunks)
        q_pos = np.full((B,), total - 1, dtype=np.int64)
    out = np.zeros((B, H, D), np.float32)
    lse = np.full((B, H), -np.inf, np.float32)
    for b in range(B):
        run_o = run_l = None
        for (k, v, c0, causal) in chunks:
            kb, vb = k[b:b + 1], v[b:b + 1]
            T = kb.shape[-2]
            mask = None
            if causal:
                allowed = (c0 + np.arange(T)) <= q_pos[b]
                if not allowed.any():
                    continue
                if not allowed.all():
                    mask = np.where(allowed, 0.0, -np.inf).astype(np.float32)[None, :]
            o_c, l_c = chunk_attention(q3[b:b + 1, :, None, :], kb, vb, scaling=scale, causal_mask=mask)
            if run_o is None:
                run_o, run_l = o_c, l_c
            else:
                run_o, run_l = lse_merge(run_o, run_l, o_c, l_c)
        if run_o is not None:
            out[b] = run_o[0, :, 0, :]
            lse[b] = run_l[0, :, 0]
    return out, lse


def update_chunk(q: np.ndarray, k: np.ndarray, v: np.ndarray, m: np.ndarray, l: np.ndarray,
                 o: np.ndarray, *, scale: float, chunk_start: int, q_pos: np.ndarray,
                 apply_causal: bool, block_n: int = 64) -> None:
    """The Triton kernel's per-(b, h) online-softmax update, in place
    (halo/triton_chunked.py:46-138), fp32: for each BLOCK_N tile, mask rows
    n >= T_c and (causal) chunk_start + n > q_pos[b]; m_new = max(m, max qk);
    l = exp(m - m_new) l + sum p; o = exp(m - m_new) o + p v.  Where the
    reference would evaluate exp(-inf - -inf) (a fully masked tile before
    any unmasked one, :122-128) this restatement uses the PyTorch route's
    zero-weight rule instead (halo/kv_cache_chunked.py:221-238).
    """
    B, H, D = q.shape
    H_kv, T_c = k.shape[1], k.shape[2]
    for b in range(B):
        for h in range(H):
            hk = h * H_kv // H
            qv = q[b, h].astype(np.float32)
            mi, li, oi = np.float32(m[b, h]), np.float32(l[b, h]), o[b, h].astype(np.float32)
            for n0 in range(0, T_c, block_n):
                n = np.arange(n0, min(n0 + block_n, T_c))
                kb = k[b, hk, n].astype(np.float32)
                vb = v[b, hk, n].astype(np.float32)
                qk = (kb @ qv) * np.float32(scale)
                mask = np.ones(len(n), bool)
                if apply_causal:
                    mask &= (chunk_start + n) <= q_pos[b]
                qk = np.where(mask, qk, -np.inf).astype(np.float32)
                m_new = np.float32(max(mi, qk.max()))
                if m_new == -np.inf:
                    continue
                alpha = np.float32(np.exp(mi - m_new))
                p = np.exp(qk - m_new).astype(np.float32)
                li = np.float32(alpha * li + p.sum())
                oi = (alpha * oi + p @ vb).astype(np.float32)
                mi = m_new
            m[b, h], l[b, h], o[b, h] = mi, li, oi


def finalize(m: np.ndarray, l: np.ndarray, o: np.ndarray):
    """halo/triton_chunked.py:195-207 plus the LSE it leaves out:
    out = o / (l > 0 ? l : 1), lse = m + log(l) (-inf where l == 0)."""
    safe = np.where(l > 0, l, 1.0).astype(np.float32)
    out = (o / safe[..., None]).astype(np.float32)
    with np.errstate(divide="ignore"):
        lse = np.where(l > 0, m + np.log(np.where(l > 0, l, 1.0)), -np.inf).astype(np.float32)
    return out, lse


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float,
                  keep: Optional[np.ndarray] = None, q_pos: Optional[np.ndarray] = None,
                  positions: Optional[np.ndarray] = None):
    """Closed-form softmax attention in float64 -- the brute force every
    restatement above is checked against.  q (B, H, D); k, v (B, H_kv, T, D);
    ``positions`` gives each row's global key position (default arange(T));
    row j of batch b is attended iff keep[j] and positions[j] <= q_pos[b].
    Returns (out (B, H, D) f64, lse (B, H) f64; out 0 / lse -inf when nothing
    is attended)."""
    B, H, D = q.shape
    H_kv, T = k.shape[1], k.shape[2]
    rep = H // H_kv
    pos = np.arange(T) if positions is None else np.asarray(positions)
    out = np.zeros((B, H, D))
    lse = np.full((B, H), -np.inf)
    for b in range(B):
        allowed = np.ones(T, bool) if keep is None else keep.copy()
        if q_pos is not None:
            allowed &= pos <= q_pos[b]
        if not allowed.any():
            continue
        for h in range(H):
            kk = k[b, h // rep][allowed].astype(np.float64)
            vv = v[b, h // rep][allowed].astype(np.float64)
            s = kk @ q[b, h].astype(np.float64) * scale
            mx = s.max()
            w = np.exp(s - mx)
            out[b, h] = (w @ vv) / w.sum()
            lse[b, h] = mx + np.log(w.sum())
    return out, lse


def prefill_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float, q_start: int):
    """Causal prefill brute force in float64: query row i sits at global
    position q_start + i and attends key rows j <= q_start + i.
    q (B, H, T_q, D); k, v (B, H_kv, T, D).  Returns (out f64, lse f64)."""
    B, H, T_q, D = q.shape
    H_kv, T = k.shape[1], k.shape[2]
    rep = H // H_kv
    qq = q.astype(np.float64)
    kk = np.repeat(k.astype(np.float64), rep, axis=1)
    vv = np.repeat(v.astype(np.float64), rep, axis=1)
    s = np.matmul(qq, np.swapaxes(kk, -1, -2)) * scale
    i = np.arange(T_q)[:, None] + q_start
    j = np.arange(T)[None, :]
    s = np.where(j <= i, s, -np.inf)
    mx = s.max(-1, keepdims=True)
    w = np.exp(s - mx)
    den = w.sum(-1, keepdims=True)
    return np.matmul(w, vv) / den, (mx + np.log(den))[..., 0]
