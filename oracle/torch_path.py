"""The reference's CPU torch op sequence, for the CPU baseline timing only.

Test infrastructure only.  This is the PyTorch route of the reference run on
the host cores: per chunk GQA repeat_interleave, fp32 matmul, logsumexp,
exp, matmul (halo/kv_cache_chunked.py:241-276), then the guarded logaddexp
merge (:194-239); mean-key scoring with topk (baselines/scorer_ablations.py:
218-268, alpha-only); KIVI dequantisation ``q.float()*s.float()+z.float()``
(baselines/kivi_cache.py:72-78) followed by the same attention.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def chunk_attention(q, k, v, scaling: Optional[float] = None, causal_mask=None):
    H, H_kv = q.shape[1], k.shape[1]
    if H != H_kv:
        rep = H // H_kv
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    if scaling is None:
        scaling = 1.0 / math.sqrt(q.shape[-1])
    qk = torch.matmul(q.to(torch.float32), k.to(torch.float32).transpose(-1, -2)) * scaling
    if causal_mask is not None:
        qk = qk + causal_mask.to(qk.dtype)
    lse = torch.logsumexp(qk, dim=-1)
    w = (qk - lse.unsqueeze(-1)).exp()
    return torch.matmul(w, v.to(torch.float32)), lse


def lse_merge(oa, la, ob, lb):
    lse = torch.logaddexp(la, lb)
    a_inf, b_inf = torch.isneginf(la), torch.isneginf(lb)
    wa = torch.where(a_inf, torch.zeros_like(la), (la - lse).exp()).unsqueeze(-1)
    wb = torch.where(b_inf, torch.zeros_like(lb), (lb - lse).exp()).unsqueeze(-1)
    oa = torch.where(a_inf.unsqueeze(-1).expand_as(oa), torch.zeros_like(oa), oa)
    ob = torch.where(b_inf.unsqueeze(-1).expand_as(ob), torch.zeros_like(ob), ob)
    return wa * oa + wb * ob, lse


def chunk_walk(q, chunks, scaling=None):
    """Attend a list of (k, v) chunks with the per-chunk LSE merge."""
    out = lse = None
    for k, v in chunks:
        oc, lc = chunk_attention(q, k, v, scaling)
        if out is None:
            out, lse = oc, lc
        else:
            out, lse = lse_merge(out, lse, oc, lc)
    return out, lse


def select_top(query, k_mean, eligible, top_k):
    """alpha-only mean-key score and topk among ``eligible`` chunk indices."""
    B, H, T_q, D = query.shape
    H_kv = k_mean.shape[1]
    q_g = query.view(B, H_kv, H // H_kv, T_q, D).mean(dim=2) if H != H_kv else query
    attn = (q_g.unsqueeze(-2).float() * k_mean.unsqueeze(-3).float()).sum(dim=-1)
    attn = attn.amax(dim=(0, 1, 2))
    sub = attn[eligible]
    return eligible[torch.topk(sub, top_k, largest=True).indices].sort().values


def kivi_dequant(codes, scale, zero):
    return (codes.float() * scale.float() + zero.float()).to(scale.dtype)
