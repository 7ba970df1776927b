"""HALOScorer on the GPU: closed-form hotness score and sorted top-k.

Reference: halo/scorer.py:36-88 (``score``, ``topk_hot``, ``jaccard``).
``score`` and ``topk_hot`` run the HIP kernels ``halo_halo_score`` and
``halo_topk_sorted``; ties in the top-k go to the lower index (torch.topk
leaves them undefined).  Inputs must be device tensors: there is no CPU path.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as nat


def topk_sorted(score: torch.Tensor, k: int, *, stream=None) -> torch.Tensor:
    """Indices (int64, ascending) of the k largest entries of a 1-D score."""
    L = nat.lib()
    score = score.reshape(-1)
    if score.dtype != torch.float32 or not score.is_contiguous():
        score = score.float().contiguous()
    K = score.numel()
    if not 1 <= k <= K:
        raise AssertionError(f"k={k} must be in [1, {K}]")
    out = torch.empty(k, dtype=torch.int64, device=score.device)
    nat.check(L.halo_topk_sorted(score.data_ptr(), K, k, out.data_ptr(), nat.stream_ptr(stream)), "halo_topk_sorted")
    return out


class HALOScorer:
    """Per-position hotness scores from an attention snapshot (GPU)."""

    def __init__(self, config) -> None:
        self.cfg = config

    def score(self, attention: torch.Tensor, *, step: int) -> torch.Tensor:
        """Hotness vector (K,) in [0, 1] for one head-mean attention snapshot
        (halo/scorer.py:36-72)."""
        L = nat.lib()
        attn = attention.reshape(-1)
        if attn.dtype != torch.float32 or not attn.is_contiguous():
            attn = attn.float().contiguous()
        if not attn.is_cuda:
            raise AssertionError("HALOScorer.score needs a device tensor")
        out = torch.empty_like(attn)
        c = self.cfg
        nat.check(L.halo_halo_score(attn.data_ptr(), attn.numel(), int(step), float(c.score_alpha),
                                    float(c.score_beta), float(c.score_gamma), int(c.sink_tokens),
                                    int(c.refresh_window), out.data_ptr(), nat.stream_ptr()), "halo_halo_score")
        return out.view(attention.shape)

    def topk_hot(self, score: torch.Tensor, *, ratio: Optional[float] = None) -> torch.Tensor:
        """Indices of the hot set, sorted; ``ratio >= 1`` returns every
        position (halo/scorer.py:74-88)."""
        ratio = self.cfg.hot_ratio if ratio is None else ratio
        K = score.shape[-1]
        if ratio >= 1.0:
            return torch.arange(K, device=score.device, dtype=torch.long)
        k = min(max(int(ratio * K), 1), K)
        return topk_sorted(score, k)

    def jaccard(self, a: torch.Tensor, b: torch.Tensor) -> float:
        """Jaccard overlap of two index sets (halo/scorer.py:92-98)."""
        sa, sb = set(a.tolist()), set(b.tolist())
        if not sa and not sb:
            return 1.0
        return len(sa & sb) / max(len(sa | sb), 1)

    def __repr__(self) -> str:  # pragma: no cover
        c = self.cfg
        return (f"HALOScorer(hot_ratio={c.hot_ratio}, alpha={c.score_alpha}, beta={c.score_beta}, "
                f"gamma={c.score_gamma}, sink={c.sink_tokens}, refresh={c.refresh_window})")
