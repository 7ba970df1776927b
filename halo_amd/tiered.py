"""One decode layer over a tiered chunk table: hot chunks plus the top-k cold
chunks a scorer picks each step.

Per step this enqueues two kernels on the current stream and nothing else:
  1. ``halo_chunk_score_topk`` scores the cold chunks' page-mean keys against
     the query and copies the chosen chunks' descriptors into the table's
     ``top_k`` selection slots;
  2. ``halo_decode_attn`` attends the hot chunks and the selection slots with
     the fused log-sum-exp merge, writing (out, lse).
There is no host round trip between the two, so a whole multi-layer decode
step can be captured in one HIP graph.

Reference: the Path-D placement loop -- a page scorer picks which pages stay
hot (halo/kv_cache_chunked.py:416-457 with baselines/scorer_ablations.py:
218-268) and the chunk walk attends them (halo/kv_cache_chunked.py:571-763);
``top_k`` of ``eligible`` cold chunks with the alpha-only mean-key score is
the workload rule "scorer picks top-k cold chunks by mean-key dot product".
Selected cold chunks must be readable by the GPU when ``step`` runs: HBM
staging copies (the refetched state) or their HBM mirrors.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from .chunk_scorer import chunk_means, score_topk
from .decode import ChunkRef, DecodePlan, build_plan, descs_to_device, launch, pack_descs


class TieredDecodeLayer:
    def __init__(self, *, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype,
                 hot: Sequence[ChunkRef], cold: Sequence[ChunkRef], top_k: int, device,
                 cold_kmean: Optional[torch.Tensor] = None, split: Optional[int] = None) -> None:
        if top_k > len(cold):
            raise AssertionError(f"top_k={top_k} > {len(cold)} cold chunks")
        self.B, self.H, self.H_kv, self.D, self.dtype = B, H, H_kv, D, dtype
        self.n_hot, self.top_k = len(hot), top_k
        self.hot, self.cold = list(hot), list(cold)
        # Selection slots start as placeholders (the first cold chunks); the
        # scorer overwrites them on the device every step.
        slots = [cold[i] for i in range(top_k)]
        self.plan: DecodePlan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype,
                                           chunks=list(hot) + slots, device=device, split=split)
        cat, keep = pack_descs(cold, B=B, H_kv=H_kv, D=D, dtype=dtype)
        self.catalog = descs_to_device(cat, device)
        self.plan.keep += keep
        self.eligible = torch.arange(len(cold), device=device, dtype=torch.int32)
        if cold_kmean is None:
            cold_kmean = self.build_means(cold)
        self.kmean = cold_kmean
        self.idx = torch.empty((1, top_k), device=device, dtype=torch.int32)
        self.scores = torch.empty((1, max(len(cold), 1)), device=device, dtype=torch.float32)

    def build_means(self, cold: Sequence[ChunkRef]) -> torch.Tensor:
        """One mean key per cold chunk (B, H_kv, n_cold, D)."""
        out = torch.empty((self.B, self.H_kv, len(cold), self.D), device=cold[0].k.device, dtype=self.dtype)
        for j, c in enumerate(cold):
            chunk_means(c.k, c.T, row0=0, n_pages=1, out=out, page_offset=j)
        return out

    @property
    def attended_rows(self) -> int:
        """K/V rows one step reads per (b, h_kv): hot rows + top_k selected."""
        per = max(c.T for c in self.cold)
        return sum(c.T for c in self.hot) + self.top_k * per

    def select(self, q: torch.Tensor) -> None:
        score_topk(q, self.kmean, self.eligible, self.top_k, catalog=self.catalog,
                   table=self.plan.descs, table_slot0=self.n_hot, idx_out=self.idx, score_out=self.scores)

    def attend(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse: Optional[torch.Tensor] = None,
               q_pos: Optional[torch.Tensor] = None) -> None:
        launch(self.plan, q, scale=scale, q_pos=q_pos, out=out, lse=lse)

    def step(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse: Optional[torch.Tensor] = None,
             q_pos: Optional[torch.Tensor] = None) -> None:
        self.select(q)
        self.attend(q, scale=scale, out=out, lse=lse, q_pos=q_pos)
