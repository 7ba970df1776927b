"""One decode layer over a tiered chunk table: hot chunks plus the top-k cold
chunks a scorer picks each step.

Per step (fused mode, the default) this enqueues one
``halo_decode_attn_tiered`` on the current stream: the workgroups of the
``top_k`` selection slots score the cold chunks' page-mean keys against the
query, take the chosen chunks' descriptors from the catalog and attend them,
while the other workgroups attend the hot chunks; the split-K merge kernel
then writes (out, lse).  Unfused mode (``fused=False``, or shapes beyond the
in-kernel selection limits) enqueues ``halo_chunk_score_topk`` (which copies
the chosen descriptors into the table's slots) followed by
``halo_decode_attn``.  Either way there is no host round trip, so a whole
multi-layer decode step can be captured in one HIP graph.

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

from . import _native as nat
from .chunk_scorer import chunk_means, score_topk
from .decode import ChunkRef, DecodePlan, build_plan, descs_to_device, launch, pack_descs

# In-kernel selection limits of halo_decode_attn_tiered (include/halo_hip.h):
# candidates and (chunk, row, KV head) triples per selection, 16-bit K/V
# (the wide form) and fp32.
_SEL_MAX_COLD = 128
_SEL_MAX_TRIPLES = 768
_SEL_MAX_COLD_F32 = 64
_SEL_MAX_TRIPLES_F32 = 512
_SEL_MAX_QBAR = 2048


def _sel_limits(dtype: torch.dtype) -> tuple[int, int]:
    if dtype == torch.float32:
        return _SEL_MAX_COLD_F32, _SEL_MAX_TRIPLES_F32
    return _SEL_MAX_COLD, _SEL_MAX_TRIPLES


class TieredDecodeLayer:
    def __init__(self, *, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype,
                 hot: Sequence[ChunkRef], cold: Sequence[ChunkRef], top_k: int, device,
                 cold_kmean: Optional[torch.Tensor] = None, split: Optional[int] = None,
                 fused: bool = True) -> None:
        if not 1 <= top_k <= len(cold):
            raise AssertionError(f"top_k={top_k} must be in [1, {len(cold)} cold chunks]")
        self.B, self.H, self.H_kv, self.D, self.dtype = B, H, H_kv, D, dtype
        self.n_hot, self.top_k = len(hot), top_k
        self.hot, self.cold = list(hot), list(cold)
        n_cold = len(cold)
        max_cold, max_triples = _sel_limits(dtype)
        self.fused = bool(fused) and n_cold <= max_cold and n_cold * B * H_kv <= max_triples \
            and B * H_kv * D <= _SEL_MAX_QBAR and D % 16 == 0
        # Selection slots come first in the table (their workgroups are
        # dispatched first, which hides the selection work behind the hot
        # chunks) and are cut into items of half the split: their rows can
        # only be read once the selection is known, so spreading them over
        # twice the workgroups shortens that critical path.  Each slot is
        # planned over the largest cold chunk, so its work items cover
        # whichever chunk is chosen; the unfused scorer overwrites the slot
        # descriptors on the device every step.
        widest = max(range(n_cold), key=lambda i: cold[i].T)
        slots = [cold[widest]] * top_k
        self.slot0 = 0
        self.plan: DecodePlan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype,
                                           chunks=slots + list(hot), device=device, split=split,
                                           first=range(top_k), first_half_split=True)
        cat, keep = pack_descs(cold, B=B, H_kv=H_kv, D=D, dtype=dtype)
        self.catalog = descs_to_device(cat, device)
        self.plan.keep += keep
        self.eligible = torch.arange(len(cold), device=device, dtype=torch.int32)
        if cold_kmean is None:
            if any(c.k.device.type == "cpu" for c in cold):
                raise AssertionError("cold chunks in pinned host memory need cold_kmean (their page means on the GPU)")
            cold_kmean = self.build_means(cold)
        self.kmean = cold_kmean
        self.idx = torch.empty((1, top_k), device=device, dtype=torch.int32)
        self.scores = torch.empty((1, max(len(cold), 1)), device=device, dtype=torch.float32)
        self.select_cfg = None
        # (residency, slot catalog, n_slots, res_out) when an HBM staging cache
        # serves the cold chunks of an unfused layer (set by ColdStaging)
        self.staging = None
        if self.fused:
            km = self.kmean
            if km.shape != (B, H_kv, n_cold, D) or km.dtype != dtype or km.stride(-1) != 1:
                raise AssertionError(f"cold_kmean must be ({B}, {H_kv}, {n_cold}, {D}) {dtype} with unit stride")
            self.select_cfg = nat.SelectCfg(
                kmean=km.data_ptr(), km_stride_b=km.stride(0), km_stride_h=km.stride(1), km_stride_p=km.stride(2),
                catalog=self.catalog.data_ptr(), catalog_stride=n_cold, n_cold_per_sel=None,
                n_cold=n_cold, top_k=top_k, slot0=self.slot0, per_row=0,
                idx_out=self.idx.data_ptr(), score_out=self.scores.data_ptr(),
                lead_items=self._lead_items())

    def _lead_items(self) -> int:
        """Number of leading work records (dispatch order) that are selection
        slots: those workgroups start the selection before reading their record."""
        d = self.plan.work_host[:, 0]
        slot = (d >= self.slot0) & (d < self.slot0 + self.top_k)
        n = 0
        while n < len(slot) and slot[n]:
            n += 1
        return n

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
        """Standalone selection (``halo_chunk_score_topk``): fills idx/scores
        and the table's selection slots."""
        score_topk(q, self.kmean, self.eligible, self.top_k, catalog=self.catalog,
                   table=self.plan.descs, table_slot0=self.slot0, idx_out=self.idx, score_out=self.scores,
                   staging=self.staging)

    def attend(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse: Optional[torch.Tensor] = None,
               q_pos: Optional[torch.Tensor] = None) -> None:
        """Attention over the table as it stands (slots as last selected)."""
        launch(self.plan, q, scale=scale, q_pos=q_pos, out=out, lse=lse)

    def step(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse: Optional[torch.Tensor] = None,
             q_pos: Optional[torch.Tensor] = None) -> None:
        if self.fused:
            launch(self.plan, q, scale=scale, q_pos=q_pos, out=out, lse=lse, select=self.select_cfg)
            return
        self.select(q)
        self.attend(q, scale=scale, out=out, lse=lse, q_pos=q_pos)



class RaggedTieredDecodeLayer:
    """Batched decode over per-sequence chunk tables (ragged contexts).

    ``rows[b] = (hot, cold)``: row b's hot chunks and cold chunks, each a
    ``ChunkRef`` with ``batch=b`` and ``(H_kv, T_c, D)`` tensors.  Every row
    selects its own ``top_k`` cold chunks by the mean-key score inside the
    attention launch (per-row selection over a ragged catalog), so one step
    is one ``halo_decode_attn_tiered`` plus its merge for the whole batch.

    Reference: the batch-uniform Triton kernel needs one call per sequence
    for ragged batches (halo/triton_chunked.py:171-177); here the chunk table
    carries per-row chunks (int32 work records) and a per-row selection.
    """

    def __init__(self, *, H: int, H_kv: int, D: int, dtype: torch.dtype, rows, top_k: int, device,
                 split: Optional[int] = None, cold_kmean: Optional[torch.Tensor] = None) -> None:
        """``cold_kmean`` (B, H_kv, max_cold, D): the cold chunks' page means,
        computed from the chunks when not given (needed when the chunks live
        in pinned host memory)."""
        from .decode import SlotRef
        B = len(rows)
        n_cold = [len(cold) for _, cold in rows]
        max_cold = max(n_cold)
        lim_cold, lim_triples = _sel_limits(dtype)
        if max_cold > lim_cold or max_cold * H_kv > lim_triples or H_kv * D > _SEL_MAX_QBAR or D % 16:
            raise AssertionError(f"per-row selection over {max_cold} cold chunks x {H_kv} KV heads (D={D}) exceeds "
                                 f"the in-kernel limits ({lim_cold} chunks, {lim_triples} rows, "
                                 f"H_kv * D <= {_SEL_MAX_QBAR}, D % 16 == 0)")
        if top_k < 1:
            raise AssertionError("top_k must be >= 1")
        for b, (hot, cold) in enumerate(rows):
            for c in list(hot) + list(cold):
                if c.batch != b:
                    raise AssertionError(f"row {b}: chunks must carry batch={b}")
        self.B, self.H, self.H_kv, self.D, self.dtype, self.top_k = B, H, H_kv, D, dtype, top_k
        self.rows = rows
        widest = max(c.T for _, cold in rows for c in cold) if max_cold else 0
        slots = [SlotRef(widest) for _ in range(top_k)]
        hot_all = [c for hot, _ in rows for c in hot]
        self.plan: DecodePlan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype, chunks=slots + hot_all,
                                           device=device, split=split, first=range(top_k))
        import numpy as np

        from .decode import DESC_DTYPE
        cat = np.zeros(B * max(max_cold, 1), dtype=DESC_DTYPE)
        for b, (_, cold) in enumerate(rows):
            if cold:
                d, keep = pack_descs(cold, B=B, H_kv=H_kv, D=D, dtype=dtype)
                cat[b * max_cold: b * max_cold + len(cold)] = d
                self.plan.keep += keep
        self.catalog = descs_to_device(cat, device)
        if cold_kmean is None:
            if any(c.k.device.type == "cpu" for _, cold in rows for c in cold):
                raise AssertionError("cold chunks in pinned host memory need cold_kmean (their page means on the GPU)")
            cold_kmean = torch.zeros((B, H_kv, max(max_cold, 1), D), device=device, dtype=dtype)
            for b, (_, cold) in enumerate(rows):
                for j, c in enumerate(cold):
                    chunk_means(c.k.unsqueeze(0), c.T, row0=0, n_pages=1, out=cold_kmean[b:b + 1], page_offset=j)
        if tuple(cold_kmean.shape) != (B, H_kv, max(max_cold, 1), D) or cold_kmean.dtype != dtype \
                or cold_kmean.stride(-1) != 1:
            raise AssertionError(f"cold_kmean must be ({B}, {H_kv}, {max(max_cold, 1)}, {D}) {dtype}")
        self.kmean = cold_kmean
        self.n_cold = torch.tensor(n_cold, dtype=torch.int32, device=device)
        self.idx = torch.empty((B, top_k), device=device, dtype=torch.int32)
        self.scores = torch.empty((B, max(max_cold, 1)), device=device, dtype=torch.float32)
        km = self.kmean
        self.select_cfg = nat.SelectCfg(
            kmean=km.data_ptr(), km_stride_b=km.stride(0), km_stride_h=km.stride(1), km_stride_p=km.stride(2),
            catalog=self.catalog.data_ptr(), catalog_stride=max(max_cold, 1), n_cold_per_sel=self.n_cold.data_ptr(),
            n_cold=max(max_cold, 1), top_k=top_k, slot0=0, per_row=1,
            idx_out=self.idx.data_ptr(), score_out=self.scores.data_ptr())

    def attended_rows(self) -> int:
        """K/V rows one step reads per KV head, summed over the batch (hot +
        the selected chunks, assuming each row fills its top_k)."""
        total = 0
        for hot, cold in self.rows:
            sizes = sorted((c.T for c in cold), reverse=True)
            total += sum(c.T for c in hot) + sum(sizes[: self.top_k])
        return total

    def step(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse: Optional[torch.Tensor] = None,
             q_pos: Optional[torch.Tensor] = None) -> None:
        launch(self.plan, q, scale=scale, q_pos=q_pos, out=out, lse=lse, select=self.select_cfg)
