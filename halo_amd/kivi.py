"""KIVI-style 2/4/8-bit cold-chunk format on the GPU.

``quantize(k, v)`` packs K (per channel over 32 tokens) and V (per token
over 32 channels) into self-contained 32-token blocks; ``dequantize``
restores them bit-exactly to the storage dtype; ``KiviChunkRef`` puts a run
of blocks into a decode chunk table, where the attention kernel dequantises
them in registers.

Reference: ``_quantize_per_group`` / ``_dequantize_per_group`` and the
quantised-buffer policy of ``KIVICache.update``
(baselines/kivi_cache.py:44-78, :121-195).  The reference keeps unpacked int8
codes; the packed block layout (include/halo_hip.h) is this library's.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as nat

GROUP = 32
# rows per work item of the unquantised recent rows in a KIVI launch
RECENT_ITEM_ROWS = 32


def block_bytes(D: int, bits: int = 2) -> int:
    n = int(nat.lib().halo_kivi_block_bytes(D, bits))
    if n == 0:
        raise AssertionError(f"unsupported KIVI shape D={D} bits={bits}")
    return n


def _check(t: torch.Tensor, name: str) -> None:
    if t.dim() != 4 or t.stride(-1) != 1:
        raise AssertionError(f"{name} must be (B, H_kv, T, D) with unit last stride")
    if t.dtype not in (torch.float16, torch.bfloat16):
        raise AssertionError(f"{name}: KIVI storage dtype must be float16 or bfloat16, got {t.dtype}")
    if not t.is_cuda:
        raise AssertionError(f"{name} must be a device tensor")


def quantize(k: torch.Tensor, v: torch.Tensor, *, bits: int = 2, out: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """(B, H_kv, T, D) K and V -> uint8 blocks (B, H_kv, T/32, block_bytes)."""
    _check(k, "k")
    _check(v, "v")
    if k.shape != v.shape or k.dtype != v.dtype:
        raise AssertionError(f"k {tuple(k.shape)} {k.dtype} and v {tuple(v.shape)} {v.dtype} must match")
    B, H, T, D = k.shape
    if T % GROUP:
        raise AssertionError(f"T={T} must be a multiple of the group size {GROUP}")
    nb = block_bytes(D, bits)
    if out is None:
        out = torch.empty((B, H, T // GROUP, nb), device=k.device, dtype=torch.uint8)
    elif out.shape != (B, H, T // GROUP, nb) or out.dtype != torch.uint8 or out.stride(-1) != 1 \
            or out.stride(-2) != nb:
        raise AssertionError(f"out must be uint8 ({B}, {H}, {T // GROUP}, {nb}) with contiguous blocks")
    nat.check(nat.lib().halo_kivi_quantize(
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        nat.dtype_code(k.dtype), B, H, T, D, bits,
        out.data_ptr(), out.stride(0), out.stride(1), nat.stream_ptr(stream)), "halo_kivi_quantize")
    return out


def dequantize(blocks: torch.Tensor, *, D: int, dtype: torch.dtype, bits: int = 2, stream=None):
    """uint8 blocks (B, H_kv, n, block_bytes) -> (k, v) (B, H_kv, 32n, D)."""
    B, H, n, nb = blocks.shape
    if nb != block_bytes(D, bits) or blocks.dtype != torch.uint8 or blocks.stride(-1) != 1 \
            or blocks.stride(-2) != nb:
        raise AssertionError("blocks must be uint8 (B, H_kv, n, block_bytes) with contiguous blocks")
    k = torch.empty((B, H, n * GROUP, D), device=blocks.device, dtype=dtype)
    v = torch.empty_like(k)
    nat.check(nat.lib().halo_kivi_dequantize(
        blocks.data_ptr(), blocks.stride(0), blocks.stride(1), nat.dtype_code(dtype), B, H, n, D, bits,
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), nat.stream_ptr(stream)), "halo_kivi_dequantize")
    return k, v


@dataclass
class KiviChunkRef:
    """A run of KIVI blocks as one decode chunk: ``blocks`` (B, H_kv, n, nb)
    covering tokens [chunk_start, chunk_start + 32n)."""

    blocks: torch.Tensor
    chunk_start: int
    causal: bool = True
    bits: int = 2
    batch: int = -1  # >= 0: blocks are (H_kv, n, nb) of that batch row only

    @property
    def T(self) -> int:
        return int(self.blocks.shape[2]) * GROUP


def plan_kivi(*, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype, cold, recent, device, split=None):
    """The work plan of one KIVI decode launch: the KIVI block runs
    ``cold`` (``KiviChunkRef``) in items of ``split`` tokens (default: about
    two per resident workgroup slot), then the unquantised ``recent`` rows
    (``decode.ChunkRef``) in items of ``RECENT_ITEM_ROWS``.

    The KIVI items fill the resident workgroup slots in the first round; the
    short recent-row items go last, into the slots that free up first,
    instead of holding back a KIVI item to a second round.  They are cut into
    32-row items (one plain tile each): they start when the first KIVI items
    end and are latency-bound, so more, shorter items end sooner (131072-token
    layer: 22.3 -> 21.6 us against one 128-row item per KV head)."""
    from .decode import _num_cus, build_plan, choose_rep_t, choose_split
    chunks = list(cold) + list(recent)
    if not cold:  # no KIVI blocks yet: a plain decode launch
        return build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype, chunks=chunks, device=device, split=split)
    if split is None:
        n_sub = -(-(H // H_kv) // choose_rep_t(H // H_kv))
        rows = sum(int(c.T) for c in chunks) * B * H_kv * n_sub
        split = choose_split(rows, _num_cus(device), kivi=True)
    return build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype, chunks=chunks, device=device,
                      split=RECENT_ITEM_ROWS, first=range(len(cold)), split_first=split)


class KiviDecodeLayer:
    """Decode over a KIVI-quantised cold region plus unquantised recent rows.

    ``cold_blocks`` (B, H_kv, n, block_bytes) hold tokens [0, 32n) (from
    :func:`quantize`); ``recent`` are plain ``decode.ChunkRef`` chunks after
    them.  One step is one attention launch plus its merge: the KIVI blocks
    and the recent rows are work items of the same table -- the
    quantised-buffer-plus-residual split of KIVICache.update
    (baselines/kivi_cache.py:137-195) without materialising the dequantised
    cache.
    """

    def __init__(self, *, B: int, H: int, H_kv: int, D: int, dtype: torch.dtype, cold_blocks: torch.Tensor,
                 recent, device, chunk_tokens: int = 2048, split=None) -> None:
        if chunk_tokens % GROUP:
            raise AssertionError(f"chunk_tokens={chunk_tokens} must be a multiple of {GROUP}")
        n = int(cold_blocks.shape[2])
        per = chunk_tokens // GROUP
        cold = [KiviChunkRef(cold_blocks[:, :, j:min(j + per, n)], j * GROUP, True) for j in range(0, n, per)]
        self.B, self.H, self.D = B, H, D
        self.plan = plan_kivi(B=B, H=H, H_kv=H_kv, D=D, dtype=dtype, cold=cold, recent=list(recent or []),
                              device=device, split=split)

    def step(self, q: torch.Tensor, *, scale: float, out: torch.Tensor, lse=None, q_pos=None) -> None:
        from .decode import launch
        launch(self.plan, q, scale=scale, q_pos=q_pos, out=out, lse=lse)