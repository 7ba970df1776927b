"""halo_amd -- MI355X-native tiered-KV chunked attention (HALO "Path D").

Public API mirrors the reference package ``halo`` (halo/__init__.py:32-54)
for the tiered-KV path: ``HALOConfig``, ``wrap_with_halo``,
``HALOCache``, ``HALOCacheChunked``, ``HALOScorer``, ``HALODemoter``,
``HALORefetcher``, ``MemoryTier``, ``TieredStorage``, and the chunked-prefill
driver (``prefill_then_generate``, ``install_preforward_peel``); the kernel
module keeps the name and call
signatures of ``halo.triton_chunked``.  Compute runs in hand-written HIP
kernels for gfx950 (``halo_amd/csrc``) behind the C-ABI in
``include/halo_hip.h``.
"""
from . import _native
from .chunked_prefill import install_preforward_peel, prefill_then_generate  # noqa: F401
from .demoter import HALODemoter  # noqa: F401
from .kv_cache import HALOCache  # noqa: F401
from .kv_cache_chunked import HALOCacheChunked  # noqa: F401
from .memory_tier import MemoryTier, TieredStorage  # noqa: F401
from .policy import HALOConfig, parse_overrides, wrap_with_halo  # noqa: F401
from .refetcher import HALORefetcher  # noqa: F401
from .scorer import HALOScorer  # noqa: F401
from .triton_chunked import (  # noqa: F401
    HAS_HIP,
    HAS_TRITON,
    finalize,
    init_acc,
    lse_merge,
    triton_chunked_attention,
    triton_chunked_attention_single_launch,
    triton_chunked_attention_streamed,
    update_chunk,
)

__version__ = "0.1.0"
