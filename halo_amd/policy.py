"""User-facing configuration and the model wrapper.

Reference: halo/policy.py:38-160 (HALOConfig with make_storage /
with_overrides), :163-217 (parse_overrides), :220-318 (wrap_with_halo) and
:321-395 (the ``halo_chunked`` attention interface).  Field names, defaults
and meaning are kept so that configurations and ``$HALO_OVERRIDES`` strings
written for the reference work unchanged.
"""
from __future__ import annotations

import ast
import os
from dataclasses import dataclass, field, replace
from typing import Any, Optional, Sequence

from .memory_tier import MemoryTier, TieredStorage


@dataclass
class HALOConfig:
    """HALO knobs (defaults as in halo/policy.py:38-126)."""

    hot_ratio: float = 0.10
    score_alpha: float = 1.0
    score_beta: float = 0.5
    score_gamma: float = 2.0
    sink_tokens: int = 4
    refresh_window: int = 64
    tiers: Sequence[str] = ("gpu", "dram")
    block_size: int = 32
    nvme_path: Optional[str] = None
    async_refetch: bool = True
    lookahead: int = 1
    layerwise_budget: str = "uniform"
    eviction: bool = False
    chunked: bool = False
    chunk_size: int = 512
    recent_window: int = 64
    use_triton: bool = False
    log_dir: Optional[str] = None
    extra: dict = field(default_factory=dict)

    def make_storage(self, *, num_layers: int, num_kv_heads: int, head_dim: int, dtype, device) -> TieredStorage:
        return TieredStorage(tiers=[MemoryTier.from_name(t) for t in self.tiers], num_layers=num_layers,
                             num_kv_heads=num_kv_heads, head_dim=head_dim, block_size=self.block_size,
                             dtype=dtype, device=device, nvme_path=self.nvme_path)

    def with_overrides(self, overrides: dict) -> "HALOConfig":
        valid = set(self.__dataclass_fields__)
        clean = {k: v for k, v in overrides.items() if k in valid}
        extras = {k: v for k, v in overrides.items() if k not in valid}
        if extras:
            clean["extra"] = {**self.extra, **extras}
        return replace(self, **clean)


def parse_overrides(s: Optional[str] = None) -> dict[str, Any]:
    """``"k1=v1,k2=v2"`` -> dict; values through ``ast.literal_eval`` when
    possible; commas inside brackets or quotes are kept (halo/policy.py:163-217)."""
    if s is None:
        s = os.environ.get("HALO_OVERRIDES", "").strip()
    if not s:
        return {}
    pairs, buf, depth, quote = [], [], 0, None
    for ch in s:
        if quote:
            buf.append(ch)
            if ch == quote and (len(buf) < 2 or buf[-2] != "\\"):
                quote = None
            continue
        if ch in ("'", '"'):
            quote = ch
        elif ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        elif ch == "," and depth == 0:
            pairs.append("".join(buf).strip())
            buf = []
            continue
        buf.append(ch)
    if buf:
        pairs.append("".join(buf).strip())
    out: dict[str, Any] = {}
    for kv in pairs:
        if "=" not in kv:
            continue
        k, v = (x.strip() for x in kv.split("=", 1))
        try:
            out[k] = ast.literal_eval(v)
        except (ValueError, SyntaxError):
            out[k] = v
    return out


def wrap_with_halo(model, config: Optional[HALOConfig] = None):
    """Attach HALO's tiered cache and its components to ``model`` in place
    (halo/policy.py:220-318): storage, scorer, demoter, refetcher and, with
    ``chunked=True``, the Path-D cache and the ``halo_chunked`` attention
    interface.  Returns the same model."""
    from .demoter import HALODemoter
    from .kv_cache_chunked import HALOCacheChunked
    from .refetcher import HALORefetcher
    from .scorer import HALOScorer

    config = config or HALOConfig()
    env = parse_overrides()
    if env:
        config = config.with_overrides(env)
    cfg_obj = getattr(model, "config", None)
    if cfg_obj is None:
        raise ValueError("`model.config` is missing; cannot wire HALO without architecture metadata.")
    num_layers = getattr(cfg_obj, "num_hidden_layers", None) or getattr(cfg_obj, "n_layer")
    num_kv_heads = getattr(cfg_obj, "num_key_value_heads", None) or getattr(cfg_obj, "num_attention_heads")
    head_dim = getattr(cfg_obj, "head_dim", None) or cfg_obj.hidden_size // cfg_obj.num_attention_heads
    p = next(model.parameters())
    storage = config.make_storage(num_layers=num_layers, num_kv_heads=num_kv_heads, head_dim=head_dim,
                                  dtype=p.dtype, device=p.device)
    scorer = HALOScorer(config)
    demoter = HALODemoter(config, storage=storage)
    refetcher = HALORefetcher(config, storage=storage)
    if config.chunked and config.eviction:
        raise ValueError("HALOConfig: cannot enable both `chunked` (Path D) and `eviction` (Path C).")
    cache = None
    if config.chunked:
        cache = HALOCacheChunked(config=config, storage=storage, scorer=scorer, demoter=demoter,
                                 refetcher=refetcher, chunk_size=config.chunk_size,
                                 recent_window=config.recent_window, use_triton=True)
        _install_chunked_attention_interface(model, cache)
    model._halo_config = config
    model._halo_cache = cache
    model._halo_scorer = scorer
    model._halo_demoter = demoter
    model._halo_refetcher = refetcher
    model._halo_storage = storage
    return model


def halo_chunked_attention(module, query, key, value, attention_mask=None, dropout=0.0, scaling=None, **kwargs):
    """The ``halo_chunked`` attention function (halo/policy.py:352-373):
    (B, H, T_q, D) query against the cache's cold chunks and recent rows;
    returns ``(out (B, T_q, H, D), None)``."""
    cache = getattr(module, "_halo_cache", None)
    if cache is None:
        raise RuntimeError("halo_chunked attention called on a module without a HALO cache")
    out = cache.compute_attention(query, module.layer_idx, scaling=scaling)
    return out.transpose(1, 2).contiguous(), None


def _install_chunked_attention_interface(model, cache) -> None:
    """Register ``halo_chunked`` in transformers' attention registry (when
    transformers is importable) and point the model's attention modules at
    the cache."""
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        ALL_ATTENTION_FUNCTIONS["halo_chunked"] = halo_chunked_attention
        if getattr(model, "config", None) is not None:
            model.config._attn_implementation = "halo_chunked"
    except Exception:  # transformers absent or without the registry
        pass
    for mod in getattr(model, "modules", lambda: [])():
        if hasattr(mod, "layer_idx"):
            mod._halo_cache = cache
