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
import re
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


_OVERRIDE_TOKEN = re.compile(r"""'(?:\\.|[^'\\])*'|"(?:\\.|[^"\\])*"|[()\[\]{},]|[^'"()\[\]{},]+""")
_CLOSERS = {")": "(", "]": "[", "}": "{"}


def _split_top_level(s: str) -> list[str]:
    """Split on commas that are outside quotes and brackets."""
    parts, cur, stack = [], [], []
    for tok in _OVERRIDE_TOKEN.findall(s):
        if tok in "([{":
            stack.append(tok)
        elif tok in _CLOSERS and stack and stack[-1] == _CLOSERS[tok]:
            stack.pop()
        elif tok == "," and not stack:
            parts.append("".join(cur))
            cur = []
            continue
        cur.append(tok)
    parts.append("".join(cur))
    return [p.strip() for p in parts if p.strip()]


def parse_overrides(s: Optional[str] = None) -> dict[str, Any]:
    """Parse ``$HALO_OVERRIDES``-style ``key=value`` pairs (halo/policy.py:
    163-212): pairs are separated by commas outside quotes and brackets, each
    value is read as a Python literal when it is one (``0.05``, ``False``,
    ``['gpu','dram']``) and kept as its text otherwise; an item without
    ``=`` is ignored."""
    if s is None:
        s = os.environ.get("HALO_OVERRIDES", "")
    out: dict[str, Any] = {}
    for item in _split_top_level(s.strip()):
        key, eq, value = item.partition("=")
        if not eq:
            continue
        key, value = key.strip(), value.strip()
        try:
            out[key] = ast.literal_eval(value)
        except (ValueError, SyntaxError):
            out[key] = value
    return out


def _model_shape(model) -> tuple[int, int, int]:
    """(layers, KV heads, head dim) from a HF model config."""
    cfg = getattr(model, "config", None)
    if cfg is None:
        raise ValueError("`model.config` is missing; cannot wire HALO without architecture metadata.")

    def first(*names):
        for n in names:
            val = getattr(cfg, n, None)
            if val:
                return val
        return None

    n_layers = first("num_hidden_layers", "n_layer")
    n_kv = first("num_key_value_heads", "num_attention_heads")
    head_dim = first("head_dim") or cfg.hidden_size // cfg.num_attention_heads
    return int(n_layers), int(n_kv), int(head_dim)


def wrap_with_halo(model, config: Optional[HALOConfig] = None):
    """Attach HALO's tiered cache and its components to ``model`` in place
    (halo/policy.py:220-318): storage, scorer, demoter, refetcher, the cache
    (Path-D ``HALOCacheChunked`` with ``chunked=True``, else ``HALOCache``),
    a ``generate`` hook that hands the cache to every call, and with
    ``chunked=True`` the ``halo_chunked`` attention interface.  Returns the
    same model."""
    from .demoter import HALODemoter
    from .kv_cache import HALOCache
    from .kv_cache_chunked import HALOCacheChunked
    from .refetcher import HALORefetcher
    from .scorer import HALOScorer

    config = config or HALOConfig()
    env = parse_overrides()
    if env:
        config = config.with_overrides(env)
    n_layers, n_kv, head_dim = _model_shape(model)
    p = next(model.parameters())
    storage = config.make_storage(num_layers=n_layers, num_kv_heads=n_kv, head_dim=head_dim,
                                  dtype=p.dtype, device=p.device)
    scorer = HALOScorer(config)
    demoter = HALODemoter(config, storage=storage)
    refetcher = HALORefetcher(config, storage=storage)
    if config.chunked and config.eviction:
        raise ValueError("HALOConfig: `chunked` (Path D, lossless) and `eviction` (Path C, pruning) "
                         "are exclusive; enable one of them.")
    if config.eviction:
        raise NotImplementedError("the eviction cache (Path C) is not part of this build; use chunked=True")
    if config.chunked:
        cache = HALOCacheChunked(config=config, storage=storage, scorer=scorer, demoter=demoter,
                                 refetcher=refetcher, chunk_size=config.chunk_size,
                                 recent_window=config.recent_window, use_triton=bool(config.use_triton))
    else:
        cache = HALOCache(config=config, storage=storage, scorer=scorer, demoter=demoter, refetcher=refetcher)
    model._halo_config = config
    model._halo_cache = cache
    model._halo_scorer = scorer
    model._halo_demoter = demoter
    model._halo_refetcher = refetcher
    model._halo_storage = storage
    _install_generate_hook(model)
    if config.chunked:
        _install_chunked_attention_interface(model, cache)
    return model


def _one_shot_attention(module, query, key, value, attention_mask=None, scaling=None, **kwargs):
    """Warm-up attention over the full (K, V) the cache returned: the
    model's own SDPA interface when transformers has one (so warm-up is
    identical to the unwrapped SDPA model, halo/policy.py:406-447), else
    torch's SDPA with the mask.  Returns (B, T_q, H, D)."""
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        sdpa = ALL_ATTENTION_FUNCTIONS["sdpa"]
    except Exception:
        sdpa = None
    if sdpa is not None:
        out, _ = sdpa(module, query, key, value, attention_mask, dropout=0.0, scaling=scaling, **kwargs)
        return out
    import torch
    H, H_kv = query.shape[1], key.shape[1]
    if H != H_kv:
        key = key.repeat_interleave(H // H_kv, dim=1)
        value = value.repeat_interleave(H // H_kv, dim=1)
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    out = torch.nn.functional.scaled_dot_product_attention(
        query, key, value, attn_mask=attention_mask, dropout_p=0.0,
        is_causal=attention_mask is None and query.shape[-2] > 1, scale=scaling)
    return out.transpose(1, 2).contiguous()


def halo_chunked_attention(module, query, key, value, attention_mask=None, dropout=0.0, scaling=None, **kwargs):
    """The ``halo_chunked`` attention function (halo/policy.py:352-373).

    In warm-up mode the cache returned every row, so this is one-shot
    attention with the model's mask (padding included).  In chunked mode
    ``key``/``value`` are only the GPU rows; the cache attends its cold
    chunks and GPU rows by global position.  Returns ``(out (B, T_q, H, D),
    None)``."""
    cache = getattr(module, "_halo_cache", None)
    if cache is None:
        raise RuntimeError("halo_chunked attention called on a module without a HALO cache")
    if getattr(cache, "_mode", "chunked") == "warmup":
        return _one_shot_attention(module, query, key, value, attention_mask=attention_mask,
                                   scaling=scaling, **kwargs), None
    out = cache.compute_attention(query, layer_idx=module.layer_idx, scaling=scaling)
    return out.transpose(1, 2).contiguous(), None


def _install_generate_hook(model) -> None:
    """Make ``model.generate`` hand the HALO cache to every call that passes
    no cache of its own, resetting the HALO cache unless the caller passes
    that cache itself (an already filled cache from a chunked prefill); a
    caller's own ``past_key_values`` is kept (halo/policy.py:450-478)."""
    if getattr(model, "_halo_generate_patched", False) or not hasattr(model, "generate"):
        return
    inner = model.generate

    def generate(*args, **kwargs):
        cache = model._halo_cache
        if kwargs.get("past_key_values") is not cache:
            cache.reset()
            if kwargs.get("past_key_values") is None:
                kwargs["past_key_values"] = cache
        kwargs.setdefault("use_cache", True)
        return inner(*args, **kwargs)

    model.generate = generate
    model._halo_generate_patched = True


def _install_chunked_attention_interface(model, cache) -> None:
    """Register ``halo_chunked`` in transformers' attention registry and
    switch the model and its submodules to it; point every attention module
    at the cache."""
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    except Exception:  # transformers absent: the modules still carry the cache
        ALL_ATTENTION_FUNCTIONS = None
    if ALL_ATTENTION_FUNCTIONS is not None:
        ALL_ATTENTION_FUNCTIONS["halo_chunked"] = halo_chunked_attention
        try:  # warm-up attention is SDPA, so the model builds SDPA-format masks for it
            from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
            ALL_MASK_ATTENTION_FUNCTIONS.register("halo_chunked", ALL_MASK_ATTENTION_FUNCTIONS["sdpa"])
        except Exception:
            pass
        for mod in [model] + list(model.modules()):
            cfg = getattr(mod, "config", None)
            if cfg is not None:
                try:
                    cfg._attn_implementation = "halo_chunked"
                except Exception:
                    pass
    for mod in model.modules():
        if hasattr(mod, "layer_idx"):
            mod._halo_cache = cache
