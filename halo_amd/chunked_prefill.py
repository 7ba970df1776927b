"""Chunked prefill then decode through the Path-D cache.

Reference: ``prefill_then_generate`` (halo/chunked_prefill.py:73-205) and
``install_preforward_peel`` (halo/preforward_peel.py:41-117).  A long prompt
is fed to the model in slices; after each slice every layer's GPU rows
beyond the recent window are peeled to the pinned cold tier, so GPU-resident
K/V stays bounded by one slice plus the recent window.  Each slice's
attention (T_q > 1) is the cache's ``compute_attention``: the cold chunks
staged behind the peel's copy event plus the GPU rows, causal by global
position, in one prefill launch.  Decoding then proceeds token by token with
the same cache (greedy or sampled), peeling as the recent rows grow.

The cache's ``get_seq_length`` reports cold + GPU rows, so the model's
``cache_position`` (and RoPE) keep the true positions.
"""
from __future__ import annotations

from typing import Any, Optional

import torch


def _peel_all_layers(cache) -> None:
    """Peel every layer whose GPU rows exceed the recent window."""
    for li, _, k, _ in list(cache._iter_layer_kv()):
        if k is not None and k.numel() and k.shape[-2] > cache.recent_window:
            cache._peel_to_cold(li)


def _pick(logits: torch.Tensor, do_sample: bool, temperature: float, top_p: float,
          generator: Optional[torch.Generator]) -> torch.Tensor:
    """Next token (B, 1): argmax, or a draw from the temperature / nucleus
    filtered distribution.  The nucleus keeps the sorted tokens whose
    cumulative probability is at most ``top_p``, and always the most likely
    one (halo/chunked_prefill.py:150-163)."""
    if not do_sample:
        return logits.argmax(dim=-1, keepdim=True)
    probs = torch.softmax(logits.float() / max(temperature, 1e-6), dim=-1)
    if top_p < 1.0:
        p_sorted, order = probs.sort(dim=-1, descending=True)
        drop = p_sorted.cumsum(dim=-1) > top_p
        drop[..., 0] = False
        p_sorted = torch.where(drop, torch.zeros_like(p_sorted), p_sorted)
        p_sorted = p_sorted / p_sorted.sum(dim=-1, keepdim=True)
        return order.gather(-1, torch.multinomial(p_sorted, 1, generator=generator))
    return torch.multinomial(probs, 1, generator=generator)


@torch.no_grad()
def prefill_then_generate(model, input_ids: torch.Tensor, *, prefill_chunk_tokens: int = 1024,
                          max_new_tokens: int = 32, do_sample: bool = False, temperature: float = 1.0,
                          top_p: float = 1.0, attention_mask: Optional[torch.Tensor] = None,
                          generator: Optional[torch.Generator] = None) -> dict:
    """Slice-by-slice prefill of ``input_ids`` (1, T) through a model wrapped
    with ``wrap_with_halo(..., HALOConfig(chunked=True))``, then
    ``max_new_tokens`` decode steps.  Returns the generated ids, the
    per-step logits, peak GPU memory of both phases and the cache
    telemetry (halo/chunked_prefill.py:194-205)."""
    cache = getattr(model, "_halo_cache", None)
    if cache is None or not hasattr(cache, "_peel_to_cold"):
        raise ValueError("prefill_then_generate needs a model wrapped with HALOConfig(chunked=True)")
    if input_ids.dim() != 2 or input_ids.shape[0] != 1:
        raise AssertionError("chunked prefill takes one sequence: input_ids (1, T)")
    if attention_mask is not None and not bool(attention_mask.all()):
        raise AssertionError("chunked prefill attends every prompt token; a padding mask is not supported")
    dev = input_ids.device
    cuda = dev.type == "cuda"
    cache.reset()
    cache._mode = "chunked"
    T = input_ids.shape[-1]
    step = max(1, int(prefill_chunk_tokens))
    if cuda:
        torch.cuda.reset_peak_memory_stats(dev)
    logits = None
    for a in range(0, T, step):
        b = min(a + step, T)
        out = model(input_ids=input_ids[:, a:b], past_key_values=cache,
                    cache_position=torch.arange(a, b, device=dev), use_cache=True, return_dict=True)
        if b == T:
            logits = out.logits[:, -1, :].clone()
        del out
        _peel_all_layers(cache)
    prefill_peak = torch.cuda.max_memory_allocated(dev) / 2**30 if cuda else 0.0
    if cuda:
        torch.cuda.reset_peak_memory_stats(dev)
    tokens, step_logits = [], []
    for _ in range(max_new_tokens):
        step_logits.append(logits)
        nxt = _pick(logits, do_sample, temperature, top_p, generator)
        tokens.append(nxt)
        pos = cache.get_seq_length()
        out = model(input_ids=nxt, past_key_values=cache, cache_position=torch.tensor([pos], device=dev),
                    use_cache=True, return_dict=True)
        logits = out.logits[:, -1, :].clone()
        del out
        _peel_all_layers(cache)
    decode_peak = torch.cuda.max_memory_allocated(dev) / 2**30 if cuda else 0.0
    return {
        "generated_ids": torch.cat([input_ids] + tokens, dim=-1),
        "prefill_peak_gib": prefill_peak,
        "decode_peak_gib": decode_peak,
        "overall_peak_gib": max(prefill_peak, decode_peak),
        "cache_telemetry": cache.telemetry(),
        "step_logits": step_logits,
    }


class PreforwardPeelResult:
    """What the patched ``generate`` returns for a long prompt: the ids as
    ``.sequences`` (and by indexing, like a plain tensor) plus the chunked
    prefill record as ``.halo_telemetry`` (halo/preforward_peel.py:120-150)."""

    def __init__(self, sequences: torch.Tensor, telemetry: dict) -> None:
        self.sequences = sequences
        self.halo_telemetry = telemetry

    def __getitem__(self, idx):
        return self.sequences[idx]

    def __len__(self) -> int:
        return len(self.sequences)

    @property
    def shape(self):
        return self.sequences.shape


def install_preforward_peel(model, *, prefill_chunk_tokens: int = 4096, activation_threshold: int = 8192):
    """Route ``model.generate`` calls with prompts longer than
    ``activation_threshold`` tokens through :func:`prefill_then_generate`
    (shorter prompts use the original ``generate``).  Needs a model wrapped
    with ``chunked=True``; idempotent (halo/preforward_peel.py:41-117)."""
    cfg = getattr(model, "_halo_config", None)
    if cfg is None or not cfg.chunked:
        raise ValueError("install_preforward_peel needs wrap_with_halo(model, HALOConfig(chunked=True)) first")
    if getattr(model, "_halo_preforward_patched", False):
        return model
    inner = model.generate

    def generate(*args: Any, **kwargs: Any):
        ids = kwargs.get("input_ids", args[0] if args else None)
        if ids is None or ids.shape[-1] <= activation_threshold:
            return inner(*args, **kwargs)
        res = prefill_then_generate(model, ids, prefill_chunk_tokens=prefill_chunk_tokens,
                                    max_new_tokens=kwargs.get("max_new_tokens", 32),
                                    do_sample=kwargs.get("do_sample", False),
                                    temperature=kwargs.get("temperature", 1.0), top_p=kwargs.get("top_p", 1.0),
                                    attention_mask=kwargs.get("attention_mask"))
        return PreforwardPeelResult(res["generated_ids"], res)

    model.generate = generate
    model._halo_preforward_patched = True
    model._halo_preforward_chunk = prefill_chunk_tokens
    model._halo_preforward_threshold = activation_threshold
    return model
