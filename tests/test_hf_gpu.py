"""Path D inside a HuggingFace model on the GPU: a tiny randomly initialised
Qwen2 (GQA 4/2, built from a local Qwen2Config, no download) wrapped with
``wrap_with_halo(chunked=True)`` against the same weights with plain full
attention (reference tests/test_path_d_identity_chunked.py:71-138 and
tests/test_chunked_wrap_integration.py).

* chunked prefill (``prefill_then_generate``) with cold chunks in pinned
  host memory: next-token logits within 5e-4 of full attention in fp32,
  argmax unchanged, and every decode step's logits within 5e-4 of a full
  recomputation over the same tokens;
* ``model.generate`` through the installed hook: warm-up prefill (SDPA),
  the transition peel on the first decode token, then chunked decode;
* ``install_preforward_peel`` routes a long prompt through chunked prefill;
* bf16 end to end within a bf16-sized bound.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers", reason="transformers is not importable on this machine")


def _models(dev, dtype):
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config
    # head_dim 64: the decode and prefill kernels are built for head dims 64 / 128.  Each model
    # gets its own config object: wrapping switches the wrapped model's attention implementation.
    def cfg():
        return Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                           num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                           rope_theta=10000.0, tie_word_embeddings=False, attn_implementation="eager")
    torch.manual_seed(0)
    ref = AutoModelForCausalLM.from_config(cfg()).eval()
    torch.manual_seed(0)
    halo = AutoModelForCausalLM.from_config(cfg()).eval()
    halo.load_state_dict(ref.state_dict())
    return ref.to(dev, dtype), halo.to(dev, dtype)


def _prompt(dev, n):
    g = torch.Generator().manual_seed(1)
    return torch.randint(10, 500, (1, n), generator=g).to(dev)


@torch.no_grad()
def _full_logits(model, ids):
    return model(ids, use_cache=False).logits[:, -1, :].float()


@pytest.mark.parametrize("hot_ratio,chunk_size,recent_window", [(0.5, 32, 8), (0.25, 16, 4)])
def test_chunked_prefill_identity_fp32(dev, hot_ratio, chunk_size, recent_window):
    from halo_amd import HALOConfig, prefill_then_generate, wrap_with_halo
    ref, halo = _models(dev, torch.float32)
    prompt = _prompt(dev, 256)
    want = _full_logits(ref, prompt)
    wrap_with_halo(halo, HALOConfig(hot_ratio=hot_ratio, chunked=True, chunk_size=chunk_size,
                                    recent_window=recent_window))
    res = prefill_then_generate(halo, prompt, prefill_chunk_tokens=64, max_new_tokens=4)
    cache = halo._halo_cache
    assert cache._mode == "chunked" and cache._cold[0].rows > 0
    assert cache.get_seq_length() == 256 + 4
    got = res["step_logits"][0].float()
    assert (got - want).abs().max().item() < 5e-4
    assert torch.equal(got.argmax(-1), want.argmax(-1))
    ids = res["generated_ids"]
    for i in range(1, 4):
        w = _full_logits(ref, ids[:, :256 + i])
        assert (res["step_logits"][i].float() - w).abs().max().item() < 5e-4


def test_generate_hook_decodes_through_the_cold_tier(dev):
    from halo_amd import HALOConfig, wrap_with_halo
    ref, halo = _models(dev, torch.float32)
    prompt = _prompt(dev, 200)
    wrap_with_halo(halo, HALOConfig(chunked=True, chunk_size=32, recent_window=8))
    out = halo.generate(prompt, max_new_tokens=6, do_sample=False, output_logits=True,
                        return_dict_in_generate=True, pad_token_id=0)
    cache = halo._halo_cache
    assert cache._mode == "chunked" and cache._cold[0].rows > 0
    seq = out.sequences
    for i, lg in enumerate(out.logits):
        w = _full_logits(ref, seq[:, :200 + i])
        assert (lg.float() - w).abs().max().item() < 5e-4, f"decode step {i}"


def test_preforward_peel_routes_long_prompts(dev):
    from halo_amd import HALOConfig, install_preforward_peel, wrap_with_halo
    ref, halo = _models(dev, torch.float32)
    prompt = _prompt(dev, 300)
    wrap_with_halo(halo, HALOConfig(chunked=True, chunk_size=32, recent_window=8))
    install_preforward_peel(halo, prefill_chunk_tokens=128, activation_threshold=256)
    res = halo.generate(input_ids=prompt, max_new_tokens=3)
    assert hasattr(res, "halo_telemetry") and res.shape == (1, 303)
    tel = res.halo_telemetry
    w = _full_logits(ref, prompt)
    assert (tel["step_logits"][0].float() - w).abs().max().item() < 5e-4
    assert tel["cache_telemetry"]["cold_layers"] == 2


def test_chunked_prefill_bf16(dev):
    from halo_amd import HALOConfig, prefill_then_generate, wrap_with_halo
    ref, halo = _models(dev, torch.bfloat16)
    prompt = _prompt(dev, 256)
    want = _full_logits(ref, prompt)
    wrap_with_halo(halo, HALOConfig(chunked=True, chunk_size=32, recent_window=8))
    res = prefill_then_generate(halo, prompt, prefill_chunk_tokens=64, max_new_tokens=2)
    got = res["step_logits"][0].float()
    # bf16 activations are rounded at every layer on both sides; the two
    # attention implementations round differently, so the bound is bf16-sized
    assert (got - want).abs().max().item() < 0.1 * max(1.0, want.abs().max().item())
