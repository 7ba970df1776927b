"""Host-side components on the CPU: configuration and overrides, tier
storage, refetch/demote bookkeeping, the Path-D cache's peel and the model
wrapper (expectations of the reference's own tests: test_policy.py,
test_overrides.py, test_memory_tier.py, test_refetcher.py:22-43,
test_demoter.py).  No kernel is launched here."""
from __future__ import annotations

import pytest
import torch


def test_default_config_matches_reference_defaults():
    from halo_amd import HALOConfig
    cfg = HALOConfig()
    assert cfg.hot_ratio == 0.10 and cfg.refresh_window == 64 and cfg.sink_tokens == 4
    assert "gpu" in cfg.tiers and "dram" in cfg.tiers
    assert (cfg.score_alpha, cfg.score_beta, cfg.score_gamma) == (1.0, 0.5, 2.0)
    assert (cfg.block_size, cfg.chunk_size, cfg.recent_window, cfg.lookahead) == (32, 512, 64, 1)


def test_make_storage_returns_tiered_storage():
    from halo_amd import HALOConfig, TieredStorage
    cfg = HALOConfig(tiers=("gpu", "dram"))
    st = cfg.make_storage(num_layers=2, num_kv_heads=2, head_dim=8, dtype=torch.float32, device=torch.device("cpu"))
    assert isinstance(st, TieredStorage) and st.num_layers == 2 and st.block_size == cfg.block_size


@pytest.mark.parametrize("text,want", [
    ("hot_ratio=0.05,score_alpha=1.0", {"hot_ratio": 0.05, "score_alpha": 1.0}),
    ("tiers=['gpu','dram','nvme'],async_refetch=False", {"tiers": ["gpu", "dram", "nvme"], "async_refetch": False}),
    ("layerwise_budget=pyramid", {"layerwise_budget": "pyramid"}),
    ("", {}), ("   ", {}),
    ("extra={'a': 1, 'b': [2, 3]},note='x,y'", {"extra": {"a": 1, "b": [2, 3]}, "note": "x,y"}),
])
def test_parse_overrides(text, want):
    from halo_amd import parse_overrides
    assert parse_overrides(text) == want


def test_with_overrides_and_env(monkeypatch):
    from halo_amd import HALOConfig, parse_overrides
    cfg = HALOConfig()
    new = cfg.with_overrides({"hot_ratio": 0.30, "lookahead": 4, "some_research_knob": 0.5})
    assert new.hot_ratio == 0.30 and new.lookahead == 4 and new.extra == {"some_research_knob": 0.5}
    assert cfg.hot_ratio == 0.10 and cfg.extra == {}
    monkeypatch.setenv("HALO_OVERRIDES", "hot_ratio=0.20,sink_tokens=8")
    assert parse_overrides() == {"hot_ratio": 0.20, "sink_tokens": 8}


def test_storage_directory_and_moves(storage_factory):
    st = storage_factory()
    assert st.locate_block(layer=0, block=0) == "gpu"
    bs = st.block_size
    keys = torch.arange(2 * bs * 8, dtype=torch.float32).reshape(2, bs, 8)
    values = torch.zeros_like(keys) - 1
    st.write_new_block(layer=0, block=1, keys=keys, values=values, tier="gpu")
    st.move_block(layer=0, block=1, src="gpu", dst="dram")
    assert st.locate_block(layer=0, block=1) == "dram"
    rk, rv = st.read_block(layer=0, block=1)
    torch.testing.assert_close(rk, keys)
    torch.testing.assert_close(rv, values)
    st.move_block(layer=0, block=0, src="gpu", dst="gpu")
    assert st.locate_block(layer=0, block=0) == "gpu"
    with pytest.raises(ValueError):
        st.write_new_block(layer=0, block=2, keys=keys, values=values, tier="nvme")


def test_nvme_tier_round_trip(tmp_path):
    from halo_amd import MemoryTier, TieredStorage
    st = TieredStorage(tiers=[MemoryTier.GPU, MemoryTier.DRAM, MemoryTier.NVME], num_layers=2, num_kv_heads=2,
                       head_dim=8, block_size=4, dtype=torch.bfloat16, device=torch.device("cpu"),
                       nvme_path=str(tmp_path), max_blocks=8)
    keys = torch.randn(2, 4, 8).to(torch.bfloat16)
    values = torch.randn(2, 4, 8).to(torch.bfloat16)
    st.write_new_block(layer=1, block=5, keys=keys, values=values, tier="gpu")
    st.move_block(layer=1, block=5, src="gpu", dst="nvme")
    assert st.locate_block(layer=1, block=5) == "nvme"
    rk, rv = st.read_block(layer=1, block=5)
    assert torch.equal(rk, keys) and torch.equal(rv, values)


def test_refetch_schedule_counts_hits_and_misses(small_config, storage_factory):
    from halo_amd import HALORefetcher
    st = storage_factory()
    bs = st.block_size
    for blk, tier in ((0, "gpu"), (1, "dram")):
        st.write_new_block(layer=0, block=blk, keys=torch.randn(2, bs, 8), values=torch.randn(2, bs, 8), tier=tier)
    r = HALORefetcher(small_config, storage=st)
    r.schedule(layer=0, predicted_indices=[0, 1, 4, 5])
    assert (r.hits, r.misses) == (1, 1)
    assert st.locate_block(layer=0, block=1) == "gpu"
    r.schedule(layer=0, predicted_indices=torch.tensor([0, 4]))
    assert (r.hits, r.misses) == (3, 1)


def test_demote_flush_and_tensor_indices(small_config, storage_factory):
    from halo_amd import HALODemoter
    st = storage_factory()
    bs = st.block_size
    for blk in (0, 1, 2):
        st.write_new_block(layer=0, block=blk, keys=torch.randn(2, bs, 8), values=torch.randn(2, bs, 8), tier="gpu")
    d = HALODemoter(small_config, storage=st)
    d.demote(layer=0, block_indices=[0, 1], src="gpu", dst="dram")
    d.demote(layer=0, block_indices=torch.tensor([2]), src="gpu", dst="dram")
    assert [st.locate_block(layer=0, block=b) for b in (0, 1, 2)] == ["dram"] * 3


def test_chunked_cache_peels_and_counts():
    """Warm-up keeps everything; the first 1-token step past 2*chunk_size
    peels all but recent_window rows into chunk_size host chunks (with their
    global positions and per-chunk key sums); later steps peel once the
    recent rows exceed recent_window + chunk_size."""
    import numpy as np

    from halo_amd import HALOCacheChunked, HALOConfig
    cfg = HALOConfig(chunk_size=16, recent_window=4, block_size=4)
    cache = HALOCacheChunked(config=cfg, chunk_size=16, recent_window=4)
    k = torch.randn(1, 2, 40, 8)
    v = torch.randn(1, 2, 40, 8)
    K, _ = cache.update(k, v, 0)
    assert K.shape[-2] == 40 and cache._mode == "warmup"
    K, _ = cache.update(torch.randn(1, 2, 1, 8), torch.randn(1, 2, 1, 8), 0)
    assert cache._mode == "chunked" and K.shape[-2] == 4
    assert cache.get_seq_length(0) == 41
    cold = cache._cold[0]
    assert cold.rows == 37 and [c.n for c in cold.chunks] == [16, 16, 5]
    got = torch.cat([c.k[..., :c.n, :] for c in cold.chunks], dim=-2)
    assert torch.equal(got, k[..., :37, :])
    assert np.array_equal(np.concatenate([c.pos[:c.n] for c in cold.chunks]), np.arange(37))
    assert np.array_equal(cache._gpu_pos[0], np.arange(37, 41))
    means = cache.cold_chunk_means(0)
    want = torch.stack([k[..., 0:16, :].mean(-2), k[..., 16:32, :].mean(-2), k[..., 32:37, :].mean(-2)], dim=2)
    torch.testing.assert_close(means, want, rtol=1e-6, atol=1e-6)
    for _ in range(16):
        cache.update(torch.randn(1, 2, 1, 8), torch.randn(1, 2, 1, 8), 0)
    assert cache.get_seq_length(0) == 57 and cache.layers[0].keys.shape[-2] <= 4 + 16
    assert cache.demoted_blocks_total > 0
    cache.reset()
    assert cache.get_seq_length(0) == 0 and cache._mode == "warmup"


def test_chunked_cache_is_a_transformers_cache():
    """The Path-D cache speaks transformers' Cache protocol (the reference
    derives it from DynamicCache, halo/kv_cache.py:69)."""
    pytest.importorskip("transformers")
    from transformers.cache_utils import Cache

    from halo_amd import HALOCacheChunked
    cache = HALOCacheChunked(chunk_size=16, recent_window=4)
    assert isinstance(cache, Cache)
    cache.update(torch.randn(1, 2, 10, 8), torch.randn(1, 2, 10, 8), 0)
    assert cache.get_seq_length() == 10 and cache.get_mask_sizes(1, 0) == (11, 0)


def test_warmup_attention_matches_unwrapped_model():
    """Before any peel the halo_chunked interface is one-shot attention with
    the model's mask: a wrapped tiny Qwen2 (fp32, CPU) gives the unwrapped
    model's logits, with and without left padding (reference
    tests/test_chunked_wrap_integration.py:72-101)."""
    pytest.importorskip("transformers")
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config

    from halo_amd import HALOConfig, wrap_with_halo
    cfg = Qwen2Config(vocab_size=256, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      tie_word_embeddings=False, attn_implementation="sdpa")
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg).eval()
    ids = torch.randint(5, 250, (2, 48), generator=torch.Generator().manual_seed(1))
    mask = torch.ones_like(ids)
    mask[1, :7] = 0
    with torch.no_grad():
        ref = model(ids, attention_mask=mask, use_cache=False).logits
    wrap_with_halo(model, HALOConfig(chunked=True, chunk_size=32, recent_window=8))
    assert model.config._attn_implementation == "halo_chunked"
    cache = model._halo_cache
    with torch.no_grad():
        got = model(ids, attention_mask=mask, past_key_values=cache, use_cache=True).logits
    assert cache._mode == "warmup" and cache.get_seq_length() == 48
    torch.testing.assert_close(got, ref, rtol=0, atol=1e-5)


def test_wrap_with_halo_attaches_components():
    from halo_amd import HALOCacheChunked, HALOConfig, wrap_with_halo

    class Cfg:
        num_hidden_layers, num_key_value_heads, num_attention_heads, hidden_size = 2, 2, 4, 32

    class Attn(torch.nn.Module):
        def __init__(self, i):
            super().__init__()
            self.layer_idx = i

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = Cfg()
            self.w = torch.nn.Linear(4, 4)
            self.layers = torch.nn.ModuleList([Attn(0), Attn(1)])

    m = wrap_with_halo(Model(), HALOConfig(chunked=True))
    assert isinstance(m._halo_cache, HALOCacheChunked)
    assert m._halo_storage.num_layers == 2 and m._halo_storage.head_dim == 8
    assert all(getattr(a, "_halo_cache", None) is m._halo_cache for a in m.layers)
    with pytest.raises(ValueError):
        wrap_with_halo(Model(), HALOConfig(chunked=True, eviction=True))


def test_host_resident_chunk_must_be_pinned():
    """A chunk in host memory is read in place only when pinned; an ordinary
    host tensor is rejected before any device call."""
    import pytest
    import torch

    from halo_amd.decode import ChunkRef, pack_descs
    k = torch.zeros((1, 2, 64, 128), dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="pinned"):
        pack_descs([ChunkRef(k, k.clone(), 0, True)], B=1, H_kv=2, D=128, dtype=torch.bfloat16)


def test_plans_used_under_capture_survive_cache_clears(monkeypatch):
    """A plan launched while a graph is being captured is kept outside the
    plan cache: clear_plan_cache() and LRU overflow do not drop it, only
    release_captured_plans() does."""
    from halo_amd import decode
    decode.release_captured_plans()

    class _Plan:  # stands for a DecodePlan; only its identity matters here
        pass

    captured, other = _Plan(), _Plan()
    monkeypatch.setattr(decode, "_capturing", lambda stream=None: True)
    decode.keep_for_capture(captured)
    decode.keep_for_capture(captured)          # kept once
    monkeypatch.setattr(decode, "_capturing", lambda stream=None: False)
    decode.keep_for_capture(other)             # not capturing: not kept
    for i in range(decode.PLAN_CACHE_SIZE + 10):
        decode._plan_cache[("k", i)] = _Plan()
        while len(decode._plan_cache) > decode.PLAN_CACHE_SIZE:
            decode._plan_cache.popitem(last=False)
    decode.clear_plan_cache()
    assert decode.captured_plans() == [captured]
    decode.release_captured_plans()
    assert decode.captured_plans() == []


def test_nucleus_filter_follows_the_reference_rule():
    """halo/chunked_prefill.py:150-163: sorted tokens with cumulative
    probability > top_p are dropped, except the most likely one.  For
    probabilities [0.5, 0.3, 0.2] and top_p 0.7 only token 0 survives; at
    top_p 0.85 tokens 0 and 1; at top_p 0.4 still token 0; at 0.999 the
    last token (cumulative 1.0) is still dropped."""
    from halo_amd.chunked_prefill import _pick
    logits = torch.log(torch.tensor([[0.2, 0.5, 0.3]]))   # token 1 most likely, then 2, then 0
    for top_p, allowed in ((0.7, {1}), (0.4, {1}), (0.85, {1, 2}), (0.999, {1, 2})):
        g = torch.Generator().manual_seed(0)
        seen = {int(_pick(logits, True, 1.0, top_p, g)) for _ in range(300)}
        assert seen == allowed, (top_p, seen)
    assert int(_pick(logits, False, 1.0, 0.1, None)) == 1


def test_generate_hook_keeps_a_callers_own_cache():
    """halo/policy.py:462-475: the HALO cache is reset unless it is the
    cache passed; it is handed in only when the caller passes none; a
    caller's own past_key_values goes through untouched."""
    from halo_amd.policy import _install_generate_hook

    class _Cache:
        resets = 0

        def reset(self):
            self.resets += 1

    class _Model:
        def generate(self, *args, **kwargs):
            return kwargs

    m = _Model()
    m._halo_cache = _Cache()
    _install_generate_hook(m)
    kw = m.generate()
    assert kw["past_key_values"] is m._halo_cache and kw["use_cache"] is True and m._halo_cache.resets == 1
    kw = m.generate(past_key_values=m._halo_cache)
    assert kw["past_key_values"] is m._halo_cache and m._halo_cache.resets == 1
    own = object()
    kw = m.generate(past_key_values=own, use_cache=False)
    assert kw["past_key_values"] is own and kw["use_cache"] is False and m._halo_cache.resets == 2


def test_kivi_from_memory_ratio_picks_bits():
    """tests/test_kivi_cache.py:99-107: memory_ratio 4 -> 4 bits, 8 -> 2, 2 -> 8
    (bits = max(16 // memory_ratio, 2))."""
    from halo_amd.kivi_cache import KIVICache
    assert KIVICache.from_memory_ratio(memory_ratio=4).bits == 4
    assert KIVICache.from_memory_ratio(memory_ratio=8).bits == 2
    assert KIVICache.from_memory_ratio(memory_ratio=2).bits == 8
    assert KIVICache.from_memory_ratio(memory_ratio=16).bits == 2
    with pytest.raises(AssertionError):
        KIVICache(bits=3)


def test_scorer_jaccard_extremes(small_config):
    """tests/test_scorer.py:43-52: identical index sets 1, disjoint 0; both
    empty 1 and a partial overlap |a & b| / |a | b| (halo/scorer.py:92-97)."""
    import torch
    from halo_amd.scorer import HALOScorer
    s = HALOScorer(small_config)
    a = torch.tensor([1, 2, 3, 4])
    assert s.jaccard(a, torch.tensor([1, 2, 3, 4])) == pytest.approx(1.0)
    assert s.jaccard(a, torch.tensor([5, 6, 7, 8])) == pytest.approx(0.0)
    assert s.jaccard(torch.tensor([], dtype=torch.long), torch.tensor([], dtype=torch.long)) == pytest.approx(1.0)
    assert s.jaccard(a, torch.tensor([3, 4, 5])) == pytest.approx(2 / 5)


def test_chunked_cache_has_no_static_bound():
    """halo/kv_cache_chunked.py:566-568: get_max_cache_shape is None."""
    from halo_amd.kv_cache_chunked import HALOCacheChunked
    assert HALOCacheChunked().get_max_cache_shape() is None
