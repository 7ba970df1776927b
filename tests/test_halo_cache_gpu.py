"""The tier-aware transformers cache ``HALOCache`` (halo/kv_cache.py:69-209)
on the GPU, with the expectations of the reference's own tests
(tests/test_kv_cache.py): an empty start, demotion of the blocks that cool
when the hot set moves, no demotion and no refetch miss at hot_ratio 1.0,
reset, and JSON-serialisable telemetry; plus the ``Cache`` protocol it
inherits (rows appended per layer)."""
from __future__ import annotations

import json

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cache(cfg, dev, *, layers=1, H_kv=2, D=8, blocks=16):
    from halo_amd import HALODemoter, HALORefetcher, HALOScorer, MemoryTier, TieredStorage
    from halo_amd.kv_cache import HALOCache
    st = TieredStorage(tiers=[MemoryTier.GPU, MemoryTier.DRAM], num_layers=layers, num_kv_heads=H_kv, head_dim=D,
                       block_size=cfg.block_size, dtype=torch.float32, device=dev, max_blocks=blocks)
    return HALOCache(config=cfg, storage=st, scorer=HALOScorer(cfg), demoter=HALODemoter(cfg, storage=st),
                     refetcher=HALORefetcher(cfg, storage=st))


def test_cache_starts_empty(dev, small_config):
    """tests/test_kv_cache.py:22-27."""
    c = _cache(small_config, dev)
    assert c.step_index == 0 and c.demoted_blocks_total == 0 and c.refetched_blocks_total == 0
    assert c.get_seq_length() == 0


def test_update_hotness_demotes_cooled_blocks(dev, small_config):
    """tests/test_kv_cache.py:30-51: the back of the cache hot, then only the
    front: the blocks that left the hot set are demoted."""
    c = _cache(small_config, dev)
    K = 64
    back = torch.zeros(K)
    back[-K // 4:] = 1.0
    c.update_hotness(layer_idx=0, attn_weights=(back / back.sum()).to(dev))
    c.step()
    front = torch.zeros(K)
    front[:K // 4] = 1.0
    c.update_hotness(layer_idx=0, attn_weights=(front / front.sum()).to(dev))
    assert c.demoted_blocks_total > 0


def test_identity_at_hot_ratio_one(dev, small_config, fake_attention):
    """tests/test_kv_cache.py:54-74: hot_ratio 1.0 never demotes and never
    misses a refetch."""
    small_config.hot_ratio = 1.0
    c = _cache(small_config, dev)
    for step in range(8):
        c.step()
        c.update_hotness(layer_idx=0, attn_weights=fake_attention(K=64, seed=step).to(dev))
    assert c.demoted_blocks_total == 0
    assert c.refetcher.misses == 0


def test_reset_and_telemetry(dev, small_config, fake_attention):
    """tests/test_kv_cache.py:77-101: reset clears the counters and the step;
    the telemetry serialises to JSON with the reference's keys."""
    c = _cache(small_config, dev)
    c.update_hotness(layer_idx=0, attn_weights=fake_attention(K=64).to(dev))
    payload = c.telemetry()
    json.dumps(payload)
    assert "demoted_blocks" in payload and "refetch_hit_rate" in payload
    c.step()
    c.step()
    assert c.step_index == 2
    k = torch.randn(1, 2, 5, 8, device=dev)
    kk, vv = c.update(k, k.clone(), 0)
    kk, vv = c.update(k[..., :3, :], k[..., :3, :].clone(), 0)
    assert kk.shape == (1, 2, 8, 8) and torch.equal(kk[..., :5, :], k) and c.get_seq_length(0) == 8
    c.reset()
    assert c.step_index == 0 and c.demoted_blocks_total == 0 and c.refetched_blocks_total == 0
    assert c.get_seq_length(0) == 0
