"""The tier machinery on the GPU: batched block moves between HBM and pinned
DRAM (``halo_copy_blocks``), the device-scheduled refetcher and demoter, and
the placement scorer plug-in (``ChunkScorer``), against the oracle's
bookkeeping and closed forms (reference tests/test_memory_tier.py,
tests/test_refetcher.py:9-43, tests/test_demoter.py, and
baselines/scorer_ablations.py:133-139, 204-268)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scoring as S
from oracle.inputs import round_to

pytestmark = pytest.mark.gpu


def _storage(dev, *, layers=2, blocks=64, H_kv=2, bs=16, D=64, dtype=torch.bfloat16):
    from halo_amd import MemoryTier, TieredStorage
    return TieredStorage(tiers=[MemoryTier.GPU, MemoryTier.DRAM], num_layers=layers, num_kv_heads=H_kv,
                         head_dim=D, block_size=bs, dtype=dtype, device=dev, max_blocks=blocks)


def _fill(st, layer, blocks, tier, seed):
    g = torch.Generator().manual_seed(seed)
    data = {}
    for b in blocks:
        k = torch.randn(st.num_kv_heads, st.block_size, st.head_dim, generator=g).to(st.dtype)
        v = torch.randn(st.num_kv_heads, st.block_size, st.head_dim, generator=g).to(st.dtype)
        st.write_new_block(layer=layer, block=b, keys=k.to(st.gpu_device) if tier == "gpu" else k,
                           values=v.to(st.gpu_device) if tier == "gpu" else v, tier=tier)
        data[b] = (k, v)
    torch.cuda.synchronize()
    return data


def test_batched_moves_round_trip(dev):
    st = _storage(dev)
    data = _fill(st, 1, range(0, 40), "gpu", 0)
    # GPU -> DRAM for a device list with padding, a duplicate and a block outside the source tier
    _fill(st, 1, [50], "dram", 1)
    lst = torch.tensor([3, 7, -1, 7, 50, 12, 39, 63], dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    st.move_blocks(layer=1, blocks=lst, src="gpu", dst="dram", stream=side)
    torch.cuda.current_stream().wait_stream(side)
    moved = {3, 7, 12, 39, 63}           # 63 was never written: an unknown block reads as GPU-resident
    for b in range(64):
        want = "dram" if b in moved or b == 50 else "gpu"
        assert st.locate_block(layer=1, block=b) == want, b
    dram = st._buffer(st.tiers[1])
    moved.discard(63)
    for b in moved:
        assert torch.equal(dram.keys[1, b], data[b][0]) and torch.equal(dram.values[1, b], data[b][1])
    # back to the GPU after clobbering the HBM copies
    gpu = st._buffer(st.tiers[0])
    gpu.keys[1].zero_()
    gpu.values[1].zero_()
    st.move_blocks(layer=1, blocks=torch.tensor(sorted(moved), dtype=torch.int32, device=dev), src="dram",
                   dst="gpu")
    torch.cuda.synchronize()
    for b in moved:
        assert st.locate_block(layer=1, block=b) == "gpu"
        assert torch.equal(gpu.keys[1, b].cpu(), data[b][0]) and torch.equal(gpu.values[1, b].cpu(), data[b][1])
    assert st.locate_block(layer=0, block=3) == "gpu"  # other layers untouched


def test_concurrent_moves_on_two_streams_keep_both_directory_updates(dev):
    """Two streams move different blocks of one layer (demotion of some, a
    refetch of others) with no ordering between them: only the listed
    directory entries are written, so neither move undoes the other's."""
    st = _storage(dev)
    _fill(st, 0, range(0, 32), "gpu", 2)
    _fill(st, 0, range(32, 64), "dram", 3)
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    a.wait_stream(torch.cuda.current_stream())
    b.wait_stream(torch.cuda.current_stream())
    down = torch.arange(0, 32, 2, dtype=torch.int32, device=dev)      # even GPU blocks -> DRAM
    up = torch.arange(33, 64, 2, dtype=torch.int32, device=dev)       # odd DRAM blocks -> GPU
    for _ in range(3):  # and back, several rounds, the two streams racing each other
        st.move_blocks(layer=0, blocks=down, src="gpu", dst="dram", stream=a)
        st.move_blocks(layer=0, blocks=up, src="dram", dst="gpu", stream=b)
        st.move_blocks(layer=0, blocks=down, src="dram", dst="gpu", stream=a)
        st.move_blocks(layer=0, blocks=up, src="gpu", dst="dram", stream=b)
    st.move_blocks(layer=0, blocks=down, src="gpu", dst="dram", stream=a)
    st.move_blocks(layer=0, blocks=up, src="dram", dst="gpu", stream=b)
    torch.cuda.synchronize()
    for blk in range(64):
        if blk < 32:
            want = "dram" if blk % 2 == 0 else "gpu"
        else:
            want = "gpu" if blk % 2 == 1 else "dram"
        assert st.locate_block(layer=0, block=blk) == want, blk


def test_refetcher_reference_expectations(dev, small_config):
    """Blocks 0 (GPU) and 1 (DRAM): positions [0, 1, 4, 5] give one hit and
    one miss, and block 1 is on the GPU afterwards (reference
    tests/test_refetcher.py:22-43), here with the asynchronous refetch."""
    from halo_amd import HALORefetcher
    cfg = small_config
    cfg.async_refetch = True
    st = _storage(dev, bs=cfg.block_size)
    data = _fill(st, 0, [0], "gpu", 2)
    data.update(_fill(st, 0, [1], "dram", 3))
    r = HALORefetcher(cfg, storage=st)
    r.schedule(layer=0, predicted_indices=[0, 1, 4, 5])
    r.schedule(layer=0, predicted_indices=torch.tensor([4, 5], device=dev))  # in flight or landed: no new miss
    r.wait()
    assert (r.hits, r.misses) in ((1, 1), (2, 1))
    assert st.locate_block(layer=0, block=1) == "gpu"
    gpu = st._buffer(st.tiers[0])
    assert torch.equal(gpu.keys[0, 1].cpu(), data[1][0]) and torch.equal(gpu.values[0, 1].cpu(), data[1][1])


def test_refetcher_counts_match_oracle_bookkeeping(dev, small_config):
    """Random directories and predictions: device hit/miss counts equal the
    oracle's per-block bookkeeping (oracle.scoring.schedule) call by call,
    synchronous refetch so the directory matches at every call."""
    from halo_amd import HALORefetcher
    cfg = small_config
    cfg.async_refetch = False
    rng = np.random.default_rng(7)
    st = _storage(dev, blocks=64, bs=cfg.block_size)
    dram_blocks = sorted(rng.choice(64, size=30, replace=False).tolist())
    _fill(st, 0, dram_blocks, "dram", 4)
    tiers = {b: "dram" for b in dram_blocks}
    r = HALORefetcher(cfg, storage=st)
    hits = misses = 0
    inflight: set = set()
    for _ in range(6):
        pred = rng.integers(0, 64 * cfg.block_size, size=40)
        h, m, fetch = S.schedule(pred.tolist(), block_size=cfg.block_size,
                                 locate=lambda layer, b: tiers.get(b, "gpu"), inflight=inflight)
        for b in fetch:
            tiers[b] = "gpu"
        hits, misses = hits + h, misses + m
        r.schedule(layer=0, predicted_indices=torch.from_numpy(pred).to(dev))
        assert (r.hits, r.misses) == (hits, misses)
    for b in range(64):
        assert st.locate_block(layer=0, block=b) == tiers.get(b, "gpu")


def test_demoter_async_then_wait(dev, small_config):
    from halo_amd import HALODemoter
    cfg = small_config
    cfg.async_refetch = True
    st = _storage(dev, bs=cfg.block_size)
    data = _fill(st, 0, [0, 1, 2, 5], "gpu", 5)
    d = HALODemoter(cfg, storage=st)
    d.demote(layer=0, block_indices=[0, 1], src="gpu", dst="dram")
    d.demote(layer=0, block_indices=torch.tensor([2, 5], device=dev), src="gpu", dst="dram")
    d.wait()
    dram = st._buffer(st.tiers[1])
    torch.cuda.synchronize()
    for b in (0, 1, 2, 5):
        assert st.locate_block(layer=0, block=b) == "dram"
        assert torch.equal(dram.keys[0, b], data[b][0])
    assert st.locate_block(layer=0, block=3) == "gpu"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunk_scorer_plugin(dev, dtype):
    """observe_keys keeps incremental page means equal to the oracle's
    (within one storage rounding); select_hot_pages returns the
    _num_hot_pages budget of pages ranked by the HALOPress score
    (min-max attention + recency + sink) with the (score desc, index asc)
    tie rule."""
    from halo_amd.chunk_scorer import ChunkScorer, ChunkScorerConfig
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    rng = np.random.default_rng(13)
    B, H, H_kv, D, p = 1, 8, 2, 128, 16
    K = round_to(rng.standard_normal((B, H_kv, 600, D)).astype(np.float32) * 2, name)
    Kd = torch.from_numpy(K).to(dev).to(dtype)
    cfg = ChunkScorerConfig(page_size=p, memory_ratio=4, min_pages_selected=4, halopress_alpha=1.0,
                            halopress_beta=0.3, halopress_gamma=0.5, halopress_refresh_window=8,
                            halopress_sink_tokens=4)
    sc = ChunkScorer(cfg)
    for T in (100, 257, 600):            # incremental: only new full pages are computed
        sc.observe_keys(0, Kd[:, :, :T])
    km = sc.page_means(0)
    want = S.page_means(K, p, name)
    P = 600 // p
    assert km.shape == (B, H_kv, P, D)
    err = np.abs(km.float().cpu().numpy() - want)
    assert err.max() <= 2.0 ** -7 * np.abs(want).max()
    q = round_to(rng.standard_normal((B, H, 1, D)).astype(np.float32), name)
    hot = sc.select_hot_pages(0, torch.from_numpy(q).to(dev).to(dtype))
    budget = S.num_hot_pages(P, 4, 4)
    attn = S.ordered_scores(q, km.float().cpu().numpy(), name)
    score = S.halopress_page_scores(attn, alpha=1.0, beta=0.3, gamma=0.5, refresh_window=8, sink_tokens=4,
                                    page_size=p)
    assert hot.tolist() == S.topk_indices(score, budget).tolist()
    assert sc.score_calls == 1 and sc.cumulative_hot_pages == budget


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nvme_tier_batched_moves(dev, tmp_path, dtype):
    """GPU <-> NVMe and DRAM <-> NVMe moves of block lists (duplicates, -1
    padding, runs and gaps) are byte-exact against the file and the written
    blocks, update the directory, skip blocks not in the source tier, and a
    block written to NVMe survives a move back into a cleared GPU tier
    (reference tests/test_memmap_nvme.py:14-74 on a GPU-backed store)."""
    from halo_amd import MemoryTier, TieredStorage
    st = TieredStorage(tiers=[MemoryTier.GPU, MemoryTier.DRAM, MemoryTier.NVME], num_layers=2, num_kv_heads=2,
                       head_dim=64, block_size=16, dtype=dtype, device=dev, max_blocks=32,
                       nvme_path=str(tmp_path / "nvme"))
    data = _fill(st, 1, range(0, 20), "gpu", 3)
    moved = [3, 4, 5, 9, 12, 13, 19]
    blocks = torch.tensor([5, 3, -1, 4, 9, 5, 13, 12, 19, 40], dtype=torch.int32, device=dev)
    st.move_blocks(layer=1, blocks=blocks, src="gpu", dst="nvme")
    torch.cuda.synchronize()
    for b in range(20):
        assert st.locate_block(layer=1, block=b) == ("nvme" if b in moved else "gpu")
    per = 2 * 16 * 64 * torch.tensor([], dtype=dtype).element_size()
    raw_k = np.fromfile(tmp_path / "nvme" / "keys.bin", dtype=np.uint8)
    for b in moved:
        s = (1 * 32 + b) * per
        assert np.array_equal(raw_k[s:s + per], data[b][0].contiguous().view(torch.uint8).numpy().reshape(-1))
    # back into a cleared GPU tier; blocks not in NVMe (0, 1) are skipped
    st._buffer(MemoryTier.GPU).keys.zero_()
    st._buffer(MemoryTier.GPU).values.zero_()
    st.move_blocks(layer=1, blocks=torch.tensor([0, 1] + moved, dtype=torch.int32, device=dev),
                   src="nvme", dst="gpu")
    torch.cuda.synchronize()
    gk = st._buffer(MemoryTier.GPU).keys[1].cpu()
    gv = st._buffer(MemoryTier.GPU).values[1].cpu()
    for b in moved:
        assert torch.equal(gk[b], data[b][0]) and torch.equal(gv[b], data[b][1])
        assert st.locate_block(layer=1, block=b) == "gpu"
    assert not gk[0].any() and not gk[1].any()
    # DRAM <-> NVMe on the same store, and single-block moves
    st.move_blocks(layer=1, blocks=torch.tensor([3, 4], dtype=torch.int32, device=dev), src="gpu", dst="dram")
    st.move_blocks(layer=1, blocks=torch.tensor([4, 3], dtype=torch.int32, device=dev), src="dram", dst="nvme")
    st.move_block(layer=1, block=3, src="nvme", dst="dram")
    torch.cuda.synchronize()
    assert st.locate_block(layer=1, block=3) == "dram" and st.locate_block(layer=1, block=4) == "nvme"
    rk, rv = st.read_block(layer=1, block=3)
    assert torch.equal(rk.cpu(), data[3][0]) and torch.equal(rv.cpu(), data[3][1])
    rk, rv = st.read_block(layer=1, block=4)
    assert torch.equal(rk.cpu(), data[4][0]) and torch.equal(rv.cpu(), data[4][1])
