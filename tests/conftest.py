"""Shared fixtures.  GPU tests are marked ``gpu``; the CPU suite runs with
``-m "not gpu"`` and never launches a kernel."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from halo_amd import _native
    _native.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


@pytest.fixture
def small_config():
    """Tiny HALOConfig (mirrors the reference fixture, tests/conftest.py:12-28)."""
    from halo_amd import HALOConfig
    return HALOConfig(hot_ratio=0.25, score_alpha=1.0, score_beta=0.5, score_gamma=2.0,
                      sink_tokens=2, refresh_window=8, tiers=("gpu", "dram"),
                      block_size=4, async_refetch=False, lookahead=1)


@pytest.fixture
def fake_attention():
    """Deterministic head-mean attention vector (reference tests/conftest.py:31-40)."""
    import torch

    def _make(K: int, *, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        return torch.softmax(torch.randn(K, generator=g), dim=0)

    return _make


@pytest.fixture
def storage_factory(small_config):
    """TieredStorage on the CPU (reference tests/conftest.py:43-63): the
    directory and tier copies are host logic and run without a GPU."""
    import torch
    from halo_amd import MemoryTier, TieredStorage

    def _make(num_layers: int = 2, num_kv_heads: int = 2, head_dim: int = 8, max_blocks: int = 16):
        return TieredStorage(tiers=[MemoryTier.GPU, MemoryTier.DRAM], num_layers=num_layers,
                             num_kv_heads=num_kv_heads, head_dim=head_dim, block_size=small_config.block_size,
                             dtype=torch.float32, device=torch.device("cpu"), max_blocks=max_blocks)

    return _make
