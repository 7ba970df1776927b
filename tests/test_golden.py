"""The committed golden fixtures (tests/golden/*.npz) against the oracle
(CPU): detects drift in the seeded generator or the restatement."""
from __future__ import annotations

import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name,cfgname", [("c1_decode", "C1"), ("c2_layer0", "C2")])
def test_golden_fixture_reproduces(name, cfgname):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    from oracle import inputs
    cfg = getattr(inputs, cfgname)
    fx = np.load(os.path.join(HERE, name + ".npz"))
    got = mg.tiered_case(cfg, cfg["seed"])
    np.testing.assert_array_equal(got["checksums"], fx["checksums"])
    np.testing.assert_array_equal(got["selected"], fx["selected"])
    np.testing.assert_array_equal(got["scores"], fx["scores"])
    np.testing.assert_allclose(got["out"], fx["out"], rtol=0, atol=1e-7)
    np.testing.assert_allclose(got["lse"], fx["lse"], rtol=0, atol=1e-7)
    # the top-k boundary is far above fp32 / bf16-mean rounding noise
    assert float(fx["margin"]) > 1e-3
