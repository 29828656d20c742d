"""The committed golden fixtures (tests/golden/*.npz) are what the CPU oracle
computes for their seeded inputs — CPU only.  The fixtures pin the oracle
against silent changes; the oracle itself is pinned in test_oracle.py."""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_oracle_reproduces_fixture(name):
    stored = np.load(GOLDEN / f"{name}.npz")  # arrays only (allow_pickle=False)
    fresh = make_golden.FIXTURES[name]()
    assert sorted(stored.files) == sorted(fresh)
    for key in stored.files:
        a, b = stored[key], np.asarray(fresh[key])
        assert a.shape == b.shape and a.dtype == b.dtype, key
        if a.dtype.kind in "iub":
            assert np.array_equal(a, b), key
        else:
            np.testing.assert_allclose(b, a, rtol=1e-10, atol=1e-13, err_msg=key)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_inputs_are_bf16_exact(name):
    stored = np.load(GOLDEN / f"{name}.npz")
    for key in stored.files:
        a = stored[key]
        if a.dtype == np.float32 and key not in ("cos", "sin", "x_scale", "q_scale", "k_scale"):
            t = torch.from_numpy(a)
            assert torch.equal(t.to(torch.bfloat16).float(), t), key
