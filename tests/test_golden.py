"""The committed golden fixtures (tests/golden/*.npz) are exactly what the
oracle produces from their recorded inputs: a change to the oracle that moves
any code, scale, dequantised bit pattern or reference product fails here."""
from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _generator():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def rebuilt():
    return _generator().build()


@pytest.mark.parametrize("fname", ["nf4_codec.npz", "nf4_lora_linear.npz", "gated_mlp.npz"])
def test_fixture_matches_oracle(rebuilt, fname):
    with np.load(GOLDEN / fname, allow_pickle=False) as f:
        stored = {k: f[k] for k in f.files}
    fresh = rebuilt[fname]
    assert sorted(stored) == sorted(fresh)
    for key, value in fresh.items():
        value = np.asarray(value)
        assert stored[key].dtype == value.dtype, key
        assert np.array_equal(stored[key], value), key


def test_codec_fixture_records_its_layout():
    with np.load(GOLDEN / "nf4_codec.npz", allow_pickle=False) as f:
        for name, shape, block, layout in _generator().CODEC_CASES:
            assert int(f[f"{name}/block"]) == block
            assert int(f[f"{name}/order"]) == (1 if layout == "bnb" else 0)
            assert f[f"{name}/w"].shape == shape
            assert (f"{name}/code2" in f.files) == (layout == "bnb")
