"""The committed golden fixtures (tests/golden/kivi_golden.*, made by
tests/golden/make_golden.py) are reproduced by the oracle bit for bit (cache
arrays) and to float64 rounding (attention outputs), and the outputs agree
with the independent numpy restatement (CPU)."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tests import kivi_numpy_ref as nref
from tests.golden import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load():
    meta = json.load(open(os.path.join(HERE, "kivi_golden.json")))
    arrays = np.load(os.path.join(HERE, "kivi_golden.npz"))
    return meta, arrays


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_oracle_reproduces_golden(oracle, name):
    meta, arrays = load()
    assert meta[name]["case"] == mg.CASES[name]
    cache, out = mg.oracle_state(mg.CASES[name])
    for a in mg.ARRAYS:
        assert mg.digest(getattr(cache, a)) == meta[name]["sha256"][a], a
    assert mg.scratch_digests(cache, mg.CASES[name]) == meta[name]["scratch_sha256"]
    np.testing.assert_allclose(out, arrays[f"{name}__out"], rtol=1e-12, atol=1e-12)
    # and the outputs agree with the numpy restatement of the read side
    _, q, tables, _, _ = mg.inputs(mg.CASES[name])
    for b, L in enumerate(mg.CASES[name]["lens"]):
        K, V = nref.dequant_sequence(cache, b, tables[b], L)
        np.testing.assert_allclose(nref.attention(q[b], K, V), out[b], rtol=1e-9, atol=1e-12)
