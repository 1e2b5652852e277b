"""The oracle's group quantiser against an independent numpy restatement (CPU).

The oracle (oracle/kivi_oracle.c, kivi_ref_pack_group) follows the
reference's age-out kernels, source_patch.py:1532-1581 (K) and :1583-1620
(V), with fminf / fmaxf semantics.  tests/kivi_numpy_quant.py restates the
same quantiser with different means (order keys + argmin, vectorised
float32).  Bit-equality is checked on random groups and on adversarial ones
(NaN / +-inf at the first and middle positions, +-0 mixes, subnormals, exact
.5 ties, values at +-65504, ties that a reciprocal multiply rounds the other
way).  Each mutant quantiser of kivi_numpy_quant.MUTANTS must disagree with
the oracle on those groups, so the agreement pins those mistakes out.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as o
from tests import kivi_numpy_quant as nq

FIELDS = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")


@pytest.fixture(scope="module", autouse=True)
def _build(oracle):
    return oracle


def oracle_group(k32, v32, page=32):
    """Age one group out through the oracle's served path (64 single-token
    writes with a 32-token residual) and return its page contents."""
    nkv, hd = k32.shape[1:]
    geo = o.Geometry(nh=nkv * 2, nkv=nkv, hd=hd, page=page, group=32, residual=32,
                     max_pages=8 * 32 // page)
    c = o.Cache.empty(geo, 8 * 32 // page, 1, fill=0xA5)
    rng = np.random.default_rng(99)
    k = np.concatenate([k32, nq._bits(rng.standard_normal((32, nkv, hd)))])
    v = np.concatenate([v32, nq._bits(rng.standard_normal((32, nkv, hd)))])
    table = np.arange(geo.max_pages, dtype=np.int32)[::-1].copy()
    for t in range(64):
        o.cache_write(c, 0, k[t], v[t], table, t + 1)
    if page == 32:
        p = table[0]
        return {f: getattr(c, f)[p] for f in FIELDS}
    pa, pb = table[0], table[1]  # one group over two 16-token pages
    out = {f: np.concatenate([getattr(c, f)[pa], getattr(c, f)[pb]], axis=1)
           for f in ("k_code", "v_code", "v_scale", "v_zero")}
    assert np.array_equal(c.k_scale[pa], c.k_scale[pb])
    assert np.array_equal(c.k_zero[pa], c.k_zero[pb])
    out["k_scale"], out["k_zero"] = c.k_scale[pa], c.k_zero[pa]
    return out


def assert_same(got, want, what):
    for f in FIELDS:
        assert got[f].shape == want[f].shape, (what, f)
        bad = np.argwhere(got[f] != want[f])
        assert bad.size == 0, f"{what}: {f} differs at {bad[:5].tolist()} " \
            f"(got {got[f][tuple(bad[0])]:#x}, want {want[f][tuple(bad[0])]:#x})"


@pytest.mark.parametrize("seed", range(6))
def test_random_groups_equal_numpy_restatement(seed):
    rng = np.random.default_rng(seed)
    scale = [1.0, 10.0, 1e-3, 300.0, 1.0, 0.05][seed]
    k = nq._bits(rng.standard_normal((32, 2, 128)) * scale)
    v = nq._bits(rng.standard_normal((32, 2, 128)) * scale)
    if seed == 4:  # outlier channels (the benchmark K recipe)
        k[:, :, ::16] = nq._bits(nq.f16(k[:, :, ::16]).astype(np.float32) * 10)
    assert_same(oracle_group(k, v), nq.quantise_group(k, v), f"seed {seed}")


@pytest.mark.parametrize("page", [32, 16])
def test_adversarial_groups_equal_numpy_restatement(page):
    rng = np.random.default_rng(1234)
    k, v = nq.adversarial_group(rng, 2, 128)
    assert_same(oracle_group(k, v, page), nq.quantise_group(k, v), "adversarial")


@pytest.mark.parametrize("name", sorted(nq.MUTANTS))
def test_adversarial_groups_reject_every_mutant(name):
    rng = np.random.default_rng(1234)
    k, v = nq.adversarial_group(rng, 2, 128)
    got = oracle_group(k, v)
    mut = nq.quantise_group(k, v, **nq.MUTANTS[name])
    assert any(not np.array_equal(got[f], mut[f]) for f in FIELDS), \
        f"the adversarial groups do not tell '{name}' apart from the oracle"


def test_fminf_semantics_closed_forms():
    """Values the reference's fminf / fmaxf fix (source_patch.py:1555-1558)."""
    nan, z, nz = nq.QNAN, nq._bits([0.0])[0], nq._bits([-0.0])[0]
    col = nq._bits(np.arange(32, dtype=np.float32) * 0.5)   # 0 .. 15.5, scale 31/30
    col[0] = nan                                              # NaN first: dropped
    k = np.repeat(np.repeat(col[:, None, None], 2, 1), 128, 2)
    v = np.ascontiguousarray(np.transpose(k, (0, 1, 2)))
    got = oracle_group(k, v)
    want_scale = nq._bits([np.float32(15.5 - 0.5) / np.float32(15)])[0]
    assert np.all(got["k_zero"] == nq._bits([0.5])[0]), "min must skip the leading NaN"
    assert np.all(got["k_scale"] == want_scale)
    codes_t0 = got["k_code"][:, 0, :]                         # token 0 is the NaN: code 0
    assert np.all(codes_t0 == 0)
    # an all-zero group with one -0: min -0, max +0 -> range 0 -> scale 1
    col = np.full(32, z, np.uint16)
    col[9] = nz
    k = np.repeat(np.repeat(col[:, None, None], 2, 1), 128, 2)
    got = oracle_group(k, k.copy())
    assert np.all(got["k_zero"] == nz) and np.all(got["k_scale"] == nq._bits([1.0])[0])
    assert np.all(got["k_code"] == 0)


def test_order_key_is_the_float_order():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(500) * 10.0 ** rng.integers(-8, 5, 500),
                        [0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45]]).astype(np.float32)
    k = nq._order_key(x)
    i, j = rng.integers(0, x.size, (2, 4000))
    lt = (x[i] < x[j]) | ((x[i] == 0) & (x[j] == 0) & np.signbit(x[i]) & ~np.signbit(x[j]))
    assert np.array_equal(k[i] < k[j], lt)
