"""The oracle's paged decode against an independent numpy restatement and
closed forms (CPU).

No reference test pins attention outputs.  The fp32 online-softmax oracle
(the reference's loop order, snapshot :51-158) and its float64 two-pass twin
are checked against
  * tests/kivi_numpy_ref.py: layout, unpack and attention re-derived in numpy;
  * uniform keys -> the plain mean of the dequantised values;
  * seq_len <= residual -> ordinary fp16 attention on the raw history;
  * physical-page permutation invariance, split-K == one pass, the LSE merge
    closed form, empty and over-long sequences;
  * sparse-retained decode (variants.rs:2620-2740): full retention == dense,
    no retention == residual-only attention, a retained subset == numpy
    attention over exactly those tokens plus the dense residual window, and
    the clamps of NUM_RETAINED_PAGES.
"""
from __future__ import annotations

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests import kivi_numpy_ref as nref

GEO = o.Geometry(nh=8, nkv=2, hd=64, page=16, group=32, residual=64, max_pages=24)


def h16(x) -> np.ndarray:
    return np.asarray(x, np.float16).view(np.uint16)


@pytest.fixture(scope="module", autouse=True)
def _build(oracle):
    return oracle


def build(geo, n, seed, outliers=True, k_override=None):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n, geo.nkv, geo.hd))
    if outliers:
        k[:, :, [3, 17]] *= 10.0
    if k_override is not None:
        k[:] = k_override
    v = rng.standard_normal((n, geo.nkv, geo.hd))
    q = h16(rng.standard_normal((geo.nh, geo.hd)))
    table = rng.permutation(geo.max_pages).astype(np.int32)
    c = o.Cache.empty(geo, geo.max_pages, 1, fill=0x55)
    o.build_sequence(c, 0, h16(k), h16(v), table)
    return c, q, table, h16(k), h16(v)


@pytest.mark.parametrize("n", [1, 40, 64, 65, 96, 97, 200, 300])
def test_oracle_matches_numpy_restatement(n):
    c, q, table, _, _ = build(GEO, n, seed=n)
    K, V = nref.dequant_sequence(c, 0, table, n)
    want = nref.attention(q, K, V)
    two = o.decode_twopass(c, 0, q, table, n)
    online = o.decode_online(c, 0, q, table, n)
    np.testing.assert_allclose(two, want, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(online, want, rtol=1e-4, atol=2e-5)


def test_uniform_keys_give_mean_of_values():
    n = 200
    rng = np.random.default_rng(7)
    krow = rng.standard_normal((GEO.nkv, GEO.hd))
    c, q, table, _, _ = build(GEO, n, seed=7, outliers=False,
                              k_override=np.broadcast_to(krow, (n, GEO.nkv, GEO.hd)))
    _, V = nref.dequant_sequence(c, 0, table, n)
    G = GEO.nh // GEO.nkv
    want = np.repeat(V.mean(axis=1), G, axis=0)
    np.testing.assert_allclose(o.decode_twopass(c, 0, q, table, n), want, rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(o.decode_online(c, 0, q, table, n), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n", [1, 17, 64])
def test_short_sequence_is_plain_fp16_attention(n):
    c, q, table, k, v = build(GEO, n, seed=100 + n)
    f = lambda x: x.view(np.float16).astype(np.float64)
    K, V = f(k).transpose(1, 0, 2), f(v).transpose(1, 0, 2)
    want = nref.attention(q, K, V)
    np.testing.assert_allclose(o.decode_twopass(c, 0, q, table, n), want, rtol=1e-10, atol=1e-12)


def test_page_permutation_invariance():
    n = 250
    c, q, table, _, _ = build(GEO, n, seed=11)
    perm = np.random.default_rng(12).permutation(GEO.max_pages)
    c2 = c.copy()
    for f in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero"):
        src = getattr(c, f)
        dst = getattr(c2, f)
        dst[perm] = src  # physical page p moves to perm[p]
    table2 = perm[table].astype(np.int32)
    a = o.decode_online(c, 0, q, table, n)
    b = o.decode_online(c2, 0, q, table2, n)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("chunk", [32, 64, 96, 160])
def test_split_k_equals_one_pass(chunk):
    n = 300
    c, q, table, _, _ = build(GEO, n, seed=13)
    one = o.decode_online(c, 0, q, table, n)
    split = o.decode_splitk(c, 0, q, table, n, chunk)
    np.testing.assert_allclose(split, one, rtol=1e-5, atol=1e-6)


def test_lse_merge_closed_form():
    rng = np.random.default_rng(14)
    s = rng.standard_normal(50) * 3
    v = rng.standard_normal((50, 8))
    parts = [(0, 20), (20, 21), (21, 50)]
    m, l, acc = [], [], []
    for a, b in parts:
        mm = s[a:b].max()
        p = np.exp(s[a:b] - mm)
        m.append(mm), l.append(p.sum()), acc.append(p @ v[a:b])
    want = np.exp(s - s.max()) @ v / np.exp(s - s.max()).sum()
    got = o.lse_merge(np.array(m), np.array(l), np.array(acc))  # natural-log domain
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_empty_and_overlong_sequences():
    n = 120
    c, q, table, _, _ = build(GEO, n, seed=15)
    assert np.all(o.decode_online(c, 0, q, table, 0) == 0)
    assert np.all(o.decode_twopass(c, 0, q, table, 0) == 0)
    # lengths beyond the cache capacity clamp to LQ + R (snapshot :74-83)
    lq = GEO.max_pages * GEO.page // 32 * 32
    cap = lq + GEO.residual
    big = o.decode_online(c, 0, q, table, cap + 1000)
    assert np.array_equal(big, o.decode_online(c, 0, q, table, cap))


def test_workload_generator_is_deterministic():
    w = wl.WORKLOADS["qwen05b"]
    r1, r2 = np.random.default_rng(w.seed), np.random.default_rng(w.seed)
    assert np.array_equal(wl.context_lens(w, r1), wl.context_lens(w, r2))


# ---------------------------------------------------------------- sparse-retained

def _sparse_case(n=400, seed=31):
    c, q, table, _, _ = build(GEO, n, seed=seed)
    lq = (GEO.max_pages * GEO.page) // 32 * 32
    dense_old, res = nref.decode_window(n, GEO.residual, lq)
    return c, q, table, dense_old, res


def test_sparse_full_retention_equals_dense():
    n = 400
    c, q, table, dense_old, _ = _sparse_case(n)
    pages = dense_old // GEO.page
    compact = np.ascontiguousarray(table[:pages])
    np.testing.assert_array_equal(o.decode_sparse_retained(c, 0, q, compact, n, pages),
                                  o.decode_online(c, 0, q, table, n))
    np.testing.assert_array_equal(o.decode_sparse_retained(c, 0, q, compact, n, pages, True),
                                  o.decode_twopass(c, 0, q, table, n))


def test_sparse_zero_retention_is_residual_attention():
    n = 400
    c, q, table, dense_old, res = _sparse_case(n)
    K, V = nref.dequant_sequence(c, 0, table, n, window=(0, res))
    want = nref.attention(q, K, V)
    # the scratch rows are the tokens after the dense boundary
    assert K.shape[1] == n - dense_old
    np.testing.assert_allclose(o.decode_sparse_retained(c, 0, q, table[:0], n, 0, True), want,
                               rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("groups", [[0], [3, 5, 9], [9, 0, 4, 2], list(range(10))])
def test_sparse_subset_matches_numpy(groups):
    """Retained groups in any order (a compact table of their pages): numpy
    attention over exactly those tokens, then the dense residual rows."""
    n = 400
    c, q, table, dense_old, res = _sparse_case(n)
    per = 32 // GEO.page
    compact = np.concatenate([table[g * per:(g + 1) * per] for g in groups]).astype(np.int32)
    npages = len(compact)
    K, V = nref.dequant_sequence(c, 0, compact, n, window=(npages * GEO.page, res))
    want = nref.attention(q, K, V)
    np.testing.assert_allclose(o.decode_sparse_retained(c, 0, q, compact, n, npages, True), want,
                               rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(o.decode_sparse_retained(c, 0, q, compact, n, npages), want,
                               rtol=1e-4, atol=2e-5)


def test_sparse_clamps_retained_pages():
    n = 400
    c, q, table, dense_old, _ = _sparse_case(n)
    pages = dense_old // GEO.page
    full = o.decode_sparse_retained(c, 0, q, table, n, pages)
    # more pages than the dense window holds -> the dense window
    np.testing.assert_array_equal(o.decode_sparse_retained(c, 0, q, table, n, pages + 3), full)
    # negative -> none retained
    np.testing.assert_array_equal(o.decode_sparse_retained(c, 0, q, table, n, -2),
                                  o.decode_sparse_retained(c, 0, q, table, n, 0))
    # page 16: an odd count covers whole groups only
    np.testing.assert_array_equal(o.decode_sparse_retained(c, 0, q, table, n, 5),
                                  o.decode_sparse_retained(c, 0, q, table, n, 4))
    lq = (GEO.max_pages * GEO.page) // 32 * 32
    assert nref.sparse_window(n, GEO.residual, lq, GEO.page, GEO.max_pages, 5) == (64, n - dense_old)
