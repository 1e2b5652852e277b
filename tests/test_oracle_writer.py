"""The oracle's cache writer against closed forms and invariants (CPU).

No reference test pins codes or scales, so the writer is pinned here by
results the quantiser's definition fixes (source_patch.py:1532-1620):
  * a constant group: scale falls back to 1.0 (`!(scale > 0)`), zero = x, codes 0;
  * an exact ramp min + k*s with s exact in fp16: scale s, codes k;
  * a group of two values {a, b}: codes {0, 15};
  * every value reconstructs to within scale/2 plus the fp16 rounding of
    scale and zero;
plus the layout (channel 2j = low nibble, variants.rs:2316-2327), the residual
window left in scratch, page 16 == page 32 codes, and batched == repeated
single writes (source_patch.py:1737-1775).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as o

GEO = o.Geometry(nh=4, nkv=2, hd=64, page=32, group=32, residual=32, max_pages=8)


def h16(x) -> np.ndarray:
    return np.asarray(x, np.float16).view(np.uint16)


def fresh(geo=GEO, pages=8, batch=1):
    return o.Cache.empty(geo, pages, batch, fill=0xAB)


def write_all(cache, k, v, table, b=0):
    for t in range(k.shape[0]):
        o.cache_write(cache, b, k[t], v[t], table, t + 1)


def unpack(codes: np.ndarray) -> np.ndarray:
    """[..., HD/2] bytes -> [..., HD] codes, channel 2j in the low nibble."""
    lo = codes & 0xF
    hi = codes >> 4
    return np.stack([lo, hi], axis=-1).reshape(*codes.shape[:-1], codes.shape[-1] * 2)


def history(geo, n, rng, scale=1.0):
    k = rng.standard_normal((n, geo.nkv, geo.hd)) * scale
    v = rng.standard_normal((n, geo.nkv, geo.hd)) * scale
    return h16(k), h16(v)


@pytest.fixture(scope="module", autouse=True)
def _build(oracle):
    return oracle


def test_constant_group_scale_one_zero_x_codes_zero():
    rng = np.random.default_rng(0)
    k, v = history(GEO, 64, rng)
    kconst = rng.standard_normal((GEO.nkv, GEO.hd))
    vconst = rng.standard_normal((GEO.nkv, GEO.hd // 32))
    k[:32] = h16(np.broadcast_to(kconst, (32, GEO.nkv, GEO.hd)))
    v[:32] = h16(np.repeat(np.broadcast_to(vconst, (32, GEO.nkv, GEO.hd // 32)), 32, axis=-1))
    c = fresh()
    table = np.array([5, 2, 7, 1], np.int32)
    write_all(c, k, v, table)  # L = 64: group 0 aged out into page 5
    p = 5
    assert np.all(c.k_scale[p] == h16(1.0)), "K scale must fall back to 1.0"
    assert np.array_equal(c.k_zero[p], k[0])
    assert np.all(c.k_code[p] == 0)
    assert np.all(c.v_scale[p] == h16(1.0))
    assert np.array_equal(c.v_zero[p], h16(vconst)[None].repeat(32, 0).transpose(1, 0, 2))
    assert np.all(c.v_code[p] == 0)


def test_exact_ramp_gives_scale_s_and_codes_k():
    rng = np.random.default_rng(1)
    k, v = history(GEO, 64, rng)
    s, m = 0.25, -1.5
    # K: per channel a permutation of 0..15 (+ 16 more draws) over the 32 tokens
    kk = np.zeros((32, GEO.nkv, GEO.hd), np.int64)
    for h in range(GEO.nkv):
        for d in range(GEO.hd):
            col = np.concatenate([np.arange(16), rng.integers(0, 16, 16)])
            kk[:, h, d] = rng.permutation(col)
    k[:32] = h16(m + kk * s)
    # V: per token, per 32-channel group, the same ramp over channels
    vk = np.zeros((32, GEO.nkv, GEO.hd), np.int64)
    for t in range(32):
        for h in range(GEO.nkv):
            for g in range(GEO.hd // 32):
                col = np.concatenate([np.arange(16), rng.integers(0, 16, 16)])
                vk[t, h, 32 * g:32 * g + 32] = rng.permutation(col)
    v[:32] = h16(m + vk * s)
    c = fresh()
    table = np.array([3, 0, 6, 4], np.int32)
    write_all(c, k, v, table)
    p = 3
    assert np.all(c.k_scale[p] == h16(s)) and np.all(c.k_zero[p] == h16(m))
    assert np.array_equal(unpack(c.k_code[p]).transpose(1, 0, 2), kk)
    assert np.all(c.v_scale[p] == h16(s)) and np.all(c.v_zero[p] == h16(m))
    assert np.array_equal(unpack(c.v_code[p]).transpose(1, 0, 2), vk)


def test_two_value_group_codes_are_0_and_15():
    rng = np.random.default_rng(2)
    k, v = history(GEO, 64, rng)
    a, b = -0.7, 2.3
    pk = rng.integers(0, 2, (32, GEO.nkv, GEO.hd))
    pk[0], pk[1] = 0, 1  # K groups run over tokens: both values in every channel
    pv = rng.integers(0, 2, (32, GEO.nkv, GEO.hd))
    for g0 in range(0, GEO.hd, 32):  # V groups run over 32 channels of one token
        pv[:, :, g0], pv[:, :, g0 + 1] = 0, 1
    k[:32] = h16(np.where(pk == 1, b, a))
    v[:32] = h16(np.where(pv == 1, b, a))
    c = fresh()
    table = np.array([1, 2, 3, 4], np.int32)
    write_all(c, k, v, table)
    assert np.array_equal(unpack(c.k_code[1]), np.where(pk == 1, 15, 0).transpose(1, 0, 2))
    assert np.array_equal(unpack(c.v_code[1]), np.where(pv == 1, 15, 0).transpose(1, 0, 2))


def test_reconstruction_error_bound():
    rng = np.random.default_rng(3)
    k, v = history(GEO, 96, rng, scale=3.0)
    c = fresh()
    table = np.array([6, 1, 4, 0], np.int32)
    write_all(c, k, v, table)  # L = 96: groups 0, 1 aged out into pages 6, 1
    f = lambda x: np.asarray(x, np.uint16).view(np.float16).astype(np.float64)
    for grp, p in ((0, 6), (1, 1)):
        xk = f(k[32 * grp:32 * grp + 32]).transpose(1, 0, 2)  # [h, t, d]
        sk, zk = f(c.k_scale[p])[:, None, :], f(c.k_zero[p])[:, None, :]
        rk = unpack(c.k_code[p]) * sk + zk
        true_s = (xk.max(1, keepdims=True) - xk.min(1, keepdims=True)) / 15
        tol = true_s / 2 + 15 * np.abs(sk - true_s) + np.abs(zk - xk.min(1, keepdims=True)) + 1e-6
        assert np.all(np.abs(rk - xk) <= tol)
        xv = f(v[32 * grp:32 * grp + 32]).transpose(1, 0, 2).reshape(GEO.nkv, 32, -1, 32)
        sv, zv = f(c.v_scale[p])[..., None], f(c.v_zero[p])[..., None]
        rv = unpack(c.v_code[p]).reshape(GEO.nkv, 32, -1, 32) * sv + zv
        true_s = (xv.max(-1, keepdims=True) - xv.min(-1, keepdims=True)) / 15
        tol = true_s / 2 + 15 * np.abs(sv - true_s) + np.abs(zv - xv.min(-1, keepdims=True)) + 1e-6
        assert np.all(np.abs(rv - xv) <= tol)


@pytest.mark.parametrize("n", [1, 31, 32, 33, 63, 64, 65, 100])
def test_scratch_holds_the_residual_window(n):
    rng = np.random.default_rng(10 + n)
    k, v = history(GEO, n, rng)
    c = fresh()
    table = np.array([0, 1, 2, 3, 4, 5, 6, 7], np.int32)
    write_all(c, k, v, table)
    old = o.split_old_tokens(n, GEO.residual, GEO.group)
    assert old == max(0, n - GEO.residual) // 32 * 32
    res = n - old
    assert np.array_equal(c.k_scr[0][:, :res].transpose(1, 0, 2), k[old:n])
    assert np.array_equal(c.v_scr[0][:, :res].transpose(1, 0, 2), v[old:n])


def test_page16_codes_equal_page32_codes():
    rng = np.random.default_rng(4)
    k, v = history(GEO, 130, rng)
    g16 = o.Geometry(GEO.nh, GEO.nkv, GEO.hd, 16, 32, GEO.residual, 16)
    c32, c16 = fresh(GEO), fresh(g16, pages=16)
    t32 = np.array([2, 0, 3, 1, 5, 4, 7, 6], np.int32)
    t16 = np.array([9, 3, 0, 12, 5, 7, 1, 14, 2, 4, 6, 8, 10, 11, 13, 15], np.int32)
    write_all(c32, k, v, t32)
    write_all(c16, k, v, t16)
    ngroups = o.split_old_tokens(130, GEO.residual, 32) // 32
    assert ngroups == 3
    for gi in range(ngroups):
        p32 = t32[gi]
        pa, pb = t16[2 * gi], t16[2 * gi + 1]
        assert np.array_equal(c16.k_code[pa], c32.k_code[p32][:, :16])
        assert np.array_equal(c16.k_code[pb], c32.k_code[p32][:, 16:])
        assert np.array_equal(c16.v_code[pa], c32.v_code[p32][:, :16])
        assert np.array_equal(c16.v_scale[pb], c32.v_scale[p32][:, 16:])
        # K scales are per group: both pages of the group carry them
        for pp in (pa, pb):
            assert np.array_equal(c16.k_scale[pp], c32.k_scale[p32])
            assert np.array_equal(c16.k_zero[pp], c32.k_zero[p32])


@pytest.mark.parametrize("start,num", [(0, 1), (0, 40), (10, 60), (31, 2), (50, 33), (63, 64)])
def test_batched_write_equals_single_writes(start, num):
    rng = np.random.default_rng(start * 100 + num)
    n = start + num
    k, v = history(GEO, n, rng)
    table = np.array([7, 3, 5, 1, 0, 2, 4, 6], np.int32)
    single, batched = fresh(), fresh()
    write_all(single, k, v, table)
    write_all(batched, k[:start], v[:start], table)
    # the planner cuts the chunk so that every launch ages out at most one group
    for sub in o.plan_batched_write(start, num, GEO.residual, GEO.group):
        s0, cnt = sub[0], sub[1]
        o.cache_write_batched(batched, 0, k[s0:s0 + cnt], v[s0:s0 + cnt], table, s0)
    for f in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero"):
        assert np.array_equal(getattr(single, f), getattr(batched, f)), f
    res = n - o.split_old_tokens(n, GEO.residual, GEO.group)
    assert np.array_equal(single.k_scr[0][:, :res], batched.k_scr[0][:, :res])
    assert np.array_equal(single.v_scr[0][:, :res], batched.v_scr[0][:, :res])


def test_fp16_conversion_matches_numpy():
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 6, 4000),
        [0.0, -0.0, 65504.0, 65519.9, 65520.0, -65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
         np.inf, -np.inf, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11],
    ]).astype(np.float32)
    got = np.array([o.f32_to_f16_bits(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    bits = rng.integers(0, 0x7C00, 3000).astype(np.uint16)
    back = np.array([o.f16_bits_to_f32(int(b)) for b in bits], np.float32)
    assert np.array_equal(back, bits.view(np.float16).astype(np.float32))
