"""Independent numpy restatement of the KIVI group quantiser, plus the
adversarial groups that pin the oracle's writer (test infrastructure).

The reference's age-out kernels (integrations/vllm_kivi/source_patch.py:
1532-1581 for K, :1583-1620 for V) compute, per 32-value group,
    mn = fminf-reduce, mx = fmaxf-reduce          (fp32 of the fp16 inputs)
    scale = (mx - mn) / 15.0f ;  if !(scale > 0) scale = 1
    code  = clamp(static_cast<int>(rintf((x - mn) / scale)), 0, 15)
and store half(scale), half(mn) with round-to-nearest-even.

This module computes the same quantities by different means than the C
oracle's loops:
  * min / max are the extremes of a total order on the non-NaN values, found
    with argmin / argmax over integer keys of the float bits (-0 < +0), NaN
    lanes masked out; a group of only NaN keeps its first element (fminf of
    two NaN is NaN);
  * the arithmetic is whole-array float32 numpy (IEEE, correctly rounded);
  * the float -> int conversion is the saturating one CUDA's cvt.rzi.s32.f32
    performs (NaN -> 0), written with np.where on the float values.

`MUTANTS` are quantisers with one plausible mistake each; the tests check
that the adversarial groups tell every one of them apart from the oracle, so
the agreement of oracle and restatement is not vacuous.
"""
from __future__ import annotations

import numpy as np

GROUP = 32
QNAN = np.uint16(0x7E00)
NEG_QNAN = np.uint16(0xFE00)


def f16(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16)


def _order_key(x: np.ndarray) -> np.ndarray:
    """int64 keys with key(a) < key(b) iff a < b for non-NaN float32, -0 < +0."""
    u = x.astype(np.float32).view(np.int32).astype(np.int64)
    return np.where(u < 0, -1 - (u & 0x7FFFFFFF), u)


def group_min_max(x: np.ndarray, axis: int = -1) -> tuple[np.ndarray, np.ndarray]:
    """fminf / fmaxf reductions of float32 `x` along `axis`."""
    x = np.moveaxis(np.asarray(x, np.float32), axis, -1)
    nan = np.isnan(x)
    key = _order_key(x)
    big = np.iinfo(np.int64).max
    imin = np.argmin(np.where(nan, big, key), axis=-1)
    imax = np.argmax(np.where(nan, -big, key), axis=-1)
    # all-NaN groups: argmin / argmax of a constant row is index 0 = the first NaN
    mn = np.take_along_axis(x, imin[..., None], -1)[..., 0]
    mx = np.take_along_axis(x, imax[..., None], -1)[..., 0]
    return mn, mx


def quantise(x16: np.ndarray, axis: int = -1, *, scale_fp16_divide=False,
             reciprocal=False, ties_away=False, compare_select=False):
    """Quantise fp16 bit groups of 32 along `axis`.

    Returns (codes uint8 shaped like x16, scale bits, zero bits) with the
    reduced axis removed from scale / zero.  The keyword switches build the
    mutants (each one plausible mistake)."""
    x = f16(x16).astype(np.float32)
    x = np.moveaxis(x, axis, -1)
    assert x.shape[-1] == GROUP
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        if compare_select:  # running `x < cur ? x : cur` from the first element
            mn = x[..., 0].copy()
            mx = x[..., 0].copy()
            for t in range(1, GROUP):
                mn = np.where(x[..., t] < mn, x[..., t], mn)
                mx = np.where(x[..., t] > mx, x[..., t], mx)
        else:
            mn, mx = group_min_max(x)
        scale = (mx - mn) / np.float32(15.0)
        scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
        div = scale.astype(np.float16).astype(np.float32) if scale_fp16_divide else scale
        if reciprocal:
            q = (x - mn[..., None]) * (np.float32(1.0) / div)[..., None]
        else:
            q = (x - mn[..., None]) / div[..., None]
        q = q.astype(np.float32)
        r = np.floor(q + np.float32(0.5)) if ties_away else np.rint(q)
        code = np.where(r >= 15, 15, np.where(r >= 0, r, 0))
        code = np.nan_to_num(code, nan=0.0).astype(np.uint8)
        scale_bits = scale.astype(np.float16).view(np.uint16)
        zero_bits = mn.astype(np.float16).view(np.uint16)
    return np.moveaxis(code, -1, axis), scale_bits, zero_bits


MUTANTS = {
    "divide by the fp16 scale": dict(scale_fp16_divide=True),
    "multiply by a reciprocal": dict(reciprocal=True),
    "round ties away from zero": dict(ties_away=True),
    "compare-select min/max (NaN kept)": dict(compare_select=True),
}


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[..., HD] codes -> [..., HD/2] bytes, channel 2j in the low nibble."""
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def quantise_group(k16: np.ndarray, v16: np.ndarray, **mut):
    """One aged group of one sequence: k16 / v16 [32, NKV, HD] fp16 bits.

    Returns dict of the page contents at page size 32 (layout of
    source_patch.py:1565-1578, :1604): k_code/v_code [NKV, 32, HD/2],
    k_scale/k_zero [NKV, HD], v_scale/v_zero [NKV, 32, HD/32]."""
    T, nkv, hd = k16.shape
    kc, ks, kz = quantise(k16, axis=0, **mut)                     # over tokens
    vg = v16.reshape(T, nkv, hd // GROUP, GROUP)
    vc, vs, vz = quantise(vg, axis=-1, **mut)                     # over 32 channels
    return {
        "k_code": pack_nibbles(kc.transpose(1, 0, 2)),
        "k_scale": ks, "k_zero": kz,
        "v_code": pack_nibbles(vc.reshape(T, nkv, hd).transpose(1, 0, 2)),
        "v_scale": vs.transpose(1, 0, 2), "v_zero": vz.transpose(1, 0, 2),
    }


# ---------------------------------------------------------------- adversarial groups

def _bits(vals) -> np.ndarray:
    return np.asarray(vals, np.float32).astype(np.float16).view(np.uint16)


def _reciprocal_ties(rng: np.random.Generator, n: int) -> list[np.ndarray]:
    """Columns where (x - mn) / s and (x - mn) * (1/s) round to different
    codes: mn = 0 and max = 15 s pin the scale to s; x is searched for."""
    out = []
    one = np.float32(1.0)
    tries = 0
    while len(out) < n and tries < 200000:
        tries += 1
        s16 = np.float16(rng.uniform(0.01, 4.0))
        s = np.float32(s16)
        top = np.float16(np.float32(15.0) * s)
        if np.float32(top) / np.float32(15) != s:
            continue
        x = np.float16(rng.uniform(0, 15) * s)
        q_div = np.float32(x) / s
        q_rec = np.float32(x) * (one / s)
        if np.rint(q_div) != np.rint(q_rec):
            col = np.concatenate([[0.0, float(top), float(x)], rng.uniform(0, float(top), 29)])
            out.append(_bits(col))
    return out


def adversarial_columns(rng: np.random.Generator) -> list[np.ndarray]:
    """32-value fp16 columns that stress the quantiser's special cases."""
    cols = []
    r = lambda n=GROUP, sc=1.0: rng.standard_normal(n) * sc
    # plain random, and spread close to the fp16 limit
    cols += [_bits(r()) for _ in range(4)]
    cols += [_bits(rng.uniform(-65504, 65504, GROUP)) for _ in range(2)]
    cols.append(_bits(np.concatenate([[65504.0, -65504.0], rng.uniform(-1, 1, 30)])))
    # NaN first, NaN mid-group, all NaN, mixed-sign NaNs
    for pos in (0, 0, 13, 31):
        c = _bits(r())
        c[pos] = QNAN
        cols.append(c)
    c = _bits(r()); c[0] = NEG_QNAN; c[7] = QNAN; cols.append(c)
    cols.append(np.full(GROUP, QNAN, np.uint16))
    c = np.full(GROUP, QNAN, np.uint16); c[5] = _bits([2.5])[0]; cols.append(c)
    # infinities
    c = _bits(r()); c[0] = _bits([np.inf])[0]; cols.append(c)
    c = _bits(r()); c[9] = _bits([-np.inf])[0]; cols.append(c)
    c = _bits(r()); c[3] = _bits([np.inf])[0]; c[4] = _bits([-np.inf])[0]; cols.append(c)
    # signed zeros
    z, nz = _bits([0.0])[0], _bits([-0.0])[0]
    cols.append(np.where(rng.integers(0, 2, GROUP) == 1, z, nz).astype(np.uint16))
    c = np.full(GROUP, z, np.uint16); c[17] = nz; cols.append(c)
    c = np.full(GROUP, nz, np.uint16); c[0] = z; cols.append(c)
    c = _bits(np.abs(r())); c[0] = nz; c[1] = z; cols.append(c)            # min is a zero
    c = _bits(-np.abs(r())); c[0] = z; c[2] = nz; cols.append(c)           # max is a zero
    # subnormal fp16 values (multiples of 2^-24)
    cols.append(rng.integers(0, 0x400, GROUP).astype(np.uint16))
    cols.append((rng.integers(0, 0x400, GROUP) | 0x8000).astype(np.uint16))
    c = np.zeros(GROUP, np.uint16); c[0] = 1; cols.append(c)               # range 2^-24
    # exact .5 ties: mn = 0, mx = 15 s, x = (k + 1/2) s, all exact in fp16
    for s in (0.25, 0.5, 2.0):
        k = rng.integers(0, 15, GROUP - 2)
        cols.append(_bits(np.concatenate([[0.0, 15 * s], (k + 0.5) * s])))
    # constant and two-valued columns
    cols.append(_bits(np.full(GROUP, 1.375)))
    cols.append(_bits(np.where(rng.integers(0, 2, GROUP) == 1, -3.0, 7.0)))
    cols += _reciprocal_ties(rng, 6)
    return cols


def adversarial_group(rng: np.random.Generator, nkv: int, hd: int):
    """K and V tiles [32, NKV, HD] (fp16 bits) whose quantisation groups are
    the adversarial columns, in every K channel (over tokens) and every V
    (token, channel group) (over channels), the rest random."""
    cols = adversarial_columns(rng)
    k = _bits(rng.standard_normal((GROUP, nkv, hd)))
    v = _bits(rng.standard_normal((GROUP, nkv, hd)))
    for i in range(nkv * hd):
        k[:, i // hd, i % hd] = cols[i % len(cols)]
    groups = hd // GROUP
    for i in range(GROUP * nkv * groups):
        t, rest = divmod(i, nkv * groups)
        h, g = divmod(rest, groups)
        v[t, h, g * GROUP:(g + 1) * GROUP] = cols[(i + 7) % len(cols)]
    return k, v
