"""GPU writer on adversarial quantisation groups: bit-exact against the oracle
and the independent numpy restatement (tests/kivi_numpy_quant.py).

The groups hold NaN / +-inf in the first and middle positions, +-0 mixes,
subnormals, exact .5 ties, values at +-65504 and reciprocal-sensitive ties
(the fminf / fmaxf semantics of source_patch.py:1555-1558, :1598-1599).
"""
from __future__ import annotations

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests import kivi_numpy_quant as nq
from tests.kivi_testlib import State, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FIELDS = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")


@pytest.fixture(scope="module")
def kivi():
    from jacq_amd import kivi as k
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    k.lib()
    return k


def _np(t):
    x = t.detach().cpu()
    if x.dtype == torch.float16:
        return x.view(torch.int16).numpy().view(np.uint16)
    return x.numpy()


def _adversarial_state(w, n_tokens, seed):
    """State whose first 32 tokens (every sequence) are an adversarial group."""
    st = State(w, lens=[n_tokens] * w.batch, seed=seed)
    rng = np.random.default_rng(seed + 1000)
    for b in range(st.batch):
        k, v = nq.adversarial_group(rng, w.nkv, w.hd)
        st.k_hist[b][:32] = k
        st.v_hist[b][:32] = v
    return st


def _check_first_group(st, got, what):
    for b in range(st.batch):
        ref = {f: getattr(st.cache, f) for f in FIELDS}
        pages = st.tables[b][: 32 // st.w.page]
        for f in FIELDS:
            g, r = got[f][pages], ref[f][pages]
            bad = np.argwhere(g != r)
            assert bad.size == 0, f"{what}: seq {b} {f} differs from the oracle at {bad[:4].tolist()}"
        # and the oracle equals the numpy restatement on the same group
        want = nq.quantise_group(st.k_hist[b][:32], st.v_hist[b][:32])
        if st.w.page == 32:
            p = pages[0]
            for f in FIELDS:
                assert np.array_equal(got[f][p], want[f]), f"{what}: seq {b} {f} vs numpy"


def test_v1_writer_adversarial_groups(kivi):
    """jac_launch_cache_write token by token (v1 geometry) ages an adversarial
    group out at L = 160: pages bit-exact against oracle and numpy."""
    w = wl.Workload("v1adv", 40, 8, 128, 1, 170, 170, page=32, residual=128, seed=3)
    st = _adversarial_state(w, 170, 3)
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    stream = kivi._stream(torch.device("cuda"))
    for t in range(170):
        nk = torch.from_numpy(st.k_hist[0][t].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][t].copy()).view(torch.float16).cuda()
        kivi.lib().jac_launch_cache_write(
            *[kivi._ptr(g[n]) for n in FIELDS], kivi._ptr(g["k_scr"][0]),
            kivi._ptr(g["v_scr"][0]), kivi._ptr(nk), kivi._ptr(nv), kivi._ptr(bt), t + 1, stream)
    st.build_oracle()
    torch.cuda.synchronize()
    _check_first_group(st, {f: _np(g[f]) for f in FIELDS}, "v1 writer")


@pytest.mark.parametrize("name", ["qwen05b", "qwen14b"])
def test_runtime_append_adversarial_groups(kivi, name):
    """jacq_kivi_cache_append of whole histories (page 16, HD 64 / 128)."""
    w = wl.WORKLOADS[name].scaled(batch=2, ctx_lo=200, ctx_hi=200)
    st = _adversarial_state(w, 200, 5)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache(geo, st.batch)
    nk = torch.from_numpy(np.stack(st.k_hist)).view(torch.float16).cuda()
    nv = torch.from_numpy(np.stack(st.v_hist)).view(torch.float16).cuda()
    cache.append(nk, nv, torch.from_numpy(st.tables).cuda(),
                 torch.zeros(st.batch, dtype=torch.int32, device="cuda"))
    st.build_oracle()
    torch.cuda.synchronize()
    got = dict(zip(FIELDS, [_np(t) for t in cache.pool()[:6]]))
    _check_first_group(st, got, f"append {name}")
    # page 16 tables: compare numpy on the group's two pages joined
    for b in range(st.batch):
        want = nq.quantise_group(st.k_hist[b][:32], st.v_hist[b][:32])
        pa, pb = st.tables[b][0], st.tables[b][1]
        assert np.array_equal(np.concatenate([got["k_code"][pa], got["k_code"][pb]], 1),
                              want["k_code"])
        assert np.array_equal(got["k_scale"][pa], want["k_scale"])
        assert np.array_equal(got["k_zero"][pb], want["k_zero"])
        assert np.array_equal(np.concatenate([got["v_zero"][pa], got["v_zero"][pb]], 1),
                              want["v_zero"])
