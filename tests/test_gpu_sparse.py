"""GPU parity of sparse-retained decode (jac_launch_sparse_retained,
crates/jac-codegen-cuda/src/variants.rs:2620-2740) through the C ABI against
the oracle's float64 two-pass attention over the same sparse window.

The compact table lists the physical pages of the retained old pages in any
order; the residual window stays at the dense SEQ_LEN boundary.  Outputs
within max-abs 2e-3 / rel 1e-2 of the reference.
"""
from __future__ import annotations

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests.kivi_testlib import State, assert_close, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V1 = wl.Workload("v1", 40, 8, 128, 1, 4096, 4096, page=32, residual=128, outliers=8,
                 outlier_scale=10.0, seed=11)
TP2 = wl.Workload("v1tp2", 20, 4, 128, 1, 4096, 4096, page=32, residual=128, outliers=8,
                  outlier_scale=10.0, seed=12)
POOL = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")


@pytest.fixture(scope="module")
def kivi():
    from jacq_amd import kivi as k
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    k.lib()
    return k


def _retained(dense_pages: int, keep: int, seed: int) -> np.ndarray:
    """logical pages kept after eviction, in a shuffled order"""
    rng = np.random.default_rng(seed)
    return rng.permutation(dense_pages)[:keep]


@pytest.mark.parametrize("w", [V1, TP2], ids=["v1", "tp2_local"])
def test_v1_sparse_retained_matches_oracle(kivi, w):
    st = State(w, lens=[4096], seed=5)
    st.build_oracle()
    g = to_torch(st)
    pool = [g[n] for n in POOL]
    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    table = st.tables[0]
    for L, keep in ((4096, 60), (4096, 124), (4096, 0), (3000, 17), (1000, 200), (200, 1)):
        print(f"[sparse v1] {w.name} L={L} keep={keep}", flush=True)
        dense_pages = max(0, (L - 128) // 32)
        logical = _retained(dense_pages, min(keep, dense_pages), seed=L + keep)
        compact = np.zeros(124, np.int32)  # the op takes an OLD_BLOCKS-entry table
        compact[:len(logical)] = table[logical]
        ct = torch.from_numpy(compact).cuda()
        n_ret = min(keep, 124)
        out = torch.empty((w.nh, 128), dtype=torch.float32, device="cuda")
        kivi.kivi_decode_sparse_retained_dsl(q, ct, *pool, g["k_scr"][0], g["v_scr"][0], L,
                                             n_ret, out)
        torch.cuda.synchronize()
        ref = o.decode_sparse_retained(st.cache, 0, st.q[0], compact, L, n_ret, twopass=True)
        assert_close(out.cpu().numpy(), ref, f"sparse {w.name} L={L} keep={keep}")
        if keep >= dense_pages and L == 4096:
            # in logical order, full retention is the dense decode
            dense = torch.empty_like(out)
            kivi.kivi_decode_dsl(q, torch.from_numpy(table).cuda(), *pool, g["k_scr"][0],
                                 g["v_scr"][0], L, dense)
            ordered = torch.empty_like(out)
            kivi.kivi_decode_sparse_retained_dsl(q, torch.from_numpy(table[:124].copy()).cuda(),
                                                 *pool,
                                                 g["k_scr"][0], g["v_scr"][0], L, n_ret,
                                                 ordered)
            torch.cuda.synchronize()
            assert torch.equal(ordered, dense)


def test_v1_sparse_validators(kivi):
    """The reference op's rejections (source_patch.py:872-951)."""
    st = State(V1, lens=[300], seed=6)
    st.build_oracle()
    g = to_torch(st)
    pool = [g[n] for n in POOL]
    q = torch.zeros((40, 128), dtype=torch.float16, device="cuda")
    out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
    ct = torch.zeros(124, dtype=torch.int32, device="cuda")
    bad = [
        (dict(n_ret=125), "NUM_RETAINED_PAGES must be in"),
        (dict(n_ret=-1), "NUM_RETAINED_PAGES must be in"),
        (dict(L=0), "SEQ_LEN must be in"),
        (dict(L=4097), "SEQ_LEN must be in"),
        (dict(table=torch.zeros(123, dtype=torch.int32, device="cuda")), "RETAINED_BLOCK_TABLE"),
        (dict(table=torch.zeros(124, dtype=torch.int64, device="cuda")), "int32"),
    ]
    for kw, msg in bad:
        with pytest.raises(kivi.KiviCheckError, match=msg):
            kivi.kivi_decode_sparse_retained_dsl(q, kw.get("table", ct), *pool, g["k_scr"][0],
                                                 g["v_scr"][0], kw.get("L", 300),
                                                 kw.get("n_ret", 1), out)


@pytest.mark.parametrize("page", [16, 32])
def test_runtime_sparse_retained_matches_oracle(kivi, page):
    """jacq_kivi_decode_sparse_retained at the 14B head shape (page 16 and 32)."""
    w = wl.WORKLOADS["qwen14b"].scaled(batch=1, ctx_lo=5000, page=page)
    st = State(w, lens=[5000], seed=9)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    table = st.tables[0]
    per = 32 // page
    dense_groups = (5000 - w.residual) // 32
    for keep_groups in (0, 1, 37, dense_groups):
        print(f"[sparse runtime] page={page} groups={keep_groups}", flush=True)
        groups = _retained(dense_groups, keep_groups, seed=keep_groups)
        compact = np.concatenate([table[gi * per:(gi + 1) * per] for gi in groups]
                                 + [np.zeros(0, np.int32)]).astype(np.int32)
        n_ret = len(compact)
        ct = torch.from_numpy(np.concatenate([compact, np.zeros(1, np.int32)])).cuda()
        out = cache.decode_sparse_retained(q, 5000, ct, n_ret)
        torch.cuda.synchronize()
        ref = o.decode_sparse_retained(st.cache, 0, st.q[0], compact, 5000, n_ret, twopass=True)
        assert_close(out.cpu().numpy(), ref, f"runtime sparse page={page} groups={keep_groups}")
