"""The fused step (jacq_kivi_write_decode): one launch appends a token to
every sequence -- aging a 32-token group out of the residual window where one
crosses it -- and decodes the new state.  The cache must end bit for bit as
the oracle's single-token write leaves it (integrations/vllm_kivi/
source_patch.py:1661-1697), stale scratch rows included, and every step's
decode must be within max-abs 2e-3 / rel 1e-2 of the float64 two-pass decode
of that state (the reference's write-then-decode order, :3259-3288)."""
from __future__ import annotations

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests.kivi_testlib import State, assert_close, geometry, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NAMES = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr")


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


def _compare_all(st: State, cache, what: str):
    for name, t in zip(NAMES, cache.pool()):
        got, want = _np(t), getattr(st.cache, name)
        assert np.array_equal(got, want), \
            f"{what}: {name} differs at {np.argwhere(got != want)[:5].tolist()}"


def _run_steps(kivi, w, lens, steps, seed, check_every=1):
    st = State(w, lens=lens, extra_tokens=steps, seed=seed)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    bt = torch.from_numpy(st.tables).cuda()
    hist_k = [torch.from_numpy(k).view(torch.float16).cuda() for k in st.k_hist]
    hist_v = [torch.from_numpy(v).view(torch.float16).cuda() for v in st.v_hist]
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    cur = np.asarray(lens).copy()
    aged = 0
    for step in range(steps):
        nk = torch.stack([hist_k[b][cur[b]] for b in range(st.batch)]).contiguous()
        nv = torch.stack([hist_v[b][cur[b]] for b in range(st.batch)]).contiguous()
        after = cur + 1
        out = cache.write_decode(q, nk, nv, torch.from_numpy(after.astype(np.int32)).cuda(), bt)
        for b in range(st.batch):
            o.cache_write(st.cache, b, st.k_hist[b][cur[b]], st.v_hist[b][cur[b]], st.tables[b],
                          int(after[b]))
            aged += int(wl.split_old_tokens(int(after[b]), w.residual)
                        > wl.split_old_tokens(int(cur[b]), w.residual))
        cur = after
        if step % check_every == 0 or step == steps - 1:
            torch.cuda.synchronize()
            _compare_all(st, cache, f"step {step}")
            assert_close(out.cpu().numpy(), st.decode_ref(cur), f"fused decode, step {step}")
    return aged


def test_write_decode_steps_cross_age_outs(kivi):
    """40 fused steps over ragged lengths that cross age-out boundaries at
    different steps (mistral geometry, page 16): after every step the whole
    pool and scratch equal the oracle's and the decode is within tolerance."""
    w = wl.WORKLOADS["mistral7b"].scaled(batch=6, ctx_lo=100)
    aged = _run_steps(kivi, w, [150, 155, 159, 190, 1, 2000], steps=40, seed=51)
    assert aged >= 5  # the steps did exercise the age-out path


@pytest.mark.parametrize("name", ["qwen14b", "qwen05b", "tinyllama"])
def test_write_decode_every_sequence_ages_out(kivi, name):
    """Age-out heavy: the first step ages a group out of every sequence at
    once (all lengths R + 31 + 32k before it), across GQA shapes and head
    dims, then steps with none and with some."""
    w = wl.WORKLOADS[name]
    R = w.residual
    lens = [R + 31 + 32 * k for k in (0, 1, 5, 30, 61, 100, 7, 2)]
    aged = _run_steps(kivi, w.scaled(batch=len(lens), ctx_lo=R), lens, steps=3, seed=52)
    assert aged >= len(lens)


def test_write_decode_equals_append_then_decode(kivi):
    """The fused step leaves the same cache bits as jacq_kivi_cache_append
    followed by jacq_kivi_decode, and decodes to the same values within the
    rounding of its own run split (its writer wavefronts take shorter runs,
    so the decode's cut differs)."""
    w = wl.WORKLOADS["qwen14b"].scaled(batch=8, ctx_lo=1000)
    lens = np.array([1000, 2207, 4095, 159, 160, 3000, 5000, 2048])
    st = State(w, lens=lens, extra_tokens=1, seed=53)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    a = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    b = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    bt = torch.from_numpy(st.tables).cuda()
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    nk = torch.stack([torch.from_numpy(st.k_hist[i][lens[i]]) for i in range(8)]).view(
        torch.float16).cuda()
    nv = torch.stack([torch.from_numpy(st.v_hist[i][lens[i]]) for i in range(8)]).view(
        torch.float16).cuda()
    after = torch.from_numpy((lens + 1).astype(np.int32)).cuda()
    fused = a.write_decode(q, nk, nv, after, bt)
    b.append(nk[:, None].contiguous(), nv[:, None].contiguous(), bt,
             torch.from_numpy(lens.astype(np.int32)).cuda())
    sep = b.decode(q, after, bt)
    torch.cuda.synchronize()
    for name, x, y in zip(NAMES, a.pool(), b.pool()):
        assert torch.equal(x.view(torch.uint8) if x.dtype == torch.uint8 else x.view(torch.int16),
                           y.view(torch.uint8) if y.dtype == torch.uint8 else y.view(torch.int16)), name
    assert torch.allclose(fused, sep, atol=1e-3, rtol=2e-3), (fused - sep).abs().max().item()
    for i in range(8):
        o.cache_write(st.cache, i, st.k_hist[i][lens[i]], st.v_hist[i][lens[i]], st.tables[i],
                      int(lens[i]) + 1)
    assert_close(fused.cpu().numpy(), st.decode_ref(lens + 1), "fused vs oracle")


def test_write_decode_graph_replays(kivi):
    """The fused step captured in a HIP graph (the writer flags are cleared by
    the wavefront or merge that finishes each aging segment, so a replay,
    which repeats the launch's epoch, starts from zero flags): replays with new
    tokens and lengths copied in between advance the cache exactly as eager
    fused steps do, bit for bit, across age-outs."""
    w = wl.WORKLOADS["qwen14b"].scaled(batch=4, ctx_lo=150)
    lens = np.array([158, 180, 1000, 2302])
    st = State(w, lens=lens, extra_tokens=8, seed=54)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    eager = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    graphed = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    bt = torch.from_numpy(st.tables).cuda()
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    hk = [torch.from_numpy(k).view(torch.float16).cuda() for k in st.k_hist]
    hv = [torch.from_numpy(v).view(torch.float16).cuda() for v in st.v_hist]
    nbytes = kivi.lib().jacq_kivi_write_decode_workspace_size(
        __import__("ctypes").byref(geo.c()), st.batch)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    nk_in = torch.empty((4, w.nkv, w.hd), dtype=torch.float16, device="cuda")
    nv_in = torch.empty_like(nk_in)
    len_in = torch.empty(4, dtype=torch.int32, device="cuda")
    out = torch.empty((4, w.nh, w.hd), dtype=torch.float32, device="cuda")
    # a throwaway cache for the capture's own launch
    spare = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    nk_in.copy_(torch.stack([hk[b][lens[b]] for b in range(4)]))
    nv_in.copy_(torch.stack([hv[b][lens[b]] for b in range(4)]))
    len_in.copy_(torch.from_numpy((lens + 1).astype(np.int32)))
    spare.write_decode(q, nk_in, nv_in, len_in, bt, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.write_decode(q, nk_in, nv_in, len_in, bt, out=out, workspace=ws)
    # the capture did not run; the graphed cache is still the initial state
    cur = lens.copy()
    for step in range(8):
        nk_in.copy_(torch.stack([hk[b][cur[b]] for b in range(4)]))
        nv_in.copy_(torch.stack([hv[b][cur[b]] for b in range(4)]))
        len_in.copy_(torch.from_numpy((cur + 1).astype(np.int32)))
        graph.replay()
        ref = eager.write_decode(q, nk_in.clone(), nv_in.clone(), len_in.clone(), bt)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {step}"
        for x, y in zip(graphed.pool(), eager.pool()):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"cache after replay {step}"
        cur += 1


FUSED_GEOMETRIES = {
    # page 32 at the v1 shape (GQA 5, the packed HD-128 kernel)
    "v1_p32": wl.Workload("fv1", 40, 8, 128, 5, 160, 160, page=32, residual=128, outliers=8,
                          outlier_scale=10.0, seed=61),
    # HD 64 with GQA 10 (the unpacked kernel), page 32
    "hd64_g10_p32": wl.Workload("f64", 40, 4, 64, 5, 160, 160, page=32, residual=128,
                                outliers=4, outlier_scale=8.0, seed=62),
    # HD 128 with GQA 16 (unpacked), page 16, and a 64-token residual window
    "hd128_g16_r64": wl.Workload("f128", 32, 2, 128, 5, 96, 96, page=16, residual=64,
                                 outliers=4, outlier_scale=8.0, seed=63),
}


@pytest.mark.parametrize("name", list(FUSED_GEOMETRIES))
def test_write_decode_other_geometries(kivi, name):
    """The fused step on the other kernel instantiations (page 32, HD 64,
    GQA above 8 -- the unpacked kernels -- and another residual window):
    bit-exact cache and in-tolerance decode over steps that cross age-outs."""
    w = FUSED_GEOMETRIES[name]
    R = w.residual
    lens = [R + 31, R + 30 + 32 * 3, R + 1, R + 17 + 32 * 40, 2]
    aged = _run_steps(kivi, w, lens, steps=34, seed=64, check_every=3)
    assert aged >= 3


def test_write_decode_merge_timeout_is_reported(kivi):
    """Failure handling in the fused step, forced from the host (the merge
    waits for a tag nobody stores and gives up after 20 us): the launch ends,
    the writer's work is complete and bit-exact (it waits for nothing), whole
    segments decode correctly and merged ones are NaN; the next fused step is
    refused without launching (cache and output untouched) until
    jacq_kivi_decode_status resets, after which the step is correct again."""
    from tests.test_gpu_parity import _segment_counts

    w = wl.WORKLOADS["qwen14b"]
    lens = np.array([3000, 159, 20, 700, 1])
    st = State(w, lens=lens, extra_tokens=2, seed=71)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    bt = torch.from_numpy(st.tables).cuda()
    q = torch.from_numpy(st.q).view(torch.float16).cuda()

    def token(i):
        nk = torch.stack([torch.from_numpy(st.k_hist[b][int(lens[b]) + i].copy())
                          for b in range(st.batch)]).view(torch.float16).cuda()
        nv = torch.stack([torch.from_numpy(st.v_hist[b][int(lens[b]) + i].copy())
                          for b in range(st.batch)]).view(torch.float16).cuda()
        return nk, nv

    def oracle_step(i):
        for b in range(st.batch):
            o.cache_write(st.cache, b, st.k_hist[b][int(lens[b]) + i],
                          st.v_hist[b][int(lens[b]) + i], st.tables[b], int(lens[b]) + i + 1)

    kivi.decode_status()  # nothing pending
    nk, nv = token(0)
    after = torch.from_numpy((lens + 1).astype(np.int32)).cuda()
    kivi.lib().jacq_kivi_test_force_merge_timeout(20)
    try:
        out = cache.write_decode(q, nk, nv, after, bt)
        torch.cuda.synchronize()
    finally:
        kivi.lib().jacq_kivi_test_force_merge_timeout(0)
    oracle_step(0)
    _compare_all(st, cache, "after the timed-out step")
    counts = _segment_counts(w, out.cpu().numpy().astype(np.float64), st.decode_ref(lens + 1))
    assert counts["other"] == 0 and counts["nan"] >= 1 and counts["match"] >= 1, counts
    # refused: nothing launched, the cache keeps the state of the step above
    nk, nv = token(1)
    after2 = torch.from_numpy((lens + 2).astype(np.int32)).cuda()
    sentinel = torch.full_like(out, 7.0)
    with pytest.raises(kivi.KiviMergeTimeout, match="timed out"):
        cache.write_decode(q, nk, nv, after2, bt, out=sentinel)
    torch.cuda.synchronize()
    assert bool((sentinel == 7.0).all()), "a refused step must not launch"
    _compare_all(st, cache, "after the refused step")
    with pytest.raises(kivi.KiviMergeTimeout, match="reset"):
        kivi.decode_status()
    out = cache.write_decode(q, nk, nv, after2, bt)
    torch.cuda.synchronize()
    oracle_step(1)
    _compare_all(st, cache, "after the reset")
    assert_close(out.cpu().numpy(), st.decode_ref(lens + 2), "fused step after the reset")


def test_write_decode_up_to_table_capacity(kivi):
    """The fused step up to exactly the block table's capacity: tables cut to
    (max_seq_len - R) / page entries, so the last step of sequence 0 ages the
    group that fills the table's last pages (255 -> 256 = max_seq_len)."""
    w = wl.WORKLOADS["qwen14b"].scaled(batch=2, ctx_lo=200)
    lens = np.array([250, 200])
    steps = 6
    st = State(w, lens=lens, extra_tokens=steps, seed=81)
    mp = (256 - w.residual) // w.page  # 8 pages of 16: max_seq_len 256
    st.tables = np.ascontiguousarray(st.tables[:, :mp])
    st.max_pages = mp
    st.geo = geometry(w, mp)
    st.cache = o.Cache.empty(st.geo, st.num_pages, st.batch)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, mp, st.num_pages)
    assert geo.max_seq_len() == 256
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    bt = torch.from_numpy(st.tables).cuda()
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    cur = lens.copy()
    for s in range(steps):
        nk = torch.stack([torch.from_numpy(st.k_hist[b][cur[b]].copy())
                          for b in range(2)]).view(torch.float16).cuda()
        nv = torch.stack([torch.from_numpy(st.v_hist[b][cur[b]].copy())
                          for b in range(2)]).view(torch.float16).cuda()
        after = cur + 1
        out = cache.write_decode(q, nk, nv, torch.from_numpy(after.astype(np.int32)).cuda(), bt)
        for b in range(2):
            o.cache_write(st.cache, b, st.k_hist[b][cur[b]], st.v_hist[b][cur[b]], st.tables[b],
                          int(after[b]))
        cur = after
        torch.cuda.synchronize()
        _compare_all(st, cache, f"step {s}")
        assert_close(out.cpu().numpy(), st.decode_ref(cur), f"capacity step {s}")
    assert int(cur[0]) == geo.max_seq_len()
