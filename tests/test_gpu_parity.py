"""GPU parity: the HIP writer and decode through the C ABI versus the CPU oracle.

Writer state (codes, scales, zeros, scratch) must be bit-exact; attention
outputs within max-abs 2e-3 / rel 1e-2 of the float64 two-pass reference.
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


@pytest.fixture(scope="module")
def kivi():
    from jacq_amd import kivi as k
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    k.lib()
    return k


def _np(t):
    x = t.detach().cpu()
    if x.dtype == torch.float16:
        x = x.view(torch.int16)
    return x.numpy().view(np.uint16) if x.dtype == torch.int16 else x.numpy()


def _compare_pool(st: State, g: dict, scratch_rows=None, what=""):
    c = st.cache
    for name in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero"):
        ref = getattr(c, name)
        got = _np(g[name])
        assert np.array_equal(got, ref), f"{what}: {name} differs at {np.argwhere(got != ref)[:5]}"
    for name in ("k_scr", "v_scr"):
        ref = getattr(c, name)
        got = _np(g[name])
        if scratch_rows is None:
            assert np.array_equal(got, ref), f"{what}: {name} differs"
        else:
            for b, r in enumerate(scratch_rows):
                assert np.array_equal(got[b, :, :r], ref[b, :, :r]), f"{what}: {name}[{b}] differs"


# ---------------------------------------------------------------- writer

def test_v1_single_token_writer_bit_exact(kivi):
    """jac_launch_cache_write token by token through 3 age-outs: pages AND the
    whole scratch (stale rows included) equal the reference's serial writer."""
    st = State(V1, lens=[256], seed=5)
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    for t in range(256):
        nk = torch.from_numpy(st.k_hist[0][t].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][t].copy()).view(torch.float16).cuda()
        kivi.lib().jac_launch_cache_write(
            *[kivi._ptr(g[n]) for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale",
                                        "v_zero")],
            kivi._ptr(g["k_scr"][0]), kivi._ptr(g["v_scr"][0]), kivi._ptr(nk), kivi._ptr(nv),
            kivi._ptr(bt), t + 1, kivi._stream(nk.device))
        o.cache_write(st.cache, 0, st.k_hist[0][t], st.v_hist[0][t], st.tables[0], t + 1)
        if (t + 1) in (159, 160, 161, 192, 224, 256):
            torch.cuda.synchronize()
            _compare_pool(st, g, what=f"after token {t + 1}")


def test_torch_op_mirrors_write_then_decode(kivi):
    """kivi_cache_write_dsl / kivi_decode_dsl (reference op surface) at the v1
    geometry, global and TP=2 local."""
    for nh, nkv in ((40, 8), (20, 4)):
        w = wl.Workload("v1op", nh, nkv, 128, 1, 300, 300, page=32, residual=128, outliers=4,
                        outlier_scale=10.0, seed=nh)
        st = State(w, lens=[300])
        g = to_torch(st)
        bt = torch.from_numpy(st.tables[0]).cuda()
        slot = torch.zeros(1, dtype=torch.int64, device="cuda")
        pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
        for t in range(300):
            nk = torch.from_numpy(st.k_hist[0][t].copy()).view(torch.float16).cuda()
            nv = torch.from_numpy(st.v_hist[0][t].copy()).view(torch.float16).cuda()
            kivi.kivi_cache_write_dsl(*pool, g["k_scr"][0], g["v_scr"][0], nk, nv, slot, bt, t + 1)
        st.build_oracle()
        torch.cuda.synchronize()
        _compare_pool(st, g, what=f"op writer {nh}/{nkv}")
        q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
        out = torch.empty((nh, 128), dtype=torch.float32, device="cuda")
        kivi.kivi_decode_dsl(q, bt, *pool, g["k_scr"][0], g["v_scr"][0], 300, out)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy()[None], st.decode_ref(), f"kivi_decode_dsl {nh}/{nkv}")


def test_batched_writer_matches_planned_single_writes(kivi):
    """kivi_cache_write_batched_dsl over plan_batched_write sub-chunks of a
    600-token prefill == the oracle's single-token writes."""
    st = State(V1, lens=[600], seed=6)
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    for (start, n, _, _, _) in kivi.plan_batched_write(0, 600):
        nk = torch.from_numpy(st.k_hist[0][start:start + n].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][start:start + n].copy()).view(torch.float16).cuda()
        slot = torch.zeros(n, dtype=torch.int64, device="cuda")
        kivi.kivi_cache_write_batched_dsl(*pool, g["k_scr"][0], g["v_scr"][0], nk, nv, slot, bt,
                                          start, n)
    st.build_oracle()
    torch.cuda.synchronize()
    _compare_pool(st, g, what="batched writer")


@pytest.mark.parametrize("name", ["tinyllama", "qwen05b", "long"])
def test_runtime_append_multi_age_out(kivi, name):
    """jacq_kivi_cache_append with whole histories in one launch (many
    age-outs per sequence), page 16, HD 64/128, R 32/128 == oracle."""
    w = wl.WORKLOADS[name].scaled(batch=3, ctx_lo=700, ctx_hi=700)
    st = State(w, lens=[700, 700, 700])
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache(geo, st.batch)
    nk = torch.from_numpy(np.stack(st.k_hist)).view(torch.float16).cuda()
    nv = torch.from_numpy(np.stack(st.v_hist)).view(torch.float16).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    cache.append(nk, nv, bt, torch.zeros(st.batch, dtype=torch.int32, device="cuda"))
    st.build_oracle()
    torch.cuda.synchronize()
    g = dict(zip(("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr"),
                 cache.pool()))
    res = [700 - wl.split_old_tokens(700, w.residual)] * 3
    _compare_pool(st, g, scratch_rows=res, what=f"append {name}")


def test_runtime_step_writes_then_decode(kivi):
    """Per-step writer (1 token per sequence, ragged lengths crossing age-out
    boundaries) then decode, mistral geometry at page 16."""
    w = wl.WORKLOADS["mistral7b"].scaled(batch=4, ctx_lo=150)
    lens = np.array([150, 155, 159, 190])
    st = State(w, lens=lens, extra_tokens=40)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache(geo, st.batch)
    bt = torch.from_numpy(st.tables).cuda()
    hist_k = [torch.from_numpy(k).view(torch.float16).cuda() for k in st.k_hist]
    hist_v = [torch.from_numpy(v).view(torch.float16).cuda() for v in st.v_hist]
    for b in range(st.batch):  # per-sequence prefill through one-sequence views
        L = int(lens[b])
        cache.sequence_view(b).append(hist_k[b][None, :L].contiguous(),
                                      hist_v[b][None, :L].contiguous(), bt[b:b + 1].contiguous(),
                                      torch.zeros(1, dtype=torch.int32, device="cuda"))
    st.build_oracle()
    cur = lens.copy()
    for step in range(40):
        nk = torch.stack([hist_k[b][cur[b]] for b in range(st.batch)])[:, None].contiguous()
        nv = torch.stack([hist_v[b][cur[b]] for b in range(st.batch)])[:, None].contiguous()
        cache.append(nk, nv, bt, torch.from_numpy(cur.astype(np.int32)).cuda())
        for b in range(st.batch):
            o.cache_write(st.cache, b, st.k_hist[b][cur[b]], st.v_hist[b][cur[b]], st.tables[b],
                          int(cur[b]) + 1)
        cur += 1
    torch.cuda.synchronize()
    g = dict(zip(("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr"),
                 cache.pool()))
    res = [int(n - wl.split_old_tokens(int(n), w.residual)) for n in cur]
    _compare_pool(st, g, scratch_rows=res, what="step writes")
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(cur.astype(np.int32)).cuda(), bt)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), st.decode_ref(cur), "decode after step writes")


# ---------------------------------------------------------------- decode

def _decode_case(kivi, w: wl.Workload, lens, seed=0):
    st = State(w, lens=lens, seed=seed)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                       torch.from_numpy(st.tables).cuda())
    torch.cuda.synchronize()
    return st, out.cpu().numpy()


@pytest.mark.parametrize("name,lens", [
    ("tinyllama", [512]),
    ("qwen05b", [2048, 1, 33, 160, 161, 191, 192, 1000]),
    ("mistral7b", [4096, 129, 4095]),
    ("qwen14b", [1024, 3000, 5001]),
    ("long", [6000, 4097]),
])
def test_runtime_decode_matches_twopass(kivi, name, lens):
    w = wl.WORKLOADS[name]
    st, out = _decode_case(kivi, w, lens)
    assert_close(out, st.decode_ref(), f"decode {name}")


def test_v1_jac_launch_all_boundaries(kivi):
    """jac_launch (40/8/128, page 32) at the boundary-probe lengths."""
    st = State(V1, lens=[4096], seed=7)
    st.build_oracle()
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    for L in (128, 129, 159, 160, 191, 192, 4096):
        out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
        kivi.kivi_decode_dsl(q, bt[:max(1, (L - 128) // 32)].contiguous() if L >= 160 else bt,
                             *pool, g["k_scr"][0], g["v_scr"][0], L, out)
        torch.cuda.synchronize()
        ref = o.decode_twopass(st.cache, 0, st.q[0], st.tables[0], L)
        assert_close(out.cpu().numpy(), ref, f"jac_launch L={L}")


def test_v1_batched_decode_equals_single(kivi):
    """jac_launch_batched equals jac_launch per query bit for bit
    (variants.rs:1211-1213): the v1 symbols cut each query's work by its own
    length alone.  60 causal queries up to the 4096-token v1 maximum need
    more than one launch of the static workspace region, which must not
    change any query's bits either."""
    st = State(V1, lens=[4096], seed=8)
    st.build_oracle()
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    nq = 60
    rng = np.random.default_rng(3)
    qs = rng.standard_normal((nq, 40, 128)).astype(np.float16)
    seq = np.arange(4096 - nq + 1, 4097).astype(np.int32)
    seq[:5] = [1, 128, 129, 160, 1000]  # short and boundary queries in the same call
    qt = torch.from_numpy(qs).cuda()
    out_b = torch.empty((nq, 40, 128), dtype=torch.float32, device="cuda")
    kivi.kivi_decode_batched_dsl(qt, torch.from_numpy(seq).cuda(), bt, *pool, g["k_scr"][0],
                                 g["v_scr"][0], nq, out_b)
    for i in range(nq):
        out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
        kivi.kivi_decode_dsl(qt[i].contiguous(), bt, *pool, g["k_scr"][0], g["v_scr"][0],
                             int(seq[i]), out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), out_b[i].view(torch.int32)), \
            f"query {i} (seq_len {seq[i]}): max diff {(out - out_b[i]).abs().max().item():.3e}"
        if i < 8 or i % 13 == 0:
            ref = o.decode_twopass(st.cache, 0, qs[i].view(np.uint16), st.tables[0], int(seq[i]))
            assert_close(out.cpu().numpy(), ref, f"batched q{i}")


def test_v1_decode_allocates_nothing_under_capture(kivi):
    """The v1 decode symbols allocate nothing (the reference's contract: every
    buffer is the caller's, source_patch.py:2391-2417).  The first v1 decode
    on a fresh stream is captured into a graph; the library's allocation count
    does not move, and every replay equals the eager decode bit for bit."""
    st = State(V1, lens=[4096], seed=12)
    st.build_oracle()
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    kivi.lib().jacq_kivi_init()
    gen = torch.Generator(device="cuda").manual_seed(9)
    qs = [torch.randn((40, 128), generator=gen, device="cuda").half() for _ in range(3)]
    q_in = qs[0].clone()
    out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    before = kivi.lib().jacq_kivi_test_device_allocations()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        kivi.kivi_decode_dsl(q_in, bt, *pool, g["k_scr"][0], g["v_scr"][0], 3000, out)
    for i, q in enumerate(qs * 2):
        q_in.copy_(q)
        graph.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(out)
        kivi.kivi_decode_dsl(q, bt, *pool, g["k_scr"][0], g["v_scr"][0], 3000, ref)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {i}"
    assert kivi.lib().jacq_kivi_test_device_allocations() == before
    refn = o.decode_twopass(st.cache, 0, _np(qs[-1]), st.tables[0], 3000)
    assert_close(out.cpu().numpy(), refn, "captured jac_launch")


def test_page16_equals_page32(kivi):
    """Separating page from group is invisible to results: the same history
    stored in 16-token and 32-token pages decodes identically."""
    outs = []
    for page in (16, 32):
        w = wl.WORKLOADS["mistral7b"].scaled(batch=2, ctx_lo=1500, page=page)
        st, out = _decode_case(kivi, w, [1500, 777], seed=21)
        outs.append(out)
    # page 16 and page 32 split the token stream differently: equal to the
    # fp16 rounding of P (see test_v1_batched_decode_equals_single)
    np.testing.assert_allclose(outs[0], outs[1], atol=1e-3, rtol=2e-3)


def test_seq_len_zero_and_clamp(kivi):
    """SEQ_LEN <= 0 gives O = 0; SEQ_LEN beyond the table's capacity is
    clamped like the reference kernel (snapshot :74-83)."""
    w = wl.WORKLOADS["qwen14b"].scaled(batch=2, ctx_lo=600)
    st, _ = _decode_case(kivi, w, [600, 600])
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    cap = geo.max_seq_len()
    out = cache.decode(q, torch.tensor([0, cap + 1000], dtype=torch.int32, device="cuda"),
                       torch.from_numpy(st.tables).cuda())
    torch.cuda.synchronize()
    o_np = out.cpu().numpy()
    assert np.all(o_np[0] == 0)
    ref = o.decode_twopass(st.cache, 1, st.q[1], st.tables[1], cap + 1000)
    assert_close(o_np[1], ref, "clamped")


_EXTREME_GEOS = {
    "hd128_g5": wl.WORKLOADS["qwen14b"],  # packed hi/lo QK columns, page 16
    "hd64_g10_p32": wl.Workload("x64", 40, 4, 64, 1, 4096, 4096, page=32, residual=128,
                                outliers=4, outlier_scale=10.0, seed=11),
    "hd128_g16_p32": wl.Workload("x128", 32, 2, 128, 1, 4096, 4096, page=32, residual=128,
                                 outliers=4, outlier_scale=10.0, seed=12),
    "hd64_g7_p16": wl.Workload("x64p", 14, 2, 64, 1, 4096, 4096, page=16, residual=128,
                               outliers=4, outlier_scale=8.0, seed=13),  # packed QK at HD 64
}


@pytest.mark.parametrize("geo_id", list(_EXTREME_GEOS))
@pytest.mark.parametrize("mults,seed,frac", [([100.0, 3000.0, 9000.0], 5, 0.3), ([30.0], 8, 0.3),
                                              ([3000.0], 7, 0.3), ([300.0], 9, 0.01)],
                         ids=["to9000", "x30", "x3000", "sparse_x300"])
def test_decode_extreme_value_scales(kivi, mults, seed, frac, geo_id):
    """V tokens scaled so that values reach 1e2..1e4 (V scales >= 64, where
    -1024*s leaves fp16, and code*s beyond 65504): the results stay within
    north_star's tolerance, max-abs 2e-3 / rel 1e-2 of the float64 two-pass
    reference.  Such groups and residual tiles get the exact correction (fp32
    P against fp32 values) after the fp16 PV step, without which the fp16
    rounding of large, cancelling terms exceeds the bound by up to 64x; the
    scores use exact integer K codes, whose matrix-core sums stay within a few
    fp32 ulps (an offset code, or subnormal codes, cost up to 3.6x the bound).
    sparse_x300 scales 1% of the tokens: most groups stay on the fp16 path and
    a few are corrected in the same segment."""
    w = _EXTREME_GEOS[geo_id]
    st = State(w, lens=[700, 333], seed=seed)
    rng = np.random.default_rng(50 + seed)
    for b in range(st.batch):
        v = st.v_hist[b].view(np.float16).astype(np.float32)
        pick = rng.random(v.shape[0]) < frac
        v[pick] *= rng.choice(mults, size=(int(pick.sum()), 1, 1))
        st.v_hist[b] = np.clip(v, -65000, 65000).astype(np.float16).view(np.uint16)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages, st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                       torch.from_numpy(st.tables).cuda())
    torch.cuda.synchronize()
    ref = st.decode_ref()
    got = out.cpu().numpy()
    assert np.abs(ref).max() > min(mults) / 100.0  # the large-value regime
    assert np.isfinite(got).all()
    assert_close(got, ref, f"values scaled by {mults}")


@pytest.mark.parametrize("geo_id", ["hd128_g5", "hd64_g10_p32", "hd64_g7_p16"])
def test_decode_nonfinite_values(kivi, geo_id):
    """+inf in V in a quantised token, -inf in an fp16 residual token.  The
    reference dequantises the first with an infinite scale, 0 * inf = NaN for
    its whole 32-channel group: every head of that kv head reads NaN there.
    The second stays -inf in its channel.  The kernel gives the float64
    reference's NaN and infinity positions (the infinite scale takes the exact
    correction; the residual tile takes the fp32 path before its PV step, since
    taking an fp16 step's -inf out again would leave inf - inf), and every
    finite output stays within the tolerance."""
    w = _EXTREME_GEOS[geo_id]
    st = State(w, lens=[700, 333], seed=21)
    v = st.v_hist[0].view(np.float16).astype(np.float32)
    v[100, 1, 3] = np.inf       # quantised group of tokens 96..127, kv head 1
    v[650, 0, 40] = -np.inf     # residual window of a 700-token sequence, kv head 0
    st.v_hist[0] = v.astype(np.float16).view(np.uint16)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages, st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                       torch.from_numpy(st.tables).cuda())
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore"):
        ref = st.decode_ref()
    got = out.cpu().numpy()
    G = w.nh // w.nkv
    assert np.isnan(ref[0, G:2 * G, 0:32]).all()
    assert (ref[0, 0:G, 40] == -np.inf).all()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN positions differ"
    assert np.array_equal(np.isinf(got), np.isinf(ref)), "infinity positions differ"
    assert (np.sign(got[np.isinf(ref)]) == np.sign(ref[np.isinf(ref)])).all()
    fin = np.isfinite(ref)
    assert_close(got[fin], ref[fin], f"finite outputs beside the non-finite groups ({geo_id})")


def test_v1_batched_and_sparse_decode_extreme_values(kivi):
    """The multi-query (jac_launch_batched) and sparse-retained entry points on
    V tokens scaled x3000 (30% of them): the same exact correction as the
    batch decode keeps every query within max-abs 2e-3 / rel 1e-2 of the
    float64 two-pass reference."""
    st = State(V1, lens=[1000], seed=31)
    rng = np.random.default_rng(31)
    v = st.v_hist[0].view(np.float16).astype(np.float32)
    pick = rng.random(v.shape[0]) < 0.3
    v[pick] *= 3000.0
    st.v_hist[0] = np.clip(v, -65000, 65000).astype(np.float16).view(np.uint16)
    st.build_oracle()
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    nq = 6
    qs = rng.standard_normal((nq, 40, 128)).astype(np.float16)
    seq = np.arange(1000 - nq + 1, 1001).astype(np.int32)
    out_b = torch.empty((nq, 40, 128), dtype=torch.float32, device="cuda")
    kivi.kivi_decode_batched_dsl(torch.from_numpy(qs).cuda(), torch.from_numpy(seq).cuda(), bt,
                                 *pool, g["k_scr"][0], g["v_scr"][0], nq, out_b)
    torch.cuda.synchronize()
    for i in range(nq):
        ref = o.decode_twopass(st.cache, 0, qs[i].view(np.uint16), st.tables[0], int(seq[i]))
        assert np.abs(ref).max() > 30.0
        assert_close(out_b[i].cpu().numpy(), ref, f"batched q{i} x3000")
    compact = np.zeros(124, np.int32)  # the v1 ABI's table width
    compact[:3] = st.tables[0][[5, 1, 9]]
    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    outs = torch.empty((40, 128), dtype=torch.float32, device="cuda")
    kivi.kivi_decode_sparse_retained_dsl(q, torch.from_numpy(compact).cuda(), *pool,
                                         g["k_scr"][0], g["v_scr"][0], 1000, 3, outs)
    torch.cuda.synchronize()
    ref = o.decode_sparse_retained(st.cache, 0, st.q[0], compact, 1000, 3, twopass=True)
    assert_close(outs.cpu().numpy(), ref, "sparse retained x3000")


def test_caller_workspace_needs_no_initial_contents(kivi):
    """A caller workspace filled with random bytes, then reused by a second
    call with other queries, decodes to the same bits as the library's own
    workspace: the merge reads only partials tagged with its own launch."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 700, 5001, 129], seed=21)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    q1 = torch.from_numpy(st.q).view(torch.float16).cuda()
    q2 = torch.randn(q1.shape, generator=torch.Generator(device="cuda").manual_seed(3),
                     device="cuda").half()
    ref1, ref2 = cache.decode(q1, lens, bt), cache.decode(q2, lens, bt)
    nbytes = kivi.lib().jacq_kivi_decode_workspace_size(ctypes_geo(kivi, geo), st.batch)
    ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    got1 = cache.decode(q1, lens, bt, workspace=ws)
    got2 = cache.decode(q2, lens, bt, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got1.view(torch.int32), ref1.view(torch.int32))
    assert torch.equal(got2.view(torch.int32), ref2.view(torch.int32))
    # leftovers of another tensor: small int64 values (positions, indices) and
    # their negatives never equal a launch tag (random, top bit set)
    n8 = nbytes // 8
    ws2 = torch.empty(n8 * 8 + 8, dtype=torch.uint8, device="cuda")
    ar = torch.arange(n8, dtype=torch.int64, device="cuda")
    ws2[:n8 * 8].view(torch.int64).copy_(torch.where(ar % 2 == 0, ar, -ar))
    got3 = cache.decode(q1, lens, bt, workspace=ws2)
    torch.cuda.synchronize()
    assert torch.equal(got3.view(torch.int32), ref1.view(torch.int32))
    assert_close(got1.cpu().numpy(), st.decode_ref(), "random workspace")


def ctypes_geo(kivi, geo):
    import ctypes
    return ctypes.byref(geo.c())


def test_decode_graph_replays_match_eager(kivi):
    """The decode captured in a HIP graph replays with one frozen launch epoch;
    every replay (new queries copied in, eager kernels in between) must equal
    the eager decode bit for bit -- the merge clears each flag it consumes, so
    a replay never sees the previous replay's partials as its own."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 700, 5001, 129, 4096, 2047], seed=23)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    gen = torch.Generator(device="cuda").manual_seed(5)
    qs = [torch.randn((st.batch, w.nh, w.hd), generator=gen, device="cuda").half()
          for _ in range(4)]
    nbytes = kivi.lib().jacq_kivi_decode_workspace_size(ctypes_geo(kivi, geo), st.batch)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    q_in = qs[0].clone()
    out = torch.empty((st.batch, w.nh, w.hd), dtype=torch.float32, device="cuda")
    cache.decode(q_in, lens, bt, out=out, workspace=ws)  # device set-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.decode(q_in, lens, bt, out=out, workspace=ws)
    for i, q in enumerate(qs * 2):
        q_in.copy_(q)
        graph.replay()
        torch.cuda.synchronize()
        ref = cache.decode(q, lens, bt)  # eager, the library's own workspace
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {i}"


def test_library_workspace_per_stream_survives_growth(kivi):
    """The library's own workspace is per stream and never freed: a graph
    captured with it (no workspace passed) still replays correctly after a
    larger decode on the same stream replaced that stream's buffer, and a
    decode on another stream meanwhile uses a buffer of its own."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 700, 129], seed=31)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    q_in = torch.from_numpy(st.q).view(torch.float16).cuda()
    ref = cache.decode(q_in, lens, bt)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    out = torch.empty_like(ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        cache.decode(q_in, lens, bt, out=out)
    # a batch of 300 sequences on the same stream outgrows its first buffer
    big = 300
    bcache = kivi.PagedKiviCache(geo, big)
    with torch.cuda.stream(s):
        bq = torch.randn((big, w.nh, w.hd), device="cuda").half()
        bl = torch.full((big,), 200, dtype=torch.int32, device="cuda")
        bbt = bt[:1].repeat(big, 1).contiguous()
        bcache.decode(bq, bl, bbt)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32))


def test_valu_decode_matches_oracle(kivi):
    """The VALU split-K decode (JACQ_KIVI_DECODE=simple, a cross-check of the
    matrix-core kernel) against the oracle, in a child process because the
    library reads the switch once when it loads."""
    import json
    import os
    import subprocess
    import sys
    env = dict(os.environ, JACQ_KIVI_DECODE="simple")
    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, os.path.join(here, "simple_decode_check.py")], env=env,
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    worst = json.loads(r.stdout.strip().splitlines()[-1])
    for name, excess in worst.items():
        assert excess <= 0.0, f"{name}: worst excess over the tolerance {excess:.3e}"


def test_caller_workspace_too_small_is_rejected(kivi):
    """A caller workspace one byte short of jacq_kivi_decode_workspace_size is
    refused before anything is launched (status JACQ_KIVI_ENOMEM, message
    naming both sizes), and the output is left untouched."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[700, 300], seed=2)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    nbytes = kivi.lib().jacq_kivi_decode_workspace_size(ctypes_geo(kivi, geo), st.batch)
    assert nbytes > 0
    ws = torch.zeros(nbytes - 1, dtype=torch.uint8, device="cuda")
    out = torch.full((st.batch, w.nh, w.hd), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(kivi.KiviLaunchError, match=f"smaller than the {nbytes} required"):
        cache.decode(torch.from_numpy(st.q).view(torch.float16).cuda(),
                     torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                     torch.from_numpy(st.tables).cuda(), out=out, workspace=ws)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


@pytest.mark.parametrize("nh,nkv,hd,page,lens", [
    (32, 2, 128, 16, [3000, 129, 700]),   # G = 16: the unpacked HD=128 kernel
    (36, 4, 128, 32, [1500, 161]),        # G = 9, page 32
    (24, 2, 64, 32, [2048, 33, 1]),       # G = 12, HD = 64
    (18, 2, 64, 16, [900, 4000]),         # G = 9, HD = 64, page 16
    (8, 8, 128, 16, [1200, 77]),          # G = 1 (multi-head attention)
], ids=["g16_hd128_p16", "g9_hd128_p32", "g12_hd64_p32", "g9_hd64_p16", "g1_hd128_p16"])
def test_decode_other_gqa_ratios(kivi, nh, nkv, hd, page, lens):
    """GQA ratios outside the benchmark configs: G > 8 runs the unpacked kernels
    (one query head per MFMA column), G = 1 the packed one with a single head."""
    w = wl.Workload(f"g{nh // nkv}", nh, nkv, hd, len(lens), min(lens), max(lens), page=page,
                    residual=128, outliers=4, outlier_scale=8.0, seed=31)
    st, out = _decode_case(kivi, w, lens, seed=31)
    assert_close(out, st.decode_ref(), f"decode G={nh // nkv} HD={hd} page={page}")


@pytest.mark.parametrize("residual", [64, 256])
def test_other_residual_windows_write_and_decode(kivi, residual):
    """Residual windows other than 32 / 128 (any multiple of 32 is accepted):
    a bulk prefill, then one-token steps crossing age-out boundaries; pool and
    scratch bit-exact, decode within tolerance.  R = 256 makes the scratch
    shift run three 128-row passes."""
    w = wl.WORKLOADS["mistral7b"].scaled(batch=3, ctx_lo=600, residual=residual)
    lens = np.array([600, residual + 31, 1000])
    st = State(w, lens=lens, extra_tokens=40, seed=41)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache(geo, st.batch)
    bt = torch.from_numpy(st.tables).cuda()
    hist_k = [torch.from_numpy(k).view(torch.float16).cuda() for k in st.k_hist]
    hist_v = [torch.from_numpy(v).view(torch.float16).cuda() for v in st.v_hist]
    for b in range(st.batch):
        L = int(lens[b])
        cache.sequence_view(b).append(hist_k[b][None, :L].contiguous(),
                                      hist_v[b][None, :L].contiguous(), bt[b:b + 1].contiguous(),
                                      torch.zeros(1, dtype=torch.int32, device="cuda"))
    st.build_oracle()
    cur = lens.copy()
    for _ in range(40):
        nk = torch.stack([hist_k[b][cur[b]] for b in range(st.batch)])[:, None].contiguous()
        nv = torch.stack([hist_v[b][cur[b]] for b in range(st.batch)])[:, None].contiguous()
        cache.append(nk, nv, bt, torch.from_numpy(cur.astype(np.int32)).cuda())
        for b in range(st.batch):
            o.cache_write(st.cache, b, st.k_hist[b][cur[b]], st.v_hist[b][cur[b]], st.tables[b],
                          int(cur[b]) + 1)
        cur += 1
    torch.cuda.synchronize()
    g = dict(zip(("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr"),
                 cache.pool()))
    res = [int(n - wl.split_old_tokens(int(n), w.residual)) for n in cur]
    _compare_pool(st, g, scratch_rows=res, what=f"R={residual}")
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(cur.astype(np.int32)).cuda(), bt)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), st.decode_ref(cur), f"decode R={residual}")


def _segment_counts(w, got, ref):
    """(sequence, kv head) segments of O that are all NaN / within tolerance / neither."""
    G = w.nh // w.nkv
    counts = {"nan": 0, "match": 0, "other": 0}
    for b in range(got.shape[0]):
        for h in range(w.nkv):
            g_, r_ = got[b, h * G:(h + 1) * G], ref[b, h * G:(h + 1) * G]
            if np.isnan(g_).all():
                counts["nan"] += 1
            elif (np.abs(g_ - r_) <= 2e-3 + 1e-2 * np.abs(r_)).all():
                counts["match"] += 1
            else:
                counts["other"] += 1
    return counts


def test_merge_timeout_drains_and_is_reported(kivi):
    """Failure handling of the in-launch merge, forced from the host: with the
    test hook the merge waits for a tag nobody stores and gives up after
    20 us.  The launch still ends; segments a single wavefront wrote whole stay
    correct and every merged segment is NaN.  The device's status word is set:
    the next decode is refused (nothing launched), jacq_kivi_decode_status
    reports the time-out once and resets, and decodes are correct again."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 129, 20, 700, 1], seed=13)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    ref = st.decode_ref()
    kivi.decode_status()  # nothing pending
    kivi.lib().jacq_kivi_test_force_merge_timeout(20)
    try:
        out = cache.decode(q, lens, bt)
        torch.cuda.synchronize()
    finally:
        kivi.lib().jacq_kivi_test_force_merge_timeout(0)
    counts = _segment_counts(w, out.cpu().numpy().astype(np.float64), ref)
    assert counts["other"] == 0 and counts["nan"] >= 1 and counts["match"] >= 1, counts
    sentinel = torch.full_like(out, 7.0)
    with pytest.raises(kivi.KiviMergeTimeout, match="timed out"):
        cache.decode(q, lens, bt, out=sentinel)
    torch.cuda.synchronize()
    assert bool((sentinel == 7.0).all()), "a refused decode must not launch"
    with pytest.raises(kivi.KiviMergeTimeout, match="reset"):
        kivi.decode_status()
    kivi.decode_status()  # reported once
    out = cache.decode(q, lens, bt)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "decode after the reset")


def test_merge_timeout_poisons_graph_replays(kivi):
    """A graph replay never passes through the host's status check, and it
    repeats its launch epoch: after a merge on its workspace timed out, flags
    that the late stream wavefronts stored would look like the replay's own.
    The timed-out merge poisons the workspace, so the replays' merged segments
    are NaN -- never finite values built from stale partials -- until
    jacq_kivi_decode_status zeroes the workspace; then replays equal the
    eager decode again."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 129, 20, 700, 1], seed=17)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    ref = st.decode_ref()
    kivi.decode_status()
    nbytes = kivi.lib().jacq_kivi_decode_workspace_size(ctypes_geo(kivi, geo), st.batch)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty((st.batch, w.nh, w.hd), dtype=torch.float32, device="cuda")
    eager = cache.decode(q, lens, bt, out=torch.empty_like(out), workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.decode(q, lens, bt, out=out, workspace=ws)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
    # an eager decode on the same workspace times out (forced from the host)
    kivi.lib().jacq_kivi_test_force_merge_timeout(20)
    try:
        cache.decode(q, lens, bt, out=torch.empty_like(out), workspace=ws)
        torch.cuda.synchronize()
    finally:
        kivi.lib().jacq_kivi_test_force_merge_timeout(0)
    for i in range(2):  # no jacq_kivi_decode_status in between
        out.fill_(5.0)
        graph.replay()
        torch.cuda.synchronize()
        counts = _segment_counts(w, out.cpu().numpy().astype(np.float64), ref)
        assert counts["other"] == 0 and counts["nan"] >= 1 and counts["match"] >= 1, (i, counts)
    with pytest.raises(kivi.KiviMergeTimeout, match="reset"):
        kivi.decode_status(ws)
    for i in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), f"replay {i} after reset"
    kivi.decode_status()


def test_merge_timeout_exits_v1_symbols(kivi):
    """The v1 symbols return void: a merge time-out is reported by the next v1
    decode on the device, which prints the error and exits(1) like the
    reference's CUDA_CHECK (child process, tests/merge_timeout_check.py)."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, os.path.join(here, "merge_timeout_check.py")],
                       capture_output=True, text=True, timeout=100)
    assert "FIRST_DECODE_RETURNED" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
    assert r.returncode == 1, r.stdout[-2000:] + r.stderr[-2000:]
    assert "jac_launch" in r.stderr and "timed out" in r.stderr, r.stderr[-2000:]


def test_wave_stamps_cover_the_stream(kivi):
    """The profiling hook (jacq_kivi_profile_wave_stamps): every stream
    workgroup stamps an end after its start, and their units add up to the
    stream's total (sum over sequences and kv heads of quantised groups plus
    three units per fp16 residual tile)."""
    from jacq_amd import cache_io
    w = wl.WORKLOADS["qwen14b"].scaled(batch=4, ctx_lo=900)
    lens = [900, 2000, 77, 3001]
    st = State(w, lens=lens, seed=3)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, g)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    cap = 8192
    stamps = torch.zeros((cap, 4), dtype=torch.int64, device="cuda")
    assert kivi.lib().jacq_kivi_profile_wave_stamps(kivi._ptr(stamps), cap) == 0
    try:
        out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                           torch.from_numpy(st.tables).cuda())
        torch.cuda.synchronize()
    finally:
        assert kivi.lib().jacq_kivi_profile_wave_stamps(None, 0) == 0
    assert_close(out.cpu().numpy(), st.decode_ref(), "decode with stamps")
    s = stamps.cpu().numpy()
    ran = s[:, 1] > 0
    assert (s[ran, 1] >= s[ran, 0]).all()
    units = s[:, 3] & 0xFFFFFFFF
    expect = 0
    for n in lens:
        ov = cache_io.old_valid(geo, n)
        tiles = max(1, -(-min(n, geo.max_seq_len()) // 32))
        nq = ov // 32
        expect += w.nkv * (nq + 3 * (tiles - nq))
    assert int(units.sum()) == expect
