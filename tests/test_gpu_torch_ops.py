"""GPU parity of the torch custom ops (libjacq_kivi_torch.so,
``torch.ops.jacq_kivi``): the reference's vLLM op surface
(source_patch.py:768-1495) driven through torch's dispatcher against the CPU
oracle.  Writer state bit-exact; decodes within max-abs 2e-3 / rel 1e-2 of
the float64 two-pass reference."""
from __future__ import annotations

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests.kivi_testlib import State, assert_close, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

POOL = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")


def _lane(nh, nkv, seed):
    return wl.Workload(f"op{nh}", nh, nkv, 128, 1, 4096, 4096, page=32, residual=128,
                       outliers=4, outlier_scale=10.0, seed=seed)


@pytest.fixture(scope="module")
def ops():
    from jacq_amd import torch_ops
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch_ops.load()


def _u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _same_pool(st: State, g: dict, what: str):
    c = st.cache
    for name in POOL:
        got = g[name].cpu().numpy() if g[name].dtype == torch.uint8 else _u16(g[name])
        assert np.array_equal(got, getattr(c, name)), f"{what}: {name}"
    for name in ("k_scr", "v_scr"):
        assert np.array_equal(_u16(g[name]), getattr(c, name)), f"{what}: {name}"


@pytest.mark.parametrize("nh,nkv", [(40, 8), (20, 4)], ids=["global", "tp2_local"])
def test_op_write_then_decode_matches_oracle(ops, nh, nkv):
    """kivi_cache_write_dsl token by token through two age-outs, then
    kivi_decode_dsl, kivi_decode_batched_dsl and kivi_decode_sparse_retained_dsl."""
    n = 230
    st = State(_lane(nh, nkv, nh + 1), lens=[n])
    g = to_torch(st)
    pool = [g[k] for k in POOL]
    bt = torch.from_numpy(st.tables[0]).cuda()
    slot = torch.zeros(1, dtype=torch.int64, device="cuda")
    for t in range(n):
        nk = torch.from_numpy(st.k_hist[0][t].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][t].copy()).view(torch.float16).cuda()
        ops.kivi_cache_write_dsl(*pool, g["k_scr"][0], g["v_scr"][0], nk, nv, slot, bt, t + 1)
    st.build_oracle()
    torch.cuda.synchronize()
    _same_pool(st, g, f"op writer {nh}/{nkv}")

    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    out = torch.empty((nh, 128), dtype=torch.float32, device="cuda")
    ops.kivi_decode_dsl(q, bt, *pool, g["k_scr"][0], g["v_scr"][0], n, out)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy()[None], st.decode_ref(), f"kivi_decode_dsl {nh}/{nkv}")

    # up to 160 causal queries of the same sequence
    nq = 6
    qs = np.random.default_rng(3).standard_normal((nq, nh, 128)).astype(np.float16)
    lens = np.arange(n - nq + 1, n + 1).astype(np.int32)
    outb = torch.empty((nq, nh, 128), dtype=torch.float32, device="cuda")
    ops.kivi_decode_batched_dsl(torch.from_numpy(qs).cuda(), torch.from_numpy(lens).cuda(), bt,
                                *pool, g["k_scr"][0], g["v_scr"][0], nq, outb)
    torch.cuda.synchronize()
    for i in range(nq):
        ref = o.decode_twopass(st.cache, 0, qs[i].view(np.uint16), st.tables[0], int(lens[i]))
        assert_close(outb[i].cpu().numpy(), ref, f"batched q{i}")

    # one of the three old pages evicted
    compact = np.zeros(124, np.int32)
    compact[:2] = st.tables[0][[2, 0]]
    outs = torch.empty_like(out)
    ops.kivi_decode_sparse_retained_dsl(q, torch.from_numpy(compact).cuda(), *pool,
                                        g["k_scr"][0], g["v_scr"][0], n, 2, outs)
    torch.cuda.synchronize()
    ref = o.decode_sparse_retained(st.cache, 0, st.q[0], compact, n, 2, twopass=True)
    assert_close(outs.cpu().numpy(), ref, "sparse op")


@pytest.mark.parametrize("hand", [True, False], ids=["hand", "jac"])
def test_op_batched_writer_over_planned_subchunks(ops, hand):
    """kivi_cache_write_batched_dsl (and its _jac comparison twin) over the
    plan_batched_write sub-chunks of a 500-token prefill == the oracle."""
    from jacq_amd import kivi
    st = State(_lane(40, 8, 5), lens=[500])
    g = to_torch(st)
    pool = [g[k] for k in POOL]
    bt = torch.from_numpy(st.tables[0]).cuda()
    op = ops.kivi_cache_write_batched_dsl if hand else ops.kivi_cache_write_batched_jac_dsl
    for (start, n, _, _, _) in kivi.plan_batched_write(0, 500):
        nk = torch.from_numpy(st.k_hist[0][start:start + n].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][start:start + n].copy()).view(torch.float16).cuda()
        op(*pool, g["k_scr"][0], g["v_scr"][0], nk, nv,
           torch.zeros(n, dtype=torch.int64, device="cuda"), bt, start, n)
    st.build_oracle()
    torch.cuda.synchronize()
    _same_pool(st, g, "batched op writer")


def test_op_jac_writer_equals_hand_writer(ops):
    """The comparison op kivi_cache_write_jac_dsl leaves the same bits as
    kivi_cache_write_dsl (the bitcheck the reference keeps it for)."""
    st = State(_lane(40, 8, 9), lens=[200])
    g1, g2 = to_torch(st), to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    slot = torch.zeros(1, dtype=torch.int64, device="cuda")
    for t in range(200):
        nk = torch.from_numpy(st.k_hist[0][t].copy()).view(torch.float16).cuda()
        nv = torch.from_numpy(st.v_hist[0][t].copy()).view(torch.float16).cuda()
        ops.kivi_cache_write_dsl(*[g1[k] for k in POOL], g1["k_scr"][0], g1["v_scr"][0], nk, nv,
                                 slot, bt, t + 1)
        ops.kivi_cache_write_jac_dsl(*[g2[k] for k in POOL], g2["k_scr"][0], g2["v_scr"][0], nk,
                                     nv, slot, bt, t + 1)
    torch.cuda.synchronize()
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k


def test_op_refuses_a_bundle_with_a_host_tensor(ops):
    """A CPU tensor among GPU ones reaches the GPU kernel and is refused
    before anything launches."""
    st = State(_lane(40, 8, 2), lens=[300])
    g = to_torch(st)
    pool = [g[k] for k in POOL]
    q = torch.zeros((40, 128), dtype=torch.float16, device="cuda")
    out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="BLOCK_TABLE must be a CUDA tensor"):
        ops.kivi_decode_dsl(q, torch.zeros(124, dtype=torch.int32), *pool, g["k_scr"][0],
                            g["v_scr"][0], 300, out)
    with pytest.raises(RuntimeError, match="Q must be fp16"):
        ops.kivi_decode_dsl(q.float(), torch.zeros(124, dtype=torch.int32, device="cuda"), *pool,
                            g["k_scr"][0], g["v_scr"][0], 300, out)
