"""jacq_kivi_decode_noalloc (the decode that allocates nothing; its split-K
workspace is the library's static device array) against jacq_kivi_decode
through the C ABI: bit-identical outputs on two calls in a row, the second
with a smaller batch, plus the size limit and the set-up requirement (a call
before jacq_kivi_init is refused, checked in a fresh child process)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from jacq_amd import workloads as wl
from tests.kivi_testlib import State, assert_close, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

POOL = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero", "k_scr", "v_scr")


@pytest.fixture(scope="module")
def kivi():
    from jacq_amd import kivi as k
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert k.lib().jacq_kivi_init() == 0, k.last_error()
    return k


def _noalloc(kivi, geo, st_g, q, lens, bt, out):
    return kivi.lib().jacq_kivi_decode_noalloc(
        ctypes.byref(geo.c()), kivi._ptr(q), kivi._ptr(lens), kivi._ptr(bt),
        *[kivi._ptr(st_g[n]) for n in POOL], int(q.shape[0]), kivi._ptr(out),
        kivi._stream(q.device))


def _library(kivi, geo, st_g, q, lens, bt, out):
    return kivi.lib().jacq_kivi_decode(
        ctypes.byref(geo.c()), kivi._ptr(q), kivi._ptr(lens), kivi._ptr(bt),
        *[kivi._ptr(st_g[n]) for n in POOL], int(q.shape[0]), kivi._ptr(out), None, 0,
        kivi._stream(q.device))


def test_noalloc_decode_equals_decode_twice(kivi):
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[5001, 3000, 700, 129, 4096, 20], seed=41)
    st.build_oracle()
    g = to_torch(st)
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    lens = torch.from_numpy(st.lens.astype(np.int32)).cuda()
    bt = torch.from_numpy(st.tables).cuda()
    ref = st.decode_ref()
    for n in (6, 3):  # the second call is smaller
        gs = {k: (v[:n].contiguous() if k in ("k_scr", "v_scr") else v) for k, v in g.items()}
        qn, ln, btn = q[:n].contiguous(), lens[:n].contiguous(), bt[:n].contiguous()
        a = torch.full((n, w.nh, w.hd), 5.0, device="cuda")
        b = torch.full((n, w.nh, w.hd), 6.0, device="cuda")
        assert _noalloc(kivi, geo, gs, qn, ln, btn, a) == 0, kivi.last_error()
        assert _library(kivi, geo, gs, qn, ln, btn, b) == 0, kivi.last_error()
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"batch {n}"
        assert_close(a.cpu().numpy(), ref[:n], f"noalloc batch {n}")
    kivi.decode_status()


def test_noalloc_rejects_batches_beyond_the_static_array(kivi):
    w = wl.WORKLOADS["qwen14b"]
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, 1024, 4096)
    big = 4096
    need = kivi.lib().jacq_kivi_decode_workspace_size(ctypes.byref(geo.c()), big)
    assert need > 32 << 20
    q = torch.zeros((big, w.nh, w.hd), dtype=torch.float16, device="cuda")
    lens = torch.ones(big, dtype=torch.int32, device="cuda")
    bt = torch.zeros((big, 1024), dtype=torch.int32, device="cuda")
    pool = {"k_code": torch.zeros(16, dtype=torch.uint8, device="cuda")}
    for n in POOL:
        pool[n] = pool["k_code"]
    out = torch.full((big, w.nh, w.hd), 3.0, device="cuda")
    rc = _noalloc(kivi, geo, pool, q, lens, bt, out)
    assert rc == 3  # JACQ_KIVI_ENOMEM
    assert "static" in kivi.last_error() and str(need) in kivi.last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())


def test_noalloc_before_init_is_refused():
    """jacq_kivi_decode_noalloc before jacq_kivi_init on the device returns
    JACQ_KIVI_EINVAL naming jacq_kivi_init and launches nothing (a fresh
    child process, tests/noalloc_before_init_check.py, in which no entry
    point has run)."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, os.path.join(here, "noalloc_before_init_check.py")],
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0 and "REFUSED_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
