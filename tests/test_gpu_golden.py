"""The HIP path against the committed golden fixtures (tests/golden/):
cache arrays bit for bit after the writer, attention outputs within the
path's tolerance."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg
from tests.kivi_testlib import assert_close

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_gpu_matches_golden(name):
    import torch
    from jacq_amd import kivi
    meta = json.load(open(os.path.join(HERE, "kivi_golden.json")))[name]
    want = np.load(os.path.join(HERE, "kivi_golden.npz"))[f"{name}__out"]
    case = mg.CASES[name]
    hist, q, tables, num_pages, max_pages = mg.inputs(case)
    print(f"[golden] {name}", flush=True)
    geo = kivi.KiviGeometry(case["nh"], case["nkv"], case["hd"], case["page"], 32,
                            case["residual"], max_pages, num_pages)
    B = len(case["lens"])
    cache = kivi.PagedKiviCache(geo, B, "cuda")
    bt = torch.from_numpy(tables).cuda()
    h = lambda a: torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    for b, (k, v) in enumerate(hist):
        if k.shape[0] == 0:
            continue
        cache.sequence_view(b).append(h(k)[None].contiguous(), h(v)[None].contiguous(),
                                      bt[b:b + 1].contiguous(),
                                      torch.zeros(1, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    host = lambda t: t.cpu().view(torch.uint8 if t.dtype == torch.uint8 else torch.int16).numpy()
    for a in mg.ARRAYS:
        arr = host(getattr(cache, a))
        if arr.dtype == np.int16:
            arr = arr.view(np.uint16)
        assert mg.digest(arr) == meta["sha256"][a], a

    class Scr:
        k_scr = host(cache.k_scr).view(np.uint16)
        v_scr = host(cache.v_scr).view(np.uint16)
    assert mg.scratch_digests(Scr, case) == meta["scratch_sha256"]
    lens = torch.tensor(case["lens"], dtype=torch.int32, device="cuda")
    out = cache.decode(h(q).contiguous(), lens, bt)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, f"golden {name}")
