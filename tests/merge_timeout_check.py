"""Child process of test_gpu_parity.test_merge_timeout_exits_v1_symbols.

With the library's test hook every merge wait of a decode runs out.  The
first jac_launch (v1 geometry, one 4096-token sequence, whose split-K pieces
need merging) returns and drains; the second sees the device's time-out
status and must print the error and exit(1), as the v1 symbols do for launch
errors.  Prints FIRST_DECODE_RETURNED between the two calls."""
from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from jacq_amd import kivi  # noqa: E402
from jacq_amd import workloads as wl  # noqa: E402
from tests.kivi_testlib import State, to_torch  # noqa: E402


def main() -> int:
    w = wl.Workload("v1", 40, 8, 128, 1, 4096, 4096, page=32, residual=128, seed=11)
    st = State(w, lens=[4096], seed=4)
    st.build_oracle()
    g = to_torch(st)
    bt = torch.from_numpy(st.tables[0]).cuda()
    q = torch.from_numpy(st.q[0].copy()).view(torch.float16).cuda()
    out = torch.empty((40, 128), dtype=torch.float32, device="cuda")
    pool = [g[n] for n in ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")]
    kivi.lib().jacq_kivi_test_force_merge_timeout(20)
    kivi.kivi_decode_dsl(q, bt, *pool, g["k_scr"][0], g["v_scr"][0], 4096, out)
    torch.cuda.synchronize()
    assert np.isnan(out.cpu().numpy()).any(), "the forced time-out merged nothing"
    print("FIRST_DECODE_RETURNED", flush=True)
    kivi.lib().jacq_kivi_test_force_merge_timeout(0)
    kivi.kivi_decode_dsl(q, bt, *pool, g["k_scr"][0], g["v_scr"][0], 4096, out)
    torch.cuda.synchronize()
    print("SECOND_DECODE_RETURNED", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
