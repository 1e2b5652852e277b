"""Child process of test_gpu_parity.test_valu_decode_matches_oracle: with
JACQ_KIVI_DECODE=simple (read once, when the library loads) the decode runs
the VALU split-K kernel; prints the worst excess over the tolerance as JSON."""
from __future__ import annotations

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from jacq_amd import kivi  # noqa: E402
from jacq_amd import workloads as wl  # noqa: E402
from tests.kivi_testlib import ATOL, RTOL, State, to_torch  # noqa: E402


def main() -> int:
    assert os.environ.get("JACQ_KIVI_DECODE") == "simple"
    res = {}
    for name, lens in (("qwen14b", [3000, 129, 700]), ("qwen05b", [2048, 1, 161])):
        w = wl.WORKLOADS[name]
        st = State(w, lens=lens, seed=9)
        st.build_oracle()
        geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                                st.num_pages)
        cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
        q = torch.from_numpy(st.q).view(torch.float16).cuda()
        out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                           torch.from_numpy(st.tables).cuda())
        torch.cuda.synchronize()
        ref = st.decode_ref()
        err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
        res[name] = float((err - (ATOL + RTOL * np.abs(ref))).max())
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
