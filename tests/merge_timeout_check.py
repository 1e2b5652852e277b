"""Child process of test_gpu_parity.test_merge_timeout_drains: with
JACQ_KIVI_TEST_MERGE_TIMEOUT_US set (read once, when the library loads) every
merge wait of the decode runs out.  Prints, as JSON, how many (sequence, kv
head) segments came out NaN (merged ones), how many match the oracle (written
whole by one wavefront) and how many are neither."""
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
    assert os.environ.get("JACQ_KIVI_TEST_MERGE_TIMEOUT_US")
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[3000, 129, 20, 700, 1], seed=13)
    st.build_oracle()
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages,
                            st.num_pages)
    cache = kivi.PagedKiviCache.from_tensors(geo, to_torch(st))
    q = torch.from_numpy(st.q).view(torch.float16).cuda()
    out = cache.decode(q, torch.from_numpy(st.lens.astype(np.int32)).cuda(),
                       torch.from_numpy(st.tables).cuda())
    torch.cuda.synchronize()
    got, ref = out.cpu().numpy().astype(np.float64), st.decode_ref()
    G = w.nh // w.nkv
    counts = {"nan": 0, "match": 0, "other": 0}
    for b in range(st.batch):
        for h in range(w.nkv):
            g_, r_ = got[b, h * G:(h + 1) * G], ref[b, h * G:(h + 1) * G]
            if np.isnan(g_).all():
                counts["nan"] += 1
            elif (np.abs(g_ - r_) <= ATOL + RTOL * np.abs(r_)).all():
                counts["match"] += 1
            else:
                counts["other"] += 1
    print(json.dumps(counts), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
