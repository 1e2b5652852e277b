"""Child process of test_zz_no_alloc.test_noalloc_before_init_is_refused.

In a fresh process in which no entry point of the library has run, a call of
jacq_kivi_decode_noalloc must be refused with JACQ_KIVI_EINVAL (1) and the
message naming jacq_kivi_init, launching nothing (its output keeps its
sentinel).  Prints REFUSED_OK on success."""
from __future__ import annotations

import ctypes
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from jacq_amd import kivi  # noqa: E402


def main() -> int:
    geo = kivi.KiviGeometry(40, 8, 128, 16, 32, 128, 64, 256)
    dev = torch.device("cuda")
    q = torch.zeros((2, 40, 128), dtype=torch.float16, device=dev)
    lens = torch.full((2,), 100, dtype=torch.int32, device=dev)
    bt = torch.zeros((2, 64), dtype=torch.int32, device=dev)
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    out = torch.full((2, 40, 128), 7.0, device=dev)
    torch.cuda.synchronize()
    rc = kivi.lib().jacq_kivi_decode_noalloc(
        ctypes.byref(geo.c()), kivi._ptr(q), kivi._ptr(lens), kivi._ptr(bt),
        *[kivi._ptr(buf)] * 8, 2, kivi._ptr(out), kivi._stream(dev))
    torch.cuda.synchronize()
    msg = kivi.last_error()
    assert rc == 1, (rc, msg)
    assert "jacq_kivi_init" in msg, msg
    assert bool((out == 7.0).all()), "a refused call must not launch"
    print("REFUSED_OK", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
