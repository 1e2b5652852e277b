"""Golden fixtures of the int4-KIVI path, produced by the oracle (oracle/).

    python tests/golden/make_golden.py      # rewrites tests/golden/kivi_golden.*

The reference holds no numeric fixture for this path (its tests pin shapes,
byte math and argument order only), so these vectors come from the oracle,
which tests/test_oracle_*.py pin against closed forms and an independent
numpy restatement.  Each case is a seeded token history written through the
reference's single-token writer order (source_patch.py:1661-1697) from an
empty cache, then one decode query per sequence (snapshot :51-158).

Inputs are regenerated from the seed (numpy PCG64); the fixture keeps the
SHA-256 of every cache array after the writes (the bit-exact part of the
contract) and the float64 two-pass attention outputs.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

CASES = {
    # 14B-like head shape at page 16 (a group spans two pages)
    "hd128_p16": dict(nh=10, nkv=2, hd=128, page=16, residual=128, lens=[0, 1, 129, 161, 300, 517],
                      seed=101, outliers=[5, 77]),
    # Qwen2.5-0.5B-like shape at page 32
    "hd64_p32": dict(nh=14, nkv=2, hd=64, page=32, residual=128, lens=[40, 200, 450],
                     seed=202, outliers=[3]),
}
ARRAYS = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")


def inputs(case: dict):
    """Histories [L, NKV, HD], queries [B, NH, HD] (fp16 bits) and block tables."""
    rng = np.random.default_rng(case["seed"])
    nkv, hd, page = case["nkv"], case["hd"], case["page"]
    lens = case["lens"]
    groups = [max(0, L - case["residual"]) // 32 for L in lens]
    need = [g * 32 // page for g in groups]
    max_pages = max(1, max(need))
    num_pages = sum(need) + 1
    perm = rng.permutation(num_pages).astype(np.int32)
    tables = np.zeros((len(lens), max_pages), np.int32)
    at = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[at:at + n]
        at += n
    hist = []
    for L in lens:
        k = rng.standard_normal((L, nkv, hd))
        k[:, :, case["outliers"]] *= 10.0
        v = rng.standard_normal((L, nkv, hd))
        hist.append((k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)))
    q = rng.standard_normal((len(lens), case["nh"], hd)).astype(np.float16).view(np.uint16)
    return hist, q, tables, num_pages, max_pages


def oracle_state(case: dict):
    from oracle import oracle as o
    hist, q, tables, num_pages, max_pages = inputs(case)
    geo = o.Geometry(case["nh"], case["nkv"], case["hd"], case["page"], 32, case["residual"],
                     max_pages)
    cache = o.Cache.empty(geo, num_pages, len(case["lens"]))
    for b, (k, v) in enumerate(hist):
        o.build_sequence(cache, b, k, v, tables[b])
    out = np.stack([o.decode_twopass(cache, b, q[b], tables[b], L)
                    for b, L in enumerate(case["lens"])])
    return cache, out


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def scratch_digests(cache, case) -> list[str]:
    """Digest of the defined scratch rows (the residual window) per sequence."""
    out = []
    for b, L in enumerate(case["lens"]):
        res = L - max(0, L - case["residual"]) // 32 * 32
        out.append(digest(np.stack([cache.k_scr[b][:, :res], cache.v_scr[b][:, :res]])))
    return out


def main() -> None:
    from oracle import oracle as o
    o.build()
    meta, arrays = {}, {}
    for name, case in CASES.items():
        cache, out = oracle_state(case)
        meta[name] = {"case": case, "sha256": {a: digest(getattr(cache, a)) for a in ARRAYS},
                      "scratch_sha256": scratch_digests(cache, case)}
        arrays[f"{name}__out"] = out
    with open(os.path.join(HERE, "kivi_golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    np.savez_compressed(os.path.join(HERE, "kivi_golden.npz"), **arrays)
    print("wrote", sorted(meta))


if __name__ == "__main__":
    main()
