"""Shared helpers of the parity tests: seeded inputs, oracle-built cache state,
and GPU mirrors of it.  The oracle (oracle/) is the checker here, never the
thing under test."""
from __future__ import annotations

import numpy as np

from jacq_amd import workloads as wl
from oracle import oracle as o

ATOL, RTOL = 2e-3, 1e-2  # attention-output tolerance vs the float64 two-pass reference


def geometry(w: wl.Workload, max_pages: int) -> o.Geometry:
    return o.Geometry(w.nh, w.nkv, w.hd, w.page, w.group, w.residual, max_pages)


class State:
    """Workload instance: histories, tables and the oracle-built cache."""

    def __init__(self, w: wl.Workload, lens=None, extra_tokens: int = 0, seed: int | None = None):
        seed = w.seed if seed is None else seed
        rng = np.random.default_rng(seed)
        self.w = w
        self.lens = np.asarray(wl.context_lens(w, rng) if lens is None else lens, np.int64)
        self.final_lens = self.lens + extra_tokens
        self.tables, self.num_pages, self.max_pages = wl.block_tables(w, self.final_lens, rng)
        # values come from their own stream: the same seed gives the same
        # tokens whatever the page size or table layout
        rng = np.random.default_rng([seed, 1])
        self.outl = wl.outlier_channels(w, rng)
        self.k_hist, self.v_hist = [], []
        for n in self.final_lens:
            k, v = wl.kv_tokens_numpy(w, rng, int(n), self.outl)
            self.k_hist.append(k)
            self.v_hist.append(v)
        self.q = wl.queries_numpy(w, rng, w.batch if lens is None else len(self.lens))
        self.geo = geometry(w, self.max_pages)
        self.cache = o.Cache.empty(self.geo, self.num_pages, len(self.lens))

    @property
    def batch(self) -> int:
        return len(self.lens)

    def build_oracle(self, upto=None) -> None:
        """Single-token writes from empty up to lens (or `upto`) per sequence."""
        upto = self.lens if upto is None else upto
        for b in range(self.batch):
            for t in range(int(upto[b])):
                o.cache_write(self.cache, b, self.k_hist[b][t], self.v_hist[b][t],
                              self.tables[b], t + 1)

    def decode_ref(self, seq_lens=None) -> np.ndarray:
        seq_lens = self.lens if seq_lens is None else seq_lens
        return np.stack([o.decode_twopass(self.cache, b, self.q[b], self.tables[b],
                                          int(seq_lens[b])) for b in range(self.batch)])


def to_torch(state: State, device="cuda"):
    """GPU copy of the oracle cache (uint16 -> float16 views)."""
    import torch
    c = state.cache

    def t(a, half=False):
        x = torch.from_numpy(np.ascontiguousarray(a))
        if half:
            x = x.view(torch.float16)
        return x.to(device)

    return {
        "k_code": t(c.k_code), "k_scale": t(c.k_scale, True), "k_zero": t(c.k_zero, True),
        "v_code": t(c.v_code), "v_scale": t(c.v_scale, True), "v_zero": t(c.v_zero, True),
        "k_scr": t(c.k_scr, True), "v_scr": t(c.v_scr, True),
    }


def assert_close(got: np.ndarray, ref: np.ndarray, what: str = "") -> None:
    err = np.abs(got.astype(np.float64) - ref)
    bound = ATOL + RTOL * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside max-abs {ATOL} / rel {RTOL}; "
        f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}")
