"""The five decode workloads of the benchmark brief, and their synthetic inputs.

Each workload fixes a geometry (query heads / kv heads / head dim, page size,
32-token group, residual window), a batch, a context-length distribution and
the K/V value model (N(0,1) with per-head outlier channels, optional +-20
spikes).  Inputs are generated from a seed so that the GPU path and the CPU
oracle see identical bits:

* ``numpy`` generators for parity-sized cases (tests, smoke);
* ``torch`` generators on the device for full-size benchmark state.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    nh: int
    nkv: int
    hd: int
    batch: int
    ctx_lo: int
    ctx_hi: int              # == ctx_lo for uniform contexts
    page: int = 16
    group: int = 32
    residual: int = 128
    outliers: int = 0        # outlier K channels per kv head
    outlier_scale: float = 1.0
    spike_frac: float = 0.0  # fraction of K entries replaced by +-spike_value
    spike_value: float = 20.0
    permuted: bool = True    # block tables: random permutation of the pool
    prefill_chunk: int = 0   # tokens appended per sequence before decoding
    decode_steps: int = 1    # decode steps (each appends one token first)
    write_before_decode: bool = False
    seed: int = 0

    @property
    def gqa(self) -> int:
        return self.nh // self.nkv

    @property
    def scratch_rows(self) -> int:
        return self.residual + self.group

    def scaled(self, batch: int | None = None, ctx_lo: int | None = None,
               ctx_hi: int | None = None, **kw) -> "Workload":
        """A smaller copy of the workload (same geometry / value model)."""
        return replace(self, batch=batch or self.batch, ctx_lo=ctx_lo or self.ctx_lo,
                       ctx_hi=ctx_hi or ctx_lo or self.ctx_hi, **kw)


WORKLOADS: dict[str, Workload] = {
    "tinyllama": Workload("tinyllama", 32, 4, 64, 1, 512, 512, page=16, residual=32,
                          permuted=False, seed=0),
    "qwen05b": Workload("qwen05b", 14, 2, 64, 16, 2048, 2048, page=16, residual=128,
                        outliers=4, outlier_scale=8.0, seed=1),
    "mistral7b": Workload("mistral7b", 32, 8, 128, 32, 4096, 4096, page=16, residual=128,
                          outliers=8, outlier_scale=10.0, write_before_decode=True, seed=2),
    "qwen14b": Workload("qwen14b", 40, 8, 128, 64, 1024, 16384, page=16, residual=128,
                        outliers=8, outlier_scale=10.0, write_before_decode=True, seed=3),
    "long": Workload("long", 64, 8, 128, 256, 4096, 32768, page=16, residual=128,
                     outliers=8, outlier_scale=10.0, spike_frac=0.01, prefill_chunk=512,
                     decode_steps=8, write_before_decode=True, seed=4),
}

HEADLINE = "qwen14b"


def split_old_tokens(seq_len: int, residual: int, group: int = 32) -> int:
    q = seq_len - residual
    return (q // group) * group if q > 0 else 0


def context_lens(w: Workload, rng: np.random.Generator) -> np.ndarray:
    if w.ctx_hi == w.ctx_lo:
        return np.full(w.batch, w.ctx_lo, np.int64)
    return rng.integers(w.ctx_lo, w.ctx_hi + 1, size=w.batch).astype(np.int64)


def pages_for(total_tokens: int, page: int) -> int:
    return max(1, math.ceil(total_tokens / page))


def block_tables(w: Workload, final_lens: np.ndarray, rng: np.random.Generator):
    """Tables [B, max_pages] int32 over a pool sized to the total tokens
    (every token of every sequence has a page, residual ones included).
    Returns (tables, num_pages, max_pages)."""
    need = [pages_for(int(n), w.page) for n in final_lens]
    max_pages = max(need)
    num_pages = int(sum(need))
    pool = rng.permutation(num_pages) if w.permuted else np.arange(num_pages)
    tables = np.zeros((len(final_lens), max_pages), np.int32)
    off = 0
    for b, k in enumerate(need):
        tables[b, :k] = pool[off:off + k]
        off += k
    return tables, num_pages, max_pages


def outlier_channels(w: Workload, rng: np.random.Generator) -> np.ndarray:
    """[NKV, outliers] channel indices per kv head."""
    if w.outliers == 0:
        return np.zeros((w.nkv, 0), np.int64)
    return np.stack([rng.choice(w.hd, w.outliers, replace=False) for _ in range(w.nkv)])


def kv_tokens_numpy(w: Workload, rng: np.random.Generator, n: int, outl: np.ndarray):
    """n tokens of K and V, [n, NKV, HD] as fp16 bit patterns (uint16)."""
    k = rng.standard_normal((n, w.nkv, w.hd), dtype=np.float32)
    v = rng.standard_normal((n, w.nkv, w.hd), dtype=np.float32)
    for h in range(w.nkv):
        if outl.shape[1]:
            k[:, h, outl[h]] *= w.outlier_scale
    if w.spike_frac > 0:
        mask = rng.random(k.shape) < w.spike_frac
        signs = np.where(rng.random(k.shape) < 0.5, -1.0, 1.0).astype(np.float32)
        k = np.where(mask, signs * w.spike_value, k)
    return (k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16))


def queries_numpy(w: Workload, rng: np.random.Generator, batch: int) -> np.ndarray:
    return rng.standard_normal((batch, w.nh, w.hd), dtype=np.float32).astype(
        np.float16).view(np.uint16)


def kv_tokens_torch(w: Workload, gen, n: int, outl, device):
    """Device-side twin of kv_tokens_numpy (different random stream)."""
    import torch
    k = torch.randn((n, w.nkv, w.hd), generator=gen, device=device, dtype=torch.float32)
    v = torch.randn((n, w.nkv, w.hd), generator=gen, device=device, dtype=torch.float32)
    if outl is not None and outl.shape[1]:
        scale = torch.ones((w.nkv, w.hd), device=device)
        for h in range(w.nkv):
            scale[h, torch.as_tensor(outl[h], device=device)] = w.outlier_scale
        k *= scale
    if w.spike_frac > 0:
        mask = torch.rand(k.shape, generator=gen, device=device) < w.spike_frac
        sign = torch.where(torch.rand(k.shape, generator=gen, device=device) < 0.5, -1.0, 1.0)
        k = torch.where(mask, sign * w.spike_value, k)
    return k.half(), v.half()
