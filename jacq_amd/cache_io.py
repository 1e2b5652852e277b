"""Cache dump / load: one self-describing file per paged KIVI cache state.

The byte layouts are the v1 ones the kernels read (layout.py:42-154 of the
reference gives the per-page byte math; ``jacq_amd.geometry.page_bytes``
computes it):

* ``k_code`` / ``v_code``   uint8   [pages, NKV, page, HD/2]   (two int4 codes a byte,
  even channel in the low nibble)
* ``k_scale`` / ``k_zero``  fp16    [pages, NKV, HD]
* ``v_scale`` / ``v_zero``  fp16    [pages, NKV, page, HD/32]
* ``k_scr`` / ``v_scr``     fp16    [batch, NKV, R + 32, HD]   (the residual scratch)
* ``block_tables``          int32   [batch, max_pages_per_seq]
* ``seq_lens``              int32   [batch]

Format ``jacq-kivi-cache/1`` is a safetensors file (a JSON header and raw
little-endian tensors; loading it executes nothing).  Its metadata holds the
format tag, the runtime geometry, the per-page byte counts and a SHA-256 of
every tensor; ``load_cache`` checks all of them before it returns.

Two forms:

* full: the whole pool and scratch.  Appends can continue after a load.
* compact: only the pages the sequences' decode windows read (the first
  ``old_valid / page`` entries of each table row, ``old_valid`` from the decode
  window of snapshot :74-83), renumbered in order of first use; table entries
  past a sequence's window are set to 0.  The same decode reads the same bytes
  from it, so it is the form for fixtures; it is not meant for further appends.
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import torch

from .kivi import KiviCheckError, KiviGeometry, PagedKiviCache

FORMAT = "jacq-kivi-cache/1"
POOL = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")
SCRATCH = ("k_scr", "v_scr")
_GEO_FIELDS = ("num_heads", "num_kv_heads", "head_dim", "page_size", "group_size", "residual",
               "max_pages_per_seq", "num_pages")


def _shapes(geo: KiviGeometry, batch: int) -> dict:
    g = geo
    return {
        "k_code": ((g.num_pages, g.num_kv_heads, g.page_size, g.head_dim // 2), torch.uint8),
        "v_code": ((g.num_pages, g.num_kv_heads, g.page_size, g.head_dim // 2), torch.uint8),
        "k_scale": ((g.num_pages, g.num_kv_heads, g.head_dim), torch.float16),
        "k_zero": ((g.num_pages, g.num_kv_heads, g.head_dim), torch.float16),
        "v_scale": ((g.num_pages, g.num_kv_heads, g.page_size, g.head_dim // g.group_size),
                    torch.float16),
        "v_zero": ((g.num_pages, g.num_kv_heads, g.page_size, g.head_dim // g.group_size),
                   torch.float16),
        "k_scr": ((batch, g.num_kv_heads, g.scratch_rows, g.head_dim), torch.float16),
        "v_scr": ((batch, g.num_kv_heads, g.scratch_rows, g.head_dim), torch.float16),
        "block_tables": ((batch, g.max_pages_per_seq), torch.int32),
        "seq_lens": ((batch,), torch.int32),
    }


def page_bytes(geo: KiviGeometry) -> dict:
    """Bytes one page holds per tensor (all kv heads)."""
    g = geo
    code = g.num_kv_heads * g.page_size * g.head_dim // 2
    return {"k_code": code, "v_code": code,
            "k_scale_zero": 2 * 2 * g.num_kv_heads * g.head_dim,
            "v_scale_zero": 2 * 2 * g.num_kv_heads * g.page_size * (g.head_dim // g.group_size)}


def old_valid(geo: KiviGeometry, seq_len: int) -> int:
    """Tokens a decode reads from pages: the decode window of snapshot :74-83
    (length clamped to [0, LQ + R], whole groups, at most LQ)."""
    lq = (geo.max_pages_per_seq * geo.page_size) // geo.group_size * geo.group_size
    bounded = min(max(int(seq_len), 0), lq + geo.residual)
    quant = max(bounded - geo.residual, 0)
    return min(quant // geo.group_size * geo.group_size, lq)


def live_pages(geo: KiviGeometry, block_tables: np.ndarray, seq_lens: np.ndarray) -> np.ndarray:
    """Distinct physical pages the decode windows read, in order of first use."""
    seen: dict[int, None] = {}
    for b in range(len(seq_lens)):
        n = old_valid(geo, int(seq_lens[b])) // geo.page_size
        for p in block_tables[b, :n].tolist():
            if not 0 <= p < geo.num_pages:
                raise ValueError(f"block_tables[{b}] names page {p} outside the pool of "
                                 f"{geo.num_pages}")
            seen.setdefault(int(p), None)
    return np.fromiter(seen.keys(), dtype=np.int64, count=len(seen))


def _check_lens(geo: KiviGeometry, sl: torch.Tensor, what: str) -> None:
    if (sl < 0).any() or (sl > geo.max_seq_len()).any():
        raise ValueError(f"{what} outside [0, {geo.max_seq_len()}]: the decode would clamp "
                         "them, the file format stores only lengths in range")


def _digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def dump_cache(path: str, cache: PagedKiviCache, block_tables: torch.Tensor,
               seq_lens: torch.Tensor, *, compact: bool = False) -> dict:
    """Write ``cache`` with its tables and lengths to ``path``; returns the metadata."""
    from safetensors.torch import save_file

    geo = cache.geo
    batch = cache.batch
    bt = block_tables.detach().to("cpu", torch.int32).contiguous()
    sl = seq_lens.detach().to("cpu", torch.int32).contiguous()
    if tuple(bt.shape) != (batch, geo.max_pages_per_seq):
        raise ValueError(f"block_tables must be [{batch}, {geo.max_pages_per_seq}], "
                         f"got {list(bt.shape)}")
    if tuple(sl.shape) != (batch,):
        raise ValueError(f"seq_lens must be [{batch}], got {list(sl.shape)}")
    _check_lens(geo, sl, "seq_lens")  # the rule load_cache applies, so every dump loads
    tensors = {k: getattr(cache, k).detach().to("cpu").contiguous() for k in POOL + SCRATCH}
    pages = live_pages(geo, bt.numpy(), sl.numpy())  # raises on an entry outside the pool
    if compact:
        remap = {int(p): i for i, p in enumerate(pages.tolist())}
        idx = torch.from_numpy(pages)
        for k in POOL:
            tensors[k] = tensors[k].index_select(0, idx).contiguous()
        new_bt = torch.zeros_like(bt)
        for b in range(batch):
            n = old_valid(geo, int(sl[b])) // geo.page_size
            new_bt[b, :n] = torch.tensor([remap[int(p)] for p in bt[b, :n].tolist()],
                                         dtype=torch.int32)
        bt = new_bt
        geo = KiviGeometry(**{**{f: getattr(geo, f) for f in _GEO_FIELDS},
                              "num_pages": max(1, len(pages))})
        if len(pages) == 0:  # keep one (unread) page so the pool is never empty
            for k in POOL:
                shape, dt = _shapes(geo, batch)[k]
                tensors[k] = torch.zeros(shape, dtype=dt)
    tensors["block_tables"] = bt
    tensors["seq_lens"] = sl
    meta = {
        "format": FORMAT,
        "geometry": json.dumps({f: int(getattr(geo, f)) for f in _GEO_FIELDS}),
        "batch": str(batch),
        "compact": "1" if compact else "0",
        "page_bytes": json.dumps(page_bytes(geo)),
        "sha256": json.dumps({k: _digest(v) for k, v in tensors.items()}),
    }
    save_file(tensors, path, metadata=meta)
    return meta


def load_cache(path: str, device="cpu"):
    """Read a file written by ``dump_cache``.  Returns (cache, block_tables,
    seq_lens) on ``device``; raises ValueError when the file is not format
    jacq-kivi-cache/1 or does not check (shapes, dtypes, digests, table range)."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path}: not a {FORMAT} file (format {meta.get('format')!r})")
    try:
        gd = json.loads(meta["geometry"])
        geo = KiviGeometry(**{f: int(gd[f]) for f in _GEO_FIELDS})
        batch = int(meta["batch"])
        digests = json.loads(meta["sha256"])
        pb = json.loads(meta["page_bytes"])
    except (KeyError, ValueError, TypeError) as e:
        raise ValueError(f"{path}: bad metadata ({e})") from None
    try:
        geo.check()
    except KiviCheckError as e:
        raise ValueError(f"{path}: {e}") from None
    if pb != page_bytes(geo):
        raise ValueError(f"{path}: page byte counts {pb} do not match the geometry")
    tensors = load_file(path)
    want = _shapes(geo, batch)
    if set(tensors) != set(want):
        raise ValueError(f"{path}: tensors {sorted(tensors)} differ from {sorted(want)}")
    for k, (shape, dt) in want.items():
        t = tensors[k]
        if tuple(t.shape) != shape or t.dtype != dt:
            raise ValueError(f"{path}: {k} is {t.dtype}{list(t.shape)}, expected "
                             f"{dt}{list(shape)}")
        if _digest(t) != digests.get(k):
            raise ValueError(f"{path}: {k} does not match its SHA-256")
    sl = tensors["seq_lens"]
    _check_lens(geo, sl, f"{path}: seq_lens")
    live_pages(geo, tensors["block_tables"].numpy(), sl.numpy())  # raises on a bad entry
    dev = torch.device(device)
    cache = PagedKiviCache.from_tensors(geo, {k: tensors[k].to(dev) for k in POOL + SCRATCH})
    return cache, tensors["block_tables"].to(dev), sl.to(dev)
