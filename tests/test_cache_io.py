"""Cache dump / load (jacq_amd.cache_io): round trips, the compact form, and
the checks load_cache makes.  The CPU tests build the cache with the oracle
writer and compare the oracle's decode over the original and the reloaded
state; the GPU test does the same with the HIP writer and decode."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from jacq_amd import cache_io, kivi
from jacq_amd import workloads as wl
from oracle import oracle as o
from tests.kivi_testlib import State, to_torch

POOL_AND_SCR = cache_io.POOL + cache_io.SCRATCH


def _state(name="qwen05b", lens=(40, 300, 700), seed=3):
    st = State(wl.WORKLOADS[name], lens=list(lens), seed=seed)
    st.build_oracle()
    return st


def _kgeo(st: State) -> kivi.KiviGeometry:
    w = st.w
    return kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, st.max_pages, st.num_pages)


def _cache(st: State, device="cpu") -> kivi.PagedKiviCache:
    return kivi.PagedKiviCache.from_tensors(_kgeo(st), to_torch(st, device))


def _to_oracle(cache: kivi.PagedKiviCache, st: State) -> o.Cache:
    def a(t):
        t = t.cpu().contiguous()
        return (t.view(torch.int16) if t.dtype == torch.float16 else t).numpy().view(
            np.uint16 if t.dtype == torch.float16 else np.uint8).copy()
    return o.Cache(st.geo, *[a(getattr(cache, k)) for k in POOL_AND_SCR])


def _lens(st):
    return torch.from_numpy(st.lens.astype(np.int32))


def test_full_round_trip_is_byte_exact(tmp_path):
    st = _state()
    c = _cache(st)
    p = str(tmp_path / "full.safetensors")
    meta = cache_io.dump_cache(p, c, torch.from_numpy(st.tables), _lens(st))
    assert meta["format"] == cache_io.FORMAT and meta["compact"] == "0"
    c2, bt, sl = cache_io.load_cache(p)
    assert c2.geo == c.geo and c2.batch == c.batch
    for k in POOL_AND_SCR:
        assert torch.equal(getattr(c2, k).view(torch.uint8), getattr(c, k).view(torch.uint8)), k
    assert torch.equal(bt, torch.from_numpy(st.tables))
    assert torch.equal(sl, _lens(st))


@pytest.mark.parametrize("name,lens", [("qwen05b", (40, 300, 700)),
                                       ("mistral7b", (129, 1000)),
                                       ("tinyllama", (512,))])
def test_compact_form_decodes_to_the_same_bits(tmp_path, name, lens):
    """The compact file keeps only the pages the decode windows read; the
    oracle's decode over it equals the decode over the full state bit for bit."""
    st = _state(name, lens)
    p = str(tmp_path / "compact.safetensors")
    cache_io.dump_cache(p, _cache(st), torch.from_numpy(st.tables), _lens(st), compact=True)
    c2, bt, sl = cache_io.load_cache(p)
    live = cache_io.live_pages(_kgeo(st), st.tables, st.lens)
    assert c2.geo.num_pages == max(1, len(live)) <= st.num_pages
    # every page a window reads, and nothing else: the distinct count equals
    # the sum of each window's pages (the tables here never share a page)
    assert len(live) == sum(cache_io.old_valid(_kgeo(st), n) // st.w.page for n in st.lens)
    oc = _to_oracle(c2, st)
    oc.geo = o.Geometry(st.w.nh, st.w.nkv, st.w.hd, st.w.page, 32, st.w.residual, st.max_pages)
    for b in range(st.batch):
        ref = o.decode_online(st.cache, b, st.q[b], st.tables[b], int(st.lens[b]))
        got = o.decode_online(oc, b, st.q[b], bt[b].numpy(), int(sl[b]))
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"seq {b}"


def test_short_sequences_compact_to_one_unread_page(tmp_path):
    """Windows with no quantised tokens (L <= R + 31) read no page: the
    compact pool keeps a single zero page."""
    st = _state("qwen05b", (20, 150))
    p = str(tmp_path / "short.safetensors")
    cache_io.dump_cache(p, _cache(st), torch.from_numpy(st.tables), _lens(st), compact=True)
    c2, bt, _ = cache_io.load_cache(p)
    assert c2.geo.num_pages == 1 and int(bt.abs().sum()) == 0
    assert torch.equal(c2.k_scr, _cache(st).k_scr)


def _resave(p, q, mutate=None, meta_update=None):
    from safetensors import safe_open
    from safetensors.torch import load_file, save_file
    with safe_open(p, framework="pt") as f:
        meta = dict(f.metadata())
    t = load_file(p)
    if mutate:
        mutate(t, meta)
    if meta_update:
        meta.update(meta_update)
    save_file(t, q, metadata=meta)


def test_load_rejects_bad_files(tmp_path):
    st = _state("qwen05b", (300,))
    p = str(tmp_path / "ok.safetensors")
    cache_io.dump_cache(p, _cache(st), torch.from_numpy(st.tables), _lens(st))
    cache_io.load_cache(p)

    q = str(tmp_path / "fmt.safetensors")
    _resave(p, q, meta_update={"format": "something-else/1"})
    with pytest.raises(ValueError, match="not a jacq-kivi-cache/1 file"):
        cache_io.load_cache(q)

    def flip(t, meta):  # one code byte changes, the digest does not
        t["k_code"].view(-1)[7] ^= 0x10
    q = str(tmp_path / "flip.safetensors")
    _resave(p, q, flip)
    with pytest.raises(ValueError, match="k_code does not match its SHA-256"):
        cache_io.load_cache(q)

    def bad_page(t, meta):  # a table entry past the pool, with a matching digest
        import json
        t["block_tables"][0, 0] = st.num_pages
        d = json.loads(meta["sha256"])
        d["block_tables"] = cache_io._digest(t["block_tables"])
        meta["sha256"] = json.dumps(d)
    q = str(tmp_path / "page.safetensors")
    _resave(p, q, bad_page)
    with pytest.raises(ValueError, match="outside the pool"):
        cache_io.load_cache(q)

    import json
    g = json.loads(_meta(p)["geometry"])
    q = str(tmp_path / "geo.safetensors")
    _resave(p, q, meta_update={"geometry": json.dumps({**g, "head_dim": 96})})
    with pytest.raises(ValueError):
        cache_io.load_cache(q)


def _meta(p):
    from safetensors import safe_open
    with safe_open(p, framework="pt") as f:
        return dict(f.metadata())


def test_dump_rejects_out_of_pool_tables(tmp_path):
    st = _state("qwen05b", (300,))
    bt = torch.from_numpy(st.tables).clone()
    bt[0, 1] = -1
    with pytest.raises(ValueError, match="outside the pool"):
        cache_io.dump_cache(str(tmp_path / "x.safetensors"), _cache(st), bt, _lens(st))


def test_dump_rejects_lengths_load_would_reject(tmp_path):
    """dump_cache and load_cache apply one length rule, so every file dump
    writes loads back: a negative length or one past max_seq_len is refused
    at dump time (the decode would clamp it; the format does not store it)."""
    st = _state("qwen05b", (300,))
    geo = _kgeo(st)
    for bad in (-1, geo.max_seq_len() + 1):
        with pytest.raises(ValueError, match="outside"):
            cache_io.dump_cache(str(tmp_path / "x.safetensors"), _cache(st),
                                torch.from_numpy(st.tables), torch.tensor([bad], dtype=torch.int32))
    p = str(tmp_path / "edge.safetensors")
    cache_io.dump_cache(p, _cache(st), torch.from_numpy(st.tables),
                        torch.tensor([geo.max_seq_len()], dtype=torch.int32))
    _, _, sl = cache_io.load_cache(p)
    assert int(sl[0]) == geo.max_seq_len()


@pytest.mark.gpu
def test_gpu_written_cache_round_trips_and_decodes_identically(tmp_path):
    """HIP writer builds the state; after a compact dump and a reload on the
    GPU, the HIP decode returns the same bits as over the original pool."""
    w = wl.WORKLOADS["qwen14b"]
    st = State(w, lens=[900, 2000, 77], seed=11)
    dev = torch.device("cuda:0")
    geo = _kgeo(st)
    cache = kivi.PagedKiviCache(geo, st.batch, dev)
    bt = torch.from_numpy(st.tables).to(dev)
    for b in range(st.batch):
        n = int(st.lens[b])
        k = torch.from_numpy(st.k_hist[b][:n]).view(torch.float16)[None].contiguous().to(dev)
        v = torch.from_numpy(st.v_hist[b][:n]).view(torch.float16)[None].contiguous().to(dev)
        cache.sequence_view(b).append(k, v, bt[b:b + 1].contiguous(),
                                      torch.zeros(1, dtype=torch.int32, device=dev))
    lens = torch.from_numpy(st.lens.astype(np.int32)).to(dev)
    q = torch.from_numpy(st.q).view(torch.float16).to(dev)
    ref = cache.decode(q, lens, bt)
    p = str(tmp_path / "gpu.safetensors")
    cache_io.dump_cache(p, cache, bt, lens, compact=True)
    c2, bt2, sl2 = cache_io.load_cache(p, dev)
    got = c2.decode(q, sl2, bt2)
    torch.cuda.synchronize()
    assert torch.equal(ref.view(torch.int32), got.view(torch.int32))


@pytest.mark.parametrize("residual,max_pages", [(128, 124), (32, 40)])
def test_old_valid_is_the_decode_window(residual, max_pages):
    """cache_io.old_valid (which pages a compact dump keeps) against the
    oracle's split rule on the clamped length, for every length from 0 to past
    the clamp: whole groups, never more than the length allows, at most LQ."""
    geo = kivi.KiviGeometry(40, 8, 128, 16, 32, residual, max_pages, 1)
    lq = max_pages * 16 // 32 * 32
    for n in range(0, lq + residual + 100):
        ov = cache_io.old_valid(geo, n)
        ref = min(o.split_old_tokens(min(n, lq + residual), residual, 32), lq)
        assert ov == ref, n
        assert ov % 32 == 0 and 0 <= ov <= max(0, min(n, lq + residual) - residual)
