"""Parity at the benchmark's full sizes.

* qwen14b (the headline config: 64 sequences, contexts U[1024,16384], page 16):
  the HIP writer builds every sequence from its history, then one step
  writes a token to every sequence and decodes (a writer launch then a decode
  launch, or one jacq_kivi_write_decode launch); the whole pool and the live scratch rows
  must equal the oracle's bit for bit, and the decode of the whole batch must
  be within max-abs 2e-3 / rel 1e-2 of the oracle's fp32 online decode.
* long (256 sequences, contexts U[4096,32768], K with 1% +-20 spikes): the
  config's own recipe -- history, a 512-token prefill chunk flushed into pages,
  then 8 steps of one-token write + decode.  The oracle re-builds a sample of
  sequences (their pages renumbered into a compact pool): their pages and
  scratch must be bit-exact and every step's decode within the tolerance.  For
  the whole batch, a size-independent property: decoding a pool whose pages are
  permuted (tables remapped) gives the same bits, since the work split depends
  on lengths only.

Token values are drawn on the GPU and copied to the host, so both sides see
the same bits.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from jacq_amd import workloads as wl
from oracle import oracle as o
from tests.kivi_testlib import assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

POOL = ("k_code", "k_scale", "k_zero", "v_code", "v_scale", "v_zero")
THREADS = 16  # the GPU box's CPU share


@pytest.fixture(scope="module")
def kivi():
    from jacq_amd import kivi as k
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    k.lib()
    return k


def _u16(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _oracle_write(cache: o.Cache, b: int, k: np.ndarray, v: np.ndarray, table: np.ndarray,
                  start: int) -> None:
    """Tokens [start, start + n) of sequence b through the reference's planned
    sub-chunks (each equal to repeated single-token writes)."""
    done, n = 0, k.shape[0]
    while done < n:
        m = min(128, n - done)
        for (s0, nn, *_r) in o.plan_batched_write(start + done, m, cache.geo.residual, 32):
            i = s0 - start
            assert o.cache_write_batched(cache, b, k[i:i + nn], v[i:i + nn], table, s0) == 0
        done += m


def _parallel(fn, items):
    o.lib()  # load (and declare) before the threads call into it
    with ThreadPoolExecutor(THREADS) as ex:
        list(ex.map(fn, items))


def _geometry(kivi, w, max_pages, num_pages):
    return kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, max_pages, num_pages)


@pytest.mark.parametrize("fused", [False, True], ids=["append_then_decode", "write_decode"])
def test_fullsize_qwen14b_writer_and_decode(kivi, fused):
    """The last token of every sequence goes in by one step: the writer
    launch then the decode launch, or the fused jacq_kivi_write_decode."""
    w = wl.WORKLOADS["qwen14b"]
    rng = np.random.default_rng(w.seed)
    lens = wl.context_lens(w, rng)
    tables, num_pages, max_pages = wl.block_tables(w, lens + 1, rng)
    outl = wl.outlier_channels(w, rng)
    dev = torch.device("cuda:0")
    print(f"qwen14b full size: B={w.batch} tokens={int(lens.sum())} pages={num_pages}", flush=True)
    cache = kivi.PagedKiviCache(_geometry(kivi, w, max_pages, num_pages), w.batch, dev)
    bt = torch.from_numpy(tables).to(dev)
    gen = torch.Generator(device=dev).manual_seed(w.seed)
    hist = []
    zero = torch.zeros(1, dtype=torch.int32, device=dev)
    for b in range(w.batch):
        k, v = wl.kv_tokens_torch(w, gen, int(lens[b]) + 1, outl, dev)
        cache.sequence_view(b).append(k[None, :-1].contiguous(), v[None, :-1].contiguous(),
                                      bt[b:b + 1].contiguous(), zero)
        hist.append((k, v))
    # one step: a token for every sequence
    nk = torch.stack([k[-1] for k, _ in hist]).contiguous()
    nv = torch.stack([v[-1] for _, v in hist]).contiguous()
    final = lens + 1
    q = torch.randn((w.batch, w.nh, w.hd), generator=gen, device=dev).half()
    after = torch.from_numpy(final.astype(np.int32)).to(dev)
    if fused:
        out = cache.write_decode(q, nk, nv, after, bt)
    else:
        cache.append(nk[:, None].contiguous(), nv[:, None].contiguous(), bt,
                     torch.from_numpy(lens.astype(np.int32)).to(dev))
        out = cache.decode(q, after, bt)
    torch.cuda.synchronize()
    ages = sum(wl.split_old_tokens(int(n) + 1, w.residual) > wl.split_old_tokens(int(n), w.residual)
               for n in lens)
    print(f"qwen14b step: {ages} of {w.batch} sequences age a group out", flush=True)

    geo = o.Geometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, max_pages)
    ref = o.Cache.empty(geo, num_pages, w.batch)
    hk = [_u16(k) for k, _ in hist]
    hv = [_u16(v) for _, v in hist]
    _parallel(lambda b: _oracle_write(ref, b, hk[b], hv[b], tables[b], 0), range(w.batch))
    for name in POOL:
        got = _u16(getattr(cache, name))
        want = getattr(ref, name)
        assert np.array_equal(got, want), f"{name} differs at {np.argwhere(got != want)[:5]}"
    for name in ("k_scr", "v_scr"):
        got, want = _u16(getattr(cache, name)), getattr(ref, name)
        for b in range(w.batch):
            r = int(final[b] - wl.split_old_tokens(int(final[b]), w.residual))
            assert np.array_equal(got[b, :, :r], want[b, :, :r]), f"{name}[{b}] differs"
    want = o.decode_batch(ref, _u16(q), final.astype(np.int32), tables, nthreads=THREADS)
    assert_close(out.cpu().numpy(), want, f"qwen14b full-size decode (fused={fused})")


@pytest.mark.parametrize("fused", [False, True], ids=["append_then_decode", "write_decode"])
def test_fullsize_long_recipe_sampled_parity_and_permutation(kivi, fused):
    """The long recipe at full size (the 8 decode steps as writer + decode
    launches, or as fused jacq_kivi_write_decode steps): sampled sequences
    bit-exact and in tolerance against the oracle, and the whole batch's last
    decode bit-identical over a permuted pool."""
    w = wl.WORKLOADS["long"]
    rng = np.random.default_rng(w.seed)
    lens = wl.context_lens(w, rng)  # context before the 8 decode steps
    steps = w.decode_steps
    tables, num_pages, max_pages = wl.block_tables(w, lens + steps, rng)
    outl = wl.outlier_channels(w, rng)
    dev = torch.device("cuda:0")
    print(f"long full size: B={w.batch} tokens={int(lens.sum())} pages={num_pages}", flush=True)
    cache = kivi.PagedKiviCache(_geometry(kivi, w, max_pages, num_pages), w.batch, dev)
    bt = torch.from_numpy(tables).to(dev)
    gen = torch.Generator(device=dev).manual_seed(w.seed)
    sample = sorted({0, 1, 97, 128, 200, w.batch - 1, int(np.argmax(lens))})
    hist = {}
    steps_k, steps_v = [], []
    zero = torch.zeros(1, dtype=torch.int32, device=dev)
    chunk = w.prefill_chunk
    for b in range(w.batch):
        L = int(lens[b])
        k, v = wl.kv_tokens_torch(w, gen, L + steps, outl, dev)
        view = cache.sequence_view(b)
        # history, then the 512-token prefill chunk flushed in one call
        view.append(k[None, :L - chunk].contiguous(), v[None, :L - chunk].contiguous(),
                    bt[b:b + 1].contiguous(), zero)
        view.append(k[None, L - chunk:L].contiguous(), v[None, L - chunk:L].contiguous(),
                    bt[b:b + 1].contiguous(),
                    torch.full((1,), L - chunk, dtype=torch.int32, device=dev))
        steps_k.append(k[L:])
        steps_v.append(v[L:])
        if b in sample:
            hist[b] = (_u16(k), _u16(v))
    qs = [torch.randn((w.batch, w.nh, w.hd), generator=gen, device=dev).half()
          for _ in range(steps)]
    outs = []
    cur = lens.copy()
    for s in range(steps):
        nk = torch.stack([t[s] for t in steps_k]).contiguous()
        nv = torch.stack([t[s] for t in steps_v]).contiguous()
        after = torch.from_numpy((cur + 1).astype(np.int32)).to(dev)
        if fused:
            outs.append(cache.write_decode(qs[s], nk, nv, after, bt))
        else:
            cache.append(nk[:, None].contiguous(), nv[:, None].contiguous(), bt,
                         torch.from_numpy(cur.astype(np.int32)).to(dev))
            outs.append(cache.decode(qs[s], after, bt))
        cur += 1
    torch.cuda.synchronize()

    # permuted pool, remapped tables: the same bits for the whole batch
    perm = torch.randperm(num_pages, generator=torch.Generator().manual_seed(9)).to(dev)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(num_pages, device=dev)
    pcache = kivi.PagedKiviCache.from_tensors(cache.geo, {
        **{n: getattr(cache, n).index_select(0, perm) for n in POOL},
        "k_scr": cache.k_scr, "v_scr": cache.v_scr})
    pbt = inv[bt.long()].to(torch.int32).contiguous()
    cur_t = torch.from_numpy(cur.astype(np.int32)).to(dev)
    pout = pcache.decode(qs[-1], cur_t, pbt)
    # the plain decode of the final state (the fused step cuts its runs
    # differently, so its own output agrees only to rounding)
    base = outs[-1] if not fused else cache.decode(qs[-1], cur_t, bt)
    torch.cuda.synchronize()
    assert torch.equal(pout.view(torch.int32), base.view(torch.int32))
    if fused:
        assert torch.allclose(outs[-1], base, atol=1e-3, rtol=2e-3), (outs[-1] - base).abs().max()
    del pcache

    # the sampled sequences, re-built by the oracle in a compact pool
    geo = o.Geometry(w.nh, w.nkv, w.hd, w.page, 32, w.residual, max_pages)
    used = [int(wl.pages_for(int(lens[b]) + steps, w.page)) for b in sample]
    ref = o.Cache.empty(geo, sum(used), len(sample))
    ctab = np.zeros((len(sample), max_pages), np.int32)
    off = 0
    for i, (b, n) in enumerate(zip(sample, used)):
        ctab[i, :n] = np.arange(off, off + n)
        off += n

    want_out = np.zeros((steps, len(sample), w.nh, w.hd), np.float32)
    qh = [_u16(t) for t in qs]

    def build(i):
        b = sample[i]
        k, v = hist[b]
        L = int(lens[b])
        _oracle_write(ref, i, k[:L], v[:L], ctab[i], 0)
        for s in range(steps):  # each step: the single-token write, then its decode
            o.cache_write(ref, i, k[L + s], v[L + s], ctab[i], L + s + 1)
            want_out[s, i] = o.decode_online(ref, i, qh[s][b], ctab[i], L + s + 1)
    _parallel(build, range(len(sample)))

    for i, (b, n) in enumerate(zip(sample, used)):
        rows = torch.from_numpy(tables[b, :n].astype(np.int64)).to(dev)
        for name in POOL:
            got = _u16(getattr(cache, name).index_select(0, rows))
            want = getattr(ref, name)[ctab[i, :n]]
            assert np.array_equal(got, want), f"seq {b}: {name} differs"
        r = int(cur[b] - wl.split_old_tokens(int(cur[b]), w.residual))
        for name in ("k_scr", "v_scr"):
            got = _u16(getattr(cache, name)[b])
            assert np.array_equal(got[:, :r], getattr(ref, name)[i][:, :r]), f"seq {b}: {name}"
        for s in range(steps):
            assert_close(outs[s][b].cpu().numpy(), want_out[s, i], f"long seq {b} step {s + 1}")
