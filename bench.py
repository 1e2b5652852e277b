"""Benchmark of the paged int4-KIVI decode step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload qwen14b]

A step is one pass of the hot path over the batch, in one launch
(jacq_kivi_write_decode): the cache writer appends one new token to every
sequence (aging out 32-token groups where a sequence crosses the residual
window), then paged decode attention runs for one query token per sequence
over the new state.  Inputs are synthetic (seeded N(0,1) with outlier K
channels, the workload definitions in jacq_amd/workloads.py) and resident
in HBM before timing starts.  A 512 MiB buffer is read (by default) before
every step so the 256 MiB MALL and the L2 start cold.

Prints ONE JSON line.  `value` is the effective KV bandwidth of the step
(the decode's algorithmic bytes / step time, GB/s; the writer's few MB are not
counted); the step time is the GPU time of the fused launch (one kernel: the
decode's stream wavefronts, the first of which do the writer's work before
their runs, then the workgroups that merge the split-K partials) from HIP events the library records on the launch
stream before and after it (jacq_kivi_profile_*), and `ms_per_step` is that
time per step.  `roofline.achieved` is the same bytes over the same time.
A second pass of the same number of steps, continuing the token stream,
launches the kernel with start / stop events that the command processor
stamps at the kernel's own start and end: `kernel_us` and
`roofline.kernel_stamped_frac` come from it (that launch form delays the next
kernel by a few microseconds, so the timed pass leaves it out).  A third pass
runs the same steps as two launches, the writer then the plain decode
(`two_launch_step`).  Before each pass's warmup and before its timed steps a
GPU spin of --lead-ms is enqueued, so the host enqueues every step ahead of
the GPU and the GPU never idles between steps waiting for Python (without it
the first pass's kernels ran about 4 us slower than the second's).
`host_bracketed_us` adds the host-side gaps (Python argument checks before
each launch) seen by events recorded around the Python calls.  The CPU
baseline runs the oracle (oracle/, a C restatement of the reference path) over
the same state on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="qwen14b")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-flush", action="store_true")
    ap.add_argument("--flush", choices=("read", "write"), default="read",
                    help="how the 512 MiB cache flush before each step touches its buffer")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--lead-ms", type=float, default=12.0,
                    help="before the warmup and before the timed steps, enqueue a GPU spin of "
                         "this many ms so the host enqueues the steps ahead of the GPU")
    ap.add_argument("--swap-passes", action="store_true",
                    help="run the command-processor-stamped pass before the plain-event pass")
    ap.add_argument("--wave-stamps", default="", metavar="NPY",
                    help="save per-workgroup start/end stamps of every timed decode of the "
                         "first pass to NPY (jacq_kivi_profile_wave_stamps)")
    ap.add_argument("--stamp-pass", choices=("fused", "decode"), default="fused",
                    help="which pass --wave-stamps records: the fused launches of the first "
                         "pass, or the plain decode launches of the two-launch pass")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the workload, copy MIB MiB device-to-device a few times "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported in this build "
              "(the decode path shards by sequence or kv head, with no exchange inside attention)",
              file=sys.stderr)
        return 2

    import torch

    from jacq_amd import geometry, kivi, workloads as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        return copy_calibration(torch, dev, args.copy_calibration)
    w = wl.WORKLOADS[args.workload]
    rng = np.random.default_rng(w.seed)
    lens0 = wl.context_lens(w, rng)            # lengths when timing starts (after prefill)
    total_steps = args.warmup + args.steps
    # three passes of warmup + steps each (below): room for all their tokens
    tables_np, num_pages, max_pages = wl.block_tables(w, lens0 + 3 * total_steps + 1, rng)
    outl = wl.outlier_channels(w, rng)
    B = w.batch
    geo = kivi.KiviGeometry(w.nh, w.nkv, w.hd, w.page, w.group, w.residual, max_pages, num_pages)
    cache = kivi.PagedKiviCache(geo, B, dev)
    bt = torch.from_numpy(tables_np).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1000 + w.seed)

    # ---- build the cache state on the GPU with the writer ----
    t0 = time.time()
    prefill = w.prefill_chunk
    for b in range(B):
        L = int(lens0[b]) - prefill
        k, v = wl.kv_tokens_torch(w, gen, L, outl, dev)
        cache.sequence_view(b).append(k[None].contiguous(), v[None].contiguous(),
                                      bt[b:b + 1].contiguous(),
                                      torch.zeros(1, dtype=torch.int32, device=dev))
        del k, v
    torch.cuda.synchronize()
    prefill_info = None
    if prefill:
        # one launch: every sequence appends a `prefill`-token chunk (many age-outs each)
        k, v = wl.kv_tokens_torch(w, gen, B * prefill, outl, dev)
        k = k.view(B, prefill, w.nkv, w.hd).contiguous()
        v = v.view(B, prefill, w.nkv, w.hd).contiguous()
        start = torch.from_numpy((lens0 - prefill).astype(np.int32)).to(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        cache.append(k, v, bt, start)
        e1.record()
        torch.cuda.synchronize()
        prefill_info = {"tokens_per_seq": prefill, "us": round(e0.elapsed_time(e1) * 1e3, 1)}
        del k, v
    log(f"[bench] state built in {time.time() - t0:.1f}s: B={B} ctx {lens0.min()}..{lens0.max()} "
        f"pages={num_pages}")

    # ---- per-step inputs ----
    qs = torch.randn((3 * total_steps, B, w.nh, w.hd), generator=gen, device=dev).half()
    nk = torch.randn((3 * total_steps, B, w.nkv, w.hd), generator=gen, device=dev).half()
    nv = torch.randn((3 * total_steps, B, w.nkv, w.hd), generator=gen, device=dev).half()
    out = torch.empty((B, w.nh, w.hd), dtype=torch.float32, device=dev)
    lens_before = torch.from_numpy(lens0.astype(np.int32)).to(dev)
    lens_after = lens_before + 1
    flush = None if args.no_flush else torch.ones(512 << 20, dtype=torch.uint8, device=dev)
    flush_sink = torch.zeros(1, dtype=torch.int64, device=dev)
    ws_bytes = max(kivi.lib().jacq_kivi_decode_workspace_size(ctypes_geo(kivi, geo), B),
                   kivi.lib().jacq_kivi_write_decode_workspace_size(ctypes_geo(kivi, geo), B))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    stream = torch.cuda.current_stream(dev)
    STAMP_CAP = 8192  # workgroups per launch the stamp buffer holds
    stamps = (torch.zeros((args.steps, STAMP_CAP, 4), dtype=torch.int64, device=dev)
              if args.wave_stamps else None)

    spin_cycles = 0
    if args.lead_ms > 0:
        # cycles of torch's spin kernel per ms on this GPU
        a_, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000000)
        a_.record()
        torch.cuda._sleep(1000000)
        b_.record()
        torch.cuda.synchronize()
        spin_cycles = int(args.lead_ms * 1000000 / max(a_.elapsed_time(b_), 1e-3))
        log(f"[bench] lead {args.lead_ms} ms = {spin_cycles} spin cycles")

    def lead():
        if spin_cycles:
            torch.cuda._sleep(spin_cycles)

    def timed_pass(step0: int, split: bool, fused: bool):
        """warmup + steps from global step step0, each a cache flush then one
        step of the hot path: the fused write + decode launch, or (not fused)
        the writer launch then the decode launch.  The library's events
        bracket the decode launch -- the fused one or the plain decode (split:
        stamped by the command processor at the kernel's own start and end).
        Returns per-step arrays of the timed steps and the wall time."""
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
               for _ in range(total_steps)]
        torch.cuda.synchronize()
        kivi.profile_start(total_steps, split)
        wall0 = None
        lead()
        for i in range(total_steps):
            gi = step0 + i
            if i == args.warmup:
                torch.cuda.synchronize()
                wall0 = time.perf_counter()
                lead()
            if flush is not None:
                # evict the pool from the 256 MiB MALL and the L2s; a read
                # leaves no dirty lines whose write-back would land in the
                # timed decode (--flush write rewrites the buffer instead)
                if args.flush == "read":
                    flush_sink.add_(flush.view(torch.int64).sum())
                else:
                    flush.fill_(gi & 0xff)
            e = evs[i]
            e[0].record(stream)
            if not fused:
                cache.append(nk[gi][:, None], nv[gi][:, None], bt, lens_before)
            e[1].record(stream)
            stamp_this = (stamps is not None and not split and i >= args.warmup
                          and fused == (args.stamp_pass == "fused"))
            if stamp_this:
                kivi.lib().jacq_kivi_profile_wave_stamps(
                    kivi._ptr(stamps[i - args.warmup]), STAMP_CAP)
            if fused:
                cache.write_decode(qs[gi], nk[gi], nv[gi], lens_after, bt, out=out,
                                   workspace=workspace)
            else:
                cache.decode(qs[gi], lens_after, bt, out=out, workspace=workspace)
            if stamp_this:
                kivi.lib().jacq_kivi_profile_wave_stamps(None, 0)
            e[2].record(stream)
            lens_before.add_(1)
            lens_after.add_(1)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        kern_ms, merge_ms = kivi.profile_stop(total_steps)
        write_ms = kivi.profile_write_ms(total_steps)
        host = [(evs[i][0].elapsed_time(evs[i][1]), evs[i][1].elapsed_time(evs[i][2]))
                for i in range(args.warmup, total_steps)]
        return (np.array(kern_ms[args.warmup:]), np.array(merge_ms[args.warmup:]),
                np.array(write_ms[args.warmup:]) if not fused else None, np.array(host), wall)

    # pass 1 (the timed region of the contract): the fused step, events only
    # around each launch, so the figure is the step exactly as a caller runs it
    # pass 2: the same steps continued, the fused kernel's own start and end
    # stamped by the command processor (kernel_us, roofline cross-check)
    # pass 3: the same steps as two launches (writer, then decode), for the
    # comparison
    p1, p2, p3 = 0, total_steps, 2 * total_steps
    if args.swap_passes:
        p1, p2 = p2, p1
        kern, _, _, _, _ = timed_pass(p2, split=True, fused=True)
        dec, _, _, host, wall = timed_pass(p1, split=False, fused=True)
    else:
        dec, _, _, host, wall = timed_pass(p1, split=False, fused=True)
        kern, _, _, _, _ = timed_pass(p2, split=True, fused=True)
    sep_dec, _, sep_wr, _, _ = timed_pass(p3, split=False, fused=False)
    if stamps is not None:
        np.save(args.wave_stamps, stamps.cpu().numpy())

    def bytes_of(step0):
        return [geometry.decode_step_bytes(lens0 + step0 + i + 1, w.nh, w.nkv, w.hd, w.page,
                                         w.residual, w.group)
                for i in range(args.warmup, total_steps)]
    step_bytes = bytes_of(p1)
    # GPU time of the launch from the events the library records on the launch
    # stream; host-side gaps before a launch (Python argument checks) are
    # excluded, host_bracketed_* keep them
    host_dec = host[:, 1]
    gbs = float(np.sum(step_bytes) / (dec.sum() * 1e-3) / 1e9)
    kern_gbs = float(np.sum(bytes_of(p2)) / (kern.sum() * 1e-3) / 1e9)
    sep_gbs = float(np.sum(bytes_of(p3)) / (sep_dec.sum() * 1e-3) / 1e9)
    bytes_per_step = float(np.mean(step_bytes))

    # ---- CPU baseline: the oracle over the same final state on this host ----
    cpu = None
    if not args.no_cpu_baseline:
        last = 3 * total_steps  # the state after the last decode of pass 3
        cpu = cpu_baseline(args, w, cache, qs[last - 1], lens0 + last, tables_np,
                           out, max_pages,
                           bytes_per_step_last=geometry.decode_step_bytes(
                               lens0 + last, w.nh, w.nkv, w.hd, w.page, w.residual, w.group))

    traffic = load_traffic(args.workload)
    line = {
        "metric": "paged int4-KIVI decode attn us/step + effective KV GB/s (% HBM peak), 14B shape",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(float(dec.mean()), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 KV, fp16 MFMA operands, fp32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.nh}q/{w.nkv}kv heads, head_dim {w.hd}, batch {B}, "
                        f"context U[{w.ctx_lo},{w.ctx_hi}], page {w.page}, group {w.group}, "
                        f"residual {w.residual}, int4 KIVI K/V, per step one fused launch "
                        f"(jacq_kivi_write_decode): append one token per sequence, aging "
                        f"32-token groups out where a sequence crosses the residual window, "
                        f"then decode one query per sequence",
            "batch": B,
            "mean_context": float(np.mean(lens0)),
            "pages": num_pages,
            "cold_cache": flush is not None,
            "cache_flush": None if flush is None else f"{args.flush} 512 MiB before each step",
        },
        "step_us": {"mean": round(float(dec.mean()) * 1e3, 2),
                    "min": round(float(dec.min()) * 1e3, 2),
                    "median": round(float(np.median(dec)) * 1e3, 2),
                    "p90": round(float(np.percentile(dec, 90)) * 1e3, 2)},
        "kernel_us": {"mean": round(float(kern.mean()) * 1e3, 2),
                      "median": round(float(np.median(kern)) * 1e3, 2),
                      "min": round(float(kern.min()) * 1e3, 2)},
        "host_bracketed_us": round(float(host_dec.mean()) * 1e3, 2),
        "two_launch_step": {
            "write_us": round(float(sep_wr.mean()) * 1e3, 2),
            "decode_us": round(float(sep_dec.mean()) * 1e3, 2),
            "write_plus_decode_us": round(float((sep_wr + sep_dec).mean()) * 1e3, 2),
            "decode_only_frac": round(sep_gbs / HBM_PEAK_GBS, 4),
        },
        "decode_bytes_per_step": int(bytes_per_step),
        # the writer's share of the step, not in `value` (new rows, age-outs, shifts)
        "writer_bytes_per_step": int(np.mean([
            geometry.write_step_bytes(lens0 + p1 + i, w.nkv, w.hd, w.residual, w.group)
            for i in range(args.warmup, total_steps)])),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "wall_s_timed_region": round(wall, 4),
        "roofline": {
            "kernel": f"kivi_decode_stream_kernel<{w.hd}, {w.page}, "
                      f"{'true' if w.nh // w.nkv <= 8 else 'false'}, false, true> "
                      f"(fused write + decode)",
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "timing": "HIP events on the launch stream around each fused launch of the timed pass",
            "kernel_stamped_frac": round(kern_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    if prefill_info:
        line["prefill_write"] = prefill_info
    print(json.dumps(line), flush=True)
    return 0


def copy_calibration(torch, dev, mib: int) -> int:
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE under
    rocprofv3 --pmc give the counters' bytes-per-unit on this GPU."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 3}), flush=True)
    return 0


def ctypes_geo(kivi, geo):
    import ctypes
    return ctypes.byref(geo.c())


def load_traffic(workload: str):
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), if one exists."""
    p = os.path.join(ROOT, "profiles", f"decode_{workload}_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def cpu_baseline(args, w, cache, q_last, lens_last, tables_np, gpu_out, max_pages,
                 bytes_per_step_last):
    """Time the oracle's batched decode on the host over the final GPU state."""
    import torch

    from oracle import oracle as o
    from tests.kivi_testlib import ATOL, RTOL

    o.lib()

    def host(t):
        x = t.detach().cpu()
        if x.dtype == torch.float16:
            return x.view(torch.int16).numpy().view(np.uint16)
        return x.numpy()

    g = o.Geometry(w.nh, w.nkv, w.hd, w.page, w.group, w.residual, max_pages)
    c = o.Cache(g, host(cache.k_code), host(cache.k_scale), host(cache.k_zero),
                host(cache.v_code), host(cache.v_scale), host(cache.v_zero),
                host(cache.k_scr), host(cache.v_scr))
    q = host(q_last)
    lens = lens_last.astype(np.int32)
    affinity = len(os.sched_getaffinity(0))
    threads = args.cpu_threads or min(16, affinity)
    t0 = time.perf_counter()
    ref = o.decode_batch(c, q, lens, tables_np, nthreads=threads)
    dt = time.perf_counter() - t0
    t0 = time.perf_counter()
    ref1 = o.decode_batch(c, q, lens, tables_np, nthreads=1)
    dt1 = time.perf_counter() - t0
    # sanity: the GPU's last step saw the same state and query
    gpu = gpu_out.cpu().numpy()
    err = np.abs(gpu - ref)
    bound = ATOL + RTOL * np.abs(ref)
    ok = bool(np.all(err <= bound))
    return {
        "value": round(bytes_per_step_last / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full last step: {w.batch} sequences, one decode query each, "
                  f"{int(lens.sum())} tokens; {dt * 1e3:.1f} ms on {threads} threads "
                  f"(OpenMP over sequence x kv head), {dt1 * 1e3:.1f} ms on 1 thread",
        "us_per_step": round(dt * 1e6, 1),
        "single_thread": {"value": round(bytes_per_step_last / dt1 / 1e9, 3), "unit": "GB/s",
                          "us_per_step": round(dt1 * 1e6, 1),
                          "same_result": bool(np.array_equal(ref, ref1))},
        "host": {"nproc": os.cpu_count(), "affinity_cpus": affinity,
                 "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
                 "cpu_model": cpu_model()},
        "matches_gpu_within_tolerance": ok,
        "max_abs_diff_vs_gpu": float(err.max()),
        "max_err_over_bound": round(float((err / bound).max()), 4),
    }


def cpu_model() -> str | None:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    sys.exit(main())
