#!/usr/bin/env python3
"""Benchmark of the llamd quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]

Headline (BASELINE.json metric "Q6_K matvec HBM GB/s (% of peak)"), on
the Q6_K expert-FFN matvecs at batch 1 -- gate and up
W [768 x 2048], down W [2048 x 768], weights from N(0, 0.02) quantized to Q6_K,
activations N(0, 1) quantized to Q8_K (resident on the device before timing).
One step = the three matvecs. value = algorithmic bytes / time over exactly
K steps of plain launches, back to back on the library stream (a rocprofv3
kernel trace of the same command gives the same per-launch time; the
graph-replay figure is reported beside it). Every launch reads a different
device copy of its weights (>= 1 GiB of copies in rotation) so the 256 MB
Infinity Cache cannot serve them.

The same JSON line carries the other configs under "extra" (Q8_0 matvec,
MoE decode layer tok/s, prefill grouped GEMM, LM head b=1/b=16), the roofline
of the dominant kernel (q6k_mv_b1: HIP events on the library stream over the
timed region) and the CPU baseline: the C oracle (1 thread, the reference's design)
timed on this host on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0        # dense int8 MFMA
QK_K = 256
GIB = 1 << 30
# HBM bytes per q6k_mv_b1 launch of configs[1] (mean of the step's three
# launches), from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this script
# scaled by the same counters on a copy of known size (x2.0 fetch, x1.0
# write); the commands and per-kernel values are in
# profiles/q6k_mv_b1.configs1.hbm_traffic.txt. Algorithmic: 1,301,504 B.
TRAFFIC_Q6K_MV_CONFIGS1 = 1398190


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def q6k_bytes(rows, k):
    return rows * k // QK_K * 210


class Timer:
    """HIP events on the library stream (where every kernel is launched)."""

    def __init__(self, L, n=2):
        self.L = L
        self.ev = [L.llamd_hip_event_create() for _ in range(n)]

    def rec(self, i):
        if self.L.llamd_hip_event_record(self.ev[i]):
            raise RuntimeError("event record failed")

    def ms(self, a, b):
        return float(self.L.llamd_hip_event_elapsed_ms(self.ev[a], self.ev[b]))

    def close(self):
        for e in self.ev:
            self.L.llamd_hip_event_destroy(e)


KERNEL_CLOCK_HZ = 100e6  # s_memrealtime on gfx950


def clocked_region(L, rocm, many, names, steps, warmup):
    """The headline's timed region once more with the in-kernel clock on
    (llamd_hip_kernel_clock): each q6k_mv_b1 launch records its earliest
    workgroup start and latest wave end, inside the same back-to-back
    enqueue. Returns per-shape mean kernel durations, their sum per step, the
    mean gap between one launch's end and the next one's start, and the
    region's HIP-event time (the clock's frequency is checked against it)."""
    n = len(names) * steps
    rec = 2048  # words per launch record: 1024 wave starts, then 1024 wave ends
    buf = rocm.DeviceBuffer.from_array(np.zeros(rec * n, np.uint64))
    warm, timed = many(names, 0, warmup), many(names, warmup, steps)
    if warm():
        raise RuntimeError("matvec_many failed")
    sync(L)
    if L.llamd_hip_kernel_clock(buf.ptr, n):
        raise RuntimeError("kernel clock")
    try:
        t = Timer(L)
        t.rec(0)
        if timed():
            raise RuntimeError("matvec_many failed")
        t.rec(1)
        sync(L)
        ms_ = t.ms(0, 1)
        t.close()
    finally:
        L.llamd_hip_kernel_clock(None, 0)
    got = buf.download(np.empty(rec * n, np.uint64)).reshape(n, 2, rec // 2)
    buf.close()
    starts = np.where(got[:, 0] > 0, got[:, 0], np.iinfo(np.uint64).max)
    st, en = starts.min(axis=1).astype(np.float64), got[:, 1].max(axis=1).astype(np.float64)
    dur = (en - st) / KERNEL_CLOCK_HZ * 1e6
    gaps = (st[1:] - en[:-1]) / KERNEL_CLOCK_HZ * 1e6
    span = (en[-1] - st[0]) / KERNEL_CLOCK_HZ * 1e3
    per = dur.reshape(steps, len(names))
    return {"us_per_launch": {nm: round(float(per[:, j].mean()), 3) for j, nm in enumerate(names)},
            "p10_p90_us": [round(float(np.percentile(dur, 10)), 3), round(float(np.percentile(dur, 90)), 3)],
            "kernel_us_per_step": round(float(per.sum(axis=1).mean()), 3),
            "gap_us": round(float(gaps.mean()), 3),
            "event_us_per_step": round(ms_ / steps * 1e3, 3),
            "clock_span_over_event": round(float(span / ms_), 4),
            "how": "llamd_hip_kernel_clock: s_memrealtime at every wave's start and end (plain vector "
                   "stores, one word per wave), the same K steps enqueued back to back once more"}


def sync(L):
    if L.llamd_fwd_sync() or L.llamd_fwd_last_error():
        from llamd_rs_amd._lib import last_error
        raise RuntimeError(f"device error: {last_error()}")


EAGER_ONLY = False  # --eager: every region on plain launches (profiler runs)


def time_region(L, fn, steps, warmup, graph=True):
    """W eager warm-up steps, then EXACTLY `steps` steps timed with HIP events
    on the library stream.

    graph=True (loops of short kernels): the timed steps are captured once
    into a HIP graph (capture records, it does not run) and replayed, so the
    figure is the device's, not the Python loop's launch rate; every step
    still runs every kernel on its own (rotating) weights, and one untimed
    replay first warms the graph's upload. graph=False (kernels long enough
    that the host keeps ahead): plain launches on the stream."""
    for i in range(warmup):
        fn(i)
    sync(L)
    if not graph or EAGER_ONLY:
        t = Timer(L)
        t.rec(0)
        for i in range(steps):
            fn(warmup + i)
        t.rec(1)
        sync(L)
        ms = t.ms(0, 1)
        t.close()
        return ms
    if L.llamd_fwd_begin_capture():
        raise RuntimeError("graph capture could not start")
    try:
        for i in range(steps):
            fn(warmup + i)
    finally:
        if L.llamd_fwd_end_capture():
            raise RuntimeError("graph capture failed")
    try:
        if L.llamd_fwd_graph_launch():
            raise RuntimeError("graph launch failed")
        sync(L)
        t = Timer(L)
        t.rec(0)
        if L.llamd_fwd_graph_launch():
            raise RuntimeError("graph launch failed")
        t.rec(1)
        sync(L)
        ms = t.ms(0, 1)
        t.close()
    finally:
        L.llamd_fwd_graph_destroy()
    return ms


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="skip the large extra configs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the in-kernel clock region (counter runs: its records add writes)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--eager", action="store_true",
                    help="plain launches everywhere, no graph replay: for rocprofv3 kernel traces, "
                         "which space graph-replayed kernels tens of microseconds apart")
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="set a kernel tune key (llamd_hip_tune) before measuring, e.g. mv_ks=4")
    args = ap.parse_args()
    global EAGER_ONLY
    EAGER_ONLY = args.eager
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (--gpus {args.gpus} requested): this build has no "
              "multi-GPU path.", file=sys.stderr)
        sys.exit(2)

    from llamd_rs_amd import rocm, synth
    from llamd_rs_amd._lib import lib
    L = lib()
    if not rocm.available():
        raise SystemExit("no ROCm device visible")
    tune = {}
    for kv in args.tune:
        key, val = kv.split("=")
        if L.llamd_hip_tune(key.encode(), int(val)) < 0:
            raise SystemExit(f"unknown tune key or value: {kv}")
        tune[key] = int(val)
    info = rocm.device_info(0)
    log(f"device: {info.name} {info.arch} CUs={info.compute_units}")
    K, W = args.steps, args.warmup
    p = lambda a: a.ctypes.data_as(C.c_void_p)

    # ---- headline: configs[1] -------------------------------------------------
    shapes = [("gate", 768, 2048, 11), ("up", 768, 2048, 12), ("down", 2048, 768, 13)]
    per_shape_bytes = {}
    mats = {}
    t0 = time.time()
    for name, rows, k, seed in shapes:
        mats[name] = synth.q6k_matrix(seed, 0.02, rows, k)
    log(f"synth weights {time.time() - t0:.1f}s")
    ncopies = int(np.ceil(1.05 * GIB / sum(len(m) for m in mats.values())))
    copies = {n: [] for n in mats}
    t0 = time.time()
    for name, rows, k, _ in shapes:
        for _ in range(ncopies):
            copies[name].append(rocm.DeviceWeights.upload(mats[name], rows, k // QK_K))
    log(f"uploaded {ncopies} copies per shape ({ncopies * sum(len(m) for m in mats.values()) / GIB:.2f} GiB) "
        f"in {time.time() - t0:.1f}s")
    xs = {2048: synth.normal(21, 1.0, 2048), 768: synth.normal(22, 1.0, 768)}
    acts = {k: rocm.quantize_q8k_on_device(x) for k, x in xs.items()}
    dq = {k: (rocm.DeviceBuffer.from_array(a.qs), rocm.DeviceBuffer.from_array(a.d)) for k, a in acts.items()}
    outs = {name: rocm.DeviceBuffer(rows * 4) for name, rows, _, _ in shapes}
    for name, rows, k, _ in shapes:
        per_shape_bytes[name] = q6k_bytes(rows, k) + k * 4 + rows * 4   # W + x + y (f32)

    def launch(name, rows, k, i):
        q, d = dq[k]
        L.llamd_fwd_matvec(copies[name][i % ncopies].ptr, q.ptr, d.ptr, outs[name].ptr, k // QK_K, rows)

    def step(i):
        for name, rows, k, _ in shapes:
            launch(name, rows, k, i)

    def many(names, i0, n):
        """steps i0 .. i0 + n - 1 of the given shapes as one llamd_hip_matvec_many call"""
        sel = [sh for sh in shapes if sh[0] in names] * n
        idx = [i0 + j // len(names) for j in range(len(sel))]
        m = len(sel)
        arr = lambda t, xs: (t * m)(*xs)
        args = (arr(C.c_void_p, [copies[sh[0]][i % ncopies].ptr for sh, i in zip(sel, idx)]),
                arr(C.c_void_p, [dq[sh[2]][0].ptr for sh in sel]),
                arr(C.c_void_p, [dq[sh[2]][1].ptr for sh in sel]),
                arr(C.c_void_p, [outs[sh[0]].ptr for sh in sel]),
                arr(C.c_int, [sh[2] // QK_K for sh in sel]),
                arr(C.c_int, [sh[1] for sh in sel]), m)
        return lambda: L.llamd_hip_matvec_many(*args)

    def time_many(names, steps, warmup):
        """W warm-up steps, then EXACTLY `steps` steps of plain launches, each
        region enqueued by one call (HIP events on the library stream)."""
        warm, timed = many(names, 0, warmup), many(names, warmup, steps)
        if warm():
            raise RuntimeError("matvec_many failed")
        sync(L)
        t = Timer(L)
        t.rec(0)
        if timed():
            raise RuntimeError("matvec_many failed")
        t.rec(1)
        sync(L)
        ms_ = t.ms(0, 1)
        t.close()
        return ms_

    # Plain launches, enqueued from C (llamd_hip_matvec_many) so the device,
    # not Python, sets the pace: the kernels run back to back, and the timed
    # interval per launch is the per-dispatch duration rocprofv3 reports
    # (profiles/q6k_mv_b1.configs1.kernel_trace.txt); a profiler run of the
    # same command reproduces the figure. The graph-replay figure (launch
    # overhead hidden further) follows in extra.
    ms = time_many([sh[0] for sh in shapes], K, W)
    in_situ = None if args.no_clock else clocked_region(L, rocm, many, [sh[0] for sh in shapes], K, W)
    bytes_step = sum(per_shape_bytes.values())
    value = bytes_step * K / (ms * 1e-3) / 1e9
    log(f"configs[1] step: {ms / K * 1e3:.2f} us, {value:.1f} GB/s")
    shape_res = {}
    for name, rows, k, _ in shapes:
        msn = time_many([name], K, W)
        shape_res[name] = {
            "rows": rows, "k": k, "bytes": per_shape_bytes[name],
            "us_back_to_back": msn / K * 1e3,
            "gbs_back_to_back": per_shape_bytes[name] * K / (msn * 1e-3) / 1e9,
        }
        log(f"  {name}: {shape_res[name]}")
    # what a launch costs here with no work, and with only the reads of one
    # configs[1] matrix (same rotating copies, same back-to-back enqueue)
    def time_reads(nbytes, grid, steps, warmup):
        arr = lambda i0, n: (C.c_void_p * n)(*[copies["gate"][i % ncopies].ptr for i in range(i0, i0 + n)])
        srcs, srcs_t = arr(0, warmup), arr(warmup, steps)
        if L.llamd_hip_read_many(srcs, nbytes, grid, warmup):
            raise RuntimeError("read_many")
        sync(L)
        t = Timer(L)
        t.rec(0)
        if L.llamd_hip_read_many(srcs_t, nbytes, grid, steps):
            raise RuntimeError("read_many")
        t.rec(1)
        sync(L)
        ms_ = t.ms(0, 1)
        t.close()
        return ms_ / steps * 1e3
    wbytes = q6k_bytes(768, 2048) // 16 * 16
    launch_floor = {
        "empty_kernel_us": round(time_reads(0, 48, K, W), 3),
        "read_only_us": {f"grid{g}": round(time_reads(wbytes, g, K, W), 3) for g in (48, 128, 512)},
        "read_bytes": wbytes,
        "how": "llamd_hip_read_many: back-to-back launches of an empty kernel, and of a kernel that "
               "only reads one 768x2048 Q6_K matrix (256-thread workgroups), from the headline's "
               "rotating weight copies",
    }
    log(f"  launch floor: {launch_floor}")

    # The graph-replay figure comes last: the plain-launch regions timed
    # right after a graph's replay ran slower (5.5 instead of 3.3 us per
    # launch for the first one).
    graph_res = None
    if not EAGER_ONLY:
        msg = time_region(L, step, K, W)
        graph_res = {"us_per_step": msg / K * 1e3, "gbs": bytes_step * K / (msg * 1e-3) / 1e9,
                     "pct_of_hbm_peak": round(100 * bytes_step * K / (msg * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
                     "how": "the same K steps captured once into a HIP graph and replayed"}
        log(f"  configs[1] graph replay: {graph_res}")

    # dominant kernel for the roofline: q6k_mv_b1, the step's three launches.
    # Average launch duration = HIP-event time of the timed region (plain
    # launches on the library stream) / launches in it.
    launches = 3 * K
    avg_us = ms * 1e3 / launches
    bytes_launch = bytes_step / 3
    achieved = bytes_launch / (avg_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_Q6K_MV_CONFIGS1,
                "kernel": "q6k_mv_b1", "bytes_per_launch": bytes_launch,
                "avg_launch_us": round(avg_us, 3), "launches": launches,
                "profile": "profiles/q6k_mv_b1.configs1.kernel_trace.txt",
                "traffic_source": "profiles/q6k_mv_b1.configs1.hbm_traffic.txt",
                "in_situ": in_situ}
    for lst in copies.values():
        for c in lst:
            c.close()
    copies = None

    extra = {"configs1_per_shape": shape_res, "configs1_graph_replay": graph_res,
             "configs1_launch_floor": launch_floor,
             "copy_calibration": bench_copy(L, rocm)}

    # ---- extra configs ---------------------------------------------------------
    if not args.quick:
        extra.update(bench_extra(L, rocm, synth, K, W, p, 0.0 if args.no_cpu else 6.0))

    # ---- CPU baseline --------------------------------------------------------------
    cpu = None
    if not args.no_cpu:
        cpu = bench_cpu(mats, shapes, xs, args.cpu_seconds)

    line = {
        "metric": "Q6_K matvec HBM GB/s (% of peak); MoE-layer decode tok/s vs llamd-cpu",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms / K, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q6_K; N(0,1) activations)",
        "config": {"workload": "configs[1]: Q6_K expert-FFN matvecs at batch 1, gate+up [768x2048] "
                               "and down [2048x768], one launch each per step, >=1 GiB of weight "
                               "copies in rotation",
                   "pct_of_hbm_peak": round(100 * value / PEAK_HBM_GBS, 2),
                   **({"tune": tune} if tune else {})},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


def moe_margin(layers):
    """Routing diagnostics over the timed calls: how many calls started
    gate/up on a certified top-k set, whether any wait gave up, and for the
    last call of each layer the certification margin min(T - E | chosen) -
    max(T + E | others) and the gap between the 8th and 9th logit estimate."""
    calls = certified = gave_up = 0
    margins, gaps = [], []
    for layer in layers:
        c, est = layer.counters()
        calls += int(c[0])
        certified += int(c[2])
        gave_up = max(gave_up, int(c[3]))
        T, E = est[0], est[1]
        order = np.argsort(-T, kind="stable")
        chosen, others = order[:8], order[8:]
        margins.append(float(np.min(T[chosen] - E[chosen]) - np.max(T[others] + E[others])))
        gaps.append(float(T[order[7]] - T[order[8]]))
    return {"calls": calls, "certified": certified, "waits_gave_up": gave_up,
            "last_call_margin": [round(m, 6) for m in margins],
            "last_call_gap_8_9": [round(g, 6) for g in gaps]}


def bench_copy(L, rocm, mib=512, reps=5):
    """A plain device copy of known size: the achievable-bandwidth reference
    and the calibration kernel for the profiler's FETCH_SIZE / WRITE_SIZE."""
    n = mib << 20
    a, b = rocm.DeviceBuffer(n), rocm.DeviceBuffer(n)
    def f(i):
        if L.llamd_hip_copy_calibration(b.ptr, a.ptr, n):
            raise RuntimeError("copy")
    ms = time_region(L, f, reps, 1, graph=False)
    a.close(); b.close()
    res = {"bytes_read": n, "bytes_written": n, "us": ms / reps * 1e3,
           "gbs_read_plus_write": 2 * n / (ms / reps * 1e-3) / 1e9}
    log(f"  copy calibration: {res}")
    return res


def host_threads():
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def cpu_median_ms(fn, seconds, max_iters=10):
    """1 warm-up call, then up to max_iters timed calls within ~seconds;
    the median in ms (the reference's CPU timing protocol)."""
    fn()
    ts = []
    t_end = time.perf_counter() + seconds
    while len(ts) < max_iters and (not ts or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return float(np.median(ts)), len(ts)


def bench_extra(L, rocm, synth, K, W, p, moe_cpu_seconds):
    out = {}
    # Q8_0 matvec, configs[0]
    rows, k = 4096, 2048
    w = synth.q8_0_matrix(7, 0.02, rows, k)
    nc = int(np.ceil(1.05 * GIB / len(w)))
    ws = [rocm.Q8_0Weights(w, rows, k) for _ in range(nc)]
    x = rocm.DeviceBuffer.from_array(synth.normal(8, 1.0, k))
    y = rocm.DeviceBuffer(rows * 4)

    def fq(i):
        L.llamd_hip_fwd_matvec_q8_0(ws[i % nc]._ptr, x.ptr, y.ptr, rows, k)
    ms = time_region(L, fq, K, W)
    by = len(w) + k * 4 + rows * 4
    out["q8_0_matvec"] = {"rows": rows, "k": k, "bytes": by, "us_back_to_back": ms / K * 1e3,
                          "gbs_back_to_back": by * K / (ms * 1e-3) / 1e9}
    if moe_cpu_seconds > 0:
        from oracle import oracle as O
        xh = synth.normal(8, 1.0, k)
        ms_c, n_c = cpu_median_ms(lambda: O.matvec_q8_0(w, rows, k, xh), 4.0)
        out["q8_0_matvec"].update({"cpu_1t_ms": ms_c, "cpu_calls": n_c,
                                   "vs_cpu_1t": ms_c / (out["q8_0_matvec"]["us_back_to_back"] * 1e-3)})
    log(f"  q8_0: {out['q8_0_matvec']}")
    for q in ws:
        q.close()
    x.close(); y.close()

    # LM head b=1 and b=16, configs[4]
    rows, k = 151936, 2048
    t0 = time.time()
    w = synth.q6k_matrix(4242, 0.02, rows, k)
    log(f"LM head synth {time.time() - t0:.1f}s")
    heads = []
    for _ in range(4):
        dw = rocm.DeviceWeights.upload(w, rows, k // QK_K)
        heads.append((dw, rocm.LmHead(dw, max_seq=16)))
    xb = rocm.DeviceBuffer.from_array(synth.normal(31, 1.0, 16 * k))
    logits = rocm.DeviceBuffer(16 * rows * 4)
    ids = rocm.DeviceBuffer(16 * 4)
    for nseq in (1, 16):
        def f(i, nseq=nseq):
            h = heads[i % 4][1]
            if L.llamd_hip_lmhead_forward(h.handle, xb.ptr, nseq, logits.ptr, ids.ptr):
                raise RuntimeError("lmhead")
        steps = max(10, K // 4)
        ms = time_region(L, f, steps, 3, graph=False)
        by = q6k_bytes(rows, k) + nseq * k * 4 + nseq * rows * 4
        out[f"lm_head_b{nseq}"] = {"us_per_call": ms / steps * 1e3, "bytes": by,
                                   "gbs": by / (ms / steps * 1e-3) / 1e9,
                                   "pct_of_hbm_peak": round(100 * by / (ms / steps * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
                                   "call": "Q8_K quantize + Q6_K matvec + argmax"}
        log(f"  lm_head b{nseq}: {out[f'lm_head_b{nseq}']}")

    def fr(i):
        h = heads[i % 4][1]
        if L.llamd_hip_lmhead_forward_ex(h.handle, xb.ptr, 16, logits.ptr, ids.ptr, 1):
            raise RuntimeError("lmhead (REDUCTION)")
    steps = max(10, K // 4)
    ms = time_region(L, fr, steps, 3, graph=False)
    by = q6k_bytes(rows, k) + 16 * k * 4 + 16 * rows * 4
    out["lm_head_b16_reduction"] = {
        "us_per_call": ms / steps * 1e3, "bytes": by, "gbs": by / (ms / steps * 1e-3) / 1e9,
        "pct_of_hbm_peak": round(100 * by / (ms / steps * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
        "call": "Q8_K quantize + REDUCTION-tolerance Q6_K matvec + certified exact argmax "
                "(LLAMD_HIP_REDUCTION)",
        "parity": "logits within tolerance::REDUCTION, ids bit-exact "
                  "(tests/test_gpu_moe.py::test_lm_head_b16_argmax_exact, ::test_lm_head_b16_reduction_near_ties)"}
    log(f"  lm_head b16 (REDUCTION): {out['lm_head_b16_reduction']}")
    # the LM-head matvec kernel alone (activation already quantized)
    a1 = rocm.quantize_q8k_on_device(synth.normal(31, 1.0, k))
    q1, d1 = rocm.DeviceBuffer.from_array(a1.qs), rocm.DeviceBuffer.from_array(a1.d)
    def fm(i):
        L.llamd_fwd_matvec(heads[i % 4][0].ptr, q1.ptr, d1.ptr, logits.ptr, k // QK_K, rows)
    steps = max(10, K // 4)
    ms = time_region(L, fm, steps, 3, graph=False)
    by = q6k_bytes(rows, k) + k + (k // QK_K) * 4 + rows * 4
    out["lm_head_matvec_b1"] = {"us_per_launch": ms / steps * 1e3, "bytes": by,
                                "gbs": by / (ms / steps * 1e-3) / 1e9,
                                "pct_of_hbm_peak": round(100 * by / (ms / steps * 1e-3) / 1e9 / PEAK_HBM_GBS, 2)}
    if moe_cpu_seconds > 0:
        from oracle import oracle as O
        ah = O.quantize_q8_k(synth.normal(31, 1.0, k))
        ms_1, n_1 = cpu_median_ms(lambda: O.matvec_q6k_act(w, rows, k, ah), 2.0, 3)
        nt = min(16, host_threads())
        ms_n, n_n = cpu_median_ms(lambda: O.matvec_q6k_act_mt(w, rows, k, ah, nt), 2.0, 5)
        out["lm_head_matvec_b1"].update({
            "cpu_1t_ms": ms_1, "cpu_nt_ms": ms_n, "cpu_threads": nt,
            "vs_cpu_1t": ms_1 / (out["lm_head_matvec_b1"]["us_per_launch"] * 1e-3),
            "vs_cpu_nt": ms_n / (out["lm_head_matvec_b1"]["us_per_launch"] * 1e-3)})
    log(f"  lm_head matvec b1: {out['lm_head_matvec_b1']}")
    q1.close(); d1.close()
    for dw, h in heads:
        h.close(); dw.close()
    xb.close(); logits.close(); ids.close()
    del w

    # MoE decode layer, configs[2]; 4 layers in rotation (2 GB of experts)
    n_embd, n_ff, n_expert, n_used = 2048, 768, 128, 8
    t0 = time.time()
    router = synth.normal(500, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(501, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(502, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(503, 0.02, n_expert * n_embd, n_ff)
    log(f"MoE synth {time.time() - t0:.1f}s")
    layers = [rocm.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used) for _ in range(4)]
    nx = 64
    X = rocm.DeviceBuffer.from_array(synth.normal(600, 1.0, nx * n_embd))
    R = rocm.DeviceBuffer.from_array(synth.normal(601, 1.0, nx * n_embd))
    O_ = rocm.DeviceBuffer(n_embd * 4)
    def f(i):
        xo = X.ptr + (i % nx) * n_embd * 4
        ro = R.ptr + (i % nx) * n_embd * 4
        if L.llamd_hip_moe_forward(layers[i % 4].handle, xo, ro, O_.ptr, 0):
            raise RuntimeError("moe")
    steps = max(20, K // 2)
    ms = time_region(L, f, steps, 5)
    by = n_expert * n_embd * 4 + 24 * q6k_bytes(n_ff, n_embd) + 3 * n_embd * 4
    out["moe_layer"] = {"us_per_token": ms / steps * 1e3, "tok_s": steps / (ms * 1e-3),
                        "bytes_per_token": by, "gbs": by / (ms / steps * 1e-3) / 1e9,
                        "routing": "bit-exact (sequential router fold every call)",
                        "routing_margin": moe_margin(layers)}
    if moe_cpu_seconds > 0:
        # the reference's CPU layer (the oracle, 1 thread) on a bounded sample
        from oracle import oracle as O
        xh, rh = synth.normal(600, 1.0, n_embd), synth.normal(601, 1.0, n_embd)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < moe_cpu_seconds:
            O.moe_layer(xh, rh, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
            n += 1
        dt = time.perf_counter() - t0
        out["moe_layer"]["cpu_tok_s"] = n / dt
        out["moe_layer"]["cpu_sample"] = f"{n} tokens in {dt:.1f}s, oracle on 1 host thread"
        out["moe_layer"]["vs_cpu"] = out["moe_layer"]["tok_s"] / (n / dt)
    log(f"  moe layer: {out['moe_layer']}")

    # configs[1] shapes without the launch floor: all 128 experts' gate
    # [768 x 2048] (and down [2048 x 768]) matrices in ONE grouped launch,
    # each on the same activation, 3 copies of each expert tensor in rotation
    # (3 x 167 MB, beyond the 256 MB Infinity Cache)
    def q8k_act(k):
        """Q8_K of a seeded N(0,1) activation of length k, on the device."""
        a = rocm.quantize_q8k_on_device(synth.normal(23 + k, 1.0, k))
        return rocm.DeviceBuffer.from_array(a.qs), rocm.DeviceBuffer.from_array(a.d)

    ids_all = rocm.DeviceBuffer.from_array(np.arange(n_expert, dtype=np.int32))
    grouped = {}
    for name, host, rows, k in (("gate", gate, n_ff, n_embd), ("down", down, n_embd, n_ff)):
        cps = [rocm.DeviceWeights.upload_experts(host, n_expert, rows, k // QK_K) for _ in range(3)]
        gq, gd = q8k_act(k)
        gy = rocm.DeviceBuffer(n_expert * rows * 4)
        def fg(i, cps=cps, gq=gq, gd=gd, gy=gy, rows=rows, k=k):
            L.llamd_fwd_matvec_grouped(cps[i % 3].ptr, ids_all.ptr, gq.ptr, gd.ptr, gy.ptr, k // QK_K,
                                       rows, n_expert)
        gsteps = max(20, K // 4)
        msg = time_region(L, fg, gsteps, 6, graph=False)
        by = n_expert * q6k_bytes(rows, k)
        us = msg / gsteps * 1e3
        grouped[name] = {"rows": rows, "k": k, "matrices_per_launch": n_expert, "bytes": by,
                         "us_per_launch": round(us, 2), "gbs": round(by / (us * 1e-6) / 1e9, 1),
                         "pct_of_hbm_peak": round(100 * by / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 2)}
        for c in cps:
            c.close()
        for b in (gq, gd, gy):
            b.close()
    grouped["how"] = ("q6k_mv_b1 over all 128 experts of one expert tensor in one launch "
                      "(llamd_fwd_matvec_grouped, ids 0..127, one activation), 3 tensors in rotation")
    out["configs1_grouped"] = grouped
    ids_all.close()
    log(f"  configs[1] shapes, 128 matrices per launch: {grouped}")

    # batched decode: 16 sequences, each routed by its own logits (past
    # batch_decode_max the experts are grouped across the batch)
    OB = rocm.DeviceBuffer(16 * n_embd * 4)
    def fb(i):
        xo = X.ptr + (i % 4) * 16 * n_embd * 4
        ro = R.ptr + (i % 4) * 16 * n_embd * 4
        if L.llamd_hip_moe_forward_batch(layers[i % 4].handle, xo, ro, OB.ptr, 16):
            raise RuntimeError("moe batch")
    bsteps = max(10, K // 10)
    ms = time_region(L, fb, bsteps, 4, graph=False)  # warm-up sizes every layer's scratch
    out["moe_layer_batch16"] = {"us_per_batch": ms / bsteps * 1e3,
                                "us_per_token": ms / bsteps * 1e3 / 16,
                                "tok_s": 16 * bsteps / (ms * 1e-3),
                                "routing": "bit-exact per sequence"}
    log(f"  moe layer batch 16: {out['moe_layer_batch16']}")

    # prefill grouped GEMM, configs[3]: 512 tokens, Zipf 1.1
    n_tok = 512
    xs = rocm.DeviceBuffer.from_array(synth.normal(700, 1.0, n_tok * n_embd))
    ids_h, w_h = synth.zipf_routing(701, 1.1, n_tok, n_expert, n_used)
    ids_d = rocm.DeviceBuffer.from_array(ids_h.astype(np.int32))
    w_d = rocm.DeviceBuffer.from_array(w_h)
    po = rocm.DeviceBuffer(n_tok * n_embd * 4)

    def fp(i):
        if L.llamd_hip_moe_prefill(layers[i % 4].handle, xs.ptr, ids_d.ptr, w_d.ptr, po.ptr, n_tok):
            raise RuntimeError("prefill")
    steps = max(5, K // 20)
    ms = time_region(L, fp, steps, 4, graph=False)  # warm-up touches all 4 layers
    ops = 2 * n_tok * n_used * (2 * n_ff * n_embd + n_embd * n_ff)
    used = len(set(ids_h.ravel().tolist()))
    wbytes = used * 3 * q6k_bytes(n_ff, n_embd)
    out["prefill_grouped"] = {"tokens": n_tok, "ms_per_pass": ms / steps, "tok_s": n_tok * steps / (ms * 1e-3),
                              "int_tops": ops / (ms / steps * 1e-3) / 1e12,
                              "experts_used": used, "weight_bytes": wbytes,
                              "weight_gbs": wbytes / (ms / steps * 1e-3) / 1e9}

    def fpr(i):
        if L.llamd_hip_moe_prefill_ex(layers[i % 4].handle, xs.ptr, ids_d.ptr, w_d.ptr, po.ptr, n_tok, 1):
            raise RuntimeError("prefill (REDUCTION)")
    ms_r = time_region(L, fpr, steps, 4, graph=False)
    out["prefill_grouped_reduction"] = {
        "tokens": n_tok, "ms_per_pass": ms_r / steps, "tok_s": n_tok * steps / (ms_r * 1e-3),
        "int_tops": ops / (ms_r / steps * 1e-3) / 1e12,
        "weight_gbs": wbytes / (ms_r / steps * 1e-3) / 1e9,
        "parity": "within tolerance::REDUCTION x rms per token (LLAMD_HIP_REDUCTION; "
                  "tests/test_gpu_moe.py::test_prefill_full_config_512_tokens)"}
    log(f"  prefill (REDUCTION): {out['prefill_grouped_reduction']}")
    if moe_cpu_seconds > 0:
        # the reference's CPU path runs moe_ffn token by token: time a sample
        # of 16 tokens (1 thread) and scale to the 512-token pass
        from oracle import oracle as O
        xh = synth.normal(700, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
        ns = 16
        t0 = time.perf_counter()
        O.moe_ffn_tokens(xh[:ns], n_embd, n_ff, n_expert, gate, up, down, ids_h[:ns], w_h[:ns])
        dt = time.perf_counter() - t0
        # and one full 512-token pass on the host's threads: 16-token slices
        # of the same call in a thread pool (the C oracle releases the GIL)
        from concurrent.futures import ThreadPoolExecutor
        nt = min(16, host_threads())
        slices = [(s0, min(n_tok, s0 + 16)) for s0 in range(0, n_tok, 16)]
        with ThreadPoolExecutor(max_workers=nt) as ex:
            t0 = time.perf_counter()
            parts = list(ex.map(lambda ab: O.moe_ffn_tokens(
                xh[ab[0]:ab[1]], n_embd, n_ff, n_expert, gate, up, down, ids_h[ab[0]:ab[1]],
                w_h[ab[0]:ab[1]]), slices))
            dt_n = time.perf_counter() - t0
        assert sum(len(q) for q in parts) == n_tok
        out["prefill_grouped"].update({
            "cpu_1t_ms_per_pass_est": dt / ns * n_tok * 1e3,
            "cpu_sample": f"{ns} tokens of moe_ffn in {dt:.2f}s on 1 host thread, scaled to {n_tok}",
            "vs_cpu_1t": (dt / ns * n_tok) / (ms / steps * 1e-3),
            "cpu_nt_ms_per_pass": dt_n * 1e3, "cpu_threads": nt,
            "cpu_nt_sample": f"one full {n_tok}-token pass of moe_ffn, {len(slices)} slices of 16 tokens "
                             f"over {nt} host threads",
            "vs_cpu_nt": dt_n / (ms / steps * 1e-3)})
    log(f"  prefill: {out['prefill_grouped']}")
    for ly in layers:
        ly.close()

    # attention front end (the adjacent decode step): RMSNorm -> Q8_K -> Q, K,
    # V (4096 / 512 / 512 rows x 2048) in one launch; 4 weight sets rotate
    blocks = n_embd // QK_K
    qkv = [(4096, 801), (512, 802), (512, 803)]
    mats = [synth.q6k_matrix(sd, 0.02, r, n_embd) for r, sd in qkv]
    nset = 24  # 24 x 10.3 MB of Q/K/V weights in rotation
    sets = [[rocm.DeviceWeights.upload(m, r, blocks) for m, (r, _) in zip(mats, qkv)] for _ in range(nset)]
    xa = rocm.DeviceBuffer.from_array(synth.normal(804, 1.0, n_embd))
    wn = rocm.DeviceBuffer.from_array((1 + 0.1 * synth.normal(805, 1.0, n_embd)).astype(np.float32))
    aq, ad = rocm.DeviceBuffer(n_embd), rocm.DeviceBuffer(blocks * 4)
    oq = [rocm.DeviceBuffer(r * 4) for r, _ in qkv]

    def fa(i):
        st_ = sets[i % nset]
        L.llamd_fwd_rms_norm_quant(xa.ptr, wn.ptr, None, aq.ptr, ad.ptr, None, n_embd, 1e-6)
        L.llamd_fwd_matvec_x3(st_[0].ptr, st_[1].ptr, st_[2].ptr, aq.ptr, ad.ptr, oq[0].ptr, oq[1].ptr,
                              oq[2].ptr, blocks, qkv[0][0], qkv[1][0], qkv[2][0])
    steps = max(20, K // 2)
    ms = time_region(L, fa, steps, 5)
    by = sum(q6k_bytes(r, n_embd) + r * 4 for r, _ in qkv) + n_embd * 8
    out["attn_front_end"] = {"us_per_token": ms / steps * 1e3, "bytes": by,
                             "gbs": by / (ms / steps * 1e-3) / 1e9,
                             "kernels": "rms_norm_quant + matvec_x3 (Q 4096, K 512, V 512 rows)",
                             "parity": "bit-exact (tests/test_gpu_norm.py)"}
    log(f"  attention front end: {out['attn_front_end']}")
    for st_ in sets:
        for d_ in st_:
            d_.close()
    # resident whole-token decode, Qwen3-30B-A3B shapes (48 layers, 128
    # experts, 151936 vocab): a synthetic GGUF whose layers share one copy of
    # their data in the file; each layer is a separate ~0.49 GB upload
    import tempfile
    from llamd_rs_amd import synth_model
    from llamd_rs_amd.gguf import Gguf
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    # --eager: the step's launches stay plain (no HIP graph capture), like
    # every other region of a profiler run; read when the model is created
    prev_graph = L.llamd_hip_tune(b"model_graph", 0 if EAGER_ONLY else 1)
    try:
        t0 = time.time()
        synth_model.write_model(path)
        with Gguf(path) as g:
            dm = rocm.DeviceModel(g, max_kv=1024)
        t_load = time.time() - t0
    except BaseException:
        os.unlink(path)
        raise
    finally:
        L.llamd_hip_tune(b"model_graph", prev_graph)
    tok = 1
    for pos in range(3):
        _, tok = dm.forward(tok, pos)
    n = 64
    t0 = time.perf_counter()
    for pos in range(3, 3 + n):
        _, tok = dm.forward(tok, pos)
    dt = time.perf_counter() - t0
    out["decode_token"] = {"model": "Qwen3-30B-A3B-shaped (48 layers, 128 experts top-8, vocab 151936), "
                                    "synthetic Q6_K weights",
                           "us_per_token": dt / n * 1e6, "tok_s": n / dt, "tokens": n,
                           "positions": f"3..{2 + n}", "load_s": round(t_load, 1),
                           "per_call": "host call incl. logits download and one sync",
                           "graph": not EAGER_ONLY,
                           "parity": "bit-identical to the CPU forward at these widths on 4 layers x 3 tokens "
                                     "(tests/test_gpu_model.py::test_decode_full_qwen3_30b_a3b_widths)"}
    log(f"  decode token: {out['decode_token']}")
    # the same model near the end of its 1024-position cache: every position
    # filled in order (untimed), then 32 timed tokens; from position 256 on
    # the step takes the split attention (logits over the whole GPU)
    for pos in range(3 + n, 992):
        _, tok = dm.forward(tok, pos)
    t0 = time.perf_counter()
    for pos in range(992, 1024):
        _, tok = dm.forward(tok, pos)
    dt = time.perf_counter() - t0
    out["decode_token_ctx1k"] = {"us_per_token": dt / 32 * 1e6, "tok_s": 32 / dt, "tokens": 32,
                                 "positions": "992..1023", "graph": not EAGER_ONLY,
                                 "parity": "bit-identical to the CPU forward through the split attention "
                                           "(tests/test_gpu_model.py::test_decode_loop_long_context)"}
    log(f"  decode token at 1k context: {out['decode_token_ctx1k']}")
    dm.close()
    try:
        out.update(bench_ffi_decode(path))
    finally:
        os.unlink(path)
    return out


def bench_ffi_decode(path):
    """The same 48-layer model through the reference's own DeviceModel call
    sequence on the exported FFI (llamd_rs_amd/ffi_replay.py: planar weights,
    llamd_fwd_* per token with its graph capture, llamd_b_* / llamd_u_* for a
    16-sequence batch): what the unchanged Rust runtime gets from this
    library."""
    from llamd_rs_amd.ffi_replay import FfiModel
    from llamd_rs_amd.gguf import Gguf
    res = {}
    t0 = time.time()
    with Gguf(path) as g:
        fm = FfiModel(g, max_kv=1024, max_seq=16, use_graph=not EAGER_ONLY)
    t_load = time.time() - t0
    try:
        tok = 1
        for pos in range(3):
            tok = fm.forward(tok, pos)
        n = 64
        t0 = time.perf_counter()
        for pos in range(3, 3 + n):
            tok = fm.forward(tok, pos)
        dt = time.perf_counter() - t0
        res["ffi_decode"] = {
            "us_per_token": dt / n * 1e6, "tok_s": n / dt, "tokens": n, "load_s": round(t_load, 1),
            "graph": not EAGER_ONLY,
            "calls": "DeviceModel::forward's sequence (device.rs:486-722) on llamd_fwd_* / planar weights",
            "parity": "bit-identical to the CPU forward at these widths on 4 layers x 3 tokens "
                      "(tests/test_gpu_ffi_model.py::test_ffi_forward_full_qwen3_30b_a3b_widths)"}
        log(f"  ffi decode: {res['ffi_decode']}")
        nseq, steps = 16, 8
        toks = list(range(1, nseq + 1))
        toks = fm.forward_batch(toks, [0] * nseq)
        t0 = time.perf_counter()
        for st_ in range(1, 1 + steps):
            toks = fm.forward_batch(toks, [st_] * nseq)
        dt = time.perf_counter() - t0
        res["ffi_decode_batch16"] = {
            "us_per_batch": dt / steps * 1e6, "us_per_token": dt / steps / nseq * 1e6,
            "tok_s": nseq * steps / dt, "steps": steps,
            "calls": "DeviceModel::forward_batch's sequence (device.rs:741-962) on llamd_b_* / llamd_u_*",
            "parity": "bit-identical per sequence to the CPU forward "
                      "(tests/test_gpu_ffi_model.py::test_ffi_forward_batch_matches_the_cpu)"}
        log(f"  ffi decode batch 16: {res['ffi_decode_batch16']}")
    finally:
        fm.close()
    return res


def bench_cpu(mats, shapes, xs, seconds):
    """The oracle (1 thread, scalar -- the reference's CPU design is
    single-threaded) on a bounded sample of the same workload: repeated
    configs[1] steps for ~`seconds`. As on the GPU, the activations are
    quantized to Q8_K before the timed steps (the step is the three matvecs).
    all_cores: the same rows split over the host threads by one OpenMP team
    inside the oracle library (same bits)."""
    from oracle import oracle as O
    acts = {k: O.quantize_q8_k(x) for k, x in xs.items()}
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for name, rows, k, _ in shapes:
            O.matvec_q6k_act(mats[name], rows, k, acts[k])
        n += 1
    dt = time.perf_counter() - t0
    bytes_step = sum(q6k_bytes(r, k) + k * 4 + r * 4 for _, r, k, _ in shapes)
    try:
        aff = len(os.sched_getaffinity(0))
    except Exception:
        aff = os.cpu_count()
    nt = min(16, host_threads())
    used = nt
    for name, rows, k, _ in shapes:  # the team starts outside the timing
        _, used = O.matvec_q6k_act_mt(mats[name], rows, k, acts[k], nt)
    t0 = time.perf_counter()
    n_n = 0
    while time.perf_counter() - t0 < seconds / 4:
        for name, rows, k, _ in shapes:
            O.matvec_q6k_act_mt(mats[name], rows, k, acts[k], nt)
        n_n += 1
    dt_n = time.perf_counter() - t0
    return {"value": round(bytes_step * n / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "all_cores": {"value": round(bytes_step * n_n / dt_n / 1e9, 4), "threads": used,
                          "ms_per_step": round(dt_n / n_n * 1e3, 3),
                          "sample": f"{n_n} steps in {dt_n:.1f}s"},
            "sample": f"{n} configs[1] steps (gate+up+down Q6_K matvec on Q8_K activations quantized "
                      f"beforehand, as on the GPU) in {dt:.1f}s on 1 of {aff} host threads",
            "ms_per_step": round(dt / n * 1e3, 3)}


if __name__ == "__main__":
    main()
