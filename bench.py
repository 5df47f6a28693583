#!/usr/bin/env python3
"""bench.py - throughput of the gfx950 quantized expert path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload: Q4 rowwise GEMV at batch 1 at
both expert shapes, down [2048 x 768] and gate [768 x 2048].  Weights are
W ~ N(0, 0.02^2) quantized per row on the device with the exporter's rule,
x ~ N(0, 1).  A step is one pass over a rotating pool of distinct matrices
(>= 1 GiB per shape, far beyond the 256 MB Infinity Cache) in one batched
launch per shape, inputs resident in HBM.  `value` is algorithmic GB/s:
weights + scales + x + y of every GEMV, each counted once.

The same line carries configs[0] (`q8_gemv`: Q8 rowwise GEMV [768 x 2048],
its own roofline and CPU baseline), configs[2] (`moe_decode_q8`), configs[3]
(`moe_prefill_q4`) and configs[4] (`model_decode_q4`), each with the
reference's CPU path timed on this host beside it.  --workload q8_gemv makes
the Q8 GEMV the headline instead.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "moe.cc_amd"))

import moehip as M  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "Q8/Q4 expert GEMV GB/s (% HBM peak); decode tok/s at 30B-A3B shape"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(dtype: int, N: int, K: int) -> int:
    """Algorithmic bytes of one batch-1 GEMV: weights + scales + x + y."""
    wbytes = N * K if dtype == 2 else N * (K // 2)
    return wbytes + 4 * N + 4 * K + 4 * N


def pool_count(dtype: int, N: int, K: int, pool_gib: float = 1.0) -> int:
    """Matrices in a GEMV pool of `pool_gib` GiB of packed weights."""
    rb = K if dtype == 2 else K // 2
    return int(np.ceil(pool_gib * (1 << 30) / (N * rb)))


class Pool:
    """`count` distinct quantized matrices [N x K] in one device allocation,
    plus a shared x and one output row per matrix, and the job table."""

    def __init__(self, dtype: int, N: int, K: int, count: int, seed: int):
        self.dtype, self.N, self.K, self.count = dtype, N, K, count
        rb = K if dtype == 2 else K // 2
        self.q = M.DeviceBuffer(count * N * rb)
        self.s = M.DeviceBuffer(count * N * 4)
        self.x = M.DeviceBuffer(K * 4)
        self.y = M.DeviceBuffer(count * N * 4)
        chunk = max(1, min(count, (512 << 20) // (N * K * 4)))
        tmp = M.DeviceBuffer(chunk * N * K * 4)
        L = M.lib()
        for c0 in range(0, count, chunk):
            n = min(chunk, count - c0)
            M.check(L.moe_fill_normal_dev(tmp.ptr, n * N * K, seed + c0, 0.0, 0.02), "fill")
            M.check(L.moe_quantize_rows_dev(dtype, tmp.ptr, n * N, K, self.q.ptr + c0 * N * rb,
                                            self.s.ptr + c0 * N * 4), "quantize")
        tmp.free()
        M.check(L.moe_fill_normal_dev(self.x.ptr, K, seed + 999983, 0.0, 1.0), "fill x")
        jobs = (M.QJob * count)()
        for i in range(count):
            jobs[i] = M.QJob(self.q.ptr + i * N * rb, self.s.ptr + i * N * 4, self.x.ptr,
                             self.y.ptr + i * N * 4)
        self.jobs = M.DeviceBuffer(ctypes.sizeof(jobs))
        M.check(L.moe_memcpy_h2d(self.jobs.ptr, ctypes.addressof(jobs), ctypes.sizeof(jobs)))
        M.synchronize()
        self.tabs = M.DeviceBuffer(L.moe_act_table_bytes(K))
        self.bytes_per_launch = count * gemv_bytes(dtype, N, K)
        self.weight_bytes = count * N * rb

    def pack(self):
        """Quantizes x into its packed tables (kernels.c:56-60 / :107-110)."""
        M.check(M.lib().moe_act_pack_dev(self.dtype, self.x.ptr, 1, self.K, self.tabs.ptr), "pack")

    def launch(self):
        """The `count` GEMVs from the packed tables, one launch."""
        M.check(M.lib().moe_matmul_q_prepacked_dev(self.dtype, self.jobs.ptr, self.count, 1,
                                                   self.N, self.K, self.tabs.ptr), "gemv")


def kernel_name(dtype, N, K):
    return M.gemv_variant(dtype, 1, N, K)


def cpu_baseline(shapes, budget_s: float):
    """Reference kernels.c (oracle/_ref, built from the reference sources) or
    the oracle restatement, single thread on this host, batch-1 GEMVs over a
    small rotating pool of each shape."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    kind = "reference" if os.path.exists(O.REF_KERNELS_LIB) else "port"
    fn = O.ref_kernels().matmul_adaptive if kind == "reference" else O.orc().orc_matmul_adaptive
    pool = 6
    tot_bytes, tot_s, calls = 0, 0.0, 0
    per = budget_s / len(shapes)
    for dtype, N, K in shapes:
        mats = []
        for i in range(pool):
            W = O.normal(N * K, 4242 + i, 0.0, 0.02).reshape(N, K)
            q, s = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
            mats.append((q, s, O.QW(q.ctypes.data, s.ctypes.data, N, K, dtype)))
        x = O.normal(K, 77, 0.0, 1.0)
        y = np.empty(N, np.float32)
        n = 0
        t0 = time.perf_counter()
        while True:
            q, s, qw = mats[n % pool]
            fn(x.ctypes.data, None, ctypes.addressof(qw), y.ctypes.data, 1, N, K)
            n += 1
            el = time.perf_counter() - t0
            if el >= per:
                break
        tot_bytes += n * gemv_bytes(dtype, N, K)
        tot_s += el
        calls += n
    return {"value": round(tot_bytes / tot_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{calls} batch-1 GEMVs over {pool} matrices per shape "
                      f"{[f'{N}x{K}' for _, N, K in shapes]}, {tot_s:.1f} s, 1 thread of "
                      f"{host_cores()} host cores"}


COPY_CALIB_BYTES = 256 << 20


def copy_calibration():
    """One device-to-device copy of known size before the timed region: the
    HBM-traffic counters (FETCH_SIZE / WRITE_SIZE) of the rocprofv3 --pmc runs
    are scaled by what they read for this copy."""
    a = M.DeviceBuffer(COPY_CALIB_BYTES)
    b = M.DeviceBuffer(COPY_CALIB_BYTES)
    M.check(M.lib().moe_memset(a.ptr, 1, COPY_CALIB_BYTES))
    M.check(M.lib().moe_memcpy_d2d(b.ptr, a.ptr, COPY_CALIB_BYTES))
    a.free()
    b.free()


def measured_traffic(kernel_name):
    """(HBM bytes per launch of `kernel_name`, the commit they were measured
    at) from the committed PMC summary (profiles/traffic.json, two rocprofv3
    --pmc runs of this script, FETCH_SIZE and WRITE_SIZE, scaled by what
    they read for the 256 MiB copy), or (None, None).  rocprofv3 cannot run
    inside this process, so the figure is not this run's own counter."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return (t["kernels"].get(kernel_name, {}).get("traffic_bytes_per_launch"),
                t.get("measured_at"))
    except (OSError, ValueError, KeyError):
        return None, None


def host_cores() -> int:
    """Host threads this process may use (the box's share, not the machine's)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def read_stream(pools, steps):
    """The plain read-only stream over each pool's weights
    (moe_stream_read_dev: the GEMV's 16-byte nontemporal loads, nothing
    else), for a pass that no cache holds.  Returns GB/s per pool.  On
    MI355X it is not an upper bound for the GEMV: the HBM read rate depends
    on the data and the access order (a constant buffer streams at ~7.1
    TB/s, these quantized weights at ~6.0, while the GEMV reads them at
    ~6.5)."""
    L = M.lib()
    sink = M.DeviceBuffer(16)
    rates = []
    for p in pools:
        M.check(L.moe_memset(sink.ptr, 0, 16))
        for _ in range(2):
            M.check(L.moe_stream_read_dev(p.q.ptr, p.weight_bytes, sink.ptr), "stream read")
        a, b = M.Event(), M.Event()
        a.record()
        for _ in range(steps):
            M.check(L.moe_stream_read_dev(p.q.ptr, p.weight_bytes, sink.ptr), "stream read")
        b.record()
        M.synchronize()
        ms = a.elapsed_ms(b) / steps
        rates.append(round(p.weight_bytes / (ms * 1e-3) / 1e9, 1))
    sink.free()
    return rates


READ_CAPS = (0, 1, 2, 3, 4, 5, 6, 8)


def read_rows(pools, steps):
    """The GEMV launch's own reads without its arithmetic (moe_rows_read_dev:
    same blocks, rows per block, lanes per row and loads in flight; weights
    and scales), over each pool, with the GEMV's blocks-per-CU cap (0) and
    with 1..8 blocks a CU.  Returns per pool {cap: (GB/s over the weight and
    scale bytes, us per launch)}; the fastest is the read ceiling of the
    GEMV's access order."""
    L = M.lib()
    sink = M.DeviceBuffer(16)
    out = []
    for p in pools:
        nbytes = p.weight_bytes + 4 * p.N * p.count
        per_cap = {}
        for cap in READ_CAPS:
            M.check(L.moe_memset(sink.ptr, 0, 16))
            for _ in range(2):
                M.check(L.moe_rows_read_dev(p.dtype, p.jobs.ptr, p.count, p.N, p.K, cap, sink.ptr),
                        "rows read")
            a, b = M.Event(), M.Event()
            a.record()
            for _ in range(steps):
                M.check(L.moe_rows_read_dev(p.dtype, p.jobs.ptr, p.count, p.N, p.K, cap, sink.ptr),
                        "rows read")
            b.record()
            M.synchronize()
            ms = a.elapsed_ms(b) / steps
            per_cap[cap] = (round(nbytes / (ms * 1e-3) / 1e9, 1), round(ms * 1e3, 2))
        out.append(per_cap)
    sink.free()
    return out


def run_gemv(args, dtype, shapes, workload):
    M.init(0)
    copy_calibration()
    pools = []
    for i, (N, K) in enumerate(shapes):
        count = pool_count(dtype, N, K, args.pool_gib)
        log(f"[bench] building pool {N}x{K} dtype {dtype}: {count} matrices")
        pools.append(Pool(dtype, N, K, count, seed=1000 * (i + 1)))
    # a step: for each shape, pack then the GEMV launch.  The K timed steps
    # carry events only at their ends (an event pair inside the loop costs
    # ~5 us of device time); a second pass of K steps brackets each pack
    # (event a -> b) and each GEMV launch (b -> c) for the per-kernel
    # figures -- the roofline is taken on the GEMV launch alone.
    evs = {i: [(M.Event(), M.Event(), M.Event()) for _ in range(args.steps)]
           for i in range(len(pools))}
    for _ in range(args.warmup):
        for p in pools:
            p.pack()
            p.launch()
    M.synchronize()
    t_start, t_end = M.Event(), M.Event()
    wall0 = time.perf_counter()
    t_start.record()
    for s in range(args.steps):
        for p in pools:
            p.pack()
            p.launch()
    t_end.record()
    M.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_ms(t_end)
    for s in range(args.steps):
        for i, p in enumerate(pools):
            a, b, c = evs[i][s]
            a.record()
            p.pack()
            b.record()
            p.launch()
            c.record()
    M.synchronize()
    per_kernel = []
    for i, p in enumerate(pools):
        ms = [b.elapsed_ms(c) for a, b, c in evs[i]]
        pack_ms = [a.elapsed_ms(b) for a, b, c in evs[i]]
        avg = float(np.mean(ms))
        per_kernel.append({"kernel": f"qgemv_{kernel_name(dtype, p.N, p.K)}",
                           "shape": f"{p.N}x{p.K}", "matrices_per_launch": p.count,
                           "avg_launch_us": round(avg * 1e3, 2),
                           "avg_pack_us": round(float(np.mean(pack_ms)) * 1e3, 2),
                           "algorithmic_bytes_per_launch": p.bytes_per_launch,
                           "achieved_GBs": round(p.bytes_per_launch / (avg * 1e-3) / 1e9, 1)})
    for k, c in zip(per_kernel, read_stream(pools, args.steps)):
        k["read_stream_GBs"] = c
    for k, per_cap in zip(per_kernel, read_rows(pools, args.steps)):
        best = min(per_cap, key=lambda c: per_cap[c][1])
        k["read_rows_GBs_by_cap"] = {str(c): v[0] for c, v in per_cap.items()}
        k["read_rows_GBs"], k["read_rows_us"], k["read_rows_best_cap"] = (per_cap[best][0],
                                                                          per_cap[best][1], best)
    bytes_step = sum(p.bytes_per_launch for p in pools)
    ms_step = total_ms / args.steps
    value = bytes_step / (ms_step * 1e-3) / 1e9
    dom = max(per_kernel, key=lambda k: k["avg_launch_us"])
    traffic, traffic_at = measured_traffic(dom["kernel"])
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": workload, "batch": 1,
                   "shapes": [f"{p.N}x{p.K}" for p in pools],
                   "pool_bytes_per_shape": [p.weight_bytes for p in pools],
                   "weights": "N(0,0.02^2) rowwise-quantized on device (export.py rule)",
                   "x": "N(0,1) fp32"},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": dom["achieved_GBs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom["achieved_GBs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_measured_at_commit": traffic_at,
                     "kernel": dom["kernel"],
                     "algorithmic_bytes": dom["algorithmic_bytes_per_launch"],
                     # the plain read-only stream over the same pool (moe_stream_read_dev)
                     "read_stream_same_pool": dom["read_stream_GBs"],
                     # the GEMV launch's own reads alone (moe_rows_read_dev, the
                     # fastest blocks-per-CU cap): the ceiling of its access
                     # order, and the GEMV's share of it (read-only launch time
                     # / GEMV launch time, the same weight and scale bytes read)
                     "read_ceiling_same_order": dom["read_rows_GBs"],
                     "read_ceiling_blocks_per_cu": dom["read_rows_best_cap"],
                     "frac_of_read_ceiling": round(dom["read_rows_us"] / dom["avg_launch_us"], 4)},
        "kernels": per_kernel,
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline([(dtype, N, K) for (N, K) in shapes], args.cpu_seconds)
    return out


def expert_bytes(dtype: int, D: int, dff: int) -> int:
    """One expert's gate + up + down weights and scales."""
    rb_g = D if dtype == 2 else D // 2
    rb_d = dff if dtype == 2 else dff // 2
    return 2 * dff * rb_g + D * rb_d + 4 * (2 * dff + D)


class LayerPool:
    """`n` device-resident MoE layers (Qwen3-30B-A3B shapes) with weights
    generated and quantized on the device."""

    def __init__(self, dtype, n, E=128, D=2048, dff=768, seed=77):
        self.dtype, self.E, self.D, self.dff = dtype, E, D, dff
        L = M.lib()
        rb_g = D if dtype == 2 else D // 2
        rb_d = dff if dtype == 2 else dff // 2
        tmp = M.DeviceBuffer(E * max(dff * D, D * dff) * 4)
        self.layers = []
        for i in range(n):
            bufs = {"rw": M.DeviceBuffer(E * D * 4), "gq": M.DeviceBuffer(E * dff * rb_g),
                    "uq": M.DeviceBuffer(E * dff * rb_g), "dq": M.DeviceBuffer(E * D * rb_d),
                    "gs": M.DeviceBuffer(E * dff * 4), "us": M.DeviceBuffer(E * dff * 4),
                    "ds": M.DeviceBuffer(E * D * 4)}
            sd = seed + 1000 * i
            M.check(L.moe_fill_normal_dev(bufs["rw"].ptr, E * D, sd, 0.0, 0.02))
            for name, rows, K in (("g", dff, D), ("u", dff, D), ("d", D, dff)):
                sd += 1
                M.check(L.moe_fill_normal_dev(tmp.ptr, E * rows * K, sd, 0.0, 0.02))
                M.check(L.moe_quantize_rows_dev(dtype, tmp.ptr, E * rows, K, bufs[name + "q"].ptr,
                                                bufs[name + "s"].ptr))
            h = ctypes.c_void_p()
            M.check(L.moe_layer_create_raw(dtype, D, dff, E, 8, bufs["rw"].ptr, None, None,
                                           bufs["gq"].ptr, bufs["gs"].ptr, bufs["uq"].ptr,
                                           bufs["us"].ptr, bufs["dq"].ptr, bufs["ds"].ptr, 1,
                                           ctypes.byref(h)), "layer_create")
            for b in bufs.values():
                b.free()
            self.layers.append(M.MoeLayer(h.value, dtype, D, dff, E, 8))
        tmp.free()
        M.synchronize()


def layer_cpu_baseline(dtype, T, runs, E=128, D=2048, dff=768, top_k=8, seed=9):
    """One MoE layer at the config shape on one host thread: the reference's
    own layer_forward_f32 MoE block (oracle/_ref, compiled from the
    reference sources: router, top-8, softmax, the per-(token, rank) GEMV
    loop, weighted sum, residual; its attention part is given zero weights
    and a 2-wide head and costs nothing) when that library is present, else
    the oracle's restatement of the same loops.  One warm-up run, then the
    median of `runs`.  The weights are random bytes with constant scales:
    the CPU loops' time does not depend on their values."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    rng = np.random.default_rng(seed)
    rb_g = D if dtype == 2 else D // 2
    rb_d = dff if dtype == 2 else dff // 2
    if dtype == 2:
        q = lambda *sh: rng.integers(-127, 128, sh, dtype=np.int8)  # noqa: E731
    else:
        q = lambda *sh: rng.integers(0, 256, sh, dtype=np.uint8)  # noqa: E731
    ex = O.ExpertSet(dtype, q(E, dff, rb_g), np.full((E, dff), 1e-3, np.float32),
                     q(E, dff, rb_g), np.full((E, dff), 1e-3, np.float32),
                     q(E, D, rb_d), np.full((E, D), 1e-3, np.float32), D, dff)
    rw = (rng.standard_normal((E, D), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal((T, D), dtype=np.float32)
    ones = np.ones(D, np.float32)
    kind = "reference" if O.ref_available() else "port"
    out = np.empty((T, D), np.float32)

    def once():
        if kind == "reference":
            xx = x.copy()
            t0 = time.perf_counter()
            O.ref_trace().ref_moe_layer(xx.ctypes.data, T, D, E, top_k, dff, ones.ctypes.data,
                                        rw.ctypes.data, None, ctypes.addressof(ex.Wg),
                                        ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd))
            return time.perf_counter() - t0
        t0 = time.perf_counter()
        O.orc_single().orc_moe_block(x.ctypes.data, x.ctypes.data, T, D, E, top_k, dff,
                                     rw.ctypes.data, None, ctypes.addressof(ex.Wg),
                                     ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd),
                                     out.ctypes.data, None, None, None)
        return time.perf_counter() - t0

    once()
    ts = [once() for _ in range(runs)]
    med = float(np.median(ts))
    return {"us_per_layer_median": round(med * 1e6, 1), "tokens_per_s_one_layer": round(T / med, 2),
            "unit": "us per layer", "cores": 1, "kind": kind,
            "sample": f"1 warm-up + median of {runs} single-thread runs of one {E}-expert "
                      f"{'Q8' if dtype == 2 else 'Q4'} layer at T={T} "
                      f"({'compiled reference layer_forward_f32 MoE block' if kind == 'reference' else 'oracle restatement'}), "
                      f"1 thread of {host_cores()} host cores"}


def run_decode(dtype, Ts, n_layers, steps, warmup):
    """One MoE layer forward per step (configs[2]: Q8 experts, T tokens,
    x ~ N(0,1)); layers and inputs rotate so expert weights stream from HBM."""
    M.init(0)
    pool = LayerPool(dtype, n_layers)
    D = pool.D
    res = []
    for T in Ts:
        n_in = 8
        xs = M.DeviceBuffer(n_in * T * D * 4)
        M.check(M.lib().moe_fill_normal_dev(xs.ptr, n_in * T * D, 4242 + T, 0.0, 1.0))
        out = M.DeviceBuffer(T * D * 4)
        idx = M.DeviceBuffer(steps * T * 8 * 4)
        for i in range(max(warmup, n_layers)):
            lay = pool.layers[i % n_layers]
            lay.forward_dev(xs.ptr + (i % n_in) * T * D * 4, xs.ptr + (i % n_in) * T * D * 4, T,
                            out.ptr)
        M.synchronize()
        # back to back (events only at the ends), then each layer between
        # its own pair of events (a pair costs device time of its own)
        s0, s1 = M.Event(), M.Event()
        s0.record()
        for i in range(steps):
            x = xs.ptr + (i % n_in) * T * D * 4
            pool.layers[i % n_layers].forward_dev(x, x, T, out.ptr, idx.ptr + i * T * 8 * 4)
        s1.record()
        M.synchronize()
        stream_ms = s0.elapsed_ms(s1) / steps
        ev = [(M.Event(), M.Event()) for _ in range(steps)]
        t0, t1 = M.Event(), M.Event()
        t0.record()
        for i in range(steps):
            lay = pool.layers[i % n_layers]
            x = xs.ptr + (i % n_in) * T * D * 4
            ev[i][0].record()
            lay.forward_dev(x, x, T, out.ptr, idx.ptr + i * T * 8 * 4)
            ev[i][1].record()
        t1.record()
        M.synchronize()
        per = [a.elapsed_ms(b) for a, b in ev]
        total_ms = t0.elapsed_ms(t1)
        ids = idx.download((steps, T * 8), np.int32)
        U = float(np.mean([len(set(r.tolist()) - {-1}) for r in ids]))
        algo = 1048576 + U * expert_bytes(dtype, D, pool.dff) + 2 * T * D * 4
        med = float(np.median(per))
        res.append({"T": T, "layers_in_pool": n_layers, "steps": steps,
                    "us_per_layer_median": round(med * 1e3, 2),
                    "us_per_layer_mean": round(total_ms / steps * 1e3, 2),
                    "us_per_layer_back_to_back": round(stream_ms * 1e3, 2),
                    "tokens_per_s_one_layer": round(T / (med * 1e-3), 1),
                    "distinct_experts_avg": U, "algorithmic_bytes": int(algo),
                    "GBs": round(algo / (med * 1e-3) / 1e9, 1),
                    "pct_hbm_peak": round(100 * algo / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)})
        log(f"[bench] decode T={T}: {res[-1]}")
    return res


def run_prefill(dtype, Ts, n_layers, steps, warmup):
    """One MoE layer forward per step at prefill (configs[3]: Q4 experts,
    T tokens, x = RMSNorm(N(0,1)) with eps 1e-6 and weight 1, residual x);
    layers rotate so expert weights stream from HBM."""
    M.init(0)
    pool = LayerPool(dtype, n_layers)
    D = pool.D
    L = M.lib()
    res = []
    for T in Ts:
        x = M.DeviceBuffer(T * D * 4)
        xn = M.DeviceBuffer(T * D * 4)
        M.check(L.moe_fill_normal_dev(x.ptr, T * D, 5151 + T, 0.0, 1.0))
        M.check(L.moe_rmsnorm_dev(x.ptr, None, xn.ptr, T, D, 1e-6))
        out = M.DeviceBuffer(T * D * 4)
        idx = M.DeviceBuffer(T * 8 * 4)
        for i in range(max(warmup, n_layers)):
            pool.layers[i % n_layers].forward_dev(xn.ptr, x.ptr, T, out.ptr)
        M.synchronize()
        s0, s1 = M.Event(), M.Event()
        s0.record()
        for i in range(steps):
            pool.layers[i % n_layers].forward_dev(xn.ptr, x.ptr, T, out.ptr, idx.ptr)
        s1.record()
        M.synchronize()
        stream_ms = s0.elapsed_ms(s1) / steps
        ev = [(M.Event(), M.Event()) for _ in range(steps)]
        t0, t1 = M.Event(), M.Event()
        t0.record()
        for i in range(steps):
            ev[i][0].record()
            pool.layers[i % n_layers].forward_dev(xn.ptr, x.ptr, T, out.ptr, idx.ptr)
            ev[i][1].record()
        t1.record()
        M.synchronize()
        per = [a.elapsed_ms(b) for a, b in ev]
        ids = idx.download((T * 8,), np.int32)
        U = len(set(ids.tolist()) - {-1})
        algo = 1048576 + U * expert_bytes(dtype, D, pool.dff) + 2 * T * D * 4
        ops = T * 76021760
        med = float(np.median(per))
        res.append({"T": T, "layers_in_pool": n_layers, "steps": steps,
                    "us_per_layer_median": round(med * 1e3, 2),
                    "us_per_layer_mean": round(t0.elapsed_ms(t1) / steps * 1e3, 2),
                    "us_per_layer_back_to_back": round(stream_ms * 1e3, 2),
                    "tokens_per_s_one_layer": round(T / (med * 1e-3), 1),
                    "distinct_experts_last_step": U, "algorithmic_bytes": int(algo),
                    "GBs": round(algo / (med * 1e-3) / 1e9, 1),
                    "pct_hbm_peak": round(100 * algo / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                    "int_TOPs": round(ops / (med * 1e-3) / 1e12, 2)})
        log(f"[bench] prefill T={T}: {res[-1]}")
        for b in (x, xn, out, idx):
            b.free()
    return res


def run_dropin(calls):
    """The drop-in matmul_adaptive (host buffers: upload of A, the GEMV,
    download of C, a stream synchronisation per call) at the reference's
    call pattern (test_model_trace.c:496-503: one call per expert
    projection), over 24 distinct Q8 gate matrices [768 x 2048] (the 3
    projections of 8 experts), in both weight-cache modes: content-verified
    (the default; every call re-hashes the 1.5 MB of weight bytes) and
    address-trusted (moe_weight_cache_mode(1)).  Microseconds per call.
    The bytes are random (the call's cost does not depend on them)."""
    N, K, n_mats = 768, 2048, 24
    L = M.lib()
    rng = np.random.default_rng(6100)
    mats = []
    for i in range(n_mats):
        q = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = np.full(N, 1e-3, np.float32)
        mats.append((q, s, M.QuantizedWeight(q.ctypes.data, s.ctypes.data, N, K, 2)))
    x = rng.standard_normal(K, dtype=np.float32)
    y = np.empty(N, np.float32)
    out = {"shape": f"{N}x{K}", "dtype": "q8", "matrices": n_mats, "calls": calls}
    for mode, key in ((0, "us_per_call_verified"), (1, "us_per_call_trusted")):
        M.check(L.moe_weight_cache_mode(mode))
        for q, s, qw in mats:   # first use uploads
            L.matmul_adaptive(x.ctypes.data, None, ctypes.byref(qw), y.ctypes.data, 1, N, K)
        t0 = time.perf_counter()
        for i in range(calls):
            qw = mats[i % n_mats][2]
            L.matmul_adaptive(x.ctypes.data, None, ctypes.byref(qw), y.ctypes.data, 1, N, K)
        out[key] = round((time.perf_counter() - t0) / calls * 1e6, 1)
    M.check(L.moe_weight_cache_mode(0))
    M.check(L.moe_weight_cache_clear())
    out["hash_share_of_verified_call"] = round(
        1.0 - out["us_per_call_trusted"] / out["us_per_call_verified"], 3)
    log(f"[bench] drop-in matmul_adaptive: {out}")
    return out


QWEN3_30B_A3B = dict(D=2048, L=48, hd=128, nq=32, nkv=4, dff=768, E=128, top_k=8, V=151936)


def model_decode_bytes(c, ctx, dtype=3):
    """Algorithmic bytes of one decode token at context length ctx: every
    dense weight once (q/k/v/o, norms, router, lm_head), the 8 routed
    experts of every layer, the embedding row, and the K/V cache read."""
    D, L, hd, nq, nkv, V = c["D"], c["L"], c["hd"], c["nq"], c["nkv"], c["V"]
    attn = (nq + 2 * nkv) * hd * D * 4 + D * nq * hd * 4
    norms = (2 * D + 2 * hd) * 4
    router = c["E"] * D * 4
    experts = c["top_k"] * expert_bytes(dtype, D, c["dff"])
    kv = 2 * nkv * ctx * hd * 4
    return L * (attn + norms + router + experts + kv) + V * D * 4 + 2 * D * 4


def run_model(args):
    """the 48-layer Qwen3-30B-A3B-shaped model, random init
    (N(0, 0.02^2), norms 1, Q4 experts), a prompt of 512 uniform-random ids,
    then greedy decode steps with a 2048-position fp32 KV cache."""
    M.init(0)
    c = QWEN3_30B_A3B
    cfg = M.qwen_config(c["D"], c["L"], c["hd"], c["nq"], c["nkv"], c["dff"], c["E"], c["top_k"],
                        c["V"])
    t0 = time.perf_counter()
    model = M.Model.synthetic(cfg, expert_dtype=3, untied_head=True, seed=2024, std=0.02,
                              max_seq=2048)
    log(f"[bench] model built in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(512)
    prompt = rng.integers(0, c["V"], args.model_prompt).astype(np.int32)
    # warm-up run (kernel loading, scratch growth), then the measured one
    model.generate(prompt[:16], 4)
    ids, ms_p, ms_d = model.generate(prompt, args.model_steps + 1)
    steps = args.model_steps
    ctx_avg = args.model_prompt + steps / 2
    per_tok = model_decode_bytes(c, ctx_avg)
    res = {"prompt_tokens": int(args.model_prompt), "decode_steps": steps,
           "prefill_ms": round(ms_p, 2), "prefill_tok_s": round(args.model_prompt / (ms_p * 1e-3), 1),
           "decode_ms_total": round(ms_d, 2), "decode_ms_per_token": round(ms_d / steps, 3),
           "decode_tok_s": round(steps / (ms_d * 1e-3), 2),
           "algorithmic_bytes_per_token": int(per_tok),
           "decode_GBs": round(per_tok * steps / (ms_d * 1e-3) / 1e9, 1),
           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / per_tok, 1),
           "generated_head": ids[:8].tolist(),
           "arithmetic": "bit-identical to the reference (sequential fp32 chains, exact integer "
                         "expert dots)"}
    model.close()
    log(f"[bench] model decode: {res}")
    return res


def model_cpu_baseline(budget_s: float, threaded: bool = False):
    """The oracle's KV-cached restatement (oracle/model_oracle.c, the
    reference's loops) on one host thread: one full-size layer's decode
    step at context 512 and the 151936-row head, timed separately and
    combined as 48 layers + head per token (the full model does not fit a
    bounded CPU sample).  threaded: the same sources built with -fopenmp
    (liboracle_omp.so), output rows, heads and tokens split over all the
    host threads, each row in the reference's order (bit-identical to the
    single-thread build)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    lib = O.orc_omp() if threaded else O.orc_single()
    threads = lib.orc_threads()
    c = QWEN3_30B_A3B
    D, hd, nq, nkv, dff, E, V = c["D"], c["hd"], c["nq"], c["nkv"], c["dff"], c["E"], c["V"]
    rng = np.random.default_rng(7)

    def w(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))

    ex = O.ExpertSet(3, rng.integers(0, 256, (E, dff, D // 2), dtype=np.uint8),
                     np.full((E, dff), 1e-3, np.float32),
                     rng.integers(0, 256, (E, dff, D // 2), dtype=np.uint8),
                     np.full((E, dff), 1e-3, np.float32),
                     rng.integers(0, 256, (E, D, dff // 2), dtype=np.uint8),
                     np.full((E, D), 1e-3, np.float32), D, dff)
    lw = {"Wq": w(nq * hd, D), "Wk": w(nkv * hd, D), "Wv": w(nkv * hd, D), "Wo": w(D, nq * hd),
          "q_norm": np.ones(hd, np.float32), "k_norm": np.ones(hd, np.float32),
          "rms1_w": np.ones(D, np.float32), "rms2_w": np.ones(D, np.float32), "router_w": w(E, D)}
    keep = []

    def ptr(a):
        if a is None:
            return None
        keep.append(a)
        return a.ctypes.data

    layer = O.OrcLayer(*[ptr(lw.get(k)) for k in (
        "Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm", "k_norm", "rms1_w", "rms2_w",
        "router_w", "router_b")], ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu),
        ctypes.addressof(ex.Wd))
    cfg = O.OrcConfig(D, 1, hd, nq, nkv, dff, E, 8, V, 1, 1e7, 1e-6)
    ctx, max_seq = 512, 520
    kc = rng.standard_normal((nkv, max_seq, hd), dtype=np.float32)
    vc = rng.standard_normal((nkv, max_seq, hd), dtype=np.float32)
    x = rng.standard_normal((1, D), dtype=np.float32)
    n_layer, t_layer = 0, 0.0
    while t_layer < budget_s * 0.6:
        xx = x.copy()
        t0 = time.perf_counter()
        lib.orc_layer_rows(ctypes.byref(cfg), ctypes.byref(layer), xx.ctypes.data, 1, ctx,
                           kc.ctypes.data, vc.ctypes.data, max_seq)
        t_layer += time.perf_counter() - t0
        n_layer += 1
    head = w(V, D)
    out = np.empty((1, V), np.float32)
    t0 = time.perf_counter()
    lib.orc_matmul_f32(x.ctypes.data, head.ctypes.data, out.ctypes.data, 1, V, D)
    t_head = time.perf_counter() - t0
    per_token = c["L"] * t_layer / n_layer + t_head
    how = (f"{threads} threads (-fopenmp build, rows split over threads)" if threaded
           else "1 thread")
    return {"value": round(1.0 / per_token, 4), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{n_layer} decode steps of one full-size layer at context {ctx} "
                      f"({t_layer / n_layer * 1e3:.1f} ms each) and one lm_head product "
                      f"({t_head * 1e3:.1f} ms), per token = 48 layers + head, {how} of "
                      f"{host_cores()} host cores"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="q4_gemv", choices=["q4_gemv", "q8_gemv"])
    ap.add_argument("--pool-gib", type=float, default=1.0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-layer-runs", type=int, default=5,
                    help="timed runs (after one warm-up) of each single-thread layer baseline")
    ap.add_argument("--cpu-prefill", default="128",
                    help="prefill T values that get a CPU baseline ('' for none)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode", default="1,4,16",
                    help="also time one Q8 MoE decode layer at these T (configs[2]); '' to skip")
    ap.add_argument("--decode-layers", type=int, default=6)
    ap.add_argument("--prefill", default="128,512,2048",
                    help="also time one Q4 MoE prefill layer at these T (configs[3]); '' to skip")
    ap.add_argument("--model-steps", type=int, default=256,
                    help="greedy decode steps of the 48-layer model (configs[4]); 0 to skip")
    ap.add_argument("--model-prompt", type=int, default=512)
    ap.add_argument("--dropin-calls", type=int, default=480,
                    help="timed drop-in matmul_adaptive calls per weight-cache mode; 0 to skip")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs the expert path on a single MI355X "
              "(multi-GPU sharding is a design note, not implemented); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    q4_args = (3, [(2048, 768), (768, 2048)],
               "q4_rowwise_gemv_batch1 down[2048x768]+gate[768x2048] (BASELINE configs[1])")
    q8_args = (2, [(768, 2048)], "q8_rowwise_gemv_batch1 gate[768x2048] (BASELINE configs[0])")
    head, other = (q4_args, q8_args) if args.workload == "q4_gemv" else (q8_args, q4_args)
    out = run_gemv(args, *head)
    sub = run_gemv(args, *other)
    out["q8_gemv" if other is q8_args else "q4_gemv"] = {
        k: sub[k] for k in ("value", "unit", "ms_per_step", "config", "pct_hbm_peak", "roofline",
                            "kernels", "cpu_baseline") if k in sub}
    if args.decode:
        Ts = [int(t) for t in args.decode.split(",") if t]
        out["moe_decode_q8"] = run_decode(2, Ts, args.decode_layers, max(args.steps, 20),
                                          args.warmup)
        if not args.no_cpu:
            for r in out["moe_decode_q8"]:
                log(f"[bench] decode layer cpu baseline T={r['T']} ...")
                r["cpu_baseline"] = layer_cpu_baseline(2, r["T"], args.cpu_layer_runs)
    if args.prefill:
        Ts = [int(t) for t in args.prefill.split(",") if t]
        out["moe_prefill_q4"] = run_prefill(3, Ts, args.decode_layers, 10, 2)
        cpu_T = {int(t) for t in args.cpu_prefill.split(",") if t}
        if not args.no_cpu:
            for r in out["moe_prefill_q4"]:
                if r["T"] in cpu_T:
                    log(f"[bench] prefill layer cpu baseline T={r['T']} ...")
                    r["cpu_baseline"] = layer_cpu_baseline(3, r["T"], args.cpu_layer_runs)
    if args.dropin_calls > 0:
        out["dropin_matmul_adaptive"] = run_dropin(args.dropin_calls)
    if args.model_steps > 0:
        out["model_decode_q4"] = run_model(args)
        if not args.no_cpu:
            log("[bench] model cpu baseline (1 thread) ...")
            out["model_decode_q4"]["cpu_baseline"] = model_cpu_baseline(args.cpu_seconds)
            log("[bench] model cpu baseline (all cores) ...")
            out["model_decode_q4"]["cpu_baseline_all_cores"] = model_cpu_baseline(
                args.cpu_seconds / 2, threaded=True)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
