"""Benchmark of the MI355X quantized-matmul hot path (BASELINE.json's five configurations).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all]

Default (`--workload all`): one JSON line whose headline is configuration 3,
the W4A16 lm_head (M=1, K=1024, V=248094, one GEMV launch per step with the
argmax folded in, 8 weight copies = 1.06 GB rotated so no step reads the
256 MB MALL): W untimed steps, then exactly K steps between one HIP event pair
on the launch stream.  `value` is HBM throughput of algorithmic bytes
(132,484,244 B per step, inputs resident in HBM).  The line's `configs` object
carries every configuration of the north star, each measured in the same run:

  1  W4A16 GEMV K=N=1024                      (1024 rotated weight sets, 562 MB)
  2  W4A16 decode MLP block, one launch        (96 rotated layer sets, 549 MB)
  3  the lm_head (the headline, repeated)
  4  W4A16 prefill GEMM, M in {128,512,2048} x (K,N) in {(1024,3584),(3584,1024)}
  5  W8A8 GEMM M in {1,256,1024}, K=1024, N=3584 (fused fp16 epilogue)

For each: `us_per_call` = mean duration of 200 back-to-back launches, enqueued
directly while a spin kernel holds the stream (so the host's launch rate does
not gate short kernels, and a rocprofv3 kernel trace of the same launches
sees them back to back as well), the median of five such timed regions
(`regions_us_per_call` lists all five), from which `value` and
`roofline.achieved` follow; `kernel_us_median` /
`kernel_us_mean` = per-launch HIP event pairs around each of >= 100 launches
(the queue is kept full by a sleep kernel, so each pair brackets one kernel);
`cpu_baseline` = the oracle's restatement of the reference's CPU path on this
host, one thread and all threads (bounded samples, stated in `sample`).

`--workload` also runs any single configuration or one of the comparison
workloads (two-launch / unfused MLPs, W8A8 MLP, projections, vendor GEMMs,
the copy calibration) for profiling.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "W4A16 M=1 GEMV HBM GB/s (% peak) + µs/call; prefill GEMM TFLOPS (% MFMA)"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
INT8_MFMA_PEAK_TOPS = 5000.0
PER_LAUNCH = 200           # event-bracketed launches per configuration
ARGS = None                # the parsed command line


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_pkg():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as ge
    return ge.load_package()


def load_oracle():
    """The CPU oracle -- loaded only for the cpu_baseline legs, as the timed
    restatement of the reference's CPU path."""
    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import load_oracle as lo
    return lo()


def f16_normal(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16).view(np.uint16)


def to_dev_f16(a_u16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).cuda().view(torch.float16)


def w4a16_bytes(K, N):
    G = K // 128
    return K * N // 2 + G * N * 2 + G * N // 2


# --------------------------------------------------------------------------- #
# GPU timing                                                                   #
# --------------------------------------------------------------------------- #
def time_queued(launch, n_sets, steps, warmup=3, regions=1):
    """Mean ms per launch over `steps` back-to-back launches enqueued directly
    on torch's current stream while a spin kernel holds it, between one event
    pair: the GPU runs them back to back however slowly the host enqueues
    (rocprofv3's kernel trace of the same launches shows them back to back
    too, so its per-kernel durations match this figure).  Returns (ms per
    launch, host enqueue ms); with regions > 1, `regions` such timed regions
    one after another and the list of their ms per launch instead."""
    import torch
    for i in range(warmup):
        launch(i % n_sets)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for i in range(20):
        launch(i % n_sets)
    host_ms = (time.perf_counter() - t) / 20 * 1e3
    torch.cuda.synchronize()
    # one untimed pass over exactly the launches timed below: every weight
    # set they use is read once before the clock starts (a set's first read
    # after it was written costs extra: page-table walks on fresh memory)
    for i in range(steps):
        launch(i % n_sets)
    torch.cuda.synchronize()
    hold = steps * host_ms * 1.5 + 1.0
    out = []
    while len(out) < regions:
        for _ in range(3):
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            _sleep_ms(hold)
            t0.record()
            th = time.perf_counter()
            for i in range(steps):
                launch(i % n_sets)
            t1.record()
            enq_ms = (time.perf_counter() - th) * 1e3
            torch.cuda.synchronize()
            if enq_ms < 0.8 * hold:          # the spin kernel outlasted the enqueue
                break
            hold *= 2.0
        else:
            # The host never got ahead of the GPU: a profiler that serialises
            # dispatches blocks each launch until the one before has finished.
            # Time the region without the hold; the figure then includes the
            # host's enqueue time (an upper bound on the kernels' own).
            sys.stderr.write(f"[time_queued] the host could not enqueue {steps} launches within a "
                             f"{hold / 2:.1f} ms hold; timing without it (host-inclusive)\n")
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for i in range(steps):
                launch(i % n_sets)
            t1.record()
            torch.cuda.synchronize()
        out.append(t0.elapsed_time(t1) / steps)
    return (out[0], enq_ms) if regions == 1 else (out, enq_ms)


def time_direct(launch, n_sets, steps, warmup):
    """`warmup` untimed launches, then exactly `steps` back-to-back host
    launches between one event pair on torch's current stream (the stream the
    bound launchers use), synchronised on both sides.  A spin kernel enqueued
    before the first event keeps the GPU busy while the host enqueues the
    first launches, so the timed region holds the `steps` kernels and not the
    host's latency to issue the first of them.  Returns total ms."""
    import torch
    for i in range(warmup):
        launch(i % n_sets)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _sleep_ms(min(steps * 0.006, 2.0) + 0.3)
    t0.record()
    for i in range(steps):
        launch(i % n_sets)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


_SLEEP_CYCLES_PER_MS = None


def _sleep_ms(ms):
    """Occupy the stream for about `ms` (torch's spin kernel, calibrated once)."""
    import torch
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1_000_000)
        a.record()
        torch.cuda._sleep(10_000_000)
        b.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 10_000_000 / max(a.elapsed_time(b), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_CYCLES_PER_MS))


_HIP = None


def _hip():
    """The HIP runtime, for timing events torch does not create: events
    without the system-scope release fence (hipEventDisableSystemFence), whose
    markers do not write back the L2 around every kernel they bracket."""
    global _HIP
    if _HIP is None:
        import ctypes
        h = ctypes.CDLL("libamdhip64.so")
        h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _HIP = h
    return _HIP


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


def time_per_launch(launch, n_sets, n=PER_LAUNCH, host_us=25.0):
    """Per-launch durations (ms): a HIP event pair (no system fence) around
    each of `n` launches on torch's current stream.  A spin kernel first keeps
    the stream busy while the host enqueues them, so the GPU runs marker,
    kernel, marker back to back; each pair still includes its markers'
    processing (measured on MI355X: +1.5 us on a 3 us kernel, +0.3 us on a
    25 us one, against rocprofv3's kernel durations)."""
    import ctypes
    import torch
    h = _hip()
    launch(0)
    torch.cuda.synchronize()
    ev = []
    for _ in range(2 * n):
        e = ctypes.c_void_p()
        if h.hipEventCreateWithFlags(ctypes.byref(e), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")
        ev.append(e)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _sleep_ms(n * host_us / 1000.0 + 2.0)
    for i in range(n):
        h.hipEventRecord(ev[2 * i], stream)
        launch(i % n_sets)
        h.hipEventRecord(ev[2 * i + 1], stream)
    torch.cuda.synchronize()
    out = []
    for i in range(n):
        f = ctypes.c_float()
        if h.hipEventElapsedTime(ctypes.byref(f), ev[2 * i], ev[2 * i + 1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        out.append(f.value)
    for e in ev:
        h.hipEventDestroy(e)
    return out


def traffic_from_profiles(workload: str):
    """HBM bytes per launch from rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, each
    scaled by the copy-kernel calibration), committed in profiles/traffic.json."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(workload, {}).get("bytes_per_launch")
    except Exception:
        return None


REGIONS = 5


def gpu_result(name, kernel, amount, unit, bound, launch, n_sets, steps, extra=None):
    """Times one configuration: REGIONS timed regions of `steps` back-to-back
    launches each, the median region's mean per launch (value, roofline), and
    the per-launch median.  One MI355X region of a few ms can differ from the
    next by up to ~7 % for the same launches (the clocks and the memory system
    change on that scale), so one region alone is a noisy figure."""
    per_r, _ = time_queued(launch, n_sets, steps, regions=REGIONS)
    per = float(np.median(per_r))
    # (--no-per-launch: profiling runs, whose kernel trace should hold only
    # the back-to-back launches)
    pl = np.array([per] if ARGS.no_per_launch else time_per_launch(launch, n_sets))
    scale = 1e9 if unit == "GB/s" else 1e12
    value = amount / (per / 1e3) / scale
    peak = HBM_PEAK_GBS if bound == "hbm" else (INT8_MFMA_PEAK_TOPS if unit == "TOP/s" else FP16_MFMA_PEAK_TFLOPS)
    r = {"kernel": kernel, "us_per_call": round(per * 1e3, 3), "value": round(value, 2), "unit": unit,
         "kernel_us_median": round(float(np.median(pl)) * 1e3, 3), "kernel_us_mean": round(float(pl.mean()) * 1e3, 3),
         "per_launch_samples": int(pl.size), "back_to_back_launches": steps,
         "regions_us_per_call": [round(v * 1e3, 3) for v in per_r],
         "roofline": {"bound": bound, "achieved": round(value, 2), "peak": peak, "unit": unit,
                      "frac": round(value / peak, 4), "traffic": traffic_from_profiles(name),
                      "algorithmic_per_launch": amount}}
    if extra:
        r.update(extra)
    log(f"[{name}] {r['us_per_call']} us/call back to back, median {r['kernel_us_median']} us per launch, "
        f"{r['value']} {unit} ({100 * r['roofline']['frac']:.1f}% of peak)")
    return r


# --------------------------------------------------------------------------- #
# CPU baseline: the oracle's restatement of the reference's CPU path           #
# --------------------------------------------------------------------------- #
def cpu_info():
    try:
        threads = len(os.sched_getaffinity(0))
    except AttributeError:
        threads = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    # the GPU box grants 16 host threads per GPU
    return {"nproc": os.cpu_count(), "affinity": threads, "threads_used": min(16, threads), "model": model}


def _median_time(fn, budget_s, max_reps=31):
    fn()                                           # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < max_reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), len(times)


def cpu_baseline(fn, amount_1, amount_all, unit, sample_1, sample_all, info, budget_s=1.0):
    """fn(nthreads) runs the sample; amount_* its bytes (or FLOPs) for one
    thread and for all threads.  `value` is the all-threads rate."""
    scale = 1e9 if unit == "GB/s" else 1e12
    t1, n1 = _median_time(lambda: fn(1, False), budget_s)
    ta, na = _median_time(lambda: fn(info["threads_used"], True), budget_s)
    digits = 3 if unit == "GB/s" else 7
    return {"value": round(amount_all / ta / scale, digits), "unit": unit, "cores": info["threads_used"],
            "kind": "port",
            "sample": f"all threads: {sample_all}, median of {na} calls, {ta * 1e3:.2f} ms/call; "
                      f"one thread: {sample_1}, median of {n1} calls, {t1 * 1e3:.2f} ms/call",
            "one_thread": {"value": round(amount_1 / t1 / scale, digits), "ms_per_call": round(t1 * 1e3, 3)},
            "all_threads": {"value": round(amount_all / ta / scale, digits), "ms_per_call": round(ta * 1e3, 3)},
            "nproc": info["nproc"], "cpu_model": info["model"]}


# --------------------------------------------------------------------------- #
# configurations                                                               #
# --------------------------------------------------------------------------- #
class Cfg:
    """One configuration: set up, time on the GPU, time the CPU baseline."""

    def __init__(self, pkg, args, info):
        self.pkg, self.args, self.info = pkg, args, info


def _clone_w4(pkg, base, n):
    return [base] + [pkg.W4A16QuantizedWeight(base.qweight.clone(), base.scales.clone(), base.zeros.clone(), base.K,
                                              base.N, base.zero_bias) for _ in range(n - 1)]


class Gemv1(Cfg):
    name = "w4a16_gemv_1024x1024"

    def setup(self):
        import torch
        pkg = self.pkg
        K = N = 1024
        self.K, self.N = K, N
        rng = np.random.default_rng(1)
        self.x = f16_normal(rng, (1, K), 1.0)
        self.qweight, self.qzeros, self.scales = pkg.quantize_int4(f16_normal(rng, (K, N), 0.02))
        base = pkg.W4A16QuantizedWeight.from_awq(self.qweight, self.qzeros, self.scales)
        self.ws = _clone_w4(pkg, base, self.args.copies or 1024)          # 1024 x 0.55 MB = 562 MB
        self.xd = to_dev_f16(self.x)
        self.out = torch.empty((1, N), dtype=torch.float16, device="cuda")
        self.bytes = w4a16_bytes(K, N) + 2 * K + 2 * N

    def gpu(self):
        pkg, ws, xd, out = self.pkg, self.ws, self.xd, self.out
        kernel = pkg.lib().mcv_w4a16_gemm_kernel_name(1, self.K, self.N, 0).decode()
        return gpu_result(self.name, kernel, self.bytes, "GB/s", "hbm",
                          lambda i: pkg.matmul_w4a16(xd, ws[i], out), len(ws), 200,
                          {"config": {"M": 1, "K": self.K, "N": self.N, "weight_sets_rotated": len(ws),
                                      "algorithmic_bytes": self.bytes}})

    def cpu(self):
        o = load_oracle()
        w8 = o.unpack_awq(self.qweight, self.qzeros)
        fn = lambda c, _: o.w4a16_matmul(self.x, w8, self.scales, nthreads=c)
        s = "K=N=1024 GEMV (fp32 group formula over unpacked int8 q-z)"
        return cpu_baseline(fn, self.bytes, self.bytes, "GB/s", s, s, self.info)


class Mlp(Cfg):
    name = "w4a16_mlp_block_decode"

    def setup(self):
        import torch
        pkg = self.pkg
        H, I = 1024, 3584
        self.H, self.I = H, I
        layers, self.host = [], []
        for s in range(24):
            rng = np.random.default_rng(100 + s)
            mats, hm = [], []
            for (K, N) in ((H, I), (H, I), (I, H)):
                q = pkg.quantize_int4(f16_normal(rng, (K, N), 0.02))
                hm.append(q)
                mats.append(pkg.W4A16QuantizedWeight.from_awq(*q))
            layers.append(mats)
            if s == 0:
                self.host = hm
        sets = list(layers)
        for _ in range((self.args.copies or 4) - 1):
            sets += [[pkg.W4A16QuantizedWeight(m.qweight.clone(), m.scales.clone(), m.zeros.clone(), m.K, m.N, 0)
                      for m in L] for L in layers]
        self.sets = sets
        self.mlps = [pkg.DecodeMlpW4A16(*L) for L in sets]
        self.x = f16_normal(np.random.default_rng(1), (1, H), 1.0)
        self.xd = to_dev_f16(self.x)
        self.y = torch.empty((1, H), dtype=torch.float16, device="cuda")
        self.bytes = 2 * w4a16_bytes(H, I) + w4a16_bytes(I, H) + 2 * H + 2 * H

    def gpu(self):
        mlps, xd, y = self.mlps, self.xd, self.y
        r = gpu_result(self.name, "w4a16_mlp_kernel (gate, up, silu*mul, down in one launch)", self.bytes, "GB/s",
                       "hbm", lambda i: mlps[i](xd, y), len(mlps), 200,
                       {"config": {"M": 1, "hidden": self.H, "intermediate": self.I,
                                   "layer_sets_rotated": len(mlps), "algorithmic_bytes": self.bytes}})
        if any(m.act_wait_gave_up() for m in mlps) or not all(m.one_launch for m in mlps):
            raise RuntimeError("decode MLP: the one-launch kernel did not run cleanly")
        return r

    def cpu(self):
        o = load_oracle()
        (gq, gz, gs), (uq, uz, us), (dq, dz, ds) = self.host
        wg, wu, wd = o.unpack_awq(gq, gz), o.unpack_awq(uq, uz), o.unpack_awq(dq, dz)

        def block(c, _):
            g = o.f2h_rne(o.w4a16_matmul(self.x, wg, gs, nthreads=c))
            u = o.f2h_rne(o.w4a16_matmul(self.x, wu, us, nthreads=c))
            a = o.silu_mul(g, u)
            return o.w4a16_matmul(a, wd, ds, nthreads=c)
        s = "one decode MLP block H=1024 I=3584 (gate, up, silu*mul, down)"
        return cpu_baseline(block, self.bytes, self.bytes, "GB/s", s, s, self.info)


class Prefill(Cfg):
    def __init__(self, pkg, args, info, M, K, N):
        super().__init__(pkg, args, info)
        self.M, self.K, self.N = M, K, N
        self.name = f"w4a16_prefill_gemm_M{M}_K{K}_N{N}"

    def setup(self, weights=None):
        import torch
        pkg, M, K, N = self.pkg, self.M, self.K, self.N
        if weights is None:
            rng = np.random.default_rng(K * 7 + N)
            q = pkg.quantize_int4(f16_normal(rng, (K, N), 0.02))
            base = pkg.W4A16QuantizedWeight.from_awq(*q)
            weights = (q, _clone_w4(pkg, base, self.args.copies or 300))     # 300 x 1.9 MB = 572 MB
        self.host, self.ws = weights
        self.x = f16_normal(np.random.default_rng(M + K), (M, K), 1.0)
        self.xd = to_dev_f16(self.x)
        self.out = torch.empty((M, N), dtype=torch.float16, device="cuda")
        self.flops = 2.0 * M * K * N
        return weights

    def gpu(self):
        pkg, ws, xd, out = self.pkg, self.ws, self.xd, self.out
        # the kernel the dispatch launches for this shape (with the workspace
        # the Python mirror passes), as the library names it
        kernel = pkg.lib().mcv_w4a16_gemm_kernel_name(self.M, self.K, self.N, 1).decode()
        return gpu_result(self.name, kernel, self.flops, "TFLOP/s", "mfma",
                          lambda i: pkg.matmul_w4a16(xd, ws[i], out), len(ws), 200,
                          {"config": {"M": self.M, "K": self.K, "N": self.N, "weight_sets_rotated": len(ws),
                                      "flops": self.flops,
                                      "k_split_workspace_bytes":
                                          int(pkg.lib().mcv_w4a16_gemm_workspace_bytes(self.M, self.K, self.N))}})

    def cpu(self):
        o = load_oracle()
        qw, qz, sc = self.host
        w8 = o.unpack_awq(qw, qz)
        m1, ma = 4, 32
        fn = lambda c, full: o.w4a16_matmul(self.x[: (ma if full else m1)], w8, sc, nthreads=c)
        per_row = 2.0 * self.K * self.N
        return cpu_baseline(fn, m1 * per_row, ma * per_row, "TFLOP/s",
                            f"{m1} of the {self.M} rows, K={self.K} N={self.N}",
                            f"{ma} of the {self.M} rows, K={self.K} N={self.N}", self.info)


class W8a8(Cfg):
    def __init__(self, pkg, args, info, M, shared=None):
        super().__init__(pkg, args, info)
        self.M, self.K, self.N = M, 1024, 3584
        self.name = f"w8a8_gemm_M{M}_K1024_N3584"
        self.shared = shared

    def setup(self):
        import torch
        pkg, M, K, N = self.pkg, self.M, self.K, self.N
        if self.shared is None:
            rng = np.random.default_rng(11)
            wf = f16_normal(rng, (K, N), 0.02)
            base = pkg.quantize_dense_weight_w8a8(to_dev_f16(wf))
            sets = [base] + [pkg.W8A8QuantizedWeight(base.w_int8.clone(), base.w_scale.clone(),
                                                     base.w_scale_f32.clone(), K, N, base.layout)
                             for _ in range((self.args.copies or 160) - 1)]          # 160 x 3.7 MB = 590 MB
            self.shared = (wf, sets)
        self.wf, self.ws = self.shared
        self.x = f16_normal(np.random.default_rng(500 + M), (M, K), 1.0)
        self.xq, self.xs, _ = pkg.w8a8_quantize(to_dev_f16(self.x))
        self.out = torch.empty((M, N), dtype=torch.float16, device="cuda")
        self.flops = 2.0 * M * K * N
        self.bytes = K * N + 4 * N + M * K + 4 * M + 2 * M * N
        return self.shared

    def gpu(self):
        pkg, ws, xq, xs, out = self.pkg, self.ws, self.xq, self.xs, self.out
        M = self.M
        kernel = pkg.lib().mcv_w8a8_gemm_kernel_name(M, self.K, self.N, ws[0].layout, 1).decode()
        if M <= 4:
            amount, unit, bound = self.bytes, "GB/s", "hbm"
        else:
            amount, unit, bound = self.flops, "TOP/s", "mfma"
        r = gpu_result(self.name, kernel, amount, unit, bound, lambda i: pkg.matmul_w8a8(xq, xs, ws[i], out), len(ws),
                       200, {"config": {"M": M, "K": self.K, "N": self.N, "weight_sets_rotated": len(ws),
                                        "scales": "fp32 per-token and per-channel", "flops": self.flops,
                                        "algorithmic_bytes": self.bytes}})
        # the MFMA-side figure for every M, the HBM-side one for M = 1
        r["tops"] = round(self.flops / (r["us_per_call"] / 1e6) / 1e12, 3)
        return r

    def cpu(self):
        o = load_oracle()
        q_o, s_o, _ = o.w8a8_quantize_act(self.x)
        wq_o, ws_o, _ = o.w8a8_quantize_weight(self.wf)
        m1 = min(self.M, 8)
        ma = min(self.M, 64)

        def fn(c, full):
            m = ma if full else m1
            return o.w8a8_dequant(o.gemm_i32(q_o[:m], wq_o, nthreads=c), s_o[:m], ws_o)
        per_row = 2.0 * self.K * self.N
        unit = "GB/s" if self.M <= 4 else "TOP/s"
        if unit == "GB/s":
            a1 = aa = self.bytes
        else:
            a1, aa = m1 * per_row, ma * per_row
        return cpu_baseline(fn, a1, aa, unit, f"{m1} of the {self.M} rows (int32 GEMM + epilogue)",
                            f"{ma} of the {self.M} rows (int32 GEMM + epilogue)", self.info)


class LmHead(Cfg):
    name = "w4a16_lm_head_gemv_argmax"

    def setup(self):
        import torch
        pkg = self.pkg
        # V: the full vocabulary, or (--V, or `vocab`) one GPU's share of a
        # column split
        K, V = 1024, getattr(self, "vocab", 0) or self.args.V or 248094
        NW = -(-V // 8) * 8
        self.K, self.V = K, V
        rng = np.random.default_rng(1)
        t = time.perf_counter()
        w = f16_normal(rng, (K, NW), 0.02)
        self.x = f16_normal(rng, (1, K), 1.0)
        self.qweight, self.qzeros, self.scales = pkg.quantize_int4(w)
        del w
        qw, sc, zr = pkg.pack_awq(self.qweight, self.qzeros, self.scales)
        log(f"[lm_head] synthetic weights quantised + packed in {time.perf_counter() - t:.1f} s")
        base = pkg.W4A16QuantizedWeight.from_packed(qw, sc, zr, K, NW, 0)
        copies = self.args.copies or max(8, -(-1_050_000_000 // (qw.nbytes + sc.nbytes + zr.nbytes)))
        self.heads = [pkg.LmHeadW4A16(w_, V) for w_ in _clone_w4(pkg, base, copies)]
        self.rotated = copies * (qw.nbytes + sc.nbytes + zr.nbytes)
        self.xd = to_dev_f16(self.x)
        self.logits = torch.empty(V, dtype=torch.float16, device="cuda")
        self.bytes = K * V // 2 + (K // 128) * V * 2 + (K // 128) * V // 2 + 2 * V + 2 * K
        # bound launchers: arguments resolved once, ~4 us of host time per launch
        self.tree = [h.bind(self.xd, self.logits) for h in self.heads]
        self.slots = [h.bind(self.xd, self.logits, route="slots") for h in self.heads]
        # every rotated copy must give copy 0's token (this is also each
        # copy's first read after the clone wrote it, which costs ~8 us more
        # than later reads and would otherwise land in a short timed region)
        toks = [int(f().item()) for f in self.tree]
        if len(set(toks)) != 1:
            raise RuntimeError(f"lm_head weight copies disagree: tokens {toks}")

    def gpu_steps(self, steps, warmup, route):
        fns = self.tree if route == "tree" else self.slots
        return time_direct(lambda i: fns[i](), len(fns), steps, warmup)

    def per_launch(self, route):
        fns = self.tree if route == "tree" else self.slots
        return np.array(time_per_launch(lambda i: fns[i](), len(fns), 200, host_us=15.0))

    def token(self):
        return int(self.heads[0].launch(self.xd, self.logits).item())

    def greedy_step_us(self, n=200):
        """The whole greedy step as a decode loop pays it (lm_head_greedy_w4a16):
        the slots launch, the copy of the 64 slots to the host, which waits
        for the kernel, and the host fold.  Host wall clock per call."""
        for i in range(5):
            self.heads[i % len(self.heads)](self.xd, self.logits)
        t = time.perf_counter()
        for i in range(n):
            self.heads[i % len(self.heads)](self.xd, self.logits)
        return (time.perf_counter() - t) / n * 1e6

    def cpu(self):
        o = load_oracle()
        w8 = o.unpack_awq(self.qweight, self.qzeros)
        V = self.V

        def fn(c, _):
            logits = o.f2h_rne(o.w4a16_matmul(self.x, w8, self.scales, nthreads=c)[0, :V])
            return o.argmax_f16(logits)
        s = f"full lm_head K=1024 V={V}: fp32 group formula over unpacked int8 (q-z) + first-max argmax"
        return cpu_baseline(fn, self.bytes, self.bytes, "GB/s", s, s, self.info, budget_s=4.0)


SHARD_V = -(-248094 // 8)          # one GPU's columns of an 8-way split of the vocabulary


def lm_head_entry(lm, args, route, steps, cpu_entry):
    """One lm_head line: `steps` timed back-to-back launches (after untimed
    ones), the other argmax route, per-launch durations and the token."""
    import torch
    other = "slots" if route == "tree" else "tree"
    total_ms = lm.gpu_steps(steps, args.warmup, route)
    alt_ms = lm.gpu_steps(max(steps, 200), args.warmup, other)
    pl = lm.per_launch(route)
    greedy_us = lm.greedy_step_us()
    token = lm.token()
    torch.cuda.synchronize()
    ms = total_ms / steps
    value = lm.bytes / (ms / 1e3) / 1e9
    spw = lm.pkg.lm_head_slabs_per_workgroup(lm.V)
    kernel = (f"w4a16_lm_head_kernel<{spw}, {0 if route == 'tree' else 1}> (GEMV + fused argmax, "
              f"{'device-token' if route == 'tree' else 'host-finished slots'} route)")
    entry = {"kernel": kernel, "us_per_call": round(ms * 1e3, 3), "value": round(value, 2), "unit": "GB/s",
             "kernel_us_median": round(float(np.median(pl)) * 1e3, 3),
             "kernel_us_mean": round(float(pl.mean()) * 1e3, 3), "per_launch_samples": int(pl.size),
             "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(value / HBM_PEAK_GBS, 4),
                          "traffic": traffic_from_profiles(lm.name if lm.V == 248094 else f"{lm.name}_V{lm.V}"),
                          "algorithmic_per_launch": lm.bytes},
             "alt_route": {other: {"us_per_call": round(alt_ms / max(steps, 200) * 1e3, 3),
                                   "value": round(lm.bytes / (alt_ms / max(steps, 200) / 1e3) / 1e9, 2)}},
             "greedy_step": {"us_per_call": round(greedy_us, 2), "calls": 200,
                             "what": "LmHeadW4A16.__call__ (the Python mirror of lm_head_greedy): slots launch + "
                                     "copy of the slots to the host + host fold, host wall clock"},
             "config": {"M": 1, "K": lm.K, "V": lm.V, "argmax": route, "launch": "direct",
                        "weight_copies_rotated": len(lm.heads), "rotated_bytes": lm.rotated,
                        "algorithmic_bytes": lm.bytes, "token": token},
             "cpu_baseline": cpu_entry}
    log(f"[lm_head V={lm.V}] {entry['us_per_call']} us/step over {steps} steps, median {entry['kernel_us_median']} "
        f"us per launch, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of peak)")
    return entry


# --------------------------------------------------------------------------- #
# the default run                                                              #
# --------------------------------------------------------------------------- #
PREFILL_SHAPES = [(M, K, N) for M in (128, 512, 2048) for (K, N) in ((1024, 3584), (3584, 1024))]


def run_all(pkg, args, info):
    import torch
    t0 = time.perf_counter()
    gemv, mlp, lm = Gemv1(pkg, args, info), Mlp(pkg, args, info), LmHead(pkg, args, info)
    pre = [Prefill(pkg, args, info, *s) for s in PREFILL_SHAPES]
    w8 = [W8a8(pkg, args, info, M) for M in (1, 256, 1024)]
    gemv.setup()
    mlp.setup()
    shared = {}
    for p in pre:
        shared[(p.K, p.N)] = p.setup(shared.get((p.K, p.N)))
    sh8 = None
    for c in w8:
        c.shared = sh8
        sh8 = c.setup()
    lm.setup()
    log(f"[setup] {time.perf_counter() - t0:.1f} s")

    cpu = {}
    if not args.no_cpu:
        t = time.perf_counter()
        for c in [gemv, mlp, lm, *pre, *w8]:
            cpu[c.name] = c.cpu()
        log(f"[cpu baselines] {time.perf_counter() - t:.1f} s on {info['threads_used']} threads ({info['model']})")

    # headline first: the lm_head, W untimed steps then exactly K timed steps.
    # Measured on MI355X with 20 timed steps after 5 untimed ones: 25.3 us as
    # the first GPU work of the run; 27.4-27.6 us after the other
    # configurations (MFMA-heavy GEMMs just before), 27.4-29.0 us after 200
    # more untimed lm_head steps -- a few ms of sustained load lower the clock
    # for the next ~10 ms, over which 5000-step runs average 23.8 us.
    route = args.argmax
    lm_entry = lm_head_entry(lm, args, route, args.steps, cpu.get(lm.name))
    value, ms, kernel = lm_entry["value"], lm_entry["us_per_call"] / 1e3, lm_entry["kernel"]

    configs = {}
    configs["1_gemv_K1024_N1024"] = gemv.gpu()
    configs["2_mlp_block_H1024_I3584"] = mlp.gpu()
    configs["3_lm_head_K1024_V248094"] = lm_entry
    configs["4_prefill_gemm"] = {p.name: p.gpu() for p in pre}
    configs["5_w8a8_gemm_K1024_N3584"] = {c.name: c.gpu() for c in w8}
    for key, c in (("1_gemv_K1024_N1024", gemv), ("2_mlp_block_H1024_I3584", mlp)):
        configs[key]["cpu_baseline"] = cpu.get(c.name)
    for p in pre:
        configs["4_prefill_gemm"][p.name]["cpu_baseline"] = cpu.get(p.name)
    for c in w8:
        configs["5_w8a8_gemm_K1024_N3584"][c.name]["cpu_baseline"] = cpu.get(c.name)
    # the same kernel on one GPU's share of an 8-way column split of the
    # vocabulary (not a BASELINE configuration; how the lm_head would run sharded)
    del lm.heads, lm.tree, lm.slots
    shard = LmHead(pkg, args, info)
    shard.vocab = SHARD_V
    shard.setup()
    sh_cpu = None if args.no_cpu else shard.cpu()
    configs[f"3s_lm_head_shard_K1024_V{SHARD_V}"] = lm_head_entry(shard, args, route, args.steps, sh_cpu)
    del shard
    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (f16 x int4, f32 accumulate)",
        "data": "synthetic (seeded N(0,1) fp16 activations, N(0,0.02) fp16 weights quantised in-build)",
        "config": {"workload": lm.name, **lm_entry["config"]},
        "roofline": {k: v for k, v in lm_entry["roofline"].items() if k != "algorithmic_per_launch"} | {
            "kernel": kernel, "kernel_us_mean": lm_entry["kernel_us_mean"],
            "kernel_us_median": lm_entry["kernel_us_median"]},
        "cpu_baseline": lm_entry["cpu_baseline"],
        "configs": configs,
        "host": info,
    }


# --------------------------------------------------------------------------- #
# single workloads (profiling runs)                                            #
# --------------------------------------------------------------------------- #
def single(pkg, args, info, which):
    """One configuration (or comparison workload) as its own JSON line."""
    import torch
    if which == "lm_head":
        lm = LmHead(pkg, args, info)
        lm.setup()
        total = lm.gpu_steps(args.steps, args.warmup, args.argmax)
        ms = total / args.steps
        return {"workload": lm.name, "us_per_call": round(ms * 1e3, 3),
                "value": round(lm.bytes / (ms / 1e3) / 1e9, 2), "unit": "GB/s"}
    if which == "gemv1":
        c = Gemv1(pkg, args, info)
    elif which == "mlp":
        c = Mlp(pkg, args, info)
    elif which == "prefill":
        c = Prefill(pkg, args, info, args.M or 2048, args.K or 1024, args.N or 3584)
    elif which == "w8a8":
        c = W8a8(pkg, args, info, args.M or 1024)
    else:
        return EXTRA[which](pkg, args)
    c.setup()
    r = c.gpu()
    if not args.no_cpu:
        r["cpu_baseline"] = c.cpu()
    torch.cuda.synchronize()
    return {"workload": c.name, **r}


def _mlp_variant(pkg, args, mode):
    """Comparison decode-MLP launch sequences over 96 rotated W4A16 layer sets:
    two launches (gate+up+silu*mul, down) or the reference's four."""
    import torch
    m = Mlp(pkg, args, None)
    m.setup()
    H, I = m.H, m.I
    a = torch.empty((1, I), dtype=torch.float16, device="cuda")
    g, u = torch.empty_like(a), torch.empty_like(a)

    def block(i):
        L = m.sets[i]
        if mode == "two":
            pkg.mlp_gate_up_silu_w4a16(m.xd, L[0], L[1], a)
        else:
            pkg.matmul_w4a16(m.xd, L[0], g)
            pkg.matmul_w4a16(m.xd, L[1], u)
            pkg.silu_mul(g, u, a)
        pkg.matmul_w4a16(a, L[2], m.y)
    return {"workload": f"w4a16_mlp_block_decode_{mode}", **gpu_result(
        f"mlp_{mode}", f"mlp block ({mode})", m.bytes, "GB/s", "hbm", block, len(m.sets), 200)}


def _mlp_w8a8(pkg, args, mode):
    """The W8A8 decode MLP block over 32 rotated layer sets (352 MB): one launch
    (reference or fp32 scales) or the reference's six launches."""
    import torch
    H, I = 1024, 3584
    sets = []
    for s in range(args.copies or 32):
        rng = np.random.default_rng(200 + s)
        sets.append([pkg.quantize_dense_weight_w8a8(to_dev_f16(f16_normal(rng, (K, N), 0.02)))
                     for (K, N) in ((H, I), (H, I), (I, H))])
    x = to_dev_f16(f16_normal(np.random.default_rng(1), (1, H), 1.0))
    y = torch.empty((1, H), dtype=torch.float16, device="cuda")
    if mode in ("block", "block_f32"):
        mlps = [pkg.DecodeMlpW8A8(*L, precision="f32" if mode == "block_f32" else "reference") for L in sets]
        fn = lambda i: mlps[i](x, y)
    else:
        xq = torch.empty((1, H), dtype=torch.int8, device="cuda")
        aq = torch.empty((1, I), dtype=torch.int8, device="cuda")
        xs, as_ = (torch.empty(1, dtype=torch.float16, device="cuda") for _ in range(2))
        g, u, a = (torch.empty((1, I), dtype=torch.float16, device="cuda") for _ in range(3))

        def fn(i):
            L = sets[i]
            pkg.w8a8_quantize(x, xq, pkg._NO_F32, xs)
            pkg.matmul_w8a8(xq, xs, L[0], g, use_f32_scale=False)
            pkg.matmul_w8a8(xq, xs, L[1], u, use_f32_scale=False)
            pkg.silu_mul(g, u, a)
            pkg.w8a8_quantize(a, aq, pkg._NO_F32, as_)
            pkg.matmul_w8a8(aq, as_, L[2], y, use_f32_scale=False)
    nbytes = 3 * H * I + 2 * (2 * I + I) + 2 * H + 2 * H
    return {"workload": f"w8a8_mlp_block_decode_{mode}", **gpu_result(
        f"mlp_w8a8_{mode}", f"w8a8 mlp ({mode})", nbytes, "GB/s", "hbm", fn, len(sets), 200)}


def _vendor(pkg, args, int8):
    """The vendor library's dense GEMM at a prefill / W8A8 shape (torch.matmul
    -> hipBLASLt, torch._int_mm), as a yardstick."""
    import torch
    M, K, N = args.M or (1024 if int8 else 2048), args.K or 1024, args.N or 3584
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    if int8:
        a = torch.randint(-128, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
        b = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=g).t()
        fn = lambda i: torch._int_mm(a, b)
    else:
        a = torch.randn(M, K, dtype=torch.float16, device="cuda", generator=g)
        b = torch.randn(N, K, dtype=torch.float16, device="cuda", generator=g).t()
        c = torch.empty(M, N, dtype=torch.float16, device="cuda")
        fn = lambda i: torch.matmul(a, b, out=c)
    unit = "TOP/s" if int8 else "TFLOP/s"
    return {"workload": f"vendor_{'int8' if int8 else 'f16'}_M{M}_K{K}_N{N}",
            **gpu_result("vendor", "vendor GEMM", 2.0 * M * K * N, unit, "mfma", fn, 1, 200)}


def _lm_head_w8a8(pkg, args, part):
    """The W8A8 lm_head step as lm_head_greedy_w8a8 runs it (language_model.cpp:
    434-480 with the argmax on the device): activation quantisation with the
    fp16 scale, then the W8A8 GEMV over V = 248094 columns with the fp16 weight
    scale and the argmax folded in (one key per slab, then their reduction);
    4 rotated weight copies (1.0 GB).  part = "step" (the whole step in one
    launch, mcv_w8a8_lm_head_argmax), "parts" (the same in three launches:
    the quantisation, the GEMV with the folded argmax, the key reduction),
    "unfused" (the quantisation, the GEMV without the fold, then the separate
    argmax over the logits), "gemv" (the GEMV alone) or "argmax" (the
    separate argmax alone)."""
    import torch
    K, V = 1024, args.V or 248094
    rng = np.random.default_rng(1)
    x = to_dev_f16(f16_normal(rng, (1, K), 1.0))
    base = pkg.quantize_dense_weight_w8a8(f16_normal(rng, (K, V), 0.02))
    ws = [base] + [pkg.W8A8QuantizedWeight(base.w_int8.clone(), base.w_scale.clone(), base.w_scale_f32.clone(), K, V,
                                           base.layout) for _ in range((args.copies or 4) - 1)]
    xq = torch.empty((1, K), dtype=torch.int8, device="cuda")
    xs = torch.empty(1, dtype=torch.float16, device="cuda")
    logits = torch.empty((1, V), dtype=torch.float16, device="cuda")
    keys = torch.empty(-(-V // 64), dtype=torch.int64, device="cuda")
    tok = torch.empty(1, dtype=torch.int64, device="cuda")
    wsp = torch.zeros(pkg.lm_head_workspace_bytes(V), dtype=torch.uint8, device="cuda")
    pkg.w8a8_quantize(x, xq, pkg._NO_F32, xs)

    def step(i):
        if part == "step":
            pkg.lm_head_argmax_w8a8_fused(x, ws[i], V, wsp, logits, tok)
            return
        if part in ("parts", "unfused"):
            pkg.w8a8_quantize(x, xq, pkg._NO_F32, xs)
        if part == "parts":
            pkg.lm_head_argmax_w8a8(xq, xs, ws[i], V, logits, keys, tok)
            return
        if part != "argmax":
            pkg.matmul_w8a8(xq, xs, ws[i], logits, use_f32_scale=False)
        if part != "gemv":
            pkg.argmax_last_dim(logits, tok)
    gemv_bytes = K * V + 2 * V + 2 * V + K                  # weights, fp16 scales, logits, int8 x
    nbytes = {"gemv": gemv_bytes, "argmax": 2 * V, "step": gemv_bytes + 2 * K, "parts": gemv_bytes + 2 * K,
              "unfused": gemv_bytes + 2 * V + 2 * K}[part]
    spw, kb = pkg.w8a8_lm_head_slabs_per_workgroup(V), -(-K // 128) * 4
    kernel = {"step": f"w8a8_lm_head_kernel<{spw}, {1 if kb <= 16 else 2 if kb <= 32 else 4}> (one launch)",
              "parts": "w8a8_quant_act_kernel + w8a8_tiled_gemv_kernel<1, 16, 2, 2, true, false, true> + "
                       "argmax_reduce_kernel",
              "unfused": "w8a8_quant_act_kernel + w8a8_tiled_gemv_kernel<1, 16, 2, 2, true, false, false> + "
                         "argmax_kernel",
              "gemv": "w8a8_tiled_gemv_kernel<1, 16, 2, 2, true, false, false>",
              "argmax": "argmax_kernel"}[part]
    return {"workload": f"w8a8_lm_head_{part}_V{V}", **gpu_result(
        f"lm_head_w8a8_{part}", kernel, nbytes, "GB/s", "hbm", step, len(ws), 200)}


def _copy(pkg, args):
    """Calibration of the HBM counters: a 128 MiB device copy reads and writes
    exactly 134,217,728 bytes each."""
    import torch
    n = 128 * 2**20
    src = [torch.ones(n, dtype=torch.uint8, device="cuda") for _ in range(4)]
    dst = torch.empty(n, dtype=torch.uint8, device="cuda")
    return {"workload": "copy_128MiB_calibration",
            **gpu_result("copy", "torch copy kernel", 2 * n, "GB/s", "hbm", lambda i: dst.copy_(src[i]), 4, 100)}


def _tiny(pkg, args):
    """The per-dispatch cost of the kernel trace itself: the library's
    smallest kernel (silu_mul over 64 elements, one workgroup) back to back.
    Its duration is almost all launch and completion, so the difference
    between this line's us_per_call and a rocprofv3 --kernel-trace average of
    the same command is the trace's own per-dispatch cost."""
    import torch
    g = torch.zeros(64, dtype=torch.float16, device="cuda")
    u = torch.zeros(64, dtype=torch.float16, device="cuda")
    o = torch.empty(64, dtype=torch.float16, device="cuda")
    return {"workload": "tiny_kernel_dispatch",
            **gpu_result("tiny", "silu_mul_kernel (64 elements)", 64 * 6, "GB/s", "hbm",
                         lambda i: pkg.silu_mul(g, u, o), 1, 200)}


EXTRA = {
    "tiny": _tiny,
    "mlp_2launch": lambda p, a: _mlp_variant(p, a, "two"),
    "mlp_unfused": lambda p, a: _mlp_variant(p, a, "unfused"),
    "mlp_w8a8": lambda p, a: _mlp_w8a8(p, a, "block"),
    "mlp_w8a8_f32": lambda p, a: _mlp_w8a8(p, a, "block_f32"),
    "mlp_w8a8_unfused": lambda p, a: _mlp_w8a8(p, a, "unfused"),
    "vendor_f16": lambda p, a: _vendor(p, a, False),
    "vendor_int8": lambda p, a: _vendor(p, a, True),
    "copy": _copy,
    "lm_head_w8a8": lambda p, a: _lm_head_w8a8(p, a, "step"),
    "lm_head_w8a8_parts": lambda p, a: _lm_head_w8a8(p, a, "parts"),
    "lm_head_w8a8_unfused": lambda p, a: _lm_head_w8a8(p, a, "unfused"),
    "lm_head_w8a8_gemv": lambda p, a: _lm_head_w8a8(p, a, "gemv"),
    "lm_head_w8a8_argmax": lambda p, a: _lm_head_w8a8(p, a, "argmax"),
}
WORKLOADS = ["all", "lm_head", "gemv1", "mlp", "prefill", "w8a8", *EXTRA]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 5000 timed steps (~0.12 s): after the synchronise that opens the timed
    # region the lm_head kernel runs slower for its first ~10 ms (kernel trace:
    # 26.2 / 25.1 / 23.8 / 23.75 us by quarter of 1100 back-to-back launches,
    # clock management), which 1000 steps would count at ~2 % of the total
    ap.add_argument("--steps", type=int, default=5000, help="timed lm_head steps (the headline)")
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="all", choices=WORKLOADS)
    ap.add_argument("--copies", type=int, default=0, help="distinct weight sets rotated (0: per-config default)")
    ap.add_argument("--M", type=int, default=0)
    ap.add_argument("--K", type=int, default=0)
    ap.add_argument("--N", type=int, default=0)
    ap.add_argument("--V", type=int, default=0, help="lm_head vocabulary (default 248094)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-per-launch", action="store_true",
                    help="skip the event-bracketed per-launch timing (profiling runs)")
    ap.add_argument("--argmax", default="tree", choices=["tree", "slots"],
                    help="lm_head: token on the device (tree) or host-finished tagged slots")
    args = ap.parse_args()
    global ARGS
    ARGS = args
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: every box in this build has a single MI355X, and this run has no "
              "multi-GPU leg (the path would shard the weights by output column; see the design notes). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP kernels have no CPU fallback)", file=sys.stderr)
        sys.exit(3)
    pkg = load_pkg()
    info = cpu_info()
    if args.workload == "all":
        line = run_all(pkg, args, info)
    else:
        line = single(pkg, args, info, args.workload)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
