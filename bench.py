"""Benchmark of the MI355X matrix-multiply engine (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]
                    [--only config2,config3,fewrows,refapi,gemm,ffn,attention,stack,layout,stackfused,
                            gemvsweep,attn32k]

Headline (BASELINE config 2 as written): the fp16-weight decode GEMV
y = W . x with W [4096 x 4096] fp16 row-major (out x in), fp32 x / y, batch 1,
through eng_gemv_f16w_nk. One step is one GEMV launch over one weight matrix;
the steps are spread over 32 distinct 32 MiB weight buffers (1 GiB) so every
launch reads cold weights (the MI355X Infinity Cache holds 256 MB). The steps
are queued behind a GPU-side hold (eng_stream_delay) and run back to back
between two HIP events on the launch stream. `value` is algorithmic bytes
(2KN + 4K + 4N per launch) over that region, in GB/s. All inputs are synthetic
and already resident in HBM when timing starts. The metric's second figure,
the FP32 GEMM at 4096^3 (config 4), is timed the same way and reported in
"gemm_4096" (TFLOP/s and fraction of the 157.3 TFLOP/s FP32 MFMA peak).

stdout carries exactly one JSON line (a few KB): the headline, "roofline",
"gemm_4096", "cpu_baseline", "timing" and a "summary" of the key secondary
figures. Everything else goes to stderr, one JSON object per line: the
secondary rows (the reference-layout GEMVs, config 3, the other config-4
GEMMs, the config-5 32-layer decode stack, the FFN, attention and layout
rows), then the environment block. Secondary rows follow the reference
harness's protocol: warm-up, batches of back-to-back calls sized to ~1.5 ms
(at most 256), 15 batches, per-call median with p25 / p75 and IQR % (flagged
"noisy" above 10%). The CPU baseline runs the scalar C oracle (a restatement
of the reference's src/cpu_ref, double accumulation) on one pinned core before
the GPU is touched: config 2 for `cpu_baseline.value`, configs 1, 3, 4, 5 in
`cpu_baseline.per_config`.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix, published
METRIC = "decode GEMV HBM GB/s (% of peak); FP32 GEMM TFLOP/s at 4096^3 (% MFMA peak)"


HEADLINE_KERNEL = "eng::gemv::gemv_rows_dma_kernel<8, 512, 8, 16>"
TRAFFIC_PROFILE = os.path.join("profiles", "gemv_rows_dma_fixed_f16w_4096x4096_cold.md")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def profiled_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-kernel calibrated), or None when the
    summary is missing or covers a different kernel."""
    import re

    try:
        with open(os.path.join(REPO, TRAFFIC_PROFILE)) as f:
            text = f.read()
    except OSError:
        return None
    if HEADLINE_KERNEL not in text:
        return None
    m = re.search(r"^traffic_bytes_per_launch: (\d+)\s*$", text, re.M)
    return int(m.group(1)) if m else None


def profiled_trace_avg_us():
    """Average duration (us) of the headline kernel in the committed
    rocprofv3 kernel-trace summary of the bench command, or None."""
    import re

    try:
        with open(os.path.join(REPO, TRAFFIC_PROFILE)) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r"^trace_avg_us: ([0-9.]+)\s*$", text, re.M)
    return float(m.group(1)) if m else None


def load_package():
    """Import bare-metal-llm-engine_amd (its directory name is not an identifier)."""
    import importlib.util

    name = "bare_metal_llm_engine_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(REPO, "bare-metal-llm-engine_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


# ------------------------------------------------------------ CPU baseline
def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_cpu(fn, reps: int, seconds: float, warm: bool = True) -> list:
    """Wall time of `fn` per call: one warm-up (unless `warm` is False, for
    multi-second calls), then at least `reps` calls and at most `seconds` of
    them (the reference's time_cpu protocol)."""
    if warm:
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < reps or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def _tiled(rng, shape, kind):
    """Cheap CPU-baseline inputs: a 1 Mi-element random block repeated to
    `shape` (scalar-loop timings do not depend on the values)."""
    n = 1 << 20
    if kind == "f16":
        base = (0.02 * rng.standard_normal(n, dtype=np.float32)).astype(np.float16).view(np.uint16)
    else:
        base = rng.uniform(-1, 1, n).astype(np.float32)
    return np.resize(base, shape)


def cpu_baseline(seconds: float = 10.0) -> dict:
    """The scalar C oracle on one pinned core, per BASELINE config: config 2
    (the headline, fp16-weight GEMV) over ~`seconds`, then configs 1, 3, 4
    (sampled rows) and 5 (one layer) at >= 3 calls each."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import helpers

    orc = helpers.oracle(0)
    cpus = sorted(os.sched_getaffinity(0))
    core = cpus[0]
    old = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {core})
    rows = []
    try:
        rng = np.random.default_rng(1)
        K = N = 4096
        W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
        x = rng.standard_normal(K, dtype=np.float32)
        times = _time_cpu(lambda: orc.gemv_f16w(W, x), 3, seconds)
        med = float(np.median(times))
        nbytes = 2 * K * N + 4 * K + 4 * N

        # config 1: 512^3 GEMM.
        r = np.random.default_rng(0)
        A = r.uniform(-1, 1, (512, 512)).astype(np.float32)
        B = r.uniform(-1, 1, (512, 512)).astype(np.float32)
        t = float(np.median(_time_cpu(lambda: orc.matmul(A, B), 3, 0.0)))
        rows.append({"config": 1, "what": "matmul 512^3", "ms_per_call": round(t * 1e3, 2),
                     "GFLOP/s": round(2 * 512 ** 3 / t / 1e9, 3)})

        # config 3: rmsnorm_linear, fp16 W [K=4096 x N=11008].
        r = np.random.default_rng(2)
        K3, N3 = 4096, 11008
        x3 = r.standard_normal((1, K3), dtype=np.float32)
        g3 = (1 + 0.1 * r.standard_normal(K3)).astype(np.float32)
        W3 = _tiled(r, (K3, N3), "f16")
        t = float(np.median(_time_cpu(lambda: orc.rmsnorm_linear(x3, g3, W3, 1e-5), 3, 0.0, warm=False)))
        b3 = 2 * K3 * N3 + 8 * K3 + 4 * N3
        rows.append({"config": 3, "what": "rmsnorm_linear fp16-W 1x11008x4096",
                     "ms_per_call": round(t * 1e3, 2), "GB/s": round(b3 / t / 1e9, 4)})
        del W3

        # config 4: 512x11008x4096 on 4 sampled rows of A, extrapolated to 512.
        r = np.random.default_rng(3)
        A4 = r.uniform(-1, 1, (4, 4096)).astype(np.float32)
        B4 = _tiled(r, (4096, 11008), "f32")
        t = float(np.median(_time_cpu(lambda: orc.matmul(A4, B4), 3, 0.0, warm=False))) * (512 / 4)
        rows.append({"config": 4, "what": "matmul 512x11008x4096 (4 of 512 rows timed, x128)",
                     "ms_per_call": round(t * 1e3, 1), "GFLOP/s": round(2 * 512 * 11008 * 4096 / t / 1e9, 3)})
        del B4

        # config 5: one decoder layer's linear stack, reported x32 per token.
        r = np.random.default_rng(4)
        H, F = 4096, 11008
        sq = _tiled(r, (H, H), "f16")
        gu = _tiled(r, (H, F), "f16")
        dn = _tiled(r, (F, H), "f16")
        xh = r.standard_normal(H, dtype=np.float32)
        g5 = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)

        def layer():
            q = orc.gemv_f16w(sq, xh)
            orc.gemv_f16w(sq, xh)
            orc.gemv_f16w(sq, xh)
            o = orc.gemv_f16w(sq, q)
            gate = orc.rmsnorm_linear(o[None, :], g5, gu, 1e-5)
            orc.rmsnorm_linear(o[None, :], g5, gu, 1e-5)
            orc.gemv_f16w(dn, gate[0])

        t = float(np.median(_time_cpu(layer, 3, 0.0, warm=False))) * 32
        b5 = 12963053568
        rows.append({"config": 5, "what": "llama7b-shape decode linear stack (1 layer timed, x32)",
                     "ms_per_token": round(t * 1e3, 1), "GB/s": round(b5 / t / 1e9, 4)})
    finally:
        os.sched_setaffinity(0, old)
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{len(times)} calls of the config-2 GEMV (4096x4096 fp16 W, fp32 x/y) by the "
                   f"scalar C oracle (oracle/oracle.c orc_gemv_f16w, double accumulation), pinned "
                   f"to core {core} of {len(cpus)} on '{_cpu_model()}'; median {med * 1e3:.1f} ms/call"),
        "per_config": rows,
        "per_config_note": ("configs 1, 3, 4, 5 by the same oracle on the same core; their large weight "
                            "matrices are a 1 Mi-element random block repeated to shape (timing does not "
                            "depend on the values); config 4 times 4 of 512 rows, config 5 one layer"),
    }


# --------------------------------------------------------------- GPU timing
def _stats(samples: list) -> dict:
    """Median and spread of per-call times (ms), as the reference's harness
    reports them (bench_harness.hpp: median, p25/p75, IQR %, flagged > 10%)."""
    a = np.sort(np.asarray(samples, dtype=np.float64))
    med = float(np.median(a))
    p25, p75 = (float(v) for v in np.percentile(a, [25, 75]))
    iqr = 100.0 * (p75 - p25) / med if med > 0 else 0.0
    return {"median_ms": med, "p25_ms": p25, "p75_ms": p75, "iqr_pct": round(iqr, 2),
            "samples": len(a), "noisy": iqr > 10.0}


CLOCK_FLOOR = 0.75  # the reference's steady-clock floor: 75% of the nominal engine clock
HEADLINE_CLOCK_FLOOR = 0.90  # the headline window waits for the steady engine clock


class Timer:
    """HIP-event timing on one stream, with the reference harness's clock
    handling (bench_harness.hpp:215-310): warm-up continues until the live
    engine clock reaches 75% of nominal (bounded), and the live engine and
    memory clocks are read while each timed batch is in flight.

    Every timed window starts behind a hold (eng_stream_delay: one wave that
    sleeps on the GPU's constant clock) sized from the host's measured issue
    time per launch, so all launches of the window are queued before the
    first one starts: the window measures the GPU running them back to back,
    not the rate at which Python issues them (which under rocprofv3 drops to
    one launch per ~12 us). Windows whose issue outran the hold are counted.
    The headline window puts LEAD untimed launches between the hold and the
    first event, so the timed launches do not include the queue's start-up
    after the hold wave retires."""

    LEAD = 2

    def __init__(self, eng, pkg):
        self.eng = eng
        self.stream = eng.stream(pkg.STREAM_NON_BLOCKING)
        self.e0 = eng.event()
        self.e1 = eng.event()
        self.calls = 0
        self.nominal_mhz = eng.clock_rate_khz() // 1000
        self.sm_samples = []   # every clock read of the run, for the environment block
        self.mem_samples = []
        self.issue_us = None   # host issue time per launch (running maximum of recent windows)
        self.windows = 0
        self.windows_unheld = 0

    def _clocks(self, record: bool = True):
        sm, mem = self.eng.live_clocks_mhz()
        if record and sm > 0:
            self.sm_samples.append(sm)
        if record and mem > 0:
            self.mem_samples.append(mem)
        return sm, mem

    def hold_us(self, n: int) -> int:
        per = self.issue_us if self.issue_us is not None else 20.0
        return int(min(1_000_000, 100 + 1.5 * per * n))

    def _window(self, launch, n: int, clocks=None, lead: int = 0) -> float:
        """Queue a GPU-side hold, then `lead` untimed launches, then the `n`
        timed ones between two events; all are issued before the hold ends, so
        the timed launches run back-to-back on an already busy queue."""
        hold = self.hold_us(n + lead)
        self.eng.call("eng_stream_delay", self.stream.handle, hold)
        for _ in range(lead):
            launch(self.calls, self.stream.handle)
            self.calls += 1
        self.e0.record(self.stream)
        t0 = time.perf_counter()
        for _ in range(n):
            launch(self.calls, self.stream.handle)
            self.calls += 1
        issued_us = (time.perf_counter() - t0) * 1e6
        self.e1.record(self.stream)
        if clocks is not None:     # read while the batch runs
            clocks.append(self._clocks())
        self.e1.sync()
        self.windows += 1
        if issued_us > hold:
            self.windows_unheld += 1
        per = issued_us / max(n, 1)
        self.issue_us = per if self.issue_us is None else max(per, 0.8 * self.issue_us)
        self.last_hold_us, self.last_issued_us = hold, issued_us
        return self.e0.elapsed_ms(self.e1)

    def _warm(self, launch, min_calls: int, warmup_ms: float, max_wait_ms: float = 500.0,
              floor_frac: float = CLOCK_FLOOR) -> None:
        """At least `min_calls` calls and `warmup_ms` of them, then until the
        engine clock read during a batch reaches `floor_frac` of nominal (or
        `max_wait_ms`)."""
        t0 = time.perf_counter()
        n = 0
        floor = floor_frac * self.nominal_mhz
        while True:
            batch = max(1, min(min_calls, 64))
            tb = time.perf_counter()
            for _ in range(batch):
                launch(self.calls, self.stream.handle)
                self.calls += 1
                n += 1
            per = (time.perf_counter() - tb) * 1e6 / batch
            self.issue_us = per if self.issue_us is None else max(per, 0.8 * self.issue_us)
            sm, _ = self._clocks(record=False)
            self.stream.sync()
            el = (time.perf_counter() - t0) * 1e3
            if n >= min_calls and el >= warmup_ms and (sm == 0 or sm >= floor or el >= max_wait_ms):
                return

    def clock_stats(self, clocks) -> dict:
        sm = sorted(c[0] for c in clocks if c[0] > 0)
        mem = sorted(c[1] for c in clocks if c[1] > 0)
        out = {}
        if sm:
            out.update({"sm_clock_min_mhz": sm[0], "sm_clock_med_mhz": sm[len(sm) // 2],
                        "sm_clock_max_mhz": sm[-1]})
            if sm[0] < CLOCK_FLOOR * self.nominal_mhz:
                out["clock_dip"] = True
        if mem:
            out["mem_clock_med_mhz"] = mem[len(mem) // 2]
        return out

    def run(self, launch, steps: int, warmup: int) -> tuple:
        """(average ms per launch over exactly `steps` back-to-back launches on
        one stream after `warmup` untimed ones, clocks read during them)."""
        for _ in range(warmup):
            launch(self.calls, self.stream.handle)
            self.calls += 1
        self.stream.sync()
        self.eng.sync()
        clocks = []
        ms = self._window(launch, steps, clocks, lead=self.LEAD) / steps
        self.eng.sync()
        return ms, self.clock_stats(clocks)

    def sampled(self, launch, samples: int = 15, target_ms: float = 1.5, max_batch: int = 256,
                warmup_ms: float = 20.0) -> dict:
        """The reference's protocol: warm up for >= `warmup_ms` and until the
        clock floor, size a batch of back-to-back calls to ~`target_ms` (at
        most `max_batch`), time `samples` batches; per-call median / quartiles
        / IQR %, and the clocks read during the batches."""
        self._warm(launch, 2, warmup_ms)
        one = self._window(launch, 4) / 4
        batch = int(max(1, min(max_batch, round(target_ms / max(one, 1e-6)))))
        clocks = []
        per_call = [self._window(launch, batch, clocks) / batch for _ in range(samples)]
        st = _stats(per_call)
        st["batch"] = batch
        st.update(self.clock_stats(clocks))
        return st


def rand_f16(rng, shape, std=0.02):
    return (std * rng.standard_normal(shape, dtype=np.float32)).astype(np.float16).view(np.uint16)


def rotating(eng, host, count):
    """`count` distinct device copies of `host` (cold-cache rotation)."""
    first = eng.upload(host)
    bufs = [first]
    for _ in range(count - 1):
        d = eng.empty(host.shape, host.dtype)
        eng.call("eng_memcpy_d2d", d.ptr, first.ptr, first.nbytes)
        bufs.append(d)
    return bufs


CLOCK_KEYS = ("sm_clock_min_mhz", "sm_clock_med_mhz", "mem_clock_med_mhz", "clock_dip")


def _spread(st: dict) -> dict:
    return {"p25_us": round(st["p25_ms"] * 1e3, 3), "p75_us": round(st["p75_ms"] * 1e3, 3),
            "iqr_pct": st["iqr_pct"], "samples": st["samples"], "batch": st["batch"],
            **({"noisy": True} if st["noisy"] else {}),
            **{k: st[k] for k in CLOCK_KEYS if k in st}}


def hbm_row(name, st, nbytes, extra=None):
    """Row for an HBM-bound call timed by Timer.sampled (median per call)."""
    ms = st["median_ms"]
    gbs = nbytes / (ms * 1e-3) / 1e9
    row = {"name": name, "us_per_call": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
           "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes}
    row.update(_spread(st))
    if extra:
        row.update(extra)
    return row


def gemm_row(name, st, M, N, K):
    ms = st["median_ms"]
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    row = {"name": name, "ms_per_call": round(ms, 4), "TFLOP/s": round(tf, 2),
           "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "flops_per_call": 2 * M * N * K}
    row.update(_spread(st))
    return row


class GemvF16w:
    """Config-2-shaped fp16-weight GEMV over `rotate` distinct weight copies.
    nk=False: reference layout out = x . W[K x N] (eng_gemv_f16w);
    nk=True: y = W[N x K] . x, W row-major out x in (eng_gemv_f16w_nk)."""

    def __init__(self, eng, rotate=32, K=4096, N=4096, seed=1, nk=False):
        rng = np.random.default_rng(seed)
        self.eng, self.rotate, self.K, self.N = eng, rotate, K, N
        self.Ws = rotating(eng, rand_f16(rng, (N, K) if nk else (K, N)), rotate)
        self.dx = eng.upload(rng.standard_normal(K, dtype=np.float32))
        self.dy = eng.empty(N, np.float32)
        self.fn = eng.lib.eng_gemv_f16w_nk if nk else eng.lib.eng_gemv_f16w
        self.nbytes = 2 * K * N + 4 * K + 4 * N

    def __call__(self, i, s):
        rc = self.fn(self.Ws[i % self.rotate].ptr, self.dx.ptr, self.dy.ptr, self.N, self.K, s)
        if rc:
            raise RuntimeError(self.eng.last_error())

    def free(self):
        for w in self.Ws:
            w.free()


def rows_config2(eng, timer) -> list:
    rows = []
    # config 2 in both weight layouts, cold, and warm (the same 32 MiB matrix
    # every call: Infinity-Cache resident, not an HBM figure).
    for nk, tag in ((False, "reference layout x.W[KxN], eng_gemv_f16w"),
                    (True, "output-major y=W[NxK].x, eng_gemv_f16w_nk")):
        for rotate, temp in ((32, "cold"), (1, "WARM (cache-resident)")):
            g = GemvF16w(eng, rotate=rotate, nk=nk)
            rows.append(hbm_row(f"config 2 gemv fp16-W 4096x4096 {temp}, {tag}", timer.sampled(g), g.nbytes))
            g.free()
    return rows


def rows_config3(eng, timer) -> list:
    rows = []
    rng = np.random.default_rng(7)
    # config 3: fused RMSNorm + linear, fp16 W, K=4096, N=11008, cold (12 x 86 MiB).
    K, N, R = 4096, 11008, 12
    dx = eng.upload(np.random.default_rng(2).standard_normal(K, dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dy = eng.empty(N, np.float32)
    for nk, f, tag in ((False, eng.lib.eng_rmsnorm_linear_f16w, "reference layout W[KxN]"),
                       (True, eng.lib.eng_rmsnorm_linear_f16w_nk, "output-major W[NxK]")):
        Ws = rotating(eng, rand_f16(np.random.default_rng(2), (N, K) if nk else (K, N)), R)
        st = timer.sampled(lambda i, s: f(dx.ptr, dg.ptr, Ws[i % R].ptr, dy.ptr, 1, N, K, 1e-5, s))
        rows.append(hbm_row(f"config 3 rmsnorm_linear fp16-W 1x11008x4096 cold, {tag}", st,
                            2 * K * N + 8 * K + 4 * N))
        for w in Ws:
            w.free()
    # Small-batch decode at the config 3 shape: up to 4 rows share passes over
    # W (GEMV kernels; 5 to 64 rows are the "fewrows" group).
    Ws = rotating(eng, rand_f16(np.random.default_rng(2), (N, K)), R)
    f = eng.lib.eng_rmsnorm_linear_f16w_nk
    for M in (4,):
        dxm = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
        dym = eng.empty((M, N), np.float32)
        st = timer.sampled(lambda i, s: f(dxm.ptr, dg.ptr, Ws[i % R].ptr, dym.ptr, M, N, K, 1e-5, s))
        rows.append(hbm_row(f"rmsnorm_linear fp16-W {M}x11008x4096 cold (small-batch decode), "
                            "output-major W[NxK]", st, 2 * K * N + 4 * M * K + 4 * K + 4 * M * N))
        dxm.free(), dym.free()
    for w in Ws:
        w.free()
    Ws = rotating(eng, rand_f16(np.random.default_rng(2), (K, N)), R)
    f = eng.lib.eng_rmsnorm_linear_f16w
    M = 4
    dxm = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dym = eng.empty((M, N), np.float32)
    st = timer.sampled(lambda i, s: f(dxm.ptr, dg.ptr, Ws[i % R].ptr, dym.ptr, M, N, K, 1e-5, s))
    rows.append(hbm_row(f"rmsnorm_linear fp16-W {M}x11008x4096 cold (small-batch decode), "
                        "reference layout W[KxN]", st, 2 * K * N + 4 * M * K + 4 * K + 4 * M * N))
    # The down-projection shape (K = 11008): the same buffers read as output-major
    # [4096 x 11008]; 2 rows per pass (90 KiB of staged rows).
    Kd, Nd = N, K
    dxd = eng.upload(rng.standard_normal((M, Kd), dtype=np.float32))
    dyd = eng.empty((M, Nd), np.float32)
    fd = eng.lib.eng_rmsnorm_linear_f16w_nk
    st = timer.sampled(lambda i, s: fd(dxd.ptr, None, Ws[i % R].ptr, dyd.ptr, M, Nd, Kd, 1e-5, s))
    rows.append(hbm_row(f"rmsnorm_linear fp16-W {M}x4096x11008 cold (small-batch decode, down-projection "
                        "shape), output-major W[NxK]", st, 2 * Kd * Nd + 4 * M * Kd + 4 * M * Nd))
    dxd.free(), dyd.free()
    dxm.free(), dym.free()
    for w in Ws:
        w.free()
    return rows


def few_rows_arith(M: int) -> str:
    """How fp16-weight RMSNorm + linear computes M rows (5 to 64)."""
    if M < 33:
        return "few rows, fp16 MFMA, activations as three fp16 terms, exact products"
    return "33-64 rows: fp16-MFMA GEMM on three fp16 planes of the rows, exact products, 64-row tiles"


def rows_few_rows(eng, timer) -> list:
    """Few-row linear layers (5 to 64 activation rows): RMSNorm + linear at
    config 3's shape in both layouts (fp16 weights: the few-row MFMA kernel
    that streams W once up to 32 rows, the fp16-MFMA GEMM from 33), the
    down-projection shape, and a few-row FP32 matmul. Bytes: W once plus
    the activation rows in and out; FLOPs 2 M N K."""
    rows = []
    rng = np.random.default_rng(9)
    K, N, R = 4096, 11008, 12
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    for nk in (True, False):
        Ws = rotating(eng, rand_f16(np.random.default_rng(2), (N, K) if nk else (K, N)), R)
        f = eng.lib.eng_rmsnorm_linear_f16w_nk if nk else eng.lib.eng_rmsnorm_linear_f16w
        tag = "output-major W[NxK]" if nk else "reference layout W[KxN]"
        for M in ((5, 8, 16, 32, 64) if nk else (16, 64)):
            dxm = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
            dym = eng.empty((M, N), np.float32)
            st = timer.sampled(lambda i, s: f(dxm.ptr, dg.ptr, Ws[i % R].ptr, dym.ptr, M, N, K, 1e-5, s))
            row = hbm_row(f"rmsnorm_linear fp16-W {M}x11008x4096 cold ({few_rows_arith(M)}), {tag}", st,
                          2 * K * N + 4 * M * K + 4 * K + 4 * M * N)
            row["TFLOP/s"] = round(2.0 * M * N * K / (st["median_ms"] * 1e-3) / 1e12, 2)
            rows.append(row)
            dxm.free(), dym.free()
        if nk:
            # the same buffers read as the down projection [4096 x 11008]
            Kd, Nd, M = N, K, 16
            dxd = eng.upload(rng.standard_normal((M, Kd), dtype=np.float32))
            dyd = eng.empty((M, Nd), np.float32)
            st = timer.sampled(lambda i, s: f(dxd.ptr, None, Ws[i % R].ptr, dyd.ptr, M, Nd, Kd, 1e-5, s))
            rows.append(hbm_row(f"rmsnorm_linear fp16-W {M}x4096x11008 cold ({few_rows_arith(M)}, "
                                "down-projection shape), output-major W[NxK]", st,
                                2 * Kd * Nd + 4 * M * Kd + 4 * M * Nd))
            dxd.free(), dyd.free()
        for w in Ws:
            w.free()
    # FP32 matmul with 16 and 64 rows (B [4096 x 4096] fp32, 8 rotating copies)
    Kf = Nf = 4096
    Bs = rotating(eng, rng.uniform(-1, 1, (Kf, Nf)).astype(np.float32), 8)
    for M in (16, 64):
        dA = eng.upload(rng.uniform(-1, 1, (M, Kf)).astype(np.float32))
        dC = eng.empty((M, Nf), np.float32)
        fm = eng.lib.eng_matmul_f32
        st = timer.sampled(lambda i, s: fm(dA.ptr, Bs[i % 8].ptr, dC.ptr, M, Nf, Kf, s))
        row = hbm_row(f"matmul_f32 {M}x4096x4096 cold B (few rows, MFMA)", st,
                      4 * Kf * Nf + 4 * M * Kf + 4 * M * Nf)
        row["TFLOP/s"] = round(2.0 * M * Nf * Kf / (st["median_ms"] * 1e-3) / 1e12, 2)
        rows.append(row)
        dA.free(), dC.free()
    for b in Bs:
        b.free()
    dg.free()
    return rows


def rows_reference_api(eng, timer) -> list:
    """The reference's published decode rows through the reference-layout API
    (W [K x N]): fp32 gemv, half-I/O gemv_fp16 and fp32-weight rmsnorm_linear
    at 1 x 4096 x 4096 and 1 x 12288 x 4096 (README / results.json rows), cold
    weights (rotating copies past the 256 MB Infinity Cache)."""
    rows = []
    rng = np.random.default_rng(8)
    K = 4096
    for N in (4096, 12288):
        Wf32 = (0.02 * rng.standard_normal((K, N), dtype=np.float32))
        R = max(2, (1 << 30) // Wf32.nbytes + 1)
        Wf = rotating(eng, Wf32, R)
        dx = eng.upload(rng.standard_normal(K, dtype=np.float32))
        dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
        dy = eng.empty(N, np.float32)
        f = eng.lib.eng_gemv_f32
        st = timer.sampled(lambda i, s: f(Wf[i % R].ptr, dx.ptr, dy.ptr, N, K, s))
        rows.append(hbm_row(f"gemv (fp32 W) {K}x{N} cold", st, 4 * K * N + 4 * K + 4 * N))
        f = eng.lib.eng_rmsnorm_linear_f32
        st = timer.sampled(lambda i, s: f(dx.ptr, dg.ptr, Wf[i % R].ptr, dy.ptr, 1, N, K, 1e-5, s))
        rows.append(hbm_row(f"rmsnorm_linear (fp32 W) 1x{N}x{K} cold", st, 4 * K * N + 8 * K + 4 * N))
        for d in Wf + [dx, dg, dy]:
            d.free()
        Wf16 = rand_f16(rng, (K, N))
        R = max(2, (1 << 30) // Wf16.nbytes + 1)
        Wh = rotating(eng, Wf16, R)
        dxh = eng.upload(rng.standard_normal(K, dtype=np.float32).astype(np.float16).view(np.uint16))
        dyh = eng.empty(N, np.uint16)
        f = eng.lib.eng_gemv_f16
        st = timer.sampled(lambda i, s: f(Wh[i % R].ptr, dxh.ptr, dyh.ptr, N, K, s))
        rows.append(hbm_row(f"gemv_fp16 (half x/out) {K}x{N} cold", st, 2 * K * N + 2 * K + 2 * N))
        for d in Wh + [dxh, dyh]:
            d.free()
    return rows


def rows_gemm(eng, timer) -> list:
    rows = []
    rng = np.random.default_rng(9)
    # configs 1 and 4: FP32 GEMMs on MFMA.
    f = eng.lib.eng_matmul_f32
    for cfg, M, N, K, seed in ((1, 512, 512, 512, 0), (4, 4096, 4096, 4096, 3), (4, 512, 11008, 4096, 3),
                               (4, 512, 4096, 11008, 3), (0, 1024, 1024, 1024, 3), (0, 2048, 2048, 2048, 3)):
        r3 = np.random.default_rng(seed)
        dA = eng.upload(r3.uniform(-1, 1, (M, K)).astype(np.float32))
        dB = eng.upload(r3.uniform(-1, 1, (K, N)).astype(np.float32))
        dC = eng.empty((M, N), np.float32)
        st = timer.sampled(lambda i, s: f(dA.ptr, dB.ptr, dC.ptr, M, N, K, s))
        # config 0: the reference's other published matmul_register_tiled sizes
        tag = f"(config {cfg})" if cfg else "(reference README size)"
        rows.append(gemm_row(f"matmul_f32 {M}x{N}x{K} {tag}", st, M, N, K))
        dA.free(), dB.free(), dC.free()

    # Reference bench shape: rmsnorm_linear (fp32 W) at M = 512, 4096 x 4096.
    M, N, K = 512, 4096, 4096
    dA = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dW = eng.upload((rng.standard_normal((K, N), dtype=np.float32) / 64).astype(np.float32))
    dC = eng.empty((M, N), np.float32)
    f = eng.lib.eng_rmsnorm_linear_f32
    st = timer.sampled(lambda i, s: f(dA.ptr, dg.ptr, dW.ptr, dC.ptr, M, N, K, 1e-5, s))
    rows.append(gemm_row("rmsnorm_linear_f32 512x4096x4096 (rmsnorm into pooled scratch + MFMA GEMM)",
                        st, M, N, K))
    dA.free(), dg.free(), dW.free(), dC.free()

    # Prefill with fp16 weights (fp32 activations, fp32 accumulate): the gate /
    # up shape of config 5 at 512 tokens, both weight layouts.
    M, N, K = 512, 11008, 4096
    dA = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dC = eng.empty((M, N), np.float32)
    for name, fn, shape in (("reference layout W[KxN]", eng.lib.eng_rmsnorm_linear_f16w, (K, N)),
                            ("output-major W[NxK]", eng.lib.eng_rmsnorm_linear_f16w_nk, (N, K))):
        dW = eng.upload(rand_f16(rng, shape))
        st = timer.sampled(lambda i, s: fn(dA.ptr, dg.ptr, dW.ptr, dC.ptr, M, N, K, 1e-5, s))
        rows.append(gemm_row(f"rmsnorm_linear_f16w {M}x{N}x{K} prefill, fp16 W {name}", st, M, N, K))
        dW.free()
    dA.free(), dg.free(), dC.free()
    # A prompt length that is not a multiple of the tile (1000 tokens).
    M = 1000
    dA = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dC = eng.empty((M, N), np.float32)
    dW = eng.upload(rand_f16(rng, (N, K)))
    fn = eng.lib.eng_rmsnorm_linear_f16w_nk
    st = timer.sampled(lambda i, s: fn(dA.ptr, dg.ptr, dW.ptr, dC.ptr, M, N, K, 1e-5, s))
    rows.append(gemm_row(f"rmsnorm_linear_f16w {M}x{N}x{K} prefill (ragged M), fp16 W output-major W[NxK]",
                         st, M, N, K))
    dA.free(), dC.free()
    # A long prompt (4096 tokens): 128 x 256 tiles on the fp16 matrix cores.
    M = 4096
    dA = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dC = eng.empty((M, N), np.float32)
    st = timer.sampled(lambda i, s: fn(dA.ptr, dg.ptr, dW.ptr, dC.ptr, M, N, K, 1e-5, s))
    rows.append(gemm_row(f"rmsnorm_linear_f16w {M}x{N}x{K} prefill, fp16 W output-major W[NxK]", st, M, N, K))
    dA.free(), dg.free(), dC.free(), dW.free()
    return rows


def rows_ffn(eng, timer) -> list:
    """The ops either side of the linear layers, and the fused gate/up + SwiGLU."""
    rows = []
    rng = np.random.default_rng(10)
    H, F = 4096, 11008
    # residual_rmsnorm: decode row and a prefill batch (reads x, residual, gain;
    # writes sum and norm).
    for R in (1, 128):
        dx = eng.upload(rng.standard_normal((R, H), dtype=np.float32))
        dr = eng.upload(rng.standard_normal((R, H), dtype=np.float32))
        dw = eng.upload((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        dn, dsum = eng.empty((R, H), np.float32), eng.empty((R, H), np.float32)
        f = eng.lib.eng_residual_rmsnorm_f32
        st = timer.sampled(lambda i, s: f(dx.ptr, dr.ptr, dw.ptr, dn.ptr, dsum.ptr, R, H, 1e-5, s))
        rows.append(hbm_row(f"residual_rmsnorm {R}x{H}", st, 16 * R * H + 4 * H))
        for d in (dx, dr, dw, dn, dsum):
            d.free()
    # swiglu over a decode row and a prefill batch of the FFN width.
    for R in (1, 128):
        dg = eng.upload(rng.standard_normal(R * F, dtype=np.float32))
        du = eng.upload(rng.standard_normal(R * F, dtype=np.float32))
        do = eng.empty(R * F, np.float32)
        f = eng.lib.eng_swiglu_f32
        st = timer.sampled(lambda i, s: f(dg.ptr, du.ptr, do.ptr, R * F, s))
        rows.append(hbm_row(f"swiglu {R}x{F}", st, 12 * R * F))
        for d in (dg, du, do):
            d.free()
    # Config-5 gate/up + SwiGLU at decode, cold (6 rotating pairs of 86 MiB):
    # one fused launch vs rmsnorm_linear x2 + swiglu.
    RW = 6
    base = rand_f16(rng, (F, H))
    Wg = rotating(eng, base, RW)
    Wu = rotating(eng, base, RW)
    dx = eng.upload(rng.standard_normal(H, dtype=np.float32))
    dgm = eng.upload((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    dgate, dup, dact = (eng.empty(F, np.float32) for _ in range(3))
    nbytes = 2 * 2 * H * F + 8 * H + 4 * F
    glu = eng.lib.eng_rmsnorm_linear_swiglu_f16w_nk
    st = timer.sampled(lambda i, s: glu(dx.ptr, dgm.ptr, Wg[i % RW].ptr, Wu[i % RW].ptr, dact.ptr,
                                        1, F, H, 1e-5, s))
    rows.append(hbm_row("FFN gate/up + SwiGLU 1x11008x4096 fp16-W cold, fused (1 launch)", st, nbytes))
    rl, sw = eng.lib.eng_rmsnorm_linear_f16w_nk, eng.lib.eng_swiglu_f32

    def unfused(i, s):
        rl(dx.ptr, dgm.ptr, Wg[i % RW].ptr, dgate.ptr, 1, F, H, 1e-5, s)
        rl(dx.ptr, dgm.ptr, Wu[i % RW].ptr, dup.ptr, 1, F, H, 1e-5, s)
        sw(dgate.ptr, dup.ptr, dact.ptr, F, s)

    st = timer.sampled(unfused)
    rows.append(hbm_row("FFN gate/up + SwiGLU 1x11008x4096 fp16-W cold, unfused (3 launches)", st, nbytes))
    # Reference layout [K x N] (the same buffers read as 4096 x 11008): one
    # split-K launch over both matrices and a reduce with the SwiGLU epilogue,
    # vs the reference's composition (two rmsnorm_linear calls and swiglu).
    glu_kn, rlk = eng.lib.eng_rmsnorm_linear_swiglu_f16w, eng.lib.eng_rmsnorm_linear_f16w
    st = timer.sampled(lambda i, s: glu_kn(dx.ptr, dgm.ptr, Wg[i % RW].ptr, Wu[i % RW].ptr, dact.ptr,
                                           1, F, H, 1e-5, s))
    rows.append(hbm_row("FFN gate/up + SwiGLU 1x11008x4096 fp16-W cold, reference layout W[KxN], "
                        "fused (2 launches)", st, nbytes))

    def unfused_kn(i, s):
        rlk(dx.ptr, dgm.ptr, Wg[i % RW].ptr, dgate.ptr, 1, F, H, 1e-5, s)
        rlk(dx.ptr, dgm.ptr, Wu[i % RW].ptr, dup.ptr, 1, F, H, 1e-5, s)
        sw(dgate.ptr, dup.ptr, dact.ptr, F, s)

    st = timer.sampled(unfused_kn)
    rows.append(hbm_row("FFN gate/up + SwiGLU 1x11008x4096 fp16-W cold, reference layout W[KxN], "
                        "unfused (5 launches)", st, nbytes))
    # Small-batch decode: 4 rows share each pass over the gate / up weights.
    M = 4
    dxm = eng.upload(rng.standard_normal((M, H), dtype=np.float32))
    dam = eng.empty((M, F), np.float32)
    st = timer.sampled(lambda i, s: glu(dxm.ptr, dgm.ptr, Wg[i % RW].ptr, Wu[i % RW].ptr, dam.ptr,
                                        M, F, H, 1e-5, s))
    rows.append(hbm_row(f"FFN gate/up + SwiGLU {M}x11008x4096 fp16-W cold (small-batch decode, 1 launch)",
                        st, 2 * 2 * H * F + 4 * M * H + 4 * H + 4 * M * F))
    for d in Wg + Wu + [dx, dgm, dgate, dup, dact, dxm, dam]:
        d.free()
    # Prefill at 512 tokens, output-major fp16 weights: the rows split once
    # into fp16 planes, gate and up on the fp16-MFMA GEMM, then SwiGLU. FLOP:
    # the two GEMMs, 2 x 2MNK.
    M = 512
    dWg, dWu = eng.upload(base), eng.upload(rand_f16(rng, (F, H)))
    dxp = eng.upload(rng.standard_normal((M, H), dtype=np.float32))
    dgp = eng.upload((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    dap = eng.empty((M, F), np.float32)
    st = timer.sampled(lambda i, s: glu(dxp.ptr, dgp.ptr, dWg.ptr, dWu.ptr, dap.ptr, M, F, H, 1e-5, s))
    rows.append(gemm_row(f"FFN gate/up + SwiGLU {M}x11008x4096 fp16-W prefill (both GEMMs' FLOP)",
                         st, M, 2 * F, H))
    for d in (dWg, dWu, dxp, dgp, dap):
        d.free()
    return rows


ATTENTION_CASES = [(512, 32, 4, 64), (2048, 32, 4, 64), (8192, 32, 4, 64), (16384, 32, 4, 64),
                   (32768, 32, 4, 64), (512, 32, 32, 128), (2048, 32, 32, 128), (8192, 32, 32, 128),
                   (8192, 32, 8, 128), (32768, 32, 8, 128)]


def rows_attention(eng, timer, cases=ATTENTION_CASES, extra_variants=True) -> list:
    """Decode attention at the reference's benchmark shapes (bench_kernels.cu:
    1079-1092): TinyLlama 32/4 heads at D = 64 and Llama-2-7B 32/32 at D = 128,
    plus GQA at D = 128 (32/8 heads, the Llama-3-8B layout, which the reference's
    kernel also takes), cold KV caches (about 1 GiB of rotating copies). Bytes:
    K and V once plus q and out, 2 (2 H_kv L D + 2 H D)."""
    rows = []
    rng = np.random.default_rng(11)
    f = eng.lib.eng_attention_decode_with_mode_f16
    for L, H, Hkv, D in cases:
        elems = 2 * Hkv * L * D
        nslots = max(2, (1 << 30) // (2 * elems) + 1)
        kv = rotating(eng, (0.5 * rng.standard_normal(elems, dtype=np.float32)).astype(np.float16).view(np.uint16),
                      nslots)
        dq = eng.upload((0.5 * rng.standard_normal(H * D, dtype=np.float32)).astype(np.float16).view(np.uint16))
        do = eng.empty(H * D, np.uint16)
        sc = 1.0 / np.sqrt(D)
        nbytes = 2 * (2 * Hkv * L * D + 2 * H * D)
        arch = "TinyLlama" if Hkv == 4 else ("Llama-2-7B" if Hkv == H else "GQA-8 (Llama-3-8B layout)")
        variants = [("auto splits", 0, 1)]
        if extra_variants and L >= 8192:
            variants.append(("split_kv=1", 1, 1))
        if extra_variants and Hkv == 4 and L == 32768:
            variants.append(("no GQA sharing", 0, 0))
        for tag, sp, share in variants:
            def launch(i, s, sp=sp, share=share):
                kp = kv[i % nslots].ptr
                rc = f(dq.ptr, kp, kp + 2 * Hkv * L * D, do.ptr, L, H, Hkv, D, L * D, sc, sp, share, s)
                if rc:
                    raise RuntimeError(eng.last_error())
            rows.append(hbm_row(f"attention_decode {arch} L={L} H={H}/{Hkv} D={D} cold, {tag}",
                                timer.sampled(launch), nbytes))
        for d in kv + [dq, do]:
            d.free()
    return rows


def rows_attention_tinyllama_32k(eng, timer) -> list:
    """Only TinyLlama L = 32768 with automatic splits (for profiling its kernels alone)."""
    return rows_attention(eng, timer, cases=[(32768, 32, 4, 64)], extra_variants=False)


def rows_stack(eng, timer) -> list:
    return [bench_llama_stack(eng, timer, nk=False),
            bench_llama_stack(eng, timer, nk=False, fused_glu=True, graph=True, fused_qkv=True),
            bench_llama_stack(eng, timer, nk=True),
            bench_llama_stack(eng, timer, nk=True, fused_glu=True),
            bench_llama_stack(eng, timer, nk=True, fused_glu=True, graph=True),
            bench_llama_stack(eng, timer, nk=True, fused_glu=True, graph=True, fused_qkv=True)]


def rows_layout(eng, timer) -> list:
    """Weight layout conversion (eng_transpose_f16): reference-layout A [K x N]
    to output-major W [N x K], once per weight at load time. Bytes: read and
    write every element (4 bytes per fp16 element)."""
    rng = np.random.default_rng(6)
    rows = []
    for K, N in ((4096, 4096), (4096, 11008), (11008, 4096)):
        host = rand_f16(rng, (K, N))
        count = max(2, (1 << 30) // host.nbytes + 1)
        srcs = rotating(eng, host, count)
        dst = eng.empty((N, K), np.uint16)
        st = timer.sampled(lambda i, s: eng.lib.eng_transpose_f16(srcs[i % count].ptr, dst.ptr, K, N, s))
        rows.append(hbm_row(f"transpose fp16 [{K} x {N}] -> [{N} x {K}] cold source", st, 4 * K * N))
        for d in srcs + [dst]:
            d.free()
    return rows


def rows_gemv_sweep(eng, timer) -> list:
    """Output-major fp16 GEMV (eng_gemv_f16w_nk) over a range of sizes, cold
    weights: time against bytes separates the per-launch fixed cost from the
    streaming rate inside a launch."""
    rng = np.random.default_rng(5)
    rows = []
    for N, K in ((4096, 512), (4096, 1024), (4096, 2048), (4096, 4096), (1024, 4096),
                 (2048, 4096), (8192, 4096), (16384, 4096), (32768, 4096), (65536, 4096)):
        host = rand_f16(rng, (N, K))
        count = max(2, (1 << 30) // host.nbytes + 1)
        Ws = rotating(eng, host, count)
        dx = eng.upload(rng.standard_normal(K, dtype=np.float32))
        dy = eng.empty(N, np.float32)
        st = timer.sampled(lambda i, s: eng.lib.eng_gemv_f16w_nk(Ws[i % count].ptr, dx.ptr, dy.ptr,
                                                                  N, K, s))
        rows.append(hbm_row(f"gemv_f16w_nk sweep N={N} K={K} cold", st, 2 * N * K + 4 * K + 4 * N,
                            {"N": N, "K": K}))
        for d in Ws + [dx, dy]:
            d.free()
    return rows


def rows_stack_fused(eng, timer) -> list:
    """Only the fastest config-5 arrangement (for profiling its kernels alone)."""
    return [bench_llama_stack(eng, timer, nk=True, fused_glu=True, graph=True, fused_qkv=True)]


# --no-graphs: rows that replay HIP graphs issue the same launches eagerly
# instead (rocprofv3's kernel trace crashes inside hipGraphLaunch on this
# image, so profiling runs use it).
NO_GRAPHS = False


# Groups that repeat or sweep a row for profiling; not part of the default run.
PROFILING_GROUPS = ("stackfused", "gemvsweep", "attn32k")

GROUPS = {"config2": rows_config2, "config3": rows_config3, "fewrows": rows_few_rows,
          "refapi": rows_reference_api,
          "gemm": rows_gemm, "ffn": rows_ffn, "attention": rows_attention, "stack": rows_stack,
          "layout": rows_layout,
          "stackfused": rows_stack_fused, "gemvsweep": rows_gemv_sweep,
          "attn32k": rows_attention_tinyllama_32k}


def bench_llama_stack(eng, timer, nk=False, fused_glu=False, graph=False, fused_qkv=False) -> dict:
    """Config 5: 32 layers of q,k,v,o (4096 -> 4096), gate/up (4096 -> 11008) via
    rmsnorm_linear, down (11008 -> 4096); fp16 weights, fp32 activations.
    nk=False stores every weight [in x out] (reference layout: each GEMV is a
    split-K launch and a reduce launch), nk=True [out x in].
    fused_glu=True runs gate, up and SwiGLU as one call
    (eng_rmsnorm_linear_swiglu_f16w[_nk]) and feeds SiLU(gate) * up to the down
    projection. graph=True captures one token's launches into a HIP graph
    (eng_graph_*) and times its replays. fused_qkv=True stores each layer's q, k
    and v weights as one matrix ([3H x H] output-major, [H x 3H] reference
    layout), so one GEMV call (N = 3H) yields q, k and v; same weights, bytes and
    arithmetic."""
    H, F, L = 4096, 11008, 32
    rng = np.random.default_rng(4)
    if nk:
        sq, gu, dn = rand_f16(rng, (H, H)), rand_f16(rng, (F, H)), rand_f16(rng, (H, F))
    else:
        sq, gu, dn = rand_f16(rng, (H, H)), rand_f16(rng, (H, F)), rand_f16(rng, (F, H))
    src = {"sq": eng.upload(sq), "gu": eng.upload(gu), "dn": eng.upload(dn)}
    if fused_qkv:
        # q, k, v stacked: output-major by rows, reference layout by columns
        src["qkv"] = eng.upload(np.concatenate([sq] * 3, axis=0 if nk else 1))
    layers = []
    for _ in range(L):
        lay = {}
        names = (("o", "sq"), ("gate", "gu"), ("up", "gu"), ("down", "dn"))
        if not fused_qkv:
            names = (("q", "sq"), ("k", "sq"), ("v", "sq")) + names
        for name, key in names:
            d = eng.empty(src[key].shape, np.uint16)
            eng.call("eng_memcpy_d2d", d.ptr, src[key].ptr, d.nbytes)
            lay[name] = d
        if fused_qkv:
            d = eng.empty(src["qkv"].shape, np.uint16)
            eng.call("eng_memcpy_d2d", d.ptr, src["qkv"].ptr, d.nbytes)
            lay["qkv"] = d
        layers.append(lay)
    for d in src.values():
        d.free()
    xh = eng.upload(rng.standard_normal(H, dtype=np.float32))
    g = eng.upload((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    q, k, v, o = (eng.empty(H, np.float32) for _ in range(4))
    qkv = eng.empty(3 * H, np.float32)
    gate, up = eng.empty(F, np.float32), eng.empty(F, np.float32)
    if nk:
        gv, rl = eng.lib.eng_gemv_f16w_nk, eng.lib.eng_rmsnorm_linear_f16w_nk
    else:
        gv, rl = eng.lib.eng_gemv_f16w, eng.lib.eng_rmsnorm_linear_f16w

    glu = eng.lib.eng_rmsnorm_linear_swiglu_f16w_nk if nk else eng.lib.eng_rmsnorm_linear_swiglu_f16w

    def token(_i, s):
        for lay in layers:
            if fused_qkv:
                gv(lay["qkv"].ptr, xh.ptr, qkv.ptr, 3 * H, H, s)
                vin = qkv.ptr + 2 * H * 4
            else:
                gv(lay["q"].ptr, xh.ptr, q.ptr, H, H, s)
                gv(lay["k"].ptr, xh.ptr, k.ptr, H, H, s)
                gv(lay["v"].ptr, xh.ptr, v.ptr, H, H, s)
                vin = v.ptr
            gv(lay["o"].ptr, vin, o.ptr, H, H, s)
            if fused_glu:
                glu(o.ptr, g.ptr, lay["gate"].ptr, lay["up"].ptr, gate.ptr, 1, F, H, 1e-5, s)
            else:
                rl(o.ptr, g.ptr, lay["gate"].ptr, gate.ptr, 1, F, H, 1e-5, s)
                rl(o.ptr, g.ptr, lay["up"].ptr, up.ptr, 1, F, H, 1e-5, s)
            gv(lay["down"].ptr, gate.ptr, xh.ptr, H, F, s)

    graph = graph and not NO_GRAPHS
    if graph:
        token(0, timer.stream.handle)         # eager first: capture needs nothing allocated
        timer.stream.sync()
        captured = eng.graph(timer.stream)
        with captured:
            token(0, timer.stream.handle)
        st = timer.sampled(lambda i, s: eng.lib.eng_graph_launch(captured.handle, s), samples=10)
        captured.destroy()
    else:
        st = timer.sampled(token, samples=10)
    wbytes = L * (4 * H * H + 3 * H * F) * 2
    abytes = L * (4 * (4 * H + 4 * H) + 2 * (8 * H + 4 * F) + (4 * F + 4 * H))
    for lay in layers:
        for d in lay.values():
            d.free()
    layout = "output-major W[out x in]" if nk else "reference layout W[in x out]"
    if fused_glu:
        layout += ", gate/up + SwiGLU fused"
    if fused_qkv:
        layout += ", q/k/v as one [3H x H] matrix" if nk else ", q/k/v as one [H x 3H] matrix"
    if graph:
        layout += ", replayed as one HIP graph"
    row = hbm_row(f"config 5 llama7b-shape decode linear stack, 32 layers, per token, {layout}",
                  st, wbytes + abytes)
    calls = 7 - (1 if fused_glu else 0) - (2 if fused_qkv else 0)
    row["launches_per_token"] = calls * L * (1 if nk else 2)  # reference layout: split-K + reduce
    return row


def vendor_gemm() -> int:
    """torch.matmul in fp32 (TF32 off) on the GEMM shapes of BASELINE configs 1
    and 4: the vendor library's figure beside eng_matmul_f32's. HIP events around
    10 back-to-back calls, median of 7 such windows, after 5 warm-up calls."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    for M, N, K in ((512, 512, 512), (4096, 4096, 4096), (512, 11008, 4096), (512, 4096, 11008)):
        a = torch.rand(M, K, device="cuda") * 2 - 1
        b = torch.rand(K, N, device="cuda") * 2 - 1
        for _ in range(5):
            a @ b
        torch.cuda.synchronize()
        ms = []
        for _ in range(7):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                a @ b
            e1.record()
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1) / 10)
        med = sorted(ms)[3]
        print(json.dumps({"name": f"torch.matmul fp32 {M}x{N}x{K}", "ms_per_call": round(med, 4),
                          "TFLOP/s": round(2.0 * M * N * K / (med * 1e-3) / 1e12, 2),
                          "frac_fp32_mfma_peak": round(2.0 * M * N * K / (med * 1e-3) / 1e12
                                                       / FP32_MFMA_PEAK_TFLOPS, 4)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (no secondary rows)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="issue the launches of graph-replay rows eagerly (for rocprofv3 kernel traces)")
    ap.add_argument("--only", default="", help="comma-separated secondary groups to run: "
                    + ", ".join(GROUPS) + " (default: all but the profiling groups "
                    + ", ".join(PROFILING_GROUPS) + ", which repeat or sweep single rows)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="time torch.matmul (hipBLASLt) in fp32 on the config-1/4 GEMM shapes and exit; "
                    "a comparison point only, run without loading the engine (a process that has "
                    "initialised HIP through the engine library does not see the GPU through torch)")
    args = ap.parse_args()
    if args.vendor_gemm:
        return vendor_gemm()

    global NO_GRAPHS
    NO_GRAPHS = args.no_graphs
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus}, WORLD_SIZE {world} requested): "
              "this engine has no multi-GPU path (the decode GEMVs would shard W by output rows "
              "across GPUs, one per rank, with x replicated and no exchange but an optional "
              "all-gather of y).",
              file=sys.stderr)
        return 2

    cpu = None if args.no_cpu_baseline else cpu_baseline()
    if cpu:
        log(f"cpu baseline: {cpu['value']} GB/s ({cpu['sample']})")

    pkg = load_package()
    eng = pkg.Engine()
    if eng.device_count() < 1:
        log("no GPU visible")
        return 1
    log(eng.device_summary())
    timer = Timer(eng, pkg)

    head = GemvF16w(eng, nk=True)
    nbytes = head.nbytes
    # Clocks up before the untimed warm-up and the window: past the reference's
    # 75% floor to the steady engine clock (90% of nominal, bounded), since
    # windows timed while the clock still ramps (1.8 GHz) read 6.7-7.2 us
    # where the same kernel reads 6.77 us at the steady 2.38 GHz.
    timer._warm(head, args.warmup, 200.0, max_wait_ms=1500.0, floor_frac=HEADLINE_CLOCK_FLOOR)
    ms, head_clocks = timer.run(head, args.steps, args.warmup)
    head_hold = {"hold_us": timer.last_hold_us, "issue_us": round(timer.last_issued_us, 1),
                 "queued_ahead": timer.last_issued_us <= timer.last_hold_us}
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"config 2 y=W.x, W[4096x4096] fp16 row-major, cold: {ms * 1e3:.3f} us/launch, {gbs:.1f} GB/s "
        f"{head_clocks} {head_hold}")
    spread = None if args.quick else _spread(timer.sampled(head))
    head.free()

    gemm = headline_gemm(eng, timer, args.steps, args.warmup)
    log(f"config 4 matmul_f32 4096^3: {gemm['ms_per_call']} ms/call, {gemm['TFLOP/s']} TFLOP/s")

    secondary = []
    if not args.quick:
        groups = [g for g in args.only.split(",") if g] or [g for g in GROUPS if g not in PROFILING_GROUPS]
        for g in groups:
            if g not in GROUPS:
                log(f"unknown group {g!r}; choose from {', '.join(GROUPS)}")
                return 2
            for r in GROUPS[g](eng, timer):
                log(json.dumps(r))
                secondary.append(r)

    env = environment(eng, timer)
    log(json.dumps({"environment": env}))
    line = result_line(steps=args.steps, warmup=args.warmup, ms=ms, nbytes=nbytes,
                       head_clocks=head_clocks, head_hold=head_hold, spread=spread, gemm=gemm,
                       cpu=cpu, secondary=secondary, env=env,
                       windows=(timer.windows, timer.windows_unheld))
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


def result_line(*, steps, warmup, ms, nbytes, head_clocks, head_hold, spread, gemm, cpu,
                secondary, env, windows) -> dict:
    """The one stdout JSON line: headline, roofline, the 4096^3 GEMM, the CPU
    baseline, timing and a summary of the secondary rows (which themselves
    go to stderr)."""
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy; weights ~N(0,0.02^2) fp16, x ~N(0,1) fp32), resident in HBM",
        "config": {
            "workload": ("BASELINE config 2: fp16-weight decode GEMV y=W.x, W [4096x4096] fp16 "
                         "(out x in), x/y fp32, fp32 accumulate, batch 1, seed 1, 32 rotating 32 MiB "
                         "weight buffers (cold); entry eng_gemv_f16w_nk"),
            "weight_dtype": "f16",
            "bytes_per_step": nbytes,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "kernel": HEADLINE_KERNEL,
            "event_avg_us": round(ms * 1e3, 3),
            "trace_avg_us": profiled_trace_avg_us(),
            "profile": TRAFFIC_PROFILE,
        },
        "gemm_4096": gemm,
        "cpu_baseline": cpu,
        "timing": {
            "value_from": (f"{steps} launches queued behind a {head_hold['hold_us']} us GPU-side "
                           f"hold and {Timer.LEAD} untimed ones, run back to back between two HIP "
                           f"events on the launch stream, after {warmup} warm-up"),
            "queued_ahead": head_hold["queued_ahead"],
            "clocks": head_clocks,
            "spread": spread,
        },
    }
    line["summary"] = summary(line, secondary, env, windows)
    return line


HEADLINE_GEMM_KERNEL = "eng::gemm_f32_mfma_dma_kernel<256, 128, false>"
GEMM_PROFILE = os.path.join("profiles", "gemm_f32_mfma_configs1_4.md")


def headline_gemm(eng, timer, steps: int, warmup: int) -> dict:
    """The metric's second figure: FP32 GEMM C = A.B at M = N = K = 4096
    (A, B ~ U[-1, 1], seed 3) through eng_matmul_f32, timed
    like the GEMV headline: max(steps, 10) launches back to back between two HIP
    events after a warm-up to the steady clock."""
    M = N = K = 4096
    r = np.random.default_rng(3)
    dA = eng.upload(r.uniform(-1, 1, (M, K)).astype(np.float32))
    dB = eng.upload(r.uniform(-1, 1, (K, N)).astype(np.float32))
    dC = eng.empty((M, N), np.float32)
    f = eng.lib.eng_matmul_f32

    def launch(_i, s):
        f(dA.ptr, dB.ptr, dC.ptr, M, N, K, s)

    n = max(steps, 10)
    timer._warm(launch, max(warmup, 4), 100.0, max_wait_ms=1000.0, floor_frac=HEADLINE_CLOCK_FLOOR)
    ms, clocks = timer.run(launch, n, max(warmup, 2))
    for d in (dA, dB, dC):
        d.free()
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"shape": "4096x4096x4096", "entry": "eng_matmul_f32", "ms_per_call": round(ms, 4),
            "TFLOP/s": round(tf, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "launches": n,
            "kernel": HEADLINE_GEMM_KERNEL, "profile": GEMM_PROFILE,
            "sm_clock_med_mhz": clocks.get("sm_clock_med_mhz")}


def _git_rev() -> str:
    import subprocess

    try:
        r = subprocess.run(["git", "-C", REPO, "describe", "--always", "--dirty", "--abbrev=12"],
                           capture_output=True, text=True, timeout=10)
        return r.stdout.strip() or "unavailable (no .git in this copy)"
    except (OSError, subprocess.SubprocessError):
        return "unavailable (no git)"


def environment(eng, timer) -> dict:
    """Run provenance (the reference's print_json environment block,
    bench_harness.hpp:679-710): device, driver, clocks read during the timed
    batches, peak bandwidth, source revision and build."""
    sm = sorted(timer.sm_samples)
    mem = sorted(timer.mem_samples)
    return {
        "device": eng.device_summary(),
        "arch": eng.device_arch(),
        "driver_version": eng.driver_version(),
        "nominal_sm_clock_mhz": timer.nominal_mhz,
        "live_sm_clock_mhz": {"min": sm[0], "median": sm[len(sm) // 2], "max": sm[-1],
                              "samples": len(sm)} if sm else None,
        "live_mem_clock_mhz": {"min": mem[0], "median": mem[len(mem) // 2], "max": mem[-1],
                               "samples": len(mem)} if mem else None,
        "clock_source": eng.live_clock_source(),
        "clock_floor": f"warm-up continues until the engine clock read during a batch is >= "
                       f"{CLOCK_FLOOR:.0%} of nominal (at most 500 ms; the headline window: >= 200 ms and "
                       f">= {HEADLINE_CLOCK_FLOOR:.0%}, at most 1.5 s); rows whose minimum read is below "
                       f"{CLOCK_FLOOR:.0%} carry clock_dip",
        "peak_bandwidth_gbs": eng.peak_bandwidth_gbs(),
        "build": eng.build_info(),
        "bench_git_rev": _git_rev(),
        "cpu": _cpu_model(),
    }


# (summary key, row-name prefix, field) for the compact end-of-line summary.
SUMMARY_ROWS = (
    ("cfg2_ref_layout_us", "config 2 gemv fp16-W 4096x4096 cold, reference layout", "us_per_call"),
    ("cfg3_out_major_us", "config 3 rmsnorm_linear fp16-W 1x11008x4096 cold, output-major", "us_per_call"),
    ("cfg3_out_major_frac", "config 3 rmsnorm_linear fp16-W 1x11008x4096 cold, output-major", "frac_hbm_peak"),
    ("cfg3_ref_layout_us", "config 3 rmsnorm_linear fp16-W 1x11008x4096 cold, reference layout", "us_per_call"),
    ("cfg1_gemm_512_ms", "matmul_f32 512x512x512 (config 1)", "ms_per_call"),
    ("cfg4_gemm_4096_tflops", "matmul_f32 4096x4096x4096 (config 4)", "TFLOP/s"),
    ("cfg4_gemm_4096_frac", "matmul_f32 4096x4096x4096 (config 4)", "frac_fp32_mfma_peak"),
    ("cfg4_gemm_512x11008x4096_tflops", "matmul_f32 512x11008x4096 (config 4)", "TFLOP/s"),
    ("cfg4_gemm_512x4096x11008_tflops", "matmul_f32 512x4096x11008 (config 4)", "TFLOP/s"),
    ("gemm_1024_tflops", "matmul_f32 1024x1024x1024", "TFLOP/s"),
    ("gemm_2048_tflops", "matmul_f32 2048x2048x2048", "TFLOP/s"),
    ("prefill_f16w_nk_512x11008_ms", "rmsnorm_linear_f16w 512x11008x4096 prefill, fp16 W output-major",
     "ms_per_call"),
    ("prefill_f16w_kn_512x11008_ms", "rmsnorm_linear_f16w 512x11008x4096 prefill, fp16 W reference layout",
     "ms_per_call"),
    ("ffn_prefill_512_ms", "FFN gate/up + SwiGLU 512x11008x4096 fp16-W prefill", "ms_per_call"),
    ("prefill_f16w_nk_4096x11008_tflops", "rmsnorm_linear_f16w 4096x11008x4096 prefill", "TFLOP/s"),
    ("gemv_fp32_4096_us", "gemv (fp32 W) 4096x4096 cold", "us_per_call"),
    ("gemv_fp32_12288_us", "gemv (fp32 W) 4096x12288 cold", "us_per_call"),
    ("gemv_fp16_halfio_4096_us", "gemv_fp16 (half x/out) 4096x4096 cold", "us_per_call"),
    ("gemv_fp16_halfio_12288_us", "gemv_fp16 (half x/out) 4096x12288 cold", "us_per_call"),
    ("rmsnorm_linear_f32_4096_us", "rmsnorm_linear (fp32 W) 1x4096x4096 cold", "us_per_call"),
    ("attn_tinyllama_512_us", "attention_decode TinyLlama L=512 H=32/4 D=64 cold, auto splits", "us_per_call"),
    ("attn_tinyllama_2048_us", "attention_decode TinyLlama L=2048 H=32/4 D=64 cold, auto splits", "us_per_call"),
    ("attn_tinyllama_32768_us", "attention_decode TinyLlama L=32768 H=32/4 D=64 cold, auto splits", "us_per_call"),
    ("attn_llama7b_8192_us", "attention_decode Llama-2-7B L=8192 H=32/32 D=128 cold, auto splits", "us_per_call"),
    ("attn_gqa_d128_8192_us", "attention_decode GQA-8 (Llama-3-8B layout) L=8192 H=32/8 D=128 cold, auto splits",
     "us_per_call"),
)


def summary(line: dict, secondary: list, env: dict, windows: tuple) -> dict:
    """Key figures of the run in a few hundred bytes."""
    out = {"cfg2_us": round(line["ms_per_step"] * 1e3, 3), "cfg2_frac": line["roofline"]["frac"]}
    for key, prefix, field in SUMMARY_ROWS:
        for r in secondary:
            if r.get("name", "").startswith(prefix) and field in r:
                out[key] = r[field]
                break
    stack = [r for r in secondary if r.get("name", "").startswith("config 5 ")]
    if stack:
        ref = [r for r in stack if r["name"].endswith("reference layout W[in x out]")]
        best = min(stack, key=lambda r: r["us_per_call"])
        if ref:
            out["cfg5_reference_call_sequence_ms"] = round(ref[0]["us_per_call"] / 1e3, 3)
        out["cfg5_best_ms"] = round(best["us_per_call"] / 1e3, 3)
        out["cfg5_best_frac"] = best["frac_hbm_peak"]
    if env.get("live_sm_clock_mhz"):
        out["sm_clock_mhz_min_med"] = [env["live_sm_clock_mhz"]["min"], env["live_sm_clock_mhz"]["median"]]
    dips = [r["name"] for r in secondary if r.get("clock_dip")]
    if dips:
        out["clock_dip_rows"] = len(dips)
    out["timed_windows"], out["windows_issue_outran_hold"] = windows
    out["secondary_rows"] = len(secondary)
    return out


if __name__ == "__main__":
    sys.exit(main())
