"""Benchmark of the MI355X matrix-multiply engine (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]

Headline (BASELINE config 2 as written): the fp16-weight decode GEMV
y = W . x with W [4096 x 4096] fp16 row-major (out x in), fp32 x / y, batch 1,
through eng_gemv_f16w_nk. One step is one GEMV launch over one weight matrix;
the steps are spread over 32 distinct 32 MiB weight buffers (1 GiB) so every
launch reads cold weights (the MI355X Infinity Cache holds 256 MB). `value` is
algorithmic bytes (2KN + 4K + 4N per launch) over the event-timed region, in
GB/s. All inputs are synthetic and already resident in HBM when timing starts.
The same GEMV through the reference-layout entry (eng_gemv_f16w, out = x . A
with A [in x out]) is reported in "secondary".

Also reported on the same JSON line (key "secondary"): the other BASELINE
configs -- fused RMSNorm+linear at K=4096, N=11008 (config 3), the FP32 GEMMs
(config 4), the 32-layer Llama-7B-shape decode linear stack (config 5) -- the
reference API's fp32 / half-I/O GEMVs and warm-cache rows, each with its
roofline fraction. The CPU baseline runs the scalar C oracle (a restatement
of the reference's src/cpu_ref, double accumulation) on one pinned core
before the GPU is touched.
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


HEADLINE_KERNEL = "eng::gemv::gemv_rows_kernel<_Float16, 8, 1, 4, false>"
TRAFFIC_PROFILE = os.path.join("profiles", "gemv_rows_f16w_4096x4096_cold.md")


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
def cpu_baseline(seconds: float = 10.0) -> dict:
    """The scalar oracle's fp16-weight GEMV (config 2 shape) on one core."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import helpers

    orc = helpers.oracle(0)
    rng = np.random.default_rng(1)
    K = N = 4096
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    cpus = sorted(os.sched_getaffinity(0))
    core = cpus[0]
    old = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {core})
    try:
        orc.gemv_f16w(W, x)  # warm-up
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end and len(times) < 200:
            t0 = time.perf_counter()
            orc.gemv_f16w(W, x)
            times.append(time.perf_counter() - t0)
    finally:
        os.sched_setaffinity(0, old)
    med = float(np.median(times))
    nbytes = 2 * K * N + 4 * K + 4 * N
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{len(times)} calls of the config-2 GEMV (4096x4096 fp16 W, fp32 x/y) by the "
                   f"scalar C oracle (oracle/oracle.c orc_gemv_f16w, double accumulation), pinned "
                   f"to core {core} of {len(cpus)} on '{cpu_model}'; median {med * 1e3:.1f} ms/call"),
    }


# --------------------------------------------------------------- GPU timing
class Timer:
    def __init__(self, eng, pkg):
        self.eng = eng
        self.stream = eng.stream(pkg.STREAM_NON_BLOCKING)
        self.e0 = eng.event()
        self.e1 = eng.event()

    def run(self, launch, steps: int, warmup: int) -> float:
        """Average ms per launch over `steps` back-to-back launches on one stream."""
        for i in range(warmup):
            launch(i, self.stream.handle)
        self.stream.sync()
        self.eng.sync()
        self.e0.record(self.stream)
        for i in range(steps):
            launch(warmup + i, self.stream.handle)
        self.e1.record(self.stream)
        self.e1.sync()
        self.eng.sync()
        return self.e0.elapsed_ms(self.e1) / steps


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


def hbm_row(name, ms, nbytes, extra=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    row = {"name": name, "us_per_call": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
           "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes}
    if extra:
        row.update(extra)
    return row


def gemm_row(name, ms, M, N, K):
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"name": name, "ms_per_call": round(ms, 4), "TFLOP/s": round(tf, 2),
            "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "flops_per_call": 2 * M * N * K}


def bench_gemv_f16w(eng, timer, steps, warmup, rotate=32, K=4096, N=4096, seed=1, nk=False):
    """nk=False: reference layout out = x . W[K x N] (eng_gemv_f16w);
    nk=True: y = W[N x K] . x, W row-major out x in (eng_gemv_f16w_nk)."""
    rng = np.random.default_rng(seed)
    Ws = rotating(eng, rand_f16(rng, (N, K) if nk else (K, N)), rotate)
    dx = eng.upload(rng.standard_normal(K, dtype=np.float32))
    dy = eng.empty(N, np.float32)
    fn = eng.lib.eng_gemv_f16w_nk if nk else eng.lib.eng_gemv_f16w

    def launch(i, s):
        rc = fn(Ws[i % rotate].ptr, dx.ptr, dy.ptr, N, K, s)
        if rc:
            raise RuntimeError(eng.last_error())

    ms = timer.run(launch, steps, warmup)
    for w in Ws:
        w.free()
    return ms, 2 * K * N + 4 * K + 4 * N


def secondary_rows(eng, timer) -> list:
    rows = []
    rng = np.random.default_rng(7)

    # config 2 in both weight layouts, cold, and warm (the same 32 MiB matrix
    # every call: Infinity-Cache resident, not an HBM figure).
    for nk, tag in ((False, "reference layout x.W[KxN], eng_gemv_f16w"),
                    (True, "output-major y=W[NxK].x, eng_gemv_f16w_nk")):
        ms, nb = bench_gemv_f16w(eng, timer, 640, 64, nk=nk)
        rows.append(hbm_row(f"config 2 gemv fp16-W 4096x4096 cold, {tag}", ms, nb))
        ms, nb = bench_gemv_f16w(eng, timer, 400, 50, rotate=1, nk=nk)
        rows.append(hbm_row(f"config 2 gemv fp16-W 4096x4096 WARM (cache-resident), {tag}", ms, nb))

    # config 3: fused RMSNorm + linear, fp16 W, K=4096, N=11008, cold (12 x 86 MiB).
    K, N, R = 4096, 11008, 12
    dx = eng.upload(np.random.default_rng(2).standard_normal(K, dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dy = eng.empty(N, np.float32)
    for nk, f, tag in ((False, eng.lib.eng_rmsnorm_linear_f16w, "reference layout W[KxN]"),
                       (True, eng.lib.eng_rmsnorm_linear_f16w_nk, "output-major W[NxK]")):
        Ws = rotating(eng, rand_f16(np.random.default_rng(2), (N, K) if nk else (K, N)), R)
        ms = timer.run(lambda i, s: f(dx.ptr, dg.ptr, Ws[i % R].ptr, dy.ptr, 1, N, K, 1e-5, s), 240, 24)
        rows.append(hbm_row(f"config 3 rmsnorm_linear fp16-W 1x11008x4096 cold, {tag}", ms,
                            2 * K * N + 8 * K + 4 * N))
        for w in Ws:
            w.free()

    # Reference-API GEMVs: fp32 gemv and half-I/O gemv_fp16, 4096x4096, cold.
    K = N = 4096
    R = 16
    Wf = rotating(eng, (0.02 * rng.standard_normal((K, N), dtype=np.float32)), R)
    dx = eng.upload(rng.standard_normal(K, dtype=np.float32))
    dy = eng.empty(N, np.float32)
    f = eng.lib.eng_gemv_f32
    ms = timer.run(lambda i, s: f(Wf[i % R].ptr, dx.ptr, dy.ptr, N, K, s), 160, 16)
    rows.append(hbm_row("gemv (fp32 W) 4096x4096 cold", ms, 4 * K * N + 8 * K))
    for w in Wf:
        w.free()
    Wh = rotating(eng, rand_f16(rng, (K, N)), 32)
    dxh = eng.upload(rng.standard_normal(K, dtype=np.float32).astype(np.float16).view(np.uint16))
    dyh = eng.empty(N, np.uint16)
    f = eng.lib.eng_gemv_f16
    ms = timer.run(lambda i, s: f(Wh[i % 32].ptr, dxh.ptr, dyh.ptr, N, K, s), 320, 32)
    rows.append(hbm_row("gemv_fp16 (half x/out) 4096x4096 cold", ms, 2 * K * N + 4 * K))
    for w in Wh:
        w.free()

    # config 4: FP32 GEMMs on MFMA.
    f = eng.lib.eng_matmul_f32
    for M, N, K, reps in ((4096, 4096, 4096, 20), (512, 11008, 4096, 40), (512, 4096, 11008, 40)):
        r3 = np.random.default_rng(3)
        dA = eng.upload(r3.uniform(-1, 1, (M, K)).astype(np.float32))
        dB = eng.upload(r3.uniform(-1, 1, (K, N)).astype(np.float32))
        dC = eng.empty((M, N), np.float32)
        ms = timer.run(lambda i, s: f(dA.ptr, dB.ptr, dC.ptr, M, N, K, s), reps, 3)
        rows.append(gemm_row(f"matmul_f32 {M}x{N}x{K} (config 4)", ms, M, N, K))
        dA.free(), dB.free(), dC.free()

    # Reference bench shape: rmsnorm_linear (fp32 W) at M = 512, 4096 x 4096.
    M, N, K = 512, 4096, 4096
    dA = eng.upload(rng.standard_normal((M, K), dtype=np.float32))
    dg = eng.upload((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dW = eng.upload((rng.standard_normal((K, N), dtype=np.float32) / 64).astype(np.float32))
    dC = eng.empty((M, N), np.float32)
    f = eng.lib.eng_rmsnorm_linear_f32
    ms = timer.run(lambda i, s: f(dA.ptr, dg.ptr, dW.ptr, dC.ptr, M, N, K, 1e-5, s), 40, 3)
    rows.append(gemm_row("rmsnorm_linear_f32 512x4096x4096 (fused MFMA GEMM)", ms, M, N, K))
    dA.free(), dg.free(), dW.free(), dC.free()
    return rows


def bench_llama_stack(eng, timer, tokens=10, warmup=3, nk=False) -> dict:
    """Config 5: 32 layers of q,k,v,o (4096 -> 4096), gate/up (4096 -> 11008) via
    rmsnorm_linear, down (11008 -> 4096); fp16 weights, fp32 activations.
    nk=False stores every weight [in x out] (reference layout), nk=True [out x in]."""
    H, F, L = 4096, 11008, 32
    rng = np.random.default_rng(4)
    if nk:
        sq, gu, dn = rand_f16(rng, (H, H)), rand_f16(rng, (F, H)), rand_f16(rng, (H, F))
    else:
        sq, gu, dn = rand_f16(rng, (H, H)), rand_f16(rng, (H, F)), rand_f16(rng, (F, H))
    src = {"sq": eng.upload(sq), "gu": eng.upload(gu), "dn": eng.upload(dn)}
    layers = []
    for _ in range(L):
        lay = {}
        for name, key in (("q", "sq"), ("k", "sq"), ("v", "sq"), ("o", "sq"), ("gate", "gu"),
                          ("up", "gu"), ("down", "dn")):
            d = eng.empty(src[key].shape, np.uint16)
            eng.call("eng_memcpy_d2d", d.ptr, src[key].ptr, d.nbytes)
            lay[name] = d
        layers.append(lay)
    for d in src.values():
        d.free()
    xh = eng.upload(rng.standard_normal(H, dtype=np.float32))
    g = eng.upload((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    q, k, v, o = (eng.empty(H, np.float32) for _ in range(4))
    gate, up = eng.empty(F, np.float32), eng.empty(F, np.float32)
    if nk:
        gv, rl = eng.lib.eng_gemv_f16w_nk, eng.lib.eng_rmsnorm_linear_f16w_nk
    else:
        gv, rl = eng.lib.eng_gemv_f16w, eng.lib.eng_rmsnorm_linear_f16w

    def token(_i, s):
        for lay in layers:
            gv(lay["q"].ptr, xh.ptr, q.ptr, H, H, s)
            gv(lay["k"].ptr, xh.ptr, k.ptr, H, H, s)
            gv(lay["v"].ptr, xh.ptr, v.ptr, H, H, s)
            gv(lay["o"].ptr, v.ptr, o.ptr, H, H, s)
            rl(o.ptr, g.ptr, lay["gate"].ptr, gate.ptr, 1, F, H, 1e-5, s)
            rl(o.ptr, g.ptr, lay["up"].ptr, up.ptr, 1, F, H, 1e-5, s)
            gv(lay["down"].ptr, gate.ptr, xh.ptr, H, F, s)

    t0 = time.perf_counter()
    ms = timer.run(token, tokens, warmup)
    host_ms = (time.perf_counter() - t0) * 1e3 / (tokens + warmup)
    wbytes = L * (4 * H * H + 3 * H * F) * 2
    abytes = L * (4 * (4 * H + 4 * H) + 2 * (8 * H + 4 * F) + (4 * F + 4 * H))
    for lay in layers:
        for d in lay.values():
            d.free()
    layout = "output-major W[out x in]" if nk else "reference layout W[in x out]"
    row = hbm_row(f"config 5 llama7b-shape decode linear stack, 32 layers, per token, {layout}",
                  ms, wbytes + abytes)
    row["launches_per_token"] = 7 * L
    row["host_ms_per_token"] = round(host_ms, 3)
    return row


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (no secondary rows)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus}, WORLD_SIZE {world} requested): "
              "this engine has no multi-GPU path; see DESIGN.md for how the path would shard.",
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

    ms, nbytes = bench_gemv_f16w(eng, timer, args.steps, args.warmup, nk=True)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"config 2 y=W.x, W[4096x4096] fp16 row-major, cold: {ms * 1e3:.2f} us/launch, {gbs:.1f} GB/s")

    secondary = []
    if not args.quick:
        secondary = secondary_rows(eng, timer)
        secondary.append(bench_llama_stack(eng, timer, nk=False))
        secondary.append(bench_llama_stack(eng, timer, nk=True))
        for r in secondary:
            log(json.dumps(r))

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy; weights ~N(0,0.02^2) fp16, x ~N(0,1) fp32), resident in HBM",
        "config": {
            "workload": ("BASELINE config 2: fp16-weight decode GEMV y=W.x, W [4096x4096] fp16 row-major "
                         "(out x in), x/y fp32, fp32 accumulate, batch 1, seed 1, cold weights "
                         "(32 rotating 32 MiB buffers); entry point eng_gemv_f16w_nk. The reference-"
                         "layout entry (eng_gemv_f16w, out=x.A with A [in x out]) is in 'secondary'"),
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
            "traffic_source": TRAFFIC_PROFILE + " (rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, "
                              "scaled by the counters of a 32 MiB device copy)",
            "kernel": HEADLINE_KERNEL,
            "achieved_from": "algorithmic bytes per launch / event-timed average launch duration on the launch stream",
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
        "host": platform.node(),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
