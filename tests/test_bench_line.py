"""bench.py's stdout contract, on the CPU: one compact JSON result line.

The driver reads bench.py's stdout for one JSON line carrying the headline,
`roofline` and `cpu_baseline`; a line of tens of KB (every secondary row and
the environment block inline) was not read as a result. These tests build the
line from realistic inputs (60 secondary rows, the CPU baseline with its
per-config rows) and check its size, that it round-trips through json, its
required keys, and that the roofline fraction follows from its own fields.
"""

from __future__ import annotations

import importlib.util
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MAX_LINE_BYTES = 4096


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _secondary(bench) -> list:
    rows = []
    for key, prefix, field in bench.SUMMARY_ROWS:
        rows.append({"name": prefix + " (a long descriptive suffix as the real rows carry)",
                     field: 12.345, "us_per_call": 12.345, "frac_hbm_peak": 0.6, "p25_us": 12.3,
                     "p75_us": 12.4, "iqr_pct": 0.5, "samples": 15, "batch": 120,
                     "sm_clock_min_mhz": 2400, "sm_clock_med_mhz": 2400, "mem_clock_med_mhz": 2000})
    for i in range(60 - len(rows)):
        rows.append({"name": f"config 5 llama7b-shape decode linear stack, 32 layers, per token, variant {i}",
                     "us_per_call": 2150.0 + i, "GB/s": 6000.0, "frac_hbm_peak": 0.75,
                     "bytes_per_call": 12963053568, "p25_us": 2149.0, "p75_us": 2151.0,
                     "iqr_pct": 0.1, "samples": 10, "batch": 1, "clock_dip": i == 3})
    return rows


def _cpu() -> dict:
    return {
        "value": 0.2922, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": "87 calls of the config-2 GEMV (4096x4096 fp16 W, fp32 x/y) by the scalar C oracle "
                  "(oracle/oracle.c orc_gemv_f16w, double accumulation), pinned to core 0 of 16 on "
                  "'AMD EPYC 9575F 64-Core Processor'; median 114.9 ms/call",
        "per_config": [
            {"config": 1, "what": "matmul 512^3", "ms_per_call": 240.11, "GFLOP/s": 1.118},
            {"config": 3, "what": "rmsnorm_linear fp16-W 1x11008x4096", "ms_per_call": 310.5, "GB/s": 0.29},
            {"config": 4, "what": "matmul 512x11008x4096 (4 of 512 rows timed, x128)",
             "ms_per_call": 51234.5, "GFLOP/s": 0.9},
            {"config": 5, "what": "llama7b-shape decode linear stack (1 layer timed, x32)",
             "ms_per_token": 45000.1, "GB/s": 0.288},
        ],
        "per_config_note": "configs 1, 3, 4, 5 by the same oracle on the same core; their large weight "
                           "matrices are a 1 Mi-element random block repeated to shape (timing does not "
                           "depend on the values); config 4 times 4 of 512 rows, config 5 one layer",
    }


def _line(bench):
    env = {"live_sm_clock_mhz": {"min": 2390, "median": 2400, "max": 2400, "samples": 900}}
    gemm = {"shape": "4096x4096x4096", "entry": "eng_matmul_f32", "ms_per_call": 1.0082,
            "TFLOP/s": 136.32, "peak": 157.3, "unit": "TFLOP/s", "frac": 0.8666, "launches": 20,
            "kernel": bench.HEADLINE_GEMM_KERNEL, "profile": bench.GEMM_PROFILE,
            "sm_clock_med_mhz": 2400}
    return bench.result_line(
        steps=640, warmup=64, ms=0.006781, nbytes=33587200,
        head_clocks={"sm_clock_min_mhz": 2400, "sm_clock_med_mhz": 2400, "sm_clock_max_mhz": 2400,
                     "mem_clock_med_mhz": 2000},
        head_hold={"hold_us": 3300, "issue_us": 2100.4, "queued_ahead": True},
        spread={"p25_us": 6.77, "p75_us": 6.79, "iqr_pct": 0.3, "samples": 15, "batch": 220},
        gemm=gemm, cpu=_cpu(), secondary=_secondary(bench), env=env, windows=(900, 0))


def test_result_line_is_compact_and_round_trips():
    bench = _bench()
    line = _line(bench)
    text = json.dumps(line, separators=(",", ":"))
    assert "\n" not in text
    assert len(text.encode()) <= MAX_LINE_BYTES, f"result line is {len(text)} bytes"
    assert json.loads(text) == line


def test_result_line_required_keys():
    bench = _bench()
    line = _line(bench)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline", "gemm_4096", "summary"):
        assert key in line, key
    assert "secondary" not in line and "environment" not in line
    roof = line["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in roof, key
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    for key in ("value", "unit", "cores", "kind", "sample", "per_config"):
        assert key in line["cpu_baseline"], key
    assert line["config"]["workload"]
    assert line["gemm_4096"]["unit"] == "TFLOP/s" and line["gemm_4096"]["peak"] == 157.3


def test_result_line_figures_follow_from_each_other():
    bench = _bench()
    line = _line(bench)
    ms = line["ms_per_step"]
    gbs = line["config"]["bytes_per_step"] / (ms * 1e-3) / 1e9
    assert line["value"] == pytest.approx(gbs, abs=0.06)
    assert line["roofline"]["achieved"] == line["value"]
    assert line["roofline"]["frac"] == pytest.approx(gbs / 8000.0, abs=1e-4)
    assert line["roofline"]["event_avg_us"] == pytest.approx(ms * 1e3, abs=1e-3)
    g = line["gemm_4096"]
    assert g["frac"] == pytest.approx(g["TFLOP/s"] / g["peak"], abs=1e-4)
    s = line["summary"]
    assert s["cfg2_frac"] == line["roofline"]["frac"]
    assert s["secondary_rows"] == 60 and s["clock_dip_rows"] == 1
    assert s["cfg5_best_ms"] == pytest.approx(2.15, abs=1e-3)


def test_committed_profile_feeds_the_roofline():
    """The traffic and trace figures come from the committed rocprofv3 summary
    of the headline kernel."""
    bench = _bench()
    assert bench.profiled_traffic() is not None
    avg = bench.profiled_trace_avg_us()
    assert avg is not None and 4.0 < avg < 12.0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU only" in r.stderr
