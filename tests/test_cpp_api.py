"""Runs the C++ drop-in API tests (tests/cpp/test_engine, built by build())."""

from __future__ import annotations

import subprocess

import pytest

import helpers

BINARY = helpers.REPO / "tests" / "cpp" / "test_engine"


def run_suite(prefix: str, timeout: int) -> None:
    if not BINARY.exists():
        helpers.ensure_built()
        subprocess.run(["make", "-C", str(BINARY.parent)], check=True, capture_output=True)
    proc = subprocess.run([str(BINARY), f"--filter={prefix}"], capture_output=True, text=True,
                          timeout=timeout)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]


def test_cpp_api_host_suites(pkg):
    run_suite("cpu_", timeout=120)


@pytest.mark.gpu
def test_cpp_api_gpu_suites(gpu):
    run_suite("gpu_", timeout=120)
