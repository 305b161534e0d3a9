"""Deterministic synthetic inputs for the golden fixtures and parity tests.

Every value comes from integer arithmetic and exact dyadic scaling, so the
same (seed, count) gives the same bits on any machine and any NumPy version:

* SplitMix64 (Steele, Lea & Flood, "Fast splittable pseudorandom number
  generators", OOPSLA 2014) produces the 64-bit stream;
* ``uniform``: the top 53 bits of a draw, scaled by 2^-53, mapped to [lo, hi);
* ``normal``: an Irwin-Hall approximation, the sum of four 24-bit uniforms
  (two per 64-bit draw) centred and scaled to unit variance. Its tails stop at
  +-2*sqrt(3), which is harmless for test data, and it needs no libm call whose
  last bit could differ between platforms.

The reference's in-test generator follows the same idea (SplitMix64 feeding a
sum of uniforms, reference tests/test_kernels.cu:2143-2162).
"""

from __future__ import annotations

import hashlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started at state `seed`."""
    with np.errstate(over="ignore"):
        state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        z = state + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """float64 values in [lo, hi)."""
    n = int(np.prod(shape, dtype=np.int64))
    u = (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0**-53)
    return (lo + (hi - lo) * u).reshape(shape)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """float64 values with the given mean and standard deviation (Irwin-Hall, 4 terms)."""
    n = int(np.prod(shape, dtype=np.int64))
    z = splitmix64(seed, 2 * n).reshape(n, 2)
    lo = (z & np.uint64(0xFFFFFFFF)) >> np.uint64(8)
    hi = z >> np.uint64(40)
    s = (lo.astype(np.float64) + hi.astype(np.float64)).sum(axis=1) * (2.0**-24)  # 4 uniforms
    unit = (s - 2.0) * np.sqrt(3.0)  # variance of the sum is 4/12
    return (mean + std * unit).reshape(shape)


def make(spec: dict) -> np.ndarray:
    """Build one input array from a manifest spec.

    spec: {"gen": "normal"|"uniform"|"zeros", "seed": int, "shape": [...],
           "mean"/"std" or "lo"/"hi", "dtype": "f32"|"f16"}
    Returns float32 for "f32" and the IEEE binary16 bit patterns (uint16) for "f16".
    """
    shape = tuple(spec["shape"])
    gen = spec["gen"]
    if gen == "normal":
        v = normal(spec["seed"], shape, spec.get("mean", 0.0), spec.get("std", 1.0))
    elif gen == "uniform":
        v = uniform(spec["seed"], shape, spec.get("lo", 0.0), spec.get("hi", 1.0))
    elif gen == "zeros":
        v = np.zeros(shape, dtype=np.float64)
    else:
        raise ValueError(f"unknown generator {gen!r}")
    if spec["dtype"] == "f32":
        return v.astype(np.float32)
    if spec["dtype"] == "f16":
        return v.astype(np.float32).astype(np.float16).view(np.uint16)
    raise ValueError(f"unknown dtype {spec['dtype']!r}")


def digest(arr: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()
