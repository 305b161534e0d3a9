"""Shared test helpers: engine/oracle loading, golden fixtures, derived tolerances.

Tolerances (stated once here, used by every parity test):

* fp32-accumulated dot product of length K against the float64 result y64,
  with a = sum_k |x_k w_k| computed in float64 (reference derivation at
  tests/test_kernels.cu:144-172; u = 2^-24):
      derived bound       |y - y64| <= K * u * a + u * |y64|
  The worst-case bound grows with K; to also catch one dropped or doubled
  term at large K, the GPU tests add a tighter statistical bound
      |y - y64| <= 16 * sqrt(K) * u * a + u * |y64|
  (rounding errors of a length-K fp32 sum of random-sign terms behave like a
  random walk, about sqrt(K) * u * a; 16x is far outside what rounding gives).
* half output: add the output rounding 2^-11 * |y64| plus 2^-25 (half of the
  smallest half subnormal).
* RMSNorm+linear: y = s * sum_k (x_k g_k) W_kn; the dot product gets the bound
  above with K + 3 terms and a = s * sum |x_k g_k W_kn|, and the fp32 row scale
  s adds (K / 2 + 4) * u * |y64| (fp32 sum of K squares, halved by the square
  root, plus the divide, root and scaling roundings).
* The C oracle accumulates in double, so against the float64 golden it must
  agree to u * |y64| + 2 * K * 2^-53 * a (output rounding plus the double sum).
"""

from __future__ import annotations

import ctypes
import importlib.util
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
GOLDEN = REPO / "tests" / "golden"
PKG_DIR = REPO / "bare-metal-llm-engine_amd"
ORACLE_DIR = REPO / "oracle"
U32 = 2.0**-24
U16 = 2.0**-11

sys.path.insert(0, str(GOLDEN))
import detgen  # noqa: E402
import engref  # noqa: E402


# ------------------------------------------------------------------ loading
def load_package():
    """Import bare-metal-llm-engine_amd (its directory name is not an identifier)."""
    name = "bare_metal_llm_engine_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def ensure_built() -> None:
    pkg = load_package()
    if not os.path.exists(pkg.LIB_PATH) or not (ORACLE_DIR / "liboracle.so").exists():
        sys.path.insert(0, str(REPO))
        import __graft_entry__

        __graft_entry__.build()


class Oracle:
    """ctypes binding of oracle/liboracle*.so (test infrastructure)."""

    def __init__(self, path: Path):
        self.path = path
        lib = ctypes.CDLL(str(path))
        p, i64, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        sig = {
            "orc_matmul": [p, p, p, i64, i64, i64],
            "orc_gemv": [p, p, p, i64, i64],
            "orc_gemv_fp16": [p, p, p, i64, i64],
            "orc_gemv_f16w": [p, p, p, i64, i64],
            "orc_rmsnorm": [p, p, p, i64, i64, f],
            "orc_rmsnorm_linear": [p, p, p, p, i64, i64, i64, f],
            "orc_rmsnorm_linear_f16w": [p, p, p, p, i64, i64, i64, f],
            "orc_f16_to_f32": [p, p, i64],
            "orc_f32_to_f16": [p, p, i64],
            "orc_vector_add": [p, p, p, i64],
            "orc_residual_rmsnorm": [p, p, p, p, p, i64, i64, f],
            "orc_swiglu": [p, p, p, i64],
            "orc_swiglu_fp16": [p, p, p, i64],
            "orc_rmsnorm_linear_swiglu": [p, p, p, p, p, i64, i64, i64, f],
            "orc_rmsnorm_linear_swiglu_f16w": [p, p, p, p, p, i64, i64, i64, f],
            "orc_ffn_subblock": [p, p, p, p, p, p, i64, i64, i64, f],
        }
        lib.orc_attention.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64, f, i64,
                                      ctypes.c_int, p]
        lib.orc_attention.restype = ctypes.c_int
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None
        lib.orc_mutation.restype = ctypes.c_int
        lib.orc_half_to_float.argtypes = [ctypes.c_uint16]
        lib.orc_half_to_float.restype = ctypes.c_float
        lib.orc_float_to_half.argtypes = [ctypes.c_float]
        lib.orc_float_to_half.restype = ctypes.c_uint16
        self.lib = lib

    @staticmethod
    def _c(a, dtype):
        return np.ascontiguousarray(a, dtype=dtype)

    def mutation(self) -> int:
        return self.lib.orc_mutation()

    def matmul(self, A, B):
        A, B = self._c(A, np.float32), self._c(B, np.float32)
        M, K = A.shape
        N = B.shape[1]
        C = np.empty((M, N), np.float32)
        self.lib.orc_matmul(A.ctypes.data, B.ctypes.data, C.ctypes.data, M, N, K)
        return C

    def gemv(self, A, x):
        A, x = self._c(A, np.float32), self._c(x, np.float32)
        K, N = A.shape
        out = np.empty(N, np.float32)
        self.lib.orc_gemv(A.ctypes.data, x.ctypes.data, out.ctypes.data, N, K)
        return out

    def gemv_fp16(self, A16, x16):
        A16, x16 = self._c(A16, np.uint16), self._c(x16, np.uint16)
        K, N = A16.shape
        out = np.empty(N, np.uint16)
        self.lib.orc_gemv_fp16(A16.ctypes.data, x16.ctypes.data, out.ctypes.data, N, K)
        return out

    def gemv_f16w(self, A16, x):
        A16, x = self._c(A16, np.uint16), self._c(x, np.float32)
        K, N = A16.shape
        out = np.empty(N, np.float32)
        self.lib.orc_gemv_f16w(A16.ctypes.data, x.ctypes.data, out.ctypes.data, N, K)
        return out

    def rmsnorm(self, x, w, eps):
        x = self._c(x, np.float32)
        rows, cols = x.shape
        out = np.empty_like(x)
        wp = None if w is None else self._c(w, np.float32)
        self.lib.orc_rmsnorm(x.ctypes.data, None if wp is None else wp.ctypes.data,
                             out.ctypes.data, rows, cols, eps)
        return out

    def rmsnorm_linear(self, x, w, W, eps):
        x = self._c(x, np.float32)
        M, K = x.shape
        half = W.dtype == np.uint16
        W = self._c(W, np.uint16 if half else np.float32)
        N = W.shape[1]
        out = np.empty((M, N), np.float32)
        wp = None if w is None else self._c(w, np.float32)
        fn = self.lib.orc_rmsnorm_linear_f16w if half else self.lib.orc_rmsnorm_linear
        fn(x.ctypes.data, None if wp is None else wp.ctypes.data, W.ctypes.data,
           out.ctypes.data, M, N, K, eps)
        return out

    @staticmethod
    def _p(a):
        return None if a is None else a.ctypes.data

    def vector_add(self, a, b):
        a, b = self._c(a, np.float32), self._c(b, np.float32)
        out = np.empty_like(a)
        self.lib.orc_vector_add(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
        return out

    def residual_rmsnorm(self, x, residual, w, eps, want_sum=True):
        """(norm_out, sum_out); residual and w may be None, want_sum=False
        passes a NULL sum_out (sum_out is then None)."""
        x = self._c(x, np.float32)
        rows, cols = x.shape
        r = None if residual is None else self._c(residual, np.float32)
        wp = None if w is None else self._c(w, np.float32)
        norm = np.empty_like(x)
        sm = np.empty_like(x) if want_sum else None
        self.lib.orc_residual_rmsnorm(x.ctypes.data, self._p(r), self._p(wp), norm.ctypes.data,
                                      self._p(sm), rows, cols, eps)
        return norm, sm

    def swiglu(self, g, u):
        g, u = self._c(g, np.float32), self._c(u, np.float32)
        out = np.empty_like(g)
        self.lib.orc_swiglu(g.ctypes.data, u.ctypes.data, out.ctypes.data, g.size)
        return out

    def swiglu_fp16(self, g16, u16):
        g16, u16 = self._c(g16, np.uint16), self._c(u16, np.uint16)
        out = np.empty_like(g16)
        self.lib.orc_swiglu_fp16(g16.ctypes.data, u16.ctypes.data, out.ctypes.data, g16.size)
        return out

    def rmsnorm_linear_swiglu(self, x, w, Wg, Wu, eps):
        """Wg, Wu [K x N] (float32, or uint16 half bits)."""
        x = self._c(x, np.float32)
        M, K = x.shape
        half = Wg.dtype == np.uint16
        dt = np.uint16 if half else np.float32
        Wg, Wu = self._c(Wg, dt), self._c(Wu, dt)
        N = Wg.shape[1]
        out = np.empty((M, N), np.float32)
        wp = None if w is None else self._c(w, np.float32)
        fn = self.lib.orc_rmsnorm_linear_swiglu_f16w if half else self.lib.orc_rmsnorm_linear_swiglu
        fn(x.ctypes.data, self._p(wp), Wg.ctypes.data, Wu.ctypes.data, out.ctypes.data, M, N, K, eps)
        return out

    def ffn_subblock(self, h, w, Wg, Wu, Wd, eps):
        h = self._c(h, np.float32)
        S, D = h.shape
        F = Wg.shape[1]
        Wg, Wu, Wd = (self._c(a, np.float32) for a in (Wg, Wu, Wd))
        wp = None if w is None else self._c(w, np.float32)
        out = np.empty_like(h)
        self.lib.orc_ffn_subblock(h.ctypes.data, self._p(wp), Wg.ctypes.data, Wu.ctypes.data,
                                  Wd.ctypes.data, out.ctypes.data, S, D, F, eps)
        return out

    def attention(self, q, k, v, n_heads, n_kv_heads, head_dim, s_kv, kv_head_stride, scale,
                  q_pos_offset=0, is_causal=False, want_lse=False):
        """Half q [s_q, H, D] and k / v (flat, kv_head_stride elements per KV
        head); returns half out [s_q, H, D] (and fp32 lse [s_q, H])."""
        q = self._c(q, np.uint16)
        k, v = self._c(k, np.uint16), self._c(v, np.uint16)
        s_q = q.size // (n_heads * head_dim)
        out = np.empty((s_q, n_heads, head_dim), np.uint16)
        lse = np.empty((s_q, n_heads), np.float32) if want_lse else None
        rc = self.lib.orc_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data,
                                    s_q, s_kv, n_heads, n_kv_heads, head_dim, kv_head_stride,
                                    scale, q_pos_offset, int(is_causal), self._p(lse))
        if rc != 0:
            raise ValueError("orc_attention: precondition failed")
        return (out, lse) if want_lse else out

    def f32_to_f16(self, a):
        a = self._c(a, np.float32)
        out = np.empty(a.shape, np.uint16)
        self.lib.orc_f32_to_f16(a.ctypes.data, out.ctypes.data, a.size)
        return out

    def f16_to_f32(self, bits):
        bits = self._c(bits, np.uint16)
        out = np.empty(bits.shape, np.float32)
        self.lib.orc_f16_to_f32(bits.ctypes.data, out.ctypes.data, bits.size)
        return out


def oracle(mutation: int = 0) -> Oracle:
    name = "liboracle.so" if mutation == 0 else f"liboracle_mut{mutation}.so"
    path = ORACLE_DIR / name
    if not path.exists():
        subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True, capture_output=True)
    return Oracle(path)


# ------------------------------------------------------------------ golden
def manifest() -> dict:
    return json.loads((GOLDEN / "manifest.json").read_text())


def cases(op: str) -> list:
    return [c for c in manifest()["cases"] if c["op"] == op]


def case(stem: str) -> dict:
    for c in manifest()["cases"]:
        if c["stem"] == stem:
            return c
    raise KeyError(stem)


def inputs(c: dict) -> dict:
    """Rebuild a case's inputs and verify them against the recorded hashes."""
    out = {}
    for name, spec in c["inputs"].items():
        arr = detgen.make(spec)
        got = detgen.digest(arr)
        if got != spec["sha256"]:
            raise AssertionError(f"{c['stem']}: input {name} regenerated with hash {got}, "
                                 f"fixture records {spec['sha256']}")
        out[name] = arr
    return out


def expected(c: dict, name: str = "expected") -> np.ndarray:
    return engref.read(GOLDEN / "data" / f"{c['stem']}.bin")[name].astype(np.float64)


def as_f64(a: np.ndarray) -> np.ndarray:
    if a.dtype == np.uint16:
        return a.view(np.float16).astype(np.float64)
    return a.astype(np.float64)


# --------------------------------------------------------------- tolerance
def absdot(x, W) -> np.ndarray:
    """sum_k |x_k W_kn| in float64 (x: [.., K], W: [K, N])."""
    return np.abs(as_f64(x)) @ np.abs(as_f64(W))


def rms_scale64(x) -> np.ndarray:
    x = as_f64(x)
    return 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-5)


def assert_within(got, exp, bound, what: str) -> float:
    """|got - exp| <= bound elementwise (NaN == NaN); returns max err/bound."""
    got = np.asarray(got, dtype=np.float64)
    exp = np.asarray(exp, dtype=np.float64)
    bound = np.broadcast_to(np.asarray(bound, dtype=np.float64), exp.shape)
    both_nan = np.isnan(got) & np.isnan(exp)
    err = np.where(both_nan, 0.0, np.abs(got - exp))
    bad = ~(err <= bound)
    if bad.any():
        idx = np.unravel_index(int(np.argmax(np.where(bad, err - bound, -np.inf))), exp.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{exp.size} elements outside the bound; first worst at "
            f"{idx}: got {got[idx]!r} expected {exp[idx]!r} err {err[idx]:.3e} bound {bound[idx]:.3e}")
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0, err / bound, 0.0)
    return float(ratio.max()) if ratio.size else 0.0


def peer_row(run, x, m):
    """Row m of run(x) recomputed in another call that must give the same bits:
    alone when x has at most 4 rows (small-batch GEMV passes: each row equals
    the single-row call), else inside a 5-row window of x (the few-row MFMA
    kernel gives a row the same bits in any batch of 5 to 32 rows of fp16
    weights, 5 to 64 of fp32)."""
    M = x.shape[0]
    if M <= 4:
        return run(x[m:m + 1])[0]
    lo = min(m, M - 5)
    return run(x[lo:lo + 5])[m - lo]


def dot_bounds(a, y64, K):
    """(derived, statistical) bounds of an fp32 dot product (see module doc)."""
    derived = K * U32 * a + U32 * np.abs(y64)
    stat = 16.0 * np.sqrt(max(K, 1)) * U32 * a + U32 * np.abs(y64)
    return derived, stat


def rmsnorm_linear_bounds(x, g, W, y64, K):
    s = rms_scale64(x)
    xs = as_f64(x) * (1.0 if g is None else as_f64(g))
    a = s * (np.abs(xs) @ np.abs(as_f64(W)))
    scale_term = (K / 2.0 + 4.0) * U32 * np.abs(y64)
    derived = (K + 3) * U32 * a + scale_term + U32 * np.abs(y64)
    stat = 16.0 * np.sqrt(K + 3) * U32 * a + scale_term + U32 * np.abs(y64)
    return derived, stat
