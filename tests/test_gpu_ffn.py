"""GPU parity of the FFN-side ops (vector_add, residual_rmsnorm, swiglu,
swiglu_fp16, the fused gate/up + SwiGLU) and of the SwiGLU FFN sub-block
composed through the C-ABI, against the float64 golden fixtures (reference
case tables) and the C oracle.

Tolerances, stated here and derived like those of tests/helpers.py (u = 2^-24):
* vector_add and sum_out: bit-exact (one fp32 addition).
* residual_rmsnorm: the sum of squares is an fp32 sum of `cols` terms, so the
  row scale carries (cols / 2 + 4) u relative error, plus the two multiplies.
* swiglu (fp32): exp (<= 2 ulp), add, correctly rounded divide, two
  multiplies: 8 u |y| relative, plus 2^-149 absolute below the normal range.
  Half output: add the rounding 2^-11 |y| + 2^-25.
* fused gate/up + SwiGLU: the RMSNorm+linear bounds of gate and up propagated
  through SwiGLU (|SiLU'| < 1.1), plus the fp32 SwiGLU evaluation.
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
EPS = 1e-5
U = helpers.U32


def silu64(g):
    e = np.exp(-np.abs(g))
    return g * np.where(g >= 0.0, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu_tol(y64, g=None):
    """8 u |y| + 2^-149; with the gate values, also |y| where exp(-g)
    overflows fp32 (g < -88.7: SiLU(g) = g / inf = -0, the true value is below
    1e-36) and 2^-126 for results in the subnormal range."""
    tol = 8 * U * np.abs(y64) + 2.0**-149
    if g is not None:
        g = np.asarray(g, dtype=np.float64)
        tol = tol + np.where(g < -88.0, np.abs(y64), 0.0) + 2.0**-126
    return tol


# ------------------------------------------------------------------ runners
def gpu_vector_add(eng, a, b):
    da, db, do = eng.upload(a), eng.upload(b), eng.empty(a.shape, np.float32)
    eng.call("eng_vector_add_f32", da.ptr, db.ptr, do.ptr, a.size, None)
    eng.sync()
    return do.download()


def gpu_residual_rmsnorm(eng, x, r, w, prefill=None):
    rows, cols = x.shape
    dx, dr = eng.upload(x), eng.upload(r)
    dw = eng.upload(w) if w is not None else None
    dn, ds = eng.empty(x.shape, np.float32), eng.empty(x.shape, np.float32)
    if prefill is not None:
        dn.upload(np.full(x.shape, prefill, np.float32))
        ds.upload(np.full(x.shape, prefill, np.float32))
    eng.call("eng_residual_rmsnorm_f32", dx.ptr, dr.ptr, dw.ptr if dw else None, dn.ptr, ds.ptr,
             rows, cols, EPS, None)
    eng.sync()
    return dn.download(), ds.download()


def gpu_swiglu(eng, g, u):
    fn = "eng_swiglu_f16" if g.dtype == np.uint16 else "eng_swiglu_f32"
    dg, du, do = eng.upload(g), eng.upload(u), eng.empty(g.shape, g.dtype)
    eng.call(fn, dg.ptr, du.ptr, do.ptr, g.size, None)
    eng.sync()
    return do.download()


def gpu_glu_nk(eng, x, g, Wg_nk, Wu_nk):
    M, K = x.shape
    N = Wg_nk.shape[0]
    fn = ("eng_rmsnorm_linear_swiglu_f16w_nk" if Wg_nk.dtype == np.uint16
          else "eng_rmsnorm_linear_swiglu_f32_nk")
    dx, dWg, dWu = eng.upload(x), eng.upload(Wg_nk), eng.upload(Wu_nk)
    dg = eng.upload(g) if g is not None else None
    da = eng.empty((M, N), np.float32)
    eng.call(fn, dx.ptr, dg.ptr if dg else None, dWg.ptr, dWu.ptr, da.ptr, M, N, K, EPS, None)
    eng.sync()
    return da.download()


def gpu_glu_kn(eng, x, g, Wg, Wu):
    """Reference-layout fused gate / up + SwiGLU (Wg, Wu [K x N])."""
    M, K = x.shape
    N = Wg.shape[1]
    fn = "eng_rmsnorm_linear_swiglu_f16w" if Wg.dtype == np.uint16 else "eng_rmsnorm_linear_swiglu_f32"
    dx, dWg, dWu = eng.upload(x), eng.upload(Wg), eng.upload(Wu)
    dg = eng.upload(g) if g is not None else None
    da = eng.empty((M, N), np.float32)
    eng.call(fn, dx.ptr, dg.ptr if dg else None, dWg.ptr, dWu.ptr, da.ptr, M, N, K, EPS, None)
    eng.sync()
    return da.download()


def gpu_glu_kn_composed(eng, x, g, Wg, Wu):
    """The reference's composition: rmsnorm_linear for gate and for up, then swiglu."""
    M, K = x.shape
    N = Wg.shape[1]
    fn = "eng_rmsnorm_linear_f16w" if Wg.dtype == np.uint16 else "eng_rmsnorm_linear_f32"
    outs = []
    for W in (Wg, Wu):
        dx, dW, dy = eng.upload(x), eng.upload(W), eng.empty((M, N), np.float32)
        dg = eng.upload(g) if g is not None else None
        eng.call(fn, dx.ptr, dg.ptr if dg else None, dW.ptr, dy.ptr, M, N, K, EPS, None)
        eng.sync()
        outs.append(dy.download())
    return gpu_swiglu(eng, outs[0], outs[1])


def rmsnorm_bound(y64, cols):
    return ((cols / 2.0 + 4.0) * U + 3 * U) * np.abs(y64) + 1e-30


def glu_reference(x, g, Wg, Wu):
    """float64 gate, up and act for reference-layout Wg, Wu [K x N], and the
    GPU bound (derived, statistical) on act."""
    K = x.shape[1]
    xs = helpers.rms_scale64(x) * helpers.as_f64(x) * (1.0 if g is None else helpers.as_f64(g))
    g64 = xs @ helpers.as_f64(Wg)
    u64 = xs @ helpers.as_f64(Wu)
    act64 = silu64(g64) * u64
    out = []
    for which in (0, 1):
        dg = helpers.rmsnorm_linear_bounds(x, g, Wg, g64, K)[which]
        du = helpers.rmsnorm_linear_bounds(x, g, Wu, u64, K)[which]
        silu = silu64(g64)
        out.append(1.1 * np.abs(u64) * dg + np.abs(silu) * du + dg * du + swiglu_tol(act64))
    return act64, out[0], out[1]


def check_glu(got, orc_act, act64, bd, bs, what):
    helpers.assert_within(got, act64, bd, what + " [derived bound]")
    helpers.assert_within(got, act64, bs, what + " [statistical bound]")
    # against the oracle: the GPU's bound plus the oracle's own (far smaller) error
    helpers.assert_within(got, orc_act, 2 * bd, what + " [vs oracle]")


# ----------------------------------------------------------------- vector_add
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("vector_add")])
def test_vector_add_golden_bit_exact(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_vector_add(gpu, x["a"], x["b"])
    assert np.array_equal(got, x["a"] + x["b"])


def test_vector_add_large_and_misaligned_bit_exact(gpu, orc):
    rng = np.random.default_rng(31)
    a = rng.standard_normal((1 << 20) + 3, dtype=np.float32)
    b = rng.standard_normal((1 << 20) + 3, dtype=np.float32)
    assert np.array_equal(gpu_vector_add(gpu, a, b), orc.vector_add(a, b))
    # offset pointers take the scalar path
    da, db = gpu.upload(a), gpu.upload(b)
    do = gpu.empty(a.shape, np.float32)
    n = a.size - 1
    gpu.call("eng_vector_add_f32", da.ptr + 4, db.ptr + 4, do.ptr + 4, n, None)
    gpu.sync()
    assert np.array_equal(do.download()[1:], a[1:] + b[1:])


# ------------------------------------------------------------ residual_rmsnorm
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("residual_rmsnorm")])
def test_residual_rmsnorm_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    norm, sm = gpu_residual_rmsnorm(gpu, x["x"], x["residual"], x.get("weight"), prefill=np.nan)
    assert np.array_equal(sm, x["x"] + x["residual"]), stem + " sum_out"
    exp = helpers.expected(c)
    helpers.assert_within(norm, exp, rmsnorm_bound(exp, c["params"]["cols"]), stem)


@pytest.mark.parametrize("rows,cols,weight,offset", [
    (3, 10000, True, False),   # rows longer than the register-resident part
    (300, 4096, True, False),  # more rows than one pass of workgroups per CU
    (7, 1001, True, False),    # cols % 4 != 0: scalar path
    (5, 2048, False, True),    # misaligned pointers: scalar path, null weight
])
def test_residual_rmsnorm_against_oracle(gpu, orc, rows, cols, weight, offset):
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    r = rng.standard_normal((rows, cols), dtype=np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32) if weight else None
    if offset:
        pad = lambda a: np.concatenate([[0.0], a.ravel()]).astype(np.float32)
        dx, dr = gpu.upload(pad(x)), gpu.upload(pad(r))
        dn, ds = gpu.empty(rows * cols + 1, np.float32), gpu.empty(rows * cols + 1, np.float32)
        gpu.call("eng_residual_rmsnorm_f32", dx.ptr + 4, dr.ptr + 4, None, dn.ptr + 4, ds.ptr + 4,
                 rows, cols, EPS, None)
        gpu.sync()
        norm = dn.download()[1:].reshape(rows, cols)
        sm = ds.download()[1:].reshape(rows, cols)
    else:
        norm, sm = gpu_residual_rmsnorm(gpu, x, r, w)
    on, osum = orc.residual_rmsnorm(x, r, w, EPS)
    assert np.array_equal(sm, osum)
    helpers.assert_within(norm, on, 2 * rmsnorm_bound(on, cols), f"residual_rmsnorm {rows}x{cols}")


def test_residual_rmsnorm_null_weight_equals_unit_weight(gpu):
    rng = np.random.default_rng(33)
    x = rng.standard_normal((32, 4096), dtype=np.float32)
    r = rng.standard_normal((32, 4096), dtype=np.float32)
    a = gpu_residual_rmsnorm(gpu, x, r, None)
    b = gpu_residual_rmsnorm(gpu, x, r, np.ones(4096, np.float32))
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# --------------------------------------------------------------------- swiglu
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("swiglu")])
def test_swiglu_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    exp = helpers.expected(c)
    helpers.assert_within(gpu_swiglu(gpu, x["gate"], x["up"]), exp, swiglu_tol(exp), stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("swiglu_fp16")])
def test_swiglu_fp16_matches_golden(gpu, orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    exp = helpers.expected(c)
    got = gpu_swiglu(gpu, x["gate"], x["up"])
    bound = helpers.U16 * np.abs(exp) + 2.0**-25 + swiglu_tol(exp)
    helpers.assert_within(helpers.as_f64(got), exp, bound, stem)
    # against the oracle's half result: at most one half ulp apart (the two
    # round different fp32 / double values to half)
    ref = orc.swiglu_fp16(x["gate"], x["up"])
    helpers.assert_within(helpers.as_f64(got), helpers.as_f64(ref),
                          2 * helpers.U16 * np.abs(helpers.as_f64(ref)) + 2.0**-24, stem + " vs oracle")


def test_swiglu_tails_ragged_and_misaligned(gpu, orc):
    rng = np.random.default_rng(34)
    n = 100003
    g = np.concatenate([rng.uniform(-90, 90, n - 6), [0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30]]).astype(np.float32)
    u = rng.standard_normal(n, dtype=np.float32)
    ref = orc.swiglu(g, u).astype(np.float64)
    got = gpu_swiglu(gpu, g, u)
    helpers.assert_within(got, ref, swiglu_tol(ref, g) + 2 * U * np.abs(ref), "swiglu tails (scalar path)")
    assert not np.isnan(got).any()
    dg, du = gpu.upload(g), gpu.upload(u)
    do = gpu.empty(n, np.float32)
    gpu.call("eng_swiglu_f32", dg.ptr + 4, du.ptr + 4, do.ptr + 4, n - 1, None)
    gpu.sync()
    helpers.assert_within(do.download()[1:], ref[1:], swiglu_tol(ref[1:], g[1:]) + 2 * U * np.abs(ref[1:]),
                          "swiglu misaligned")
    g16, u16 = orc.f32_to_f16(g / 8), orc.f32_to_f16(u)
    ref16 = helpers.as_f64(orc.swiglu_fp16(g16, u16))
    got16 = helpers.as_f64(gpu_swiglu(gpu, g16, u16))
    helpers.assert_within(got16, ref16, 2 * helpers.U16 * np.abs(ref16) + 2.0**-24, "swiglu_fp16 ragged")


# --------------------------------------------- fused gate/up + SwiGLU (nk)
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear_swiglu")
                                  + helpers.cases("rmsnorm_linear_swiglu_f16w")])
def test_rmsnorm_linear_swiglu_nk_matches_golden(gpu, orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    g = x.get("weight")
    Wg, Wu = x["Wg"], x["Wu"]
    got = gpu_glu_nk(gpu, x["input"], g, np.ascontiguousarray(Wg.T), np.ascontiguousarray(Wu.T))
    act64, bd, bs = glu_reference(x["input"], g, Wg, Wu)
    helpers.assert_within(act64, helpers.expected(c), 4 * U * np.abs(act64) + 1e-30, stem + " golden")
    check_glu(got, orc.rmsnorm_linear_swiglu(x["input"], g, Wg, Wu, EPS), act64, bd, bs, stem)


@pytest.mark.parametrize("M,N,K,dtype,gamma", [
    (1, 11008, 4096, "f16", True),   # BASELINE config 5 gate/up shape: fused launch
    (1, 1376, 4096, "f16", False),   # one GPU's share of it under 8-way TP; null gain
    (1, 300, 1000, "f16", True),     # ragged last piece
    (1, 257, 1024, "f32", True),     # fp32 weights: fused launch
    (1, 64, 100, "f16", True),       # K % 8 != 0: GEMV fallback with arena scratch
    (1, 64, 20000, "f16", True),     # 80 KiB of staged x: fused launch past the default LDS size
    (1, 64, 33000, "f16", True),     # K past the 128 KiB budget: GEMV fallback
    (5, 200, 512, "f16", True),      # few rows: MFMA kernel for gate and up + SwiGLU kernel
    (4, 11008, 4096, "f16", True),   # small batch at the config 5 gate/up shape
    (3, 300, 1000, "f32", False),    # small batch, fp32 weights, null gain
    (40, 200, 512, "f16", True),     # 33-64 rows of fp16 W: fp16-MFMA GEMMs on 64-row tiles
    (40, 200, 520, "f16", True),     # K % 32 != 0 past 32 rows: rmsnorm + FP32 MFMA GEMMs
    (128, 512, 256, "f16", True),    # prefill, whole tiles: direct-to-LDS GEMM with fp16 B
    (64, 256, 512, "f16", False),    # 64 rows: the 64-row fp16-MFMA tiles' largest batch
    (65, 256, 512, "f16", True),     # past it: 128-row fp16-MFMA tiles
    (65, 256, 500, "f16", True),     # K % 32 != 0: rmsnorm + FP32 MFMA GEMMs on fp16 B
    (130, 300, 200, "f32", True),    # fp32 weights past the few-row kernel: FP32 MFMA GEMMs
])
def test_rmsnorm_linear_swiglu_nk_against_oracle(gpu, orc, M, N, K, dtype, gamma):
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
    # (float32 / np.float64 scalar is float64 under NumPy 2: cast back)
    Wgf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wuf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wg, Wu = (orc.f32_to_f16(W) if dtype == "f16" else W for W in (Wgf, Wuf))
    got = gpu_glu_nk(gpu, x, g, Wg, Wu)
    Wg_kn, Wu_kn = np.ascontiguousarray(Wg.T), np.ascontiguousarray(Wu.T)
    act64, bd, bs = glu_reference(x, g, Wg_kn, Wu_kn)
    check_glu(got, orc.rmsnorm_linear_swiglu(x, g, Wg_kn, Wu_kn, EPS), act64, bd, bs,
              f"rmsnorm_linear_swiglu nk {M}x{N}x{K} {dtype}")


@pytest.mark.parametrize("M,N,K", [(1000, 2816, 1024), (300, 11008, 512), (33, 11008, 1024),
                                   (64, 2816, 512), (48, 1004, 512)])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_swiglu_prefill_fp16_mfma(gpu, orc, M, N, K, layout):
    # Prefill and batches past 32 rows with fp16 weights in either layout: the
    # rows split once into three fp16 planes, gate and up on the fp16-MFMA
    # GEMM (ragged M and N on the first shape; 258 tiles and the stream-K
    # split on the second; 64-row tiles, every tile split by K, on the 33- and
    # 64-row shapes; N = 1004 in the reference layout, N % 8 != 0, takes
    # rmsnorm and the FP32 GEMM). Eight rows of every 128-row tile against
    # every column.
    rng = np.random.default_rng(M + 3 * N + K + (layout == "kn"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wg = orc.f32_to_f16((rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32))
    Wu = orc.f32_to_f16((rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32))
    Wg_kn, Wu_kn = np.ascontiguousarray(Wg.T), np.ascontiguousarray(Wu.T)
    got = gpu_glu_nk(gpu, x, g, Wg, Wu) if layout == "nk" else gpu_glu_kn(gpu, x, g, Wg_kn, Wu_kn)
    rows = []
    for m0 in range(0, M, 128):
        last = min(m0 + 127, M - 1)
        rows += [m0, m0 + 1, min(m0 + 63, last), min(m0 + 64, last), last]
        rows += list(rng.integers(m0, last + 1, 3))
    rows = np.unique(rows)
    act64, bd, bs = glu_reference(x[rows], g, Wg_kn, Wu_kn)
    check_glu(got[rows], orc.rmsnorm_linear_swiglu(x[rows], g, Wg_kn, Wu_kn, EPS), act64, bd, bs,
              f"rmsnorm_linear_swiglu {layout} prefill {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,dtype", [(2, 11008, 4096, "f16"), (3, 1000, 2048, "f16"),
                                         (5, 4096, 4096, "f16"), (16, 11008, 4096, "f16"),
                                         (4, 512, 1024, "f32")])
def test_rmsnorm_linear_swiglu_small_batch_rows_match_single_row_calls(gpu, orc, M, N, K, dtype):
    # Up to 4 rows share each pass over Wg and Wu (fused SwiGLU epilogue), each
    # row's act equal to the M = 1 fused call bit for bit; 5 or more take the
    # few-row MFMA kernel for gate and up, each row the same bits in any batch
    # of 5 to 32 rows (fp16 weights; 5 to 64 for fp32).
    rng = np.random.default_rng(M * 13 + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wgf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wuf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wg, Wu = (orc.f32_to_f16(W) if dtype == "f16" else W for W in (Wgf, Wuf))
    got = gpu_glu_nk(gpu, x, g, Wg, Wu)
    for m in sorted({0, M // 2, M - 1}):
        one = helpers.peer_row(lambda xs: gpu_glu_nk(gpu, xs, g, Wg, Wu), x, m)
        assert np.array_equal(got[m], one), f"row {m} of {M}"
    rows = np.array(sorted({0, M - 1}))
    Wg_kn, Wu_kn = np.ascontiguousarray(Wg.T), np.ascontiguousarray(Wu.T)
    act64, bd, bs = glu_reference(x[rows], g, Wg_kn, Wu_kn)
    check_glu(got[rows], orc.rmsnorm_linear_swiglu(x[rows], g, Wg_kn, Wu_kn, EPS), act64, bd, bs,
              f"small batch glu {M}x{N}x{K} {dtype}")


def test_rmsnorm_linear_swiglu_equals_separate_calls(gpu):
    """Fused act == SwiGLU of the two RMSNorm+linear outputs, within rounding."""
    rng = np.random.default_rng(35)
    N, K = 1408, 512
    x = rng.standard_normal((1, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wg = (rng.standard_normal((N, K), dtype=np.float32) / 23).astype(np.float16).view(np.uint16)
    Wu = (rng.standard_normal((N, K), dtype=np.float32) / 23).astype(np.float16).view(np.uint16)
    fused = gpu_glu_nk(gpu, x, g, Wg, Wu)
    outs = []
    for W in (Wg, Wu):
        dx, dg, dW, dy = gpu.upload(x), gpu.upload(g), gpu.upload(W), gpu.empty((1, N), np.float32)
        gpu.call("eng_rmsnorm_linear_f16w_nk", dx.ptr, dg.ptr, dW.ptr, dy.ptr, 1, N, K, EPS, None)
        gpu.sync()
        outs.append(dy.download())
    sep = gpu_swiglu(gpu, outs[0], outs[1])
    act64, bd, _ = glu_reference(x, g, np.ascontiguousarray(Wg.T), np.ascontiguousarray(Wu.T))
    helpers.assert_within(fused, sep, 2 * bd, "fused vs separate")
    assert np.array_equal(fused, gpu_glu_nk(gpu, x, g, Wg, Wu)), "fused launch is deterministic"


# ---------------------------------- fused gate/up + SwiGLU (reference layout)
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear_swiglu")
                                  + helpers.cases("rmsnorm_linear_swiglu_f16w")])
def test_rmsnorm_linear_swiglu_kn_matches_golden(gpu, orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    g = x.get("weight")
    got = gpu_glu_kn(gpu, x["input"], g, x["Wg"], x["Wu"])
    act64, bd, bs = glu_reference(x["input"], g, x["Wg"], x["Wu"])
    check_glu(got, orc.rmsnorm_linear_swiglu(x["input"], g, x["Wg"], x["Wu"], EPS), act64, bd, bs,
              stem + " (kn)")


@pytest.mark.parametrize("M,N,K,dtype,gamma", [
    (1, 11008, 4096, "f16", True),   # config 5 gate/up shape: one launch over both matrices + reduce
    (1, 1376, 4096, "f16", False),   # null gain
    (1, 4096, 16384, "f16", True),   # long K: 64 splits
    (1, 64, 300, "f16", True),       # one column block per matrix
    (1, 257, 1024, "f32", True),     # N % 4 != 0: composition (scalar split-K kernel)
    (1, 1000, 1024, "f32", True),    # fp32 weights: fused
    (1, 36, 20, "f16", True),        # N % 8 != 0 for fp16: composition
    (3, 300, 1000, "f16", True),     # small batch: one fused pass of 3 rows
    (4, 1024, 512, "f16", False),    # one fused pass of 4 rows
    (16, 1024, 512, "f16", False),   # few rows: MFMA kernel for gate and up + SwiGLU kernel
    (6, 400, 256, "f32", True),      # few rows, fp32 weights
    (17, 256, 512, "f32", True),
    (40, 200, 512, "f16", True),     # fp16-MFMA GEMMs on 64-row tiles
    (40, 200, 520, "f16", True),     # K % 32 != 0 past 32 rows: rmsnorm + FP32 MFMA GEMMs
    (24, 200, 520, "f16", True),     # few rows (two m-blocks), K % 32 != 0
    (12, 36, 20, "f16", True),       # N % 8 != 0: GEMV passes of up to 4 rows + SwiGLU kernel
    (80, 200, 512, "f16", True),     # prefill: rmsnorm + MFMA GEMMs + SwiGLU kernel
])
def test_rmsnorm_linear_swiglu_kn_against_oracle_and_composition(gpu, orc, M, N, K, dtype, gamma):
    # Against the oracle, and bit for bit against the reference's composition
    # (two rmsnorm_linear calls and swiglu): the fused decode path sums each
    # plane exactly as rmsnorm_linear does.
    rng = np.random.default_rng(3 * M + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
    Wgf = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wuf = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    Wg, Wu = (orc.f32_to_f16(W) if dtype == "f16" else W for W in (Wgf, Wuf))
    got = gpu_glu_kn(gpu, x, g, Wg, Wu)
    rows = np.array(sorted({0, M // 2, M - 1}))
    act64, bd, bs = glu_reference(x[rows], g, Wg, Wu)
    check_glu(got[rows], orc.rmsnorm_linear_swiglu(x[rows], g, Wg, Wu, EPS), act64, bd, bs,
              f"rmsnorm_linear_swiglu kn {M}x{N}x{K} {dtype}")
    assert np.array_equal(got, gpu_glu_kn_composed(gpu, x, g, Wg, Wu)), "fused == composition"


def test_rmsnorm_linear_swiglu_kn_zero_sizes_and_contracts(gpu):
    dx = gpu.upload(np.ones((1, 64), np.float32))
    dW = gpu.upload(np.zeros((64, 64), np.uint16))
    da = gpu.empty((1, 64), np.float32)
    fn = "eng_rmsnorm_linear_swiglu_f16w"
    for M, N, K in ((0, 64, 64), (1, 0, 64), (1, 64, 0)):
        gpu.call(fn, dx.ptr, None, dW.ptr, dW.ptr, da.ptr, M, N, K, EPS, None)
    gpu.sync()
    with pytest.raises(RuntimeError, match="negative dimension"):
        gpu.call(fn, dx.ptr, None, dW.ptr, dW.ptr, da.ptr, -1, 64, 64, EPS, None)
    with pytest.raises(RuntimeError, match="null device pointer"):
        gpu.call(fn, dx.ptr, None, None, dW.ptr, da.ptr, 1, 64, 64, EPS, None)
    with pytest.raises(RuntimeError, match="eps must be non-negative"):
        gpu.call(fn, dx.ptr, None, dW.ptr, dW.ptr, da.ptr, 1, 64, 64, -1.0, None)


# ------------------------------------------------------------ FFN sub-block
def ffn_bound(x, w, Wg, Wu, Wd):
    """GPU bound on the FFN sub-block output against float64 (reference-layout weights)."""
    D = x.shape[1]
    F = Wg.shape[1]
    act64, bd, _ = glu_reference(x, w, Wg, Wu)
    wd = np.abs(helpers.as_f64(Wd))
    down64 = act64 @ helpers.as_f64(Wd)
    down_b = bd @ wd + (F * U) * (np.abs(act64) @ wd) + U * np.abs(down64)
    out64 = helpers.as_f64(x) + down64
    return out64, down_b + U * np.abs(out64)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("ffn_subblock")])
def test_ffn_subblock_reference_composition(gpu, stem):
    """The reference's GPU composition (tests/test_kernels.cu:2867-2898): rmsnorm,
    gate / up GEMV (S == 1) or GEMM, swiglu, down, vector_add -- through this
    engine's reference-API entry points."""
    c = helpers.case(stem)
    x = helpers.inputs(c)
    S, D, F = (c["params"][k] for k in ("S", "D", "F"))
    h, w = x["x"], x["ffn_rms_w"]
    dh, dw = gpu.upload(h), gpu.upload(w)
    dWg, dWu, dWd = gpu.upload(x["w_gate"]), gpu.upload(x["w_up"]), gpu.upload(x["w_down"])
    dn = gpu.empty((S, D), np.float32)
    dgate, dup, dact = (gpu.empty((S, F), np.float32) for _ in range(3))
    ddown, dout = gpu.empty((S, D), np.float32), gpu.empty((S, D), np.float32)
    gpu.call("eng_rmsnorm_f32", dh.ptr, dw.ptr, dn.ptr, S, D, EPS, None)
    if S > 1:
        gpu.call("eng_matmul_f32", dn.ptr, dWg.ptr, dgate.ptr, S, F, D, None)
        gpu.call("eng_matmul_f32", dn.ptr, dWu.ptr, dup.ptr, S, F, D, None)
    else:
        gpu.call("eng_gemv_f32", dWg.ptr, dn.ptr, dgate.ptr, F, D, None)
        gpu.call("eng_gemv_f32", dWu.ptr, dn.ptr, dup.ptr, F, D, None)
    gpu.call("eng_swiglu_f32", dgate.ptr, dup.ptr, dact.ptr, S * F, None)
    if S > 1:
        gpu.call("eng_matmul_f32", dact.ptr, dWd.ptr, ddown.ptr, S, D, F, None)
    else:
        gpu.call("eng_gemv_f32", dWd.ptr, dact.ptr, ddown.ptr, D, F, None)
    gpu.call("eng_vector_add_f32", dh.ptr, ddown.ptr, dout.ptr, S * D, None)
    gpu.sync()
    out64, bound = ffn_bound(h, w, x["w_gate"], x["w_up"], x["w_down"])
    helpers.assert_within(out64, helpers.expected(c), 4 * U * np.abs(out64) + 1e-30, stem + " golden")
    # rmsnorm writes the normalised rows in fp32 first: one more rounding per term
    helpers.assert_within(dout.download(), out64, 2 * bound, stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("ffn_subblock")])
def test_ffn_subblock_fused_composition(gpu, stem):
    """The engine's own decode FFN: fused gate/up + SwiGLU (output-major
    weights), down projection, residual add -- three launches."""
    c = helpers.case(stem)
    x = helpers.inputs(c)
    S, D, F = (c["params"][k] for k in ("S", "D", "F"))
    h, w = x["x"], x["ffn_rms_w"]
    Wg_nk, Wu_nk = np.ascontiguousarray(x["w_gate"].T), np.ascontiguousarray(x["w_up"].T)
    Wd_nk = np.ascontiguousarray(x["w_down"].T)  # [D x F]
    dh, dw = gpu.upload(h), gpu.upload(w)
    dWg, dWu, dWd = gpu.upload(Wg_nk), gpu.upload(Wu_nk), gpu.upload(Wd_nk)
    dact = gpu.empty((S, F), np.float32)
    ddown, dout = gpu.empty((S, D), np.float32), gpu.empty((S, D), np.float32)
    gpu.call("eng_rmsnorm_linear_swiglu_f32_nk", dh.ptr, dw.ptr, dWg.ptr, dWu.ptr, dact.ptr, S, F, D,
             EPS, None)
    for s in range(S):
        gpu.call("eng_gemv_f32_nk", dWd.ptr, dact.ptr + 4 * s * F, ddown.ptr + 4 * s * D, D, F, None)
    gpu.call("eng_vector_add_f32", dh.ptr, ddown.ptr, dout.ptr, S * D, None)
    gpu.sync()
    out64, bound = ffn_bound(h, w, x["w_gate"], x["w_up"], x["w_down"])
    helpers.assert_within(dout.download(), out64, bound, stem + " fused")
    helpers.assert_within(dout.download(), helpers.expected(c), bound + 2 * U * np.abs(out64),
                          stem + " fused vs golden")
