"""GPU parity of the HIP kernels, called through the C-ABI.

Tier 1: against the float64 golden fixtures (reference case tables).
Tier 2: against the C oracle at the BASELINE configs' full sizes (sampled
        rows for the 4096^3 GEMM) and on odd / misaligned shapes that take the
        fallback paths.
Properties: determinism, K == 0 / zero-size contracts, M = 1 equivalences,
fused == separate, null gain == unit gain, linearity.
Every comparison uses the derived bound and the tighter statistical bound of
tests/helpers.py.
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
EPS = 1e-5


# ------------------------------------------------------------------ runners
def gpu_matmul(eng, A, B):
    M, K = A.shape
    N = B.shape[1]
    dA, dB, dC = eng.upload(A), eng.upload(B), eng.empty((M, N), np.float32)
    eng.call("eng_matmul_f32", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    eng.sync()
    return dC.download()


def gpu_gemv(eng, A, x):
    K, N = A.shape
    half_w = A.dtype == np.uint16
    half_x = x.dtype == np.uint16
    dA, dx = eng.upload(A), eng.upload(x)
    dy = eng.empty(N, np.uint16 if half_x else np.float32)
    fn = "eng_gemv_f16" if half_x else ("eng_gemv_f16w" if half_w else "eng_gemv_f32")
    eng.call(fn, dA.ptr, dx.ptr, dy.ptr, N, K, None)
    eng.sync()
    return dy.download()


def gpu_rmsnorm(eng, x, w):
    rows, cols = x.shape
    dx, dy = eng.upload(x), eng.empty(x.shape, np.float32)
    dw = eng.upload(w) if w is not None else None
    eng.call("eng_rmsnorm_f32", dx.ptr, dw.ptr if dw else None, dy.ptr, rows, cols, EPS, None)
    eng.sync()
    return dy.download()


def gpu_rmsnorm_linear(eng, x, w, W, fn=None):
    M, K = x.shape
    N = W.shape[1]
    half_w = W.dtype == np.uint16
    fn = fn or ("eng_rmsnorm_linear_f16w" if half_w else "eng_rmsnorm_linear_f32")
    dx, dW, dy = eng.upload(x), eng.upload(W), eng.empty((M, N), np.float32)
    dw = eng.upload(w) if w is not None else None
    eng.call(fn, dx.ptr, dw.ptr if dw else None, dW.ptr, dy.ptr, M, N, K, EPS, None)
    eng.sync()
    return dy.download()


def check_dot(got, y64, a, K, what):
    derived, stat = helpers.dot_bounds(a, y64, K)
    helpers.assert_within(got, y64, derived, what + " [derived K*u bound]")
    helpers.assert_within(got, y64, stat, what + " [statistical 16*sqrt(K)*u bound]")


def check_rmsnorm_linear(got, y64, x, g, W, K, what):
    derived, stat = helpers.rmsnorm_linear_bounds(x, g, W, y64, K)
    helpers.assert_within(got, y64, derived, what + " [derived bound]")
    helpers.assert_within(got, y64, stat, what + " [statistical bound]")


# ------------------------------------------------------------- tier 1 golden
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("matmul")])
def test_matmul_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_matmul(gpu, x["A"], x["B"])
    # golden is float32-rounded: its rounding is one more u|y|
    y = helpers.expected(c)
    check_dot(got, y, helpers.absdot(x["A"], x["B"]) + np.abs(y), c["params"]["K"], stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv")])
def test_gemv_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_gemv(gpu, x["A"], x["x"])
    y = helpers.expected(c)
    check_dot(got, y, helpers.absdot(x["x"], x["A"]) + np.abs(y), c["params"]["K"], stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv_f16w")])
def test_gemv_f16w_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_gemv(gpu, x["A"], x["x"])
    y = helpers.expected(c)
    check_dot(got, y, helpers.absdot(x["x"], x["A"]) + np.abs(y), c["params"]["K"], stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv_fp16")])
def test_gemv_fp16_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = helpers.as_f64(gpu_gemv(gpu, x["A"], x["x"]))
    y = helpers.expected(c)
    K = c["params"]["K"]
    derived, _ = helpers.dot_bounds(helpers.absdot(x["x"], x["A"]) + np.abs(y), y, K)
    bound = derived + helpers.U16 * np.abs(y) + 2.0**-25
    helpers.assert_within(got, y, bound, stem + " [derived bound + half output rounding]")


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm")])
def test_rmsnorm_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_rmsnorm(gpu, x["input"], x.get("weight"))
    y = helpers.expected(c)
    cols = c["params"]["cols"]
    # fp32 sum of `cols` squares (cols*u relative, halved by the root) + divide,
    # root, two multiplies, golden rounding
    bound = (cols / 2.0 + 6) * helpers.U32 * np.abs(y) + 1e-30
    helpers.assert_within(got, y, bound, stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear")
                                  + helpers.cases("rmsnorm_linear_f16w")])
def test_rmsnorm_linear_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = gpu_rmsnorm_linear(gpu, x["input"], x.get("weight"), x["W"])
    y = helpers.expected(c)
    check_rmsnorm_linear(got, y, x["input"], x.get("weight"), x["W"], c["params"]["K"], stem)


# --------------------------------------------------- tier 2 BASELINE configs
def test_config1_matmul_512_uniform(gpu, orc):
    rng = np.random.default_rng(0)
    A = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    B = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    y = orc.matmul(A, B).astype(np.float64)
    check_dot(got, y, helpers.absdot(A, B) + np.abs(y), 512, "config 1 512^3")


def test_config2_gemv_f16w_4096(gpu, orc):
    rng = np.random.default_rng(1)
    K = N = 4096
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    got = gpu_gemv(gpu, W, x)
    y = orc.gemv_f16w(W, x).astype(np.float64)
    check_dot(got, y, helpers.absdot(x, W) + np.abs(y), K, "config 2 gemv_f16w 4096x4096")


def test_config3_rmsnorm_linear_f16w(gpu, orc):
    rng = np.random.default_rng(2)
    K, N = 4096, 11008
    x = rng.standard_normal((1, K), dtype=np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear(gpu, x, g, W)
    y = orc.rmsnorm_linear(x, g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, W, K, "config 3 rmsnorm_linear_f16w 4096x11008")


@pytest.mark.parametrize("M,N,K", [(256, 512, 1024), (96, 320, 512), (512, 1024, 2048), (480, 480, 768)])
def test_matmul_small_single_launch(gpu, orc, M, N, K):
    # At most half a round of 64 x 64 tiles (config 1's 512^3 is another):
    # one 32 x 32 tile per workgroup, its four waves splitting K and summing
    # through LDS in wave order. Every row, and the same bits on a second
    # call.
    rng = np.random.default_rng(M + 3 * N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    y = orc.matmul(A, B).astype(np.float64)
    check_dot(got, y, helpers.absdot(A, B) + np.abs(y), K, f"matmul {M}x{N}x{K}")
    assert np.array_equal(got, gpu_matmul(gpu, A, B)), "same inputs, different bits"


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (512, 11008, 4096), (512, 4096, 11008)])
def test_config4_matmul_sampled_rows(gpu, orc, M, N, K):
    rng = np.random.default_rng(3)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    rows = np.unique(np.concatenate([[0, 1, 127, 128, M - 1], rng.integers(0, M, 3)]))
    y = orc.matmul(A[rows], B).astype(np.float64)
    check_dot(got[rows], y, helpers.absdot(A[rows], B) + np.abs(y), K, f"config 4 {M}x{N}x{K} rows {rows}")
    # Column sums as a second, full-matrix property: sum_i C[i, :] = (sum_i A[i, :]) . B
    colsum = got.astype(np.float64).sum(axis=0)
    ref = A.astype(np.float64).sum(axis=0) @ B.astype(np.float64)
    bound = (K + M) * helpers.U32 * (np.abs(A).astype(np.float64).sum(axis=0) @ np.abs(B).astype(np.float64))
    helpers.assert_within(colsum, ref, bound, f"config 4 {M}x{N}x{K} column sums")


@pytest.mark.parametrize("M,N,K", [(256, 16640, 512), (384, 19200, 256), (1024, 4224, 1024)])
def test_matmul_stream_k_tail(gpu, orc, M, N, K):
    # 128 x 128 tile counts between one and two rounds of one tile per CU
    # (260, 450 and 264 tiles on 256 CUs): a data-parallel round plus the
    # remaining tiles' k-iterations split over as many workgroups, partial
    # tiles added by the fix-up kernel in workgroup order. Sampled rows of
    # every row tile against the oracle, column sums over the whole matrix,
    # and bit-equal results on a second call.
    rng = np.random.default_rng(M + N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    rows = np.unique(np.concatenate([np.arange(0, M, 64), np.arange(63, M, 64), rng.integers(0, M, 4)]))
    y = orc.matmul(A[rows], B).astype(np.float64)
    check_dot(got[rows], y, helpers.absdot(A[rows], B) + np.abs(y), K, f"stream-K {M}x{N}x{K}")
    colsum = got.astype(np.float64).sum(axis=0)
    ref = A.astype(np.float64).sum(axis=0) @ B.astype(np.float64)
    bound = (K + M) * helpers.U32 * (np.abs(A).astype(np.float64).sum(axis=0) @ np.abs(B).astype(np.float64))
    helpers.assert_within(colsum, ref, bound, f"stream-K {M}x{N}x{K} column sums")
    again = gpu_matmul(gpu, A, B)
    assert np.array_equal(again, got), "stream-K result not deterministic"


# -------------------------------------------------------- odd / fallback paths
@pytest.mark.parametrize("M,N,K", [(3, 7, 11), (65, 137, 73), (129, 257, 65), (1, 65, 127),
                                   (71, 97, 113), (2, 5, 1), (300, 8, 4), (130, 130, 33)])
def test_matmul_non_tile_multiples(gpu, orc, M, N, K):
    i = np.arange(M * K, dtype=np.float32)
    j = np.arange(K * N, dtype=np.float32)
    A = (np.sin((i + 1) * 0.1) / np.sqrt(K)).astype(np.float32).reshape(M, K)
    B = (np.cos((j + 1) * 0.1) / np.sqrt(K)).astype(np.float32).reshape(K, N)
    got = gpu_matmul(gpu, A, B)
    y = orc.matmul(A, B).astype(np.float64)
    check_dot(got, y, helpers.absdot(A, B) + np.abs(y), K, f"matmul {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(100, 300, 256), (65, 132, 512), (1, 4096, 64), (200, 64, 96),
                                   (1000, 11008, 4096), (513, 4100, 128)])
def test_matmul_ragged_tiles_take_direct_loads(gpu, orc, M, N, K):
    # K % 32 == 0, aligned, N % 4 == 0: the direct-to-LDS GEMM with clamped
    # edge loads and masked stores (M / N not multiples of the tile).
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 12).astype(int), [M - 1]]))
    y = orc.matmul(A[rows], B).astype(np.float64)
    check_dot(got[rows], y, helpers.absdot(A[rows], B) + np.abs(y), K, f"matmul {M}x{N}x{K}")


def big_tile_rows(M, rng):
    # every 64-row wave band of the first two 256-row tiles, a middle and the
    # last tile, and a few random rows
    fixed = [0, 63, 64, 127, 128, 191, 192, 255, 256, 319, 320, 383, 384, 447, 448, 511, M // 2, M - 1]
    return np.unique(np.concatenate([fixed, rng.integers(0, M, 4)]))


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 32), (2048, 4096, 64), (2048, 4096, 96),
                                   (2048, 4096, 288), (2000, 4000, 256)])
def test_matmul_256_row_tiles(gpu, orc, M, N, K):
    # 2048 x 4096 (and 4096^3) take 256 x 128 tiles: 8 waves, three LDS
    # stages, the K loop unrolled by three. 1, 2, 3 and 9 K tiles cover the
    # loop's remainders and a ring that wraps; 2000 x 4000 is the ragged form.
    rng = np.random.default_rng(M + N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    rows = big_tile_rows(M, rng)
    y = orc.matmul(A[rows], B).astype(np.float64)
    check_dot(got[rows], y, helpers.absdot(A[rows], B) + np.abs(y), K, f"matmul {M}x{N}x{K} rows {rows}")
    colsum = got.astype(np.float64).sum(axis=0)
    ref = A.astype(np.float64).sum(axis=0) @ B.astype(np.float64)
    bound = (K + M) * helpers.U32 * (np.abs(A).astype(np.float64).sum(axis=0) @ np.abs(B).astype(np.float64))
    helpers.assert_within(colsum, ref, bound, f"matmul {M}x{N}x{K} column sums")


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 256), (2000, 4000, 160)])
@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_rmsnorm_linear_256_row_tiles(gpu, orc, M, N, K, wdtype, layout):
    # The 256 x 128 tile with B given [N x K] and with fp16 B (converted as
    # fragments are read), whole and ragged.
    rng = np.random.default_rng(5 * M + N + K + (layout == "nk") + 2 * (wdtype == "f16"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    if wdtype == "f16":
        W = W.astype(np.float16).view(np.uint16)
    if layout == "kn":
        got = gpu_rmsnorm_linear(gpu, x, g, W)
    else:
        got = gpu_rmsnorm_linear_nk(gpu, x, g, np.ascontiguousarray(W.T))
    rows = big_tile_rows(M, rng)
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear {wdtype} {layout} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(100, 11008, 4096), (77, 200, 512), (3, 136, 64)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_rmsnorm_linear_f16w_ragged_tiles(gpu, orc, M, N, K, layout):
    # fp16 weights with M (and N) not multiples of the tile: the EDGE form of
    # the direct-load GEMM for both weight layouts.
    rng = np.random.default_rng(5 * M + N + K + (layout == "nk"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    if layout == "kn":
        got = gpu_rmsnorm_linear(gpu, x, g, W)
    else:
        got = gpu_rmsnorm_linear_nk(gpu, x, g, np.ascontiguousarray(W.T))
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 12).astype(int), [M - 1]]))
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear f16w {layout} {M}x{N}x{K}")


def gpu_rmsnorm_linear_f16w(eng, x, g, W, layout):
    """fp16 W given [K x N]: through the reference-layout entry point, or
    transposed through the output-major one."""
    if layout == "kn":
        return gpu_rmsnorm_linear(eng, x, g, W)
    return gpu_rmsnorm_linear_nk(eng, x, g, np.ascontiguousarray(W.T))


@pytest.mark.parametrize("M,N,K", [(65, 128, 32), (128, 128, 64), (200, 136, 96), (256, 256, 128),
                                   (130, 304, 160), (1000, 264, 224), (130, 300, 160),
                                   (130, 1000, 512), (33, 128, 32), (64, 256, 96), (48, 136, 160),
                                   (40, 300, 224), (64, 2048, 1024), (37, 1000, 512)])
@pytest.mark.parametrize("with_gamma", [True, False])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_f16w_fp16_mfma_every_row(gpu, orc, M, N, K, with_gamma, layout):
    # M >= 33, fp16 W in either layout, K % 32 == 0: the rows are split into
    # three K-blocked fp16 planes and multiplied on the fp16 matrix cores
    # ([K x N] weights through transposing LDS reads; N % 8 == 0 there, so
    # N = 300 takes the FP32 GEMM in that layout). K = 32 .. 224 is 1 to 7 K
    # steps (every remainder of the four-stage ring of the 128-row tiles and
    # of the three-stage ring of the 64-row tiles that take 33-64 rows), M
    # and N whole and ragged; 130 x 1000 x 512 (16 tiles, fewer than the
    # CUs), 64 x 2048 x 1024 and 37 x 1000 x 512 split every tile by K.
    # Every row is checked.
    rng = np.random.default_rng(13 * M + N + K + with_gamma + (layout == "kn"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if with_gamma else None
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_f16w(gpu, x, g, W, layout)
    y = orc.rmsnorm_linear(x, g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, W, K, f"rmsnorm_linear f16w {layout} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(300, 12760, 256), (384, 11008, 256), (1000, 4104, 384),
                                   (1000, 9000, 256), (2000, 8296, 256), (2000, 8296, 96),
                                   (2000, 8296, 64), (2048, 8448, 256), (2048, 8192, 64)])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_f16w_fp16_mfma_stream_k(gpu, orc, M, N, K, layout):
    # Tile counts past one round of one tile per CU (256 on MI355X): whole
    # rounds data-parallel, the last round's tiles split over the CUs by K
    # tile and added by the fix-up pass. 128 x 128 tiles: 300, 258 and 264
    # (ragged M and N on the first and third shapes; on the second, 2 tail
    # tiles split into 8-K-tile pieces). 128 x 256 tiles: 1000 x 9000, 288 of
    # them, the last 32 split; 2000 x 8296, 528 tiles ragged both ways, splits
    # the last 16 after two whole rounds at K = 256 and runs unsplit through
    # the three-stage ring's remainders at 3 and 2 K steps; 2048 x 8448 and
    # 2048 x 8192 are the whole-tile forms, split and not.
    # Both weight layouts. Eight rows of every 128-row tile (its edges and
    # random ones) against every column, so every tile is checked.
    rng = np.random.default_rng(17 * M + N + K + (layout == "kn"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_f16w(gpu, x, g, W, layout)
    rows = []
    for m0 in range(0, M, 128):
        last = min(m0 + 127, M - 1)
        rows += [m0, m0 + 1, min(m0 + 63, last), min(m0 + 64, last), last]
        rows += list(rng.integers(m0, last + 1, 3))
    rows = np.unique(rows)
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear f16w {layout} stream-K {M}x{N}x{K}")


@pytest.mark.parametrize("case", ["k_not_32", "kn_n_not_8", "misaligned_x"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_f16w_prefill_fallbacks(gpu, orc, case, layout):
    # Prefill calls the fp16-MFMA path does not take run RMSNorm into fp32
    # scratch and the FP32 MFMA GEMM on converted weights: K % 32 != 0, a
    # reference-layout N % 8 != 0, and activations not 16-byte aligned.
    M, N, K = {"k_not_32": (100, 300, 200), "kn_n_not_8": (100, 302, 256),
               "misaligned_x": (130, 256, 256)}[case]
    rng = np.random.default_rng(M + N + K + (layout == "kn"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    if case == "misaligned_x":
        Wd = gpu.upload(W if layout == "kn" else np.ascontiguousarray(W.T))
        dxb = gpu.upload(np.concatenate([[0.0], x.reshape(-1)]).astype(np.float32))
        dg, dy = gpu.upload(g), gpu.empty((M, N), np.float32)
        fn = "eng_rmsnorm_linear_f16w" if layout == "kn" else "eng_rmsnorm_linear_f16w_nk"
        gpu.call(fn, dxb.ptr + 4, dg.ptr, Wd.ptr, dy.ptr, M, N, K, EPS, None)
        gpu.sync()
        got = dy.download()
    else:
        got = gpu_rmsnorm_linear_f16w(gpu, x, g, W, layout)
    y = orc.rmsnorm_linear(x, g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, W, K, f"rmsnorm_linear f16w {layout} {case} {M}x{N}x{K}")


@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_f16w_fp16_mfma_long_prompt(gpu, orc, layout):
    # 4096 x 11008 x 4096 (a 4096-token prompt at the FFN width): 128 x 256
    # tiles, 1376 of them, the last 96 split by K. Sampled rows of every
    # 1024-row quarter against the oracle, and the column sums of all rows
    # against float64: sum_r y[r] = (sum_r xn[r]) . W with xn the normalised
    # rows.
    M, N, K = 4096, 11008, 4096
    rng = np.random.default_rng(4096 + (layout == "kn"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_f16w(gpu, x, g, W, layout)
    rows = np.unique(np.concatenate([[0, 128, 1023, 2048, M - 1], rng.integers(0, M, 2)]))
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear f16w {layout} {M}x{N}x{K}")
    W64 = helpers.as_f64(W)
    xn = helpers.rms_scale64(x) * helpers.as_f64(x) * helpers.as_f64(g)
    colsum = got.astype(np.float64).sum(axis=0)
    ref = xn.sum(axis=0) @ W64
    bound = (K + M + 8) * helpers.U32 * (np.abs(xn).sum(axis=0) @ np.abs(W64))
    helpers.assert_within(colsum, ref, bound, f"rmsnorm_linear f16w {layout} {M}x{N}x{K} column sums")


@pytest.mark.parametrize("gscale", [1e-30, 1e-3, 1.0, 1e25])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_rmsnorm_linear_f16w_fp16_mfma_row_scales(gpu, orc, gscale, layout):
    # The planes hold each row times its own power of two (row maximum moved
    # into [2^14, 2^15)): gamma far below and above fp16's range keeps the
    # FP32 bound, rows of very different size share a tile, and an all-zero
    # row stays exactly zero.
    M, N, K = 96, 160, 256
    rng = np.random.default_rng(int(np.log10(gscale)) + 40)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[::7] *= np.float32(1e-6)   # eps-dominated: normalised rows ~3e-4 of the others
    x[3::7] *= np.float32(1e15)
    x[5] = 0.0
    x[40] = 0.0
    g = (gscale * (1 + 0.1 * rng.standard_normal(K))).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_f16w(gpu, x, g, W, layout)
    assert np.all(got[5] == 0.0) and np.all(got[40] == 0.0)
    y = orc.rmsnorm_linear(x, g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, W, K, f"rmsnorm_linear f16w {layout} row scales, gamma x {gscale:g}")


@pytest.mark.parametrize("N,K,dtype", [(127, 31, "f32"), (73, 125, "f16w"), (4100, 4096, "f16w"),
                                       (11008, 4096, "f32"), (8, 20000, "f16w"), (1, 1, "f32"),
                                       (3000, 7, "f16"), (64, 1, "f16w")])
def test_gemv_shapes_against_oracle(gpu, orc, N, K, dtype):
    rng = np.random.default_rng(N * 7 + K)
    A = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal(K, dtype=np.float32)
    if dtype == "f32":
        got, y = gpu_gemv(gpu, A, x), orc.gemv(A, x)
        check_dot(got, y.astype(np.float64), helpers.absdot(x, A) + np.abs(y), K, f"gemv {N}x{K}")
    elif dtype == "f16w":
        A16 = orc.f32_to_f16(A)
        got, y = gpu_gemv(gpu, A16, x), orc.gemv_f16w(A16, x)
        check_dot(got, y.astype(np.float64), helpers.absdot(x, A16) + np.abs(y), K, f"gemv_f16w {N}x{K}")
    else:
        A16, x16 = orc.f32_to_f16(A), orc.f32_to_f16(x)
        got = helpers.as_f64(gpu_gemv(gpu, A16, x16))
        y = helpers.as_f64(x16) @ helpers.as_f64(A16)
        derived, _ = helpers.dot_bounds(helpers.absdot(x16, A16), y, K)
        helpers.assert_within(got, y, derived + helpers.U16 * np.abs(y) + 2.0**-25, f"gemv_fp16 {N}x{K}")


@pytest.mark.parametrize("N,K,dtype", [(64, 16384, "f16w"), (300, 16384, "f32"), (4100, 4096, "f16w"),
                                       (11008, 96, "f16w")])
def test_rmsnorm_linear_split_k_reduce_regimes(gpu, orc, N, K, dtype):
    # Reference-layout decode: the split count ranges from 256 (N = 64: every
    # reduce wave sums four groups of 8 partials, wave 0 folds four sums of
    # squares per lane) down to 2 (K = 96); rows of a 3-row batch equal the
    # single-row calls bit for bit whatever the split count.
    rng = np.random.default_rng(N + 5 * K)
    x = rng.standard_normal((3, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    if dtype == "f16w":
        W = orc.f32_to_f16(W)
    one = gpu_rmsnorm_linear(gpu, x[:1], g, W)
    y = orc.rmsnorm_linear(x[:1], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(one, y, x[:1], g, W, K, f"rmsnorm_linear kn {N}x{K} {dtype}")
    three = gpu_rmsnorm_linear(gpu, x, g, W)
    for m in range(3):
        assert np.array_equal(three[m], gpu_rmsnorm_linear(gpu, x[m:m + 1], g, W)[0]), f"row {m}"


def test_misaligned_pointers_take_the_scalar_path(gpu, orc):
    """A weight pointer off 16-byte alignment must still give the right answer."""
    rng = np.random.default_rng(12)
    K, N = 512, 1024
    A = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal(K, dtype=np.float32)
    dbig = gpu.upload(np.concatenate([[0.0], A.ravel()]).astype(np.float32))
    dx, dy = gpu.upload(x), gpu.empty(N, np.float32)
    gpu.call("eng_gemv_f32", dbig.ptr + 4, dx.ptr, dy.ptr, N, K, None)
    gpu.sync()
    y = orc.gemv(A, x).astype(np.float64)
    check_dot(dy.download(), y, helpers.absdot(x, A) + np.abs(y), K, "misaligned gemv")
    Ab = np.concatenate([[0.0], A.ravel()]).astype(np.float32)
    B = (rng.standard_normal((K, 96)) / np.sqrt(K)).astype(np.float32)
    dA, dB, dC = gpu.upload(Ab), gpu.upload(B), gpu.empty((K // 2, 96), np.float32)
    gpu.call("eng_matmul_f32", dA.ptr + 4, dB.ptr, dC.ptr, K // 2, 96, K, None)
    gpu.sync()
    Am = A.ravel()[: (K // 2) * K].reshape(K // 2, K)
    y = orc.matmul(Am, B).astype(np.float64)
    check_dot(dC.download(), y, helpers.absdot(Am, B) + np.abs(y), K, "misaligned matmul")


# ------------------------------------------------------------------ properties
def test_results_are_deterministic(gpu):
    rng = np.random.default_rng(13)
    K, N = 4096, 11008
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((1, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    a = gpu_rmsnorm_linear(gpu, x, g, W)
    b = gpu_rmsnorm_linear(gpu, x, g, W)
    assert np.array_equal(a, b)
    A = rng.uniform(-1, 1, (700, 900)).astype(np.float32)
    B = rng.uniform(-1, 1, (900, 600)).astype(np.float32)
    assert np.array_equal(gpu_matmul(gpu, A, B), gpu_matmul(gpu, A, B))


def test_matmul_m1_is_gemv_bit_exact(gpu):
    rng = np.random.default_rng(14)
    A = rng.standard_normal((2048, 3000), dtype=np.float32)
    x = rng.standard_normal(2048, dtype=np.float32)
    assert np.array_equal(gpu_matmul(gpu, x[None, :], A)[0], gpu_gemv(gpu, A, x))


def test_gemv_is_linear_in_x(gpu):
    rng = np.random.default_rng(15)
    K, N = 4096, 4096
    W = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x1 = rng.standard_normal(K, dtype=np.float32)
    x2 = rng.standard_normal(K, dtype=np.float32)
    y1, y2, y12 = gpu_gemv(gpu, W, x1), gpu_gemv(gpu, W, x2), gpu_gemv(gpu, W, x1 + x2)
    a = helpers.absdot(np.abs(x1) + np.abs(x2), W)
    helpers.assert_within(y12, y1.astype(np.float64) + y2, 2 * 16 * np.sqrt(K) * helpers.U32 * a,
                          "gemv(x1 + x2) = gemv(x1) + gemv(x2)")
    assert np.all(gpu_gemv(gpu, W, np.zeros(K, np.float32)) == 0.0)


def test_rmsnorm_linear_fused_equals_separate(gpu):
    rng = np.random.default_rng(16)
    for M in (1, 32, 80):
        x = rng.standard_normal((M, 512), dtype=np.float32)
        g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
        W = (rng.standard_normal((512, 256)) / np.sqrt(512)).astype(np.float32)
        fused = gpu_rmsnorm_linear(gpu, x, g, W)
        sep = gpu_matmul(gpu, gpu_rmsnorm(gpu, x, g), W) if M > 1 else gpu_gemv(gpu, W, gpu_rmsnorm(gpu, x, g)[0])[None]
        y = helpers.rms_scale64(x) * helpers.as_f64(x) * g @ W.astype(np.float64)
        check_rmsnorm_linear(fused, y, x, g, W, 512, f"fused M={M}")
        check_rmsnorm_linear(sep, y, x, g, W, 512, f"separate M={M}")
        direct = gpu_rmsnorm_linear(gpu, x, g, W, fn="eng_rmsnorm_linear_fused_direct_f32")
        assert np.array_equal(direct, fused)
        if M > 64:
            # past the few-row kernel (M <= 64, RMS scale applied after its
            # sums): rmsnorm into scratch, then the GEMM -- the same launches.
            assert np.array_equal(fused, sep)


def test_rmsnorm_linear_null_weight_equals_unit_weight(gpu):
    rng = np.random.default_rng(17)
    for M in (1, 32):
        x = rng.standard_normal((M, 512), dtype=np.float32)
        W = (rng.standard_normal((512, 256)) / np.sqrt(512)).astype(np.float32)
        assert np.array_equal(gpu_rmsnorm_linear(gpu, x, None, W),
                              gpu_rmsnorm_linear(gpu, x, np.ones(512, np.float32), W))


def test_rmsnorm_zero_row_is_zero(gpu):
    assert np.all(gpu_rmsnorm(gpu, np.zeros((2, 256), np.float32), None) == 0.0)
    W = np.ones((256, 64), np.float32)
    assert np.all(gpu_rmsnorm_linear(gpu, np.zeros((1, 256), np.float32), None, W) == 0.0)
    assert np.all(gpu_rmsnorm_linear(gpu, np.zeros((3, 256), np.float32), None, W) == 0.0)


# ---------------------------------------------------------------- contracts
def test_k_zero_zero_fills_and_empty_is_untouched(gpu):
    poison = np.full(12, 7.0, np.float32)
    d1 = gpu.upload(np.zeros(4, np.float32))
    for fn, args in (("eng_matmul_f32", (4, 3, 0)), ("eng_gemv_f32", (12, 0)), ("eng_gemv_f16w", (12, 0))):
        dy = gpu.upload(poison)
        gpu.call(fn, d1.ptr, d1.ptr, dy.ptr, *args, None)
        gpu.sync()
        assert np.all(dy.download() == 0.0), fn
    dh = gpu.upload(np.full(13, 0x4700, np.uint16))  # 7.0 in half
    gpu.call("eng_gemv_f16", d1.ptr, d1.ptr, dh.ptr, 13, 0, None)
    gpu.sync()
    assert np.all(dh.download() == 0)
    # rmsnorm_linear with any zero dimension, and N == 0 GEMVs, write nothing.
    dy = gpu.upload(poison)
    gpu.call("eng_rmsnorm_linear_f32", d1.ptr, None, d1.ptr, dy.ptr, 4, 3, 0, EPS, None)
    gpu.call("eng_gemv_f32", d1.ptr, d1.ptr, dy.ptr, 0, 5, None)
    gpu.call("eng_matmul_f32", d1.ptr, d1.ptr, dy.ptr, 0, 3, 5, None)
    gpu.sync()
    assert np.all(dy.download() == 7.0)


def test_split_k_workspace_survives_shape_changes_and_streams(gpu, orc):
    """Many GEMVs of varying shape on two streams share per-stream scratch arenas."""
    rng = np.random.default_rng(18)
    shapes = [(4096, 4096), (11008, 4096), (4096, 11008), (64, 8192), (1000, 3000)]
    cases = []
    for N, K in shapes:
        A = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
        x = rng.standard_normal(K, dtype=np.float32)
        cases.append((N, K, A, x, gpu.upload(A), gpu.upload(x), gpu.empty(N, np.float32)))
    streams = [gpu.stream(), gpu.stream()]
    try:
        for rep in range(3):
            for i, (N, K, _, _, dA, dx, dy) in enumerate(cases):
                gpu.call("eng_gemv_f16w", dA.ptr, dx.ptr, dy.ptr, N, K, streams[(i + rep) % 2].handle)
        for s in streams:
            s.sync()
        for N, K, A, x, _, _, dy in cases:
            y = orc.gemv_f16w(A, x).astype(np.float64)
            check_dot(dy.download(), y, helpers.absdot(x, A) + np.abs(y), K, f"stream gemv {N}x{K}")
    finally:
        for s in streams:
            s.destroy()


def test_scratch_arena_with_threads_sharing_one_stream(gpu, orc):
    """Split-K GEMVs from four host threads on ONE stream. Each call's partial
    and reduce kernels hold the stream's scratch arena while they are queued,
    so no call's reduce can read another call's partials; the shapes differ so
    the arena also grows while other threads wait for it."""
    import threading
    rng = np.random.default_rng(19)
    shapes = [(64, 8192), (1000, 3000), (512, 11008), (2048, 16384)]
    cases = []
    for N, K in shapes:
        A = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
        x = rng.standard_normal(K, dtype=np.float32)
        cases.append((N, K, A, x, gpu.upload(A), gpu.upload(x), gpu.empty(N, np.float32)))
    s = gpu.stream()
    errors = []

    def worker(case):
        N, K, _, _, dA, dx, dy = case
        try:
            for _ in range(25):
                gpu.call("eng_gemv_f16w", dA.ptr, dx.ptr, dy.ptr, N, K, s.handle)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    try:
        threads = [threading.Thread(target=worker, args=(c,)) for c in cases]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        s.sync()
        assert not errors, errors
        for N, K, A, x, _, _, dy in cases:
            y = orc.gemv_f16w(A, x).astype(np.float64)
            check_dot(dy.download(), y, helpers.absdot(x, A) + np.abs(y), K, f"threaded gemv {N}x{K}")
    finally:
        s.destroy()


# ------------------------------------------------- output-major ([N x K]) path
def gpu_gemv_nk(eng, W, x):
    N, K = W.shape
    dW, dx, dy = eng.upload(W), eng.upload(x), eng.empty(N, np.float32)
    fn = "eng_gemv_f16w_nk" if W.dtype == np.uint16 else "eng_gemv_f32_nk"
    eng.call(fn, dW.ptr, dx.ptr, dy.ptr, N, K, None)
    eng.sync()
    return dy.download()


def gpu_rmsnorm_linear_nk(eng, x, g, W):
    M, K = x.shape
    N = W.shape[0]
    fn = "eng_rmsnorm_linear_f16w_nk" if W.dtype == np.uint16 else "eng_rmsnorm_linear_f32_nk"
    dx, dW, dy = eng.upload(x), eng.upload(W), eng.empty((M, N), np.float32)
    dg = eng.upload(g) if g is not None else None
    eng.call(fn, dx.ptr, dg.ptr if dg else None, dW.ptr, dy.ptr, M, N, K, EPS, None)
    eng.sync()
    return dy.download()


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv_f16w")])
def test_gemv_f16w_nk_matches_golden(gpu, stem):
    """The golden's A is [K x N]; its transpose is the output-major W."""
    c = helpers.case(stem)
    x = helpers.inputs(c)
    W = np.ascontiguousarray(x["A"].T)
    got = gpu_gemv_nk(gpu, W, x["x"])
    y = helpers.expected(c)
    check_dot(got, y, helpers.absdot(x["x"], x["A"]) + np.abs(y), c["params"]["K"], stem + " (nk)")


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear_f16w")
                                  + helpers.cases("rmsnorm_linear")])
def test_rmsnorm_linear_nk_matches_golden(gpu, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    W = np.ascontiguousarray(x["W"].T)
    got = gpu_rmsnorm_linear_nk(gpu, x["input"], x.get("weight"), W)
    y = helpers.expected(c)
    check_rmsnorm_linear(got, y, x["input"], x.get("weight"), x["W"], c["params"]["K"], stem + " (nk)")


def test_config2_gemv_f16w_nk_4096(gpu, orc):
    """BASELINE config 2 as written: y = W.x, W [4096 x 4096] fp16 row-major."""
    rng = np.random.default_rng(1)
    N = K = 4096
    W = (0.02 * rng.standard_normal((N, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    got = gpu_gemv_nk(gpu, W, x)
    Wt = np.ascontiguousarray(W.T)
    y = orc.gemv_f16w(Wt, x).astype(np.float64)
    check_dot(got, y, helpers.absdot(x, Wt) + np.abs(y), K, "config 2 nk")


def test_config3_rmsnorm_linear_f16w_nk(gpu, orc):
    """BASELINE config 3 as written: W [11008 x 4096] fp16 row-major."""
    rng = np.random.default_rng(2)
    N, K = 11008, 4096
    x = rng.standard_normal((1, K), dtype=np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((N, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_nk(gpu, x, g, W)
    Wt = np.ascontiguousarray(W.T)
    y = orc.rmsnorm_linear(x, g, Wt, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, Wt, K, "config 3 nk")


@pytest.mark.parametrize("N,K,dtype", [(4096, 11008, "f16"), (7, 13, "f16"), (33, 1000, "f32"),
                                       (4097, 4096, "f16"), (1, 8, "f16"), (300, 4100, "f32")])
def test_gemv_nk_shapes_against_oracle(gpu, orc, N, K, dtype):
    rng = np.random.default_rng(N + 3 * K)
    Wf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal(K, dtype=np.float32)
    W = orc.f32_to_f16(Wf) if dtype == "f16" else Wf
    got = gpu_gemv_nk(gpu, W, x)
    Wt = np.ascontiguousarray(W.T)
    y = (orc.gemv_f16w(Wt, x) if dtype == "f16" else orc.gemv(Wt, x)).astype(np.float64)
    check_dot(got, y, helpers.absdot(x, Wt) + np.abs(y), K, f"gemv nk {N}x{K} {dtype}")


@pytest.mark.parametrize("N,K,rms,gamma", [
    (5, 8, True, True),          # K below one 512-element piece
    (333, 1000, True, True),     # ragged last piece, N not a multiple of 4 rows
    (333, 1000, True, False),    # null gain
    (4099, 520, True, True),     # N beyond one resident round, odd N: last 16-wave workgroup partly idle
    (64, 16384, True, True),     # largest K whose staged vector fits the default 64 KiB of LDS
    (64, 16392, True, True),     # just past it: LDS allowed up to 128 KiB
    (300, 8200, False, False),   # K > 4096 without RMSNorm: LDS-staged, 16 loads per row in flight
    (5000, 1000, False, False),  # many rows, small K: LDS-staged, 4 loads per row in flight
    (64, 20000, False, False),   # 80 KiB of staged x
    (96, 32768, True, True),     # largest K whose staged vector fits 128 KiB
    (64, 32776, True, False),    # just past it: register kernel fallback
    (64, 40000, False, False),   # register kernel, 4 loads in flight
])
def test_nk_fp16_kernel_selection_against_oracle(gpu, orc, N, K, rms, gamma):
    """Every output-major fp16 launch variant (LDS-staged x, register x,
    fallbacks) against the oracle at the shapes that select it."""
    rng = np.random.default_rng(7 * N + K)
    W = orc.f32_to_f16(rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K))
    Wt = np.ascontiguousarray(W.T)
    if rms:
        x = rng.standard_normal((1, K), dtype=np.float32)
        g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
        got = gpu_rmsnorm_linear_nk(gpu, x, g, W)
        y = orc.rmsnorm_linear(x, g, Wt, EPS).astype(np.float64)
        check_rmsnorm_linear(got, y, x, g, Wt, K, f"rmsnorm_linear nk {N}x{K}")
    else:
        x = rng.standard_normal(K, dtype=np.float32)
        got = gpu_gemv_nk(gpu, W, x)
        y = orc.gemv_f16w(Wt, x).astype(np.float64)
        check_dot(got, y, helpers.absdot(x, Wt) + np.abs(y), K, f"gemv nk {N}x{K}")


@pytest.mark.parametrize("N,K,gamma", [
    (8193, 4096, True),    # one row past one resident round of 16-wave workgroups (256 CUs)
    (9000, 2048, True),    # ring of 4 pieces; some waves with one row, some with two
    (8200, 4096, False),   # null gain
    (16389, 4096, True),   # three rows for a few waves, N not a multiple of 16
])
def test_rmsnorm_linear_nk_persistent_grid(gpu, orc, N, K, gamma):
    """Fixed-K RMSNorm GEMV past one resident round (the persistent grid whose
    waves stream a second and third row through their ring) against the
    oracle, and each row equal bit for bit to the 2-row kernel's first row
    (the staged kernels' arithmetic)."""
    rng = np.random.default_rng(N + K)
    W = orc.f32_to_f16(rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K))
    Wt = np.ascontiguousarray(W.T)
    x2 = rng.standard_normal((2, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
    got = gpu_rmsnorm_linear_nk(gpu, x2[:1], g, W)
    y = orc.rmsnorm_linear(x2[:1], g, Wt, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x2[:1], g, Wt, K, f"rmsnorm_linear nk persistent {N}x{K}")
    two = gpu_rmsnorm_linear_nk(gpu, x2, g, W)
    assert np.array_equal(np.asarray(got, np.float32).reshape(-1).view(np.uint32),
                          np.asarray(two[0], np.float32).reshape(-1).view(np.uint32)), \
        f"{N}x{K}: single-row and 2-row results differ"


def test_gemv_nk_misaligned_x_takes_scalar_path(gpu, orc):
    rng = np.random.default_rng(21)
    N, K = 256, 2048
    W = orc.f32_to_f16(rng.standard_normal((N, K), dtype=np.float32) / 45)
    x = rng.standard_normal(K, dtype=np.float32)
    dW = gpu.upload(W)
    dxb = gpu.upload(np.concatenate([[0.0], x]).astype(np.float32))
    dy = gpu.empty(N, np.float32)
    gpu.call("eng_gemv_f16w_nk", dW.ptr, dxb.ptr + 4, dy.ptr, N, K, None)
    gpu.sync()
    Wt = np.ascontiguousarray(W.T)
    y = orc.gemv_f16w(Wt, x).astype(np.float64)
    check_dot(dy.download(), y, helpers.absdot(x, Wt) + np.abs(y), K, "misaligned x nk")


@pytest.mark.parametrize("M,N,K,dtype", [(32, 256, 512, "f16"), (17, 127, 31, "f32"), (512, 4096, 4096, "f16"),
                                         (130, 300, 200, "f32"), (3, 11008, 4096, "f16")])
def test_rmsnorm_linear_nk_prefill_against_oracle(gpu, orc, M, N, K, dtype):
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wf = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    W = orc.f32_to_f16(Wf) if dtype == "f16" else Wf
    got = gpu_rmsnorm_linear_nk(gpu, x, g, W)
    Wt = np.ascontiguousarray(W.T)
    rows = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
    y = orc.rmsnorm_linear(x[rows], g, Wt, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, Wt, K, f"rmsnorm_linear nk {M}x{N}x{K} {dtype}")


@pytest.mark.parametrize("M,N,K", [(192, 256, 512), (128, 512, 256), (256, 128, 1024)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("with_gamma", [True, False])
def test_rmsnorm_linear_f32_full_tiles_against_oracle(gpu, orc, M, N, K, layout, with_gamma):
    # M > 64 normalises into scratch; whole 64/128-row tiles with
    # K % 32 == 0 then take the direct-to-LDS GEMM.
    rng = np.random.default_rng(7 * M + N + K + (layout == "nk"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if with_gamma else None
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    if layout == "kn":
        got = gpu_rmsnorm_linear(gpu, x, g, W)
    else:
        got = gpu_rmsnorm_linear_nk(gpu, x, g, np.ascontiguousarray(W.T))
    rows = np.unique(np.linspace(0, M - 1, 16).astype(int))
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear f32 {layout} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(192, 256, 512), (128, 512, 256), (256, 128, 1024),
                                   (512, 11008, 4096)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("with_gamma", [True, False])
def test_rmsnorm_linear_f16w_full_tiles_against_oracle(gpu, orc, M, N, K, layout, with_gamma):
    # fp16 weights at M > 64: whole tiles take the direct-to-LDS GEMM with the
    # B tile loaded as halves and converted while the fragments are read.
    rng = np.random.default_rng(11 * M + N + K + (layout == "nk"))
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if with_gamma else None
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float16).view(np.uint16)
    if layout == "kn":
        got = gpu_rmsnorm_linear(gpu, x, g, W)
    else:
        got = gpu_rmsnorm_linear_nk(gpu, x, g, np.ascontiguousarray(W.T))
    rows = np.unique(np.linspace(0, M - 1, 16).astype(int))
    y = orc.rmsnorm_linear(x[rows], g, W, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, W, K, f"rmsnorm_linear f16w {layout} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(2, 4096, 4096), (3, 11008, 4096), (4, 300, 4096), (5, 4096, 4096),
                                   (8, 11008, 4096), (13, 1000, 2048), (16, 4096, 4096),
                                   (2, 4096, 11008), (4, 4096, 11008)])
@pytest.mark.parametrize("with_gamma", [True, False])
def test_rmsnorm_linear_f16w_nk_small_batch_rows_match_single_row_calls(gpu, orc, M, N, K, with_gamma):
    # Small-batch decode: up to 4 rows share passes over W (multi-row kernel),
    # each row the single-row call's bits; 5 to 32 take the few-row MFMA
    # kernel, each row the same bits in any batch of 5 to 32 rows.
    rng = np.random.default_rng(M * 100 + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if with_gamma else None
    W = (0.02 * rng.standard_normal((N, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    got = gpu_rmsnorm_linear_nk(gpu, x, g, W)
    for m in sorted({0, M // 2, M - 1}):
        one = helpers.peer_row(lambda xs: gpu_rmsnorm_linear_nk(gpu, xs, g, W), x, m)
        assert np.array_equal(got[m], one), f"row {m} of {M}"
    Wt = np.ascontiguousarray(W.T)
    rows = np.array(sorted({0, M - 1}))
    y = orc.rmsnorm_linear(x[rows], g, Wt, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, Wt, K, f"small batch f16w nk {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,dtype", [(2, 4096, 4096, "f16"), (3, 11008, 4096, "f16"),
                                         (4, 300, 1000, "f16"), (6, 4096, 11008, "f16"),
                                         (16, 4096, 4096, "f16"), (5, 4096, 4096, "f32"),
                                         (4, 257, 100, "f32")])
def test_rmsnorm_linear_kn_small_batch_rows_match_single_row_calls(gpu, orc, M, N, K, dtype):
    # Reference-layout weights A [K x N]: up to 4 rows take the split-K kernel
    # with several activation rows, each row equal to the single-row call bit
    # for bit; 5 or more the few-row MFMA kernel (same bits in any batch).
    rng = np.random.default_rng(M * 77 + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    A = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    if dtype == "f16":
        A = orc.f32_to_f16(A)
    got = gpu_rmsnorm_linear(gpu, x, g, A)
    for m in sorted({0, M // 2, M - 1}):
        one = helpers.peer_row(lambda xs: gpu_rmsnorm_linear(gpu, xs, g, A), x, m)
        assert np.array_equal(got[m], one), f"row {m} of {M}"
    rows = np.array(sorted({0, M - 1}))
    y = orc.rmsnorm_linear(x[rows], g, A, EPS).astype(np.float64)
    check_rmsnorm_linear(got[rows], y, x[rows], g, A, K, f"small batch kn {dtype} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(2, 4096, 4096), (3, 130, 77), (8, 11008, 4096), (16, 64, 1000)])
def test_matmul_small_m_rows_match_gemv(gpu, orc, M, N, K):
    # matmul with up to 4 rows shares GEMV passes over B (row m equals the
    # M = 1 product of A[m] bit for bit); with 5 to 64 the few-row MFMA kernel
    # (row m has the same bits in any such batch).
    rng = np.random.default_rng(M + N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = gpu_matmul(gpu, A, B)
    for m in sorted({0, M - 1}):
        one = helpers.peer_row(lambda a: gpu_matmul(gpu, a, B), A, m)
        assert np.array_equal(got[m], one), f"row {m} of {M}"
    y = orc.matmul(A, B).astype(np.float64)
    check_dot(got, y, helpers.absdot(A, B) + np.abs(y), K, f"matmul small M {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(2, 4096, 4096), (7, 11008, 4096), (16, 512, 1024)])
def test_rmsnorm_linear_f32_nk_small_batch_against_oracle(gpu, orc, M, N, K):
    rng = np.random.default_rng(M * 10 + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    got = gpu_rmsnorm_linear_nk(gpu, x, g, W)
    Wt = np.ascontiguousarray(W.T)
    y = orc.rmsnorm_linear(x, g, Wt, EPS).astype(np.float64)
    check_rmsnorm_linear(got, y, x, g, Wt, K, f"small batch f32 nk {M}x{N}x{K}")


def test_nk_k_zero_contract(gpu):
    d1 = gpu.upload(np.zeros(4, np.float32))
    dy = gpu.upload(np.full(12, 7.0, np.float32))
    gpu.call("eng_gemv_f16w_nk", d1.ptr, d1.ptr, dy.ptr, 12, 0, None)
    gpu.sync()
    assert np.all(dy.download() == 0.0)
    dy = gpu.upload(np.full(12, 7.0, np.float32))
    gpu.call("eng_rmsnorm_linear_f16w_nk", d1.ptr, None, d1.ptr, dy.ptr, 4, 3, 0, EPS, None)
    gpu.sync()
    assert np.all(dy.download() == 7.0)


def test_nk_results_are_deterministic(gpu):
    rng = np.random.default_rng(22)
    W = (0.02 * rng.standard_normal((11008, 4096), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((1, 4096), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    assert np.array_equal(gpu_rmsnorm_linear_nk(gpu, x, g, W), gpu_rmsnorm_linear_nk(gpu, x, g, W))
