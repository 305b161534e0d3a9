"""GPU parity of the few-row linear path (5 <= M <= 64 activation rows on
FP32 MFMA, W streamed once: csrc/kernels/skinny.hip), through the C-ABI.

rmsnorm_linear (fp16 / fp32 weights, reference layout [K x N] and
output-major [N x K], with and without a gain), matmul and the FFN's
gate / up + SwiGLU with 5 to 64 rows are checked against the C oracle under
the derived bound (K + 3) u sum|t W| + (K/2 + 4) u |y| + u |y| and the tighter
statistical bound of tests/helpers.py, on the BASELINE shapes (config 3's
11008 x 4096, the down projection 4096 x 11008) and on shapes that take the
kernel's edge cases: a ragged last column tile, K % 32 != 0 (a partial last
k-group), fp32 weights whose second 16-byte piece is past N, one K chunk
(no partial sums, RMS scale applied in the kernel), K = 8.

fp16 weights take the few-row kernel at 5 to 32 rows (activations as three
fp16 terms that add up to them exactly) and, from 33 rows, the fp16-MFMA GEMM
(64-row tiles up to 64 rows) or, with K % 32 != 0, rmsnorm and the FP32 GEMM.
test_fp16_weight_paths_keep_every_activation_bit pins the exactness of both
fp16 paths bit for bit.

Batch invariance: each row's result involves only its own activation row and
the chunking of K depends on N, K and the CU count only, so a row computed in
a call of any M within one path (fp16 weights: 5 to 32 rows, 33 to 64 rows;
fp32 weights: 5 to 64) has the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
EPS = 1e-5


def run_rmsnorm_linear(eng, x, g, W, layout):
    """W [K x N] ('kn') or [N x K] ('nk'), fp16 bits (uint16) or fp32."""
    M, K = x.shape
    N = W.shape[1] if layout == "kn" else W.shape[0]
    half = W.dtype == np.uint16
    fn = "eng_rmsnorm_linear_" + ("f16w" if half else "f32") + ("_nk" if layout == "nk" else "")
    dx, dW, dy = eng.upload(x), eng.upload(W), eng.empty((M, N), np.float32)
    dg = eng.upload(g) if g is not None else None
    eng.call(fn, dx.ptr, dg.ptr if dg else None, dW.ptr, dy.ptr, M, N, K, EPS, None)
    eng.sync()
    out = dy.download()
    for d in (dx, dW, dy) + ((dg,) if dg else ()):
        d.free()
    return out


def run_matmul(eng, A, B):
    M, K = A.shape
    N = B.shape[1]
    dA, dB, dC = eng.upload(A), eng.upload(B), eng.empty((M, N), np.float32)
    eng.call("eng_matmul_f32", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    eng.sync()
    out = dC.download()
    for d in (dA, dB, dC):
        d.free()
    return out


def make_weights(orc, rng, N, K, dtype, layout):
    Wf = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float32)
    W_kn = orc.f32_to_f16(Wf) if dtype == "f16" else Wf
    return W_kn, (W_kn if layout == "kn" else np.ascontiguousarray(W_kn.T))


def check_rows(orc, got, x, g, W_kn, rows, what):
    K = x.shape[1]
    y64 = helpers.as_f64(orc.rmsnorm_linear(x[rows], g, W_kn, EPS))
    derived, stat = helpers.rmsnorm_linear_bounds(x[rows], g, W_kn, y64, K)
    helpers.assert_within(got[rows], y64, derived, what + " [derived bound]")
    helpers.assert_within(got[rows], y64, stat, what + " [statistical bound]")


@pytest.mark.parametrize("M,N,K,dtype,layout,gamma", [
    (5, 11008, 4096, "f16", "kn", True),    # config 3 shape, the smallest few-row batch
    (16, 11008, 4096, "f16", "kn", True),
    (16, 11008, 4096, "f16", "nk", True),
    # 33-64 rows of fp16 W with K % 32 == 0 take the fp16-MFMA GEMM (64-row tiles)
    (64, 11008, 4096, "f16", "nk", False),  # null gain
    (64, 11008, 4096, "f16", "kn", True),
    (33, 4096, 11008, "f16", "nk", True),   # down-projection shape
    # ... and with K % 32 = 8 rmsnorm and the FP32 GEMM on the fp16 weights
    (64, 11008, 4104, "f16", "nk", False),
    (49, 4096, 4104, "f16", "kn", True),
    (17, 4096, 11008, "f16", "kn", True),
    (8, 1000, 776, "f16", "kn", True),      # ragged last column tile, K % 32 = 8 (partial k-group)
    (20, 300, 1000, "f16", "nk", True),     # rows of W past N read row N - 1, K % 32 = 8
    (12, 4096, 4096, "f32", "kn", True),
    (40, 1004, 1000, "f32", "kn", True),    # fp32, N % 8 = 4: a lane's second piece is past N
    (64, 1000, 1024, "f32", "nk", False),
    (6, 65536, 256, "f16", "kn", True),     # one K chunk: RMS scale applied in the kernel
    (7, 40000, 256, "f16", "nk", True),
    (9, 64, 8, "f16", "kn", True),          # K = 8: a single partial k-group
    (9, 1000, 776, "f16", "nk", True),      # one m-block, weights through LDS: ragged tile and unit
    (36, 1000, 776, "f16", "kn", False),    # K % 32 != 0 past 32 rows: the FP32 GEMM
    (32, 1000, 776, "f16", "kn", True),     # two m-blocks, one X' buffer: ragged tile and unit
    (17, 1000, 776, "f16", "nk", False),    # two m-blocks, weights in registers: ragged
    (50, 11008, 4096, "f16", "kn", True),   # config-3 shape (fp16-MFMA GEMM)
])
def test_rmsnorm_linear_few_rows_against_oracle(gpu, orc, M, N, K, dtype, layout, gamma):
    rng = np.random.default_rng(M * 1000 + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32) if gamma else None
    W_kn, W = make_weights(orc, rng, N, K, dtype, layout)
    got = run_rmsnorm_linear(gpu, x, g, W, layout)
    rows = np.array(sorted({0, M // 2, M - 1}))
    check_rows(orc, got, x, g, W_kn, rows, f"few-row rmsnorm_linear {layout} {dtype} {M}x{N}x{K}")


@pytest.mark.parametrize("M", [5, 16, 17, 32, 33, 64, 130])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_fp16_weight_paths_keep_every_activation_bit(gpu, M, layout):
    # Both fp16-weight paths for M > 4 carry every fp32 activation into the
    # fp16 matrix instruction as three fp16 terms that add up to it exactly
    # (the few-row kernel per unit of 128 values of k, the fp16-MFMA GEMM per
    # row), with exact products. With a weight matrix that selects one
    # activation per output (a single 1.0 per column) the output is that
    # activation times the row's RMS factor s, rounded once:
    # y[m][n] = fp32(x[m][k_n] s_m). Column 64 t of each 64-column tile selects
    # x[m][0] = 1.0, which reads back the s_m that tile applied. Two fp16
    # terms (22 bits) would round most of these activations.
    rng = np.random.default_rng(500 + M + (layout == "nk"))
    K, N = 4096, 512
    mag = rng.uniform(0.5, 1.0, (M, K)) * 2.0 ** rng.integers(-8, 1, (M, K))
    x = (mag * rng.choice([-1.0, 1.0], (M, K))).astype(np.float32)  # full 24-bit significands
    x[:, 0] = 1.0
    sel = rng.integers(1, K, N)
    sel[::64] = 0
    W_kn = np.zeros((K, N), np.float16)
    W_kn[sel, np.arange(N)] = 1.0
    W = W_kn.view(np.uint16) if layout == "kn" else np.ascontiguousarray(W_kn.T).view(np.uint16)
    got = run_rmsnorm_linear(gpu, x, None, W, layout)
    for t in range(N // 64):
        cols = np.arange(64 * t, 64 * t + 64)
        s = got[:, 64 * t]
        want = x[:, sel[cols]] * s[:, None]  # float32 x float32: one rounding
        assert want.dtype == np.float32
        bad = np.argwhere(got[:, cols] != want)
        assert bad.size == 0, (f"{layout} M={M}: tile {t}, {len(bad)} outputs differ, first "
                               f"(row, col) {tuple(bad[0])}: {got[:, cols][tuple(bad[0])]!r} "
                               f"!= {want[tuple(bad[0])]!r}")


@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_few_row_results_do_not_depend_on_the_batch(gpu, orc, layout):
    # A row's bits do not depend on the other rows of the call within each
    # path: 5-32 rows of fp16 W (the few-row kernel) and 33-64 rows (the
    # fp16-MFMA GEMM on one row of 64-row tiles, whose split plan depends on
    # N and K only).
    rng = np.random.default_rng(71)
    N, K = 11008, 4096
    x = rng.standard_normal((64, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W_kn, W = make_weights(orc, rng, N, K, "f16", layout)
    full = run_rmsnorm_linear(gpu, x, g, W, layout)
    for lo, hi in ((0, 33), (20, 64), (31, 64)):
        part = run_rmsnorm_linear(gpu, x[lo:hi], g, W, layout)
        assert np.array_equal(part, full[lo:hi]), f"rows {lo}:{hi} of a {hi - lo}-row call"
    again = run_rmsnorm_linear(gpu, x, g, W, layout)
    assert np.array_equal(again, full), "deterministic"
    few = run_rmsnorm_linear(gpu, x[:32], g, W, layout)
    for lo, hi in ((0, 5), (8, 25), (27, 32), (16, 32)):
        part = run_rmsnorm_linear(gpu, x[lo:hi], g, W, layout)
        assert np.array_equal(part, few[lo:hi]), f"rows {lo}:{hi} of a {hi - lo}-row call"
    rows = np.array([0, 17, 31])
    check_rows(orc, few, x[:32], g, W_kn, rows, f"few-row rmsnorm_linear {layout} 32x{N}x{K}")
    check_rows(orc, full, x, g, W_kn, np.array([0, 40, 63]), f"rmsnorm_linear {layout} 64x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(5, 4096, 4096), (24, 11008, 4096), (64, 1000, 1000),
                                   (37, 4096, 11008)])
def test_matmul_few_rows_against_oracle(gpu, orc, M, N, K):
    rng = np.random.default_rng(M + 7 * N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = run_matmul(gpu, A, B)
    rows = np.array(sorted({0, M // 2, M - 1}))
    y = orc.matmul(A[rows], B).astype(np.float64)
    a = helpers.absdot(A[rows], B)
    derived, stat = helpers.dot_bounds(a, y, K)
    helpers.assert_within(got[rows], y, derived, f"few-row matmul {M}x{N}x{K} [derived]")
    helpers.assert_within(got[rows], y, stat, f"few-row matmul {M}x{N}x{K} [statistical]")
    part = run_matmul(gpu, A[M - 5:], B)
    assert np.array_equal(part, got[M - 5:]), "rows of a 5-row call"


def test_few_rows_k_zero_and_contracts(gpu):
    # K == 0 zero-fills a matmul; rmsnorm_linear writes nothing (the
    # reference's contracts) whatever M.
    dA = gpu.upload(np.ones((8, 4), np.float32))
    dC = gpu.upload(np.full((8, 64), 7.0, np.float32))
    gpu.call("eng_matmul_f32", dA.ptr, dA.ptr, dC.ptr, 8, 64, 0, None)
    gpu.sync()
    assert np.all(dC.download() == 0.0)
    dy = gpu.upload(np.full((8, 64), 7.0, np.float32))
    gpu.call("eng_rmsnorm_linear_f16w", dA.ptr, None, dA.ptr, dy.ptr, 8, 64, 0, EPS, None)
    gpu.sync()
    assert np.all(dy.download() == 7.0)
