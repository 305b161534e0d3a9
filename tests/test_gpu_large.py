"""Maximum-size cases: operands of more than 2^31 elements.

Index arithmetic past 32 bits is exercised where it matters for the decode
path: an output-major fp16 GEMV with W [N x K] of 2^31 + 2^18 elements, the
transpose of that W into the reference layout, and the reference-layout
split-K GEMV over it; and for the MFMA GEMM, whose direct loads address each
tile through a buffer descriptor (a 64-bit base and a 32-bit range clamped at
4 GiB): fp16 B [N x K] of the same size through rmsnorm_linear_f16w_nk at 128
rows, and an fp32 A [M x 4096] of 4 GiB + 1 MiB through matmul. W repeats every 64 rows (built on the device by
doubling copies of one 64-row block), so every output equals the output of
its row modulo 64, bit for bit (the kernels compute each row / column with
the same arithmetic in the same order); the first 64 outputs are checked
against the C oracle with the GEMV bound.
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu

PERIOD = 64
K = 4096
N = (1 << 19) + PERIOD  # N * K = 2^31 + 2^18 elements (4 GiB + 512 KiB of fp16)


def tiled_rows(eng, block, rows):
    """Device [rows x cols] matrix repeating `block` ([PERIOD x cols]) by rows."""
    d = eng.empty((rows, block.shape[1]), block.dtype)
    eng.call("eng_memcpy_h2d", d.ptr, block.ctypes.data, block.nbytes)
    have = block.shape[0]
    row_bytes = block.shape[1] * block.itemsize
    while have < rows:
        n = min(have, rows - have)
        eng.call("eng_memcpy_d2d", d.ptr + have * row_bytes, d.ptr, n * row_bytes)
        have += n
    return d


def check_periodic(got, y64_block, what):
    got = np.asarray(got)
    blocks = got[: (len(got) // PERIOD) * PERIOD].reshape(-1, PERIOD)
    bad = np.nonzero(~(blocks == blocks[0]).all(axis=1))[0]
    assert bad.size == 0, f"{what}: block {bad[:4]} differs from block 0"
    return blocks[0]


def test_gemv_past_2_31_elements_both_layouts(gpu, orc):
    assert N * K > (1 << 31)
    rng = np.random.default_rng(31)
    W0 = (0.02 * rng.standard_normal((PERIOD, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    W = tiled_rows(gpu, W0, N)
    dx = gpu.upload(x)
    y = gpu.empty(N, np.float32)
    print(f"large: output-major gemv N={N} K={K} ({N * K} elements)", flush=True)
    gpu.call("eng_gemv_f16w_nk", W.ptr, dx.ptr, y.ptr, N, K, None)
    gpu.sync()
    y_nk = y.download()
    block = check_periodic(y_nk, None, "output-major gemv")
    A0 = np.ascontiguousarray(W0.T)  # [K x PERIOD]
    y64 = orc.gemv_f16w(A0, x).astype(np.float64)
    a = helpers.absdot(x, A0) + np.abs(y64)
    derived, stat = helpers.dot_bounds(a, y64, K)
    helpers.assert_within(block, y64, derived, "output-major gemv block 0 [derived bound]")
    helpers.assert_within(block, y64, stat, "output-major gemv block 0 [statistical bound]")

    # reference layout A [K x N] = W^T: columns repeat every 64
    print("large: transpose to the reference layout", flush=True)
    A = gpu.empty((K, N), np.uint16)
    gpu.call("eng_transpose_f16", W.ptr, A.ptr, N, K, None)
    W.free()
    row = np.empty(N, np.uint16)
    for k in (0, 1, K // 2, K - 1):  # spot rows of A: A[k][n] = W0[n % 64][k]
        gpu.call("eng_memcpy_d2h", row.ctypes.data, A.ptr + 2 * k * N, 2 * N)
        assert np.array_equal(row, np.tile(W0[:, k], N // PERIOD + 1)[:N]), k
    print("large: reference-layout split-K gemv", flush=True)
    gpu.call("eng_gemv_f16w", A.ptr, dx.ptr, y.ptr, N, K, None)
    gpu.sync()
    y_kn = y.download()
    block_kn = check_periodic(y_kn, None, "reference-layout gemv")
    helpers.assert_within(block_kn, y64, derived, "reference-layout gemv block 0 [derived bound]")
    helpers.assert_within(block_kn, y64, stat, "reference-layout gemv block 0 [statistical bound]")
    A.free()


def test_gemm_operands_past_4_gib(gpu, orc):
    rng = np.random.default_rng(32)
    # fp16 B [N x K] (4 GiB + 512 KiB) at M = 128: the GEMM path of rmsnorm_linear
    M = 128
    W0 = (0.02 * rng.standard_normal((PERIOD, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((M, K), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    W = tiled_rows(gpu, W0, N)
    dx, dg = gpu.upload(x), gpu.upload(g)
    out = gpu.empty((M, N), np.float32)
    print(f"large: rmsnorm_linear_f16w_nk M={M} N={N} K={K}", flush=True)
    gpu.call("eng_rmsnorm_linear_f16w_nk", dx.ptr, dg.ptr, W.ptr, out.ptr, M, N, K, 1e-5, None)
    gpu.sync()
    got = out.download().reshape(M, N // PERIOD, PERIOD)
    W.free()
    out.free()
    # Every 64-column block against the oracle's block (W's rows repeat every
    # 64). Not bit for bit across blocks: 4097 tiles of 128 columns leave a
    # last round of one tile, which the GEMM splits over the CUs by K tile
    # and adds in another order.
    Wt = np.ascontiguousarray(W0.T)  # [K x PERIOD]
    y64 = orc.rmsnorm_linear(x, g, Wt, 1e-5).astype(np.float64)
    derived, stat = helpers.rmsnorm_linear_bounds(x, g, Wt, y64, K)
    for b0 in range(0, got.shape[1], 1024):
        blk = got[:, b0:b0 + 1024, :]
        exp = np.broadcast_to(y64[:, None, :], blk.shape)
        what = f"rmsnorm_linear_f16w_nk blocks {b0}.. "
        helpers.assert_within(blk, exp, derived[:, None, :], what + "[derived bound]")
        helpers.assert_within(blk, exp, stat[:, None, :], what + "[statistical bound]")

    # fp32 A [M x K] of 4 GiB + 1 MiB, B [K x 128]
    MA, NB = (1 << 18) + PERIOD, 128
    A0 = rng.uniform(-1, 1, (PERIOD, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, NB)).astype(np.float32)
    A = tiled_rows(gpu, A0, MA)
    dB = gpu.upload(B)
    C = gpu.empty((MA, NB), np.float32)
    print(f"large: matmul_f32 M={MA} N={NB} K={K}", flush=True)
    gpu.call("eng_matmul_f32", A.ptr, dB.ptr, C.ptr, MA, NB, K, None)
    gpu.sync()
    got = C.download().reshape(MA // PERIOD, PERIOD, NB)
    A.free()
    C.free()
    assert np.array_equal(got, np.broadcast_to(got[:1], got.shape)), "rows not periodic"
    y64 = orc.matmul(A0, B).astype(np.float64)
    derived, stat = helpers.dot_bounds(helpers.absdot(A0, B) + np.abs(y64), y64, K)
    helpers.assert_within(got[0], y64, derived, "matmul block 0 [derived bound]")
    helpers.assert_within(got[0], y64, stat, "matmul block 0 [statistical bound]")
