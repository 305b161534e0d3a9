"""Weight layout conversion (eng_transpose_f16 / _f32) on the GPU.

Bit-exact against NumPy's transpose for square, ragged, single-row and
single-column shapes, on the 16-byte path and the per-element path
(dimensions not multiples of the vector, pointers off 16-byte alignment),
with NaN / infinity / signed-zero bit patterns carried unchanged. End to end:
reference-layout fp16 weights A [K x N] transposed on the device feed the
output-major GEMV, which then matches the reference-layout GEMV on the
original A within the GEMV bound against the C oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu


def gpu_transpose(eng, a, src_off=0, dst_off=0):
    """Transpose `a` (uint16 or float32 bits) on the device, optionally with
    the source / destination shifted by a few elements off alignment."""
    rows, cols = a.shape
    fn = "eng_transpose_f16" if a.dtype == np.uint16 else "eng_transpose_f32"
    esz = a.dtype.itemsize
    src = eng.empty(a.size + src_off, a.dtype)
    dst = eng.empty(a.size + dst_off, a.dtype)
    if a.size:
        eng.call("eng_memcpy_h2d", src.ptr + esz * src_off, np.ascontiguousarray(a).ctypes.data, a.nbytes)
    dst.fill_bytes(0x5A)
    eng.call(fn, src.ptr + esz * src_off, dst.ptr + esz * dst_off, rows, cols, None)
    eng.sync()
    out = dst.download()[dst_off:].reshape(cols, rows)
    src.free()
    dst.free()
    return out


SHAPES = [(1, 1), (1, 17), (17, 1), (63, 65), (64, 64), (128, 4096), (4096, 128), (257, 1000),
          (4096, 11008)]


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("dtype", [np.uint16, np.uint32])
def test_transpose_is_bit_exact(gpu, rows, cols, dtype):
    rng = np.random.default_rng(rows * 7 + cols)
    a = rng.integers(0, np.iinfo(dtype).max, (rows, cols), dtype=dtype, endpoint=True)
    if dtype == np.uint32:
        a = a.view(np.float32)
    got = gpu_transpose(gpu, a)
    assert np.array_equal(got.view(dtype), np.ascontiguousarray(a.T).view(dtype))


@pytest.mark.parametrize("src_off,dst_off", [(1, 0), (0, 3), (5, 7)])
def test_transpose_off_alignment(gpu, src_off, dst_off):
    rng = np.random.default_rng(src_off * 10 + dst_off)
    for dtype in (np.uint16, np.float32):
        a = rng.standard_normal((96, 200)).astype(dtype if dtype == np.float32 else np.float16)
        if dtype == np.uint16:
            a = a.view(np.uint16)
        got = gpu_transpose(gpu, a, src_off, dst_off)
        assert np.array_equal(got, np.ascontiguousarray(a.T))


def test_special_values_are_moved_not_converted(gpu):
    h = np.array([0x7E00, 0x7C01, 0xFC00, 0x8000, 0x0001, 0x7BFF, 0xFFFF, 0x0000], np.uint16)
    a = np.tile(h, (16, 3))
    assert np.array_equal(gpu_transpose(gpu, a), np.ascontiguousarray(a.T))
    f = np.array([0x7FC00001, 0xFF800000, 0x80000000, 0x00000001, 0x7F7FFFFF, 0xFFFFFFFF],
                 np.uint32).view(np.float32)
    b = np.tile(f, (9, 5))
    assert np.array_equal(gpu_transpose(gpu, b).view(np.uint32), np.ascontiguousarray(b.T).view(np.uint32))


@pytest.mark.parametrize("K,N", [(4096, 4096), (1000, 1536)])
def test_reference_layout_weights_feed_the_output_major_gemv(gpu, orc, K, N):
    rng = np.random.default_rng(K + N)
    A = (0.02 * rng.standard_normal((K, N), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    dA, dx = gpu.upload(A), gpu.upload(x)
    dW = gpu.empty((N, K), np.uint16)
    y_ref, y_nk = gpu.empty(N, np.float32), gpu.empty(N, np.float32)
    gpu.call("eng_transpose_f16", dA.ptr, dW.ptr, K, N, None)
    gpu.call("eng_gemv_f16w", dA.ptr, dx.ptr, y_ref.ptr, N, K, None)
    gpu.call("eng_gemv_f16w_nk", dW.ptr, dx.ptr, y_nk.ptr, N, K, None)
    gpu.sync()
    assert np.array_equal(dW.download(), np.ascontiguousarray(A.T))
    y64 = orc.gemv_f16w(A, x).astype(np.float64)
    a = helpers.absdot(x, A) + np.abs(y64)
    derived, stat = helpers.dot_bounds(a, y64, K)
    for name, d in (("reference layout", y_ref), ("output-major after transpose", y_nk)):
        got = d.download()
        helpers.assert_within(got, y64, derived, f"{name} {K}x{N} [derived bound]")
        helpers.assert_within(got, y64, stat, f"{name} {K}x{N} [statistical bound]")
