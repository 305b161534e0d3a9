"""ENGREF01 weight slabs on the GPU: eng_engref_upload through the C-ABI.

Bit-exact: every tensor's bytes in the slab equal the file's, over files that
take several staging chunks, with mixed dtypes, odd sizes and zero-size
tensors; padding between tensors is left untouched. Parity: a decode GEMV
run on fp16 weights and fp32 activations read straight from the slab matches
the C oracle within the GEMV bound.
"""

from __future__ import annotations

import sys
import time

import numpy as np
import pytest

import helpers

sys.path.insert(0, str(helpers.REPO / "tests" / "golden"))
import engref  # noqa: E402

pytestmark = pytest.mark.gpu


def upload_and_check(gpu, path, stream=None):
    with gpu.engref(path) as f:
        slab = gpu.empty(f.slab_bytes(), np.uint8)
        slab.fill_bytes(0xAB)
        t0 = time.perf_counter()
        f.upload(slab, stream)
        dt = time.perf_counter() - t0
        got = slab.download()
        covered = np.zeros(got.size, dtype=bool)
        for t in f.tensors:
            region = got[t.slab_offset:t.slab_offset + t.nbytes]
            assert np.array_equal(region, t.host.reshape(-1).view(np.uint8)), t.name
            covered[t.slab_offset:t.slab_offset + t.nbytes] = True
        assert (got[~covered] == 0xAB).all(), "padding bytes were written"
        slab.free()
        return f.slab_bytes(), dt


def test_multi_chunk_mixed_dtype_upload_is_bit_exact(gpu, tmp_path):
    rng = np.random.default_rng(7)
    tensors = {
        "w_f16": rng.standard_normal((3001, 2503)).astype(np.float16).view(np.uint16),  # 15 MB
        "odd_f32": rng.standard_normal(1_234_567).astype(np.float32),                  # 4.9 MB
        "empty": np.zeros((0, 17), np.float32),
        "tiny_f16": np.arange(3, dtype=np.uint16),
        "f64": rng.standard_normal((129, 7)),
        "tail_f32": rng.standard_normal(2_097_153).astype(np.float32),                 # 8 MiB + 4 B
    }
    path = tmp_path / "mixed.bin"
    engref.write(path, tensors)
    nbytes, dt = upload_and_check(gpu, path)
    print(f"engref upload: {nbytes / 2**20:.1f} MiB in {dt * 1e3:.1f} ms "
          f"({nbytes / dt / 1e9:.2f} GB/s host file -> HBM)", flush=True)


def test_upload_on_a_created_stream_and_reuse_of_a_slab(gpu, tmp_path):
    rng = np.random.default_rng(8)
    a = tmp_path / "a.bin"
    b = tmp_path / "b.bin"
    engref.write(a, {"x": rng.standard_normal(1000).astype(np.float32)})
    engref.write(b, {"y": rng.standard_normal((64, 64)).astype(np.float16).view(np.uint16),
                     "z": rng.standard_normal(5).astype(np.float32)})
    with gpu.stream() as s:
        upload_and_check(gpu, a, s)
        upload_and_check(gpu, b, s)
    # one slab holding a's layout, overwritten by b's upload
    with gpu.engref(a) as fa, gpu.engref(b) as fb:
        slab = gpu.empty(max(fa.slab_bytes(), fb.slab_bytes()), np.uint8)
        fa.upload(slab)
        fb.upload(slab)
        got = slab.download()
        for t in fb.tensors:
            assert np.array_equal(got[t.slab_offset:t.slab_offset + t.nbytes],
                                  t.host.reshape(-1).view(np.uint8))


@pytest.mark.parametrize("N,K", [(4096, 4096), (1000, 1536)])
def test_gemv_on_slab_resident_fp16_weights(gpu, orc, tmp_path, N, K):
    rng = np.random.default_rng(N + K)
    W = (0.02 * rng.standard_normal((N, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K, dtype=np.float32)
    path = tmp_path / "layer.bin"
    engref.write(path, {"x": x, "W": W})  # x first: W starts at a 256-byte boundary after it
    with gpu.engref(path) as f:
        slab = gpu.empty(f.slab_bytes(), np.uint8)
        f.upload(slab)
        w_ptr = slab.ptr + f.at("W").slab_offset
        x_ptr = slab.ptr + f.at("x").slab_offset
        y = gpu.empty(N, np.float32)
        gpu.call("eng_gemv_f16w_nk", w_ptr, x_ptr, y.ptr, N, K, None)
        gpu.sync()
        got = y.download()
        slab.free()
    Wt = np.ascontiguousarray(W.T)
    y64 = orc.gemv_f16w(Wt, x).astype(np.float64)
    a = helpers.absdot(x, Wt) + np.abs(y64)
    derived, stat = helpers.dot_bounds(a, y64, K)
    helpers.assert_within(got, y64, derived, f"slab gemv {N}x{K} [derived K*u bound]")
    helpers.assert_within(got, y64, stat, f"slab gemv {N}x{K} [statistical bound]")
