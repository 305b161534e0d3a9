"""The C-ABI library: it loads, exports every declared symbol, and keeps the
reference's launch contract (status codes and message substrings) on paths
that are decided on the host before any device call.
"""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

import helpers

HEADER = helpers.REPO / "include" / "engine_hip.h"


def declared_functions() -> list:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eng_\w+)\s*\(", text)))


def test_header_declares_the_hot_path_entry_points():
    names = declared_functions()
    for fn in ("eng_matmul_f32", "eng_gemv_f32", "eng_gemv_f16", "eng_gemv_f16w",
               "eng_rmsnorm_f32", "eng_rmsnorm_linear_f32", "eng_rmsnorm_linear_f16w",
               "eng_rmsnorm_linear_fused_direct_f32", "eng_last_error", "eng_vector_add_f32",
               "eng_residual_rmsnorm_f32", "eng_swiglu_f32", "eng_swiglu_f16",
               "eng_rmsnorm_linear_swiglu_f16w_nk", "eng_rmsnorm_linear_swiglu_f32_nk",
               "eng_rmsnorm_linear_swiglu_f16w", "eng_rmsnorm_linear_swiglu_f32"):
        assert fn in names


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(pkg.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in engine_hip.h but not exported: {missing}"


def test_python_binding_covers_the_header(pkg):
    bound = set(pkg.SIGNATURES) | set(pkg.STRING_FUNCTIONS)
    assert set(declared_functions()) <= bound


def test_build_info_names_the_target(eng):
    assert "gfx950" in eng.lib.eng_build_info().decode()


# ------------------------------------------------------------------ contract
P = 0x1000  # dummy non-null "device" pointer; never dereferenced on these paths


@pytest.mark.parametrize("call,code,substr", [
    (("eng_gemv_f32", None, P, P, 4, 4, None), 1, "gemv: A is null"),
    (("eng_gemv_f32", P, None, P, 4, 4, None), 1, "gemv: x is null"),
    (("eng_gemv_f32", P, P, None, 4, 4, None), 1, "gemv: out is null"),
    (("eng_gemv_f32", P, P, P, -1, 4, None), 1, "non-negative"),
    (("eng_gemv_f32", P, P, P, 4, -1, None), 1, "non-negative"),
    (("eng_gemv_f16", None, P, P, 4, 4, None), 1, "gemv_fp16: A is null"),
    (("eng_gemv_f16", P, P, P, -1, 4, None), 1, "non-negative"),
    (("eng_gemv_f16w", P, P, None, 4, 4, None), 1, "null"),
    (("eng_gemv_f16w", P, P, P, 4, -1, None), 1, "non-negative"),
    (("eng_matmul_f32", None, P, P, 2, 2, 2, None), 1, "matmul_register_tiled: A is null"),
    (("eng_matmul_f32", P, P, None, 2, 2, 2, None), 1, "C is null"),
    (("eng_matmul_f32", P, P, P, -1, 4, 4, None), 1, "M must be non-negative"),
    (("eng_matmul_f32", P, P, P, 4, 4, -1, None), 1, "K must be non-negative"),
    (("eng_rmsnorm_f32", None, P, P, 2, 2, 1e-5, None), 1, "rmsnorm: null device pointer"),
    (("eng_rmsnorm_f32", P, P, P, -1, 4, 1e-5, None), 1, "rmsnorm: negative dimension"),
    (("eng_rmsnorm_f32", P, P, P, 4, 4, -1.0, None), 1, "eps"),
    (("eng_rmsnorm_linear_f32", None, P, P, P, 2, 2, 2, 1e-5, None), 1, "null device pointer"),
    (("eng_rmsnorm_linear_f32", P, P, None, P, 2, 2, 2, 1e-5, None), 1, "null"),
    (("eng_rmsnorm_linear_f32", P, P, P, P, 4, -1, 4, 1e-5, None), 1, "negative dimension"),
    (("eng_rmsnorm_linear_f16w", P, P, P, P, 4, 4, -1, 1e-5, None), 1, "negative"),
    (("eng_rmsnorm_linear_f16w", P, P, P, P, 4, 4, 4, -1.0, None), 1, "eps must be non-negative"),
    (("eng_rmsnorm_linear_fused_direct_f32", P, P, P, P, 4, 4, 4, float("nan"), None), 1, "eps"),
    (("eng_gemv_f16w_nk", None, P, P, 4, 4, None), 1, "A is null"),
    (("eng_gemv_f16w_nk", P, P, P, 4, -1, None), 1, "non-negative"),
    (("eng_gemv_f32_nk", P, None, P, 4, 4, None), 1, "x is null"),
    (("eng_rmsnorm_linear_f16w_nk", P, P, None, P, 2, 2, 2, 1e-5, None), 1, "null device pointer"),
    (("eng_rmsnorm_linear_f32_nk", P, P, P, P, 2, -2, 2, 1e-5, None), 1, "negative dimension"),
    (("eng_rmsnorm_linear_f32_nk", P, P, P, P, 2, 2, 2, -1e-5, None), 1, "eps"),
    (("eng_vector_add_f32", P, P, P, -1, None), 1, "vector_add: n must be non-negative"),
    (("eng_vector_add_f32", None, P, P, 4, None), 1, "vector_add: null device pointer"),
    (("eng_vector_add_f32", P, P, None, 4, None), 1, "null"),
    (("eng_residual_rmsnorm_f32", P, P, P, P, P, -1, 4, 1e-5, None), 1, "residual_rmsnorm: negative dimension"),
    (("eng_residual_rmsnorm_f32", P, P, P, P, P, 4, -1, 1e-5, None), 1, "negative dimension"),
    (("eng_residual_rmsnorm_f32", None, P, P, P, P, 2, 2, 1e-5, None), 1, "null device pointer"),
    (("eng_residual_rmsnorm_f32", P, None, P, P, P, 2, 2, 1e-5, None), 1, "null"),
    (("eng_residual_rmsnorm_f32", P, P, P, None, P, 2, 2, 1e-5, None), 1, "null"),
    (("eng_residual_rmsnorm_f32", P, P, P, P, None, 2, 2, 1e-5, None), 1, "null"),
    (("eng_residual_rmsnorm_f32", P, P, P, P, P, 4, 4, -1.0, None), 1, "eps"),
    (("eng_swiglu_f32", None, P, P, 4, None), 1, "swiglu: gate is null"),
    (("eng_swiglu_f32", P, None, P, 4, None), 1, "swiglu: up is null"),
    (("eng_swiglu_f32", P, P, None, 4, None), 1, "swiglu: out is null"),
    (("eng_swiglu_f32", P, P, P, -1, None), 1, "swiglu: n must be non-negative"),
    (("eng_swiglu_f16", None, P, P, 4, None), 1, "swiglu_fp16: gate is null"),
    (("eng_swiglu_f16", P, P, P, -1, None), 1, "swiglu_fp16: n must be non-negative"),
    (("eng_rmsnorm_linear_swiglu_f16w_nk", P, P, None, P, P, 1, 4, 4, 1e-5, None), 1, "null device pointer"),
    (("eng_rmsnorm_linear_swiglu_f16w_nk", P, P, P, None, P, 1, 4, 4, 1e-5, None), 1, "null"),
    (("eng_rmsnorm_linear_swiglu_f32_nk", P, P, P, P, P, 1, -4, 4, 1e-5, None), 1, "negative dimension"),
    (("eng_rmsnorm_linear_swiglu_f32_nk", P, P, P, P, P, 1, 4, 4, -1.0, None), 1, "eps"),
    (("eng_rmsnorm_linear_swiglu_f16w", P, P, None, P, P, 1, 4, 4, 1e-5, None), 1, "null device pointer"),
    (("eng_rmsnorm_linear_swiglu_f32", P, P, P, P, P, 1, -4, 4, 1e-5, None), 1, "negative dimension"),
    (("eng_rmsnorm_linear_swiglu_f32", P, P, P, P, P, 1, 4, 4, -1.0, None), 1, "eps"),
    (("eng_attention_decode_f16", None, P, P, P, 4, 8, 2, 64, 256, 0.125, 0, None), 1, "attention_decode: q is null"),
    (("eng_attention_decode_f16", P, None, P, P, 4, 8, 2, 64, 256, 0.125, 0, None), 1, "k is null"),
    (("eng_attention_decode_f16", P, P, None, P, 4, 8, 2, 64, 256, 0.125, 0, None), 1, "v is null"),
    (("eng_attention_decode_f16", P, P, P, None, 4, 8, 2, 64, 256, 0.125, 0, None), 1, "out is null"),
    (("eng_attention_decode_f16", P, P, P, P, -1, 8, 2, 64, 256, 0.125, 0, None), 1, "kv_len must be non-negative"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 0, 2, 64, 256, 0.125, 0, None), 1, "n_heads must be positive"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 8, 0, 64, 256, 0.125, 0, None), 1, "n_kv_heads must be positive"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 6, 4, 64, 256, 0.125, 0, None), 1, "divisible by n_kv_heads"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 8, 2, 32, 128, 0.125, 0, None), 1, "head_dim must be 64 or 128"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 8, 2, 64, 256, float("inf"), 0, None), 1, "scale must be finite"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 8, 2, 64, 256, 0.125, -1, None), 1, "split_kv must be non-negative"),
    (("eng_attention_decode_f16", P, P, P, P, 4, 8, 2, 64, 255, 0.125, 0, None), 1, "kv_head_stride < kv_len * head_dim"),
    (("eng_attention_decode_with_mode_f16", P, P, P, P, 4, 8, 2, 128, 256, 0.125, 0, 0, None), 1, "kv_head_stride"),
    (("eng_cast_f32_to_f16", P, P, -1, None), 1, "cast_f32_to_f16: n must be non-negative"),
    (("eng_cast_f32_to_f16", None, P, 4, None), 1, "in is null"),
    (("eng_cast_f16_to_f32", P, None, 4, None), 1, "cast_f16_to_f32: out is null"),
    (("eng_kv_cache_write_f16", P, P, P, P, -1, 2, 64, 0, 8, None), 1, "s_new must be non-negative"),
    (("eng_kv_cache_write_f16", P, P, P, P, 1, 0, 64, 0, 8, None), 1, "n_kv_heads must be positive"),
    (("eng_kv_cache_write_f16", P, P, P, P, 1, 2, 0, 0, 8, None), 1, "head_dim must be positive"),
    (("eng_kv_cache_write_f16", P, P, P, P, 1, 2, 64, -1, 8, None), 1, "pos_offset must be non-negative"),
    (("eng_kv_cache_write_f16", P, P, P, P, 4, 2, 64, 5, 8, None), 1, "kv_max_seq_len < pos_offset + s_new"),
    (("eng_kv_cache_write_f16", None, P, P, P, 1, 2, 64, 0, 8, None), 1, "k_new/v_new is null"),
    (("eng_kv_cache_write_f16", P, P, P, None, 1, 2, 64, 0, 8, None), 1, "k_cache/v_cache is null"),
    (("eng_graph_capture_begin", None), 1, "capture needs a created stream"),
    (("eng_graph_capture_end", None, P), 1, "eng_graph_capture_end: stream is null"),
    (("eng_graph_capture_end", P, None), 1, "eng_graph_capture_end: graph is null"),
    (("eng_graph_launch", None, None), 1, "eng_graph_launch: graph is null"),
    (("eng_transpose_f16", P, P + 4096, -1, 4, None), 1, "transpose: negative dimension"),
    (("eng_transpose_f16", None, P, 4, 4, None), 1, "transpose: null device pointer"),
    (("eng_transpose_f32", P, None, 4, 4, None), 1, "transpose: null device pointer"),
    (("eng_transpose_f16", P, P, 4, 4, None), 1, "src and dst overlap"),
    (("eng_transpose_f32", P, P + 60, 4, 4, None), 1, "src and dst overlap"),
    (("eng_transpose_f32", P + 60, P, 4, 4, None), 1, "src and dst overlap"),
])
def test_preconditions_fail_before_launch(eng, call, code, substr):
    name, *args = call
    rc = eng.status(name, *args)
    msg = eng.last_error()
    assert rc == code, (rc, msg)
    assert substr in msg
    assert msg.startswith("[engine] ") and "\n  check failed: " in msg


@pytest.mark.parametrize("call", [
    ("eng_gemv_f32", P, P, P, 0, 8, None),
    ("eng_gemv_f16", P, P, P, 0, 8, None),
    ("eng_gemv_f16w", P, P, P, 0, 8, None),
    ("eng_matmul_f32", P, P, P, 0, 8, 8, None),
    ("eng_matmul_f32", P, P, P, 8, 0, 8, None),
    ("eng_rmsnorm_f32", P, P, P, 0, 8, 1e-5, None),
    ("eng_rmsnorm_f32", P, None, P, 8, 0, 1e-5, None),
    ("eng_rmsnorm_linear_f32", P, P, P, P, 0, 8, 8, 1e-5, None),
    ("eng_rmsnorm_linear_f32", P, None, P, P, 8, 0, 8, 1e-5, None),
    ("eng_rmsnorm_linear_f32", P, P, P, P, 8, 8, 0, 1e-5, None),
    ("eng_rmsnorm_linear_f16w", P, P, P, P, 8, 8, 0, 1e-5, None),
    ("eng_gemv_f16w_nk", P, P, P, 0, 8, None),
    ("eng_rmsnorm_linear_f16w_nk", P, P, P, P, 8, 0, 8, 1e-5, None),
    ("eng_rmsnorm_linear_f32_nk", P, P, P, P, 0, 8, 8, 1e-5, None),
    ("eng_vector_add_f32", None, None, None, 0, None),
    ("eng_residual_rmsnorm_f32", P, P, None, P, P, 0, 8, 1e-5, None),
    ("eng_residual_rmsnorm_f32", P, P, P, P, P, 8, 0, 1e-5, None),
    ("eng_swiglu_f32", P, P, P, 0, None),
    ("eng_swiglu_f16", P, P, P, 0, None),
    ("eng_rmsnorm_linear_swiglu_f16w_nk", P, None, P, P, P, 1, 0, 8, 1e-5, None),
    ("eng_rmsnorm_linear_swiglu_f32_nk", P, P, P, P, P, 1, 8, 0, 1e-5, None),
    ("eng_rmsnorm_linear_swiglu_f16w", P, None, P, P, P, 0, 8, 8, 1e-5, None),
    ("eng_rmsnorm_linear_swiglu_f32", P, P, P, P, P, 1, 8, 0, 1e-5, None),
    ("eng_cast_f32_to_f16", None, None, 0, None),
    ("eng_cast_f16_to_f32", None, None, 0, None),
    ("eng_kv_cache_write_f16", None, None, None, None, 0, 2, 64, 3, 3, None),
    ("eng_graph_destroy", None),
    ("eng_transpose_f16", None, None, 0, 7, None),
    ("eng_transpose_f32", None, None, 7, 0, None),
])
def test_empty_work_is_a_no_op(eng, call):
    name, *args = call
    assert eng.status(name, *args) == 0, eng.last_error()


# ---------------------------------------------------------------- host fp16
def test_host_f16_conversions_match_numpy(eng):
    import test_oracle

    f = test_oracle.half_probe_floats()
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16)
    got = eng.f32_to_f16(f)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], ref[~nan].view(np.uint16))
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = eng.f16_to_f32(bits)
    r = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(back), np.isnan(r))
    assert np.array_equal(back[~np.isnan(r)].view(np.uint32), r[~np.isnan(r)].view(np.uint32))


# ----------------------------------------------------------- host pool (C-ABI)
def test_host_pool_contract_through_c_abi(eng, pkg):
    pool = ctypes.c_void_p()
    eng.call("eng_pool_create", ctypes.byref(pool), pkg.DEVICE_CPU, 64 * 1024)
    try:
        ptrs = []
        for nbytes in (1, 256, 257, 5000):
            p = ctypes.c_void_p()
            eng.call("eng_pool_allocate", pool, nbytes, ctypes.byref(p))
            assert p.value % 256 == 0
            ptrs.append(p.value)
        st = pkg.AllocStats()
        eng.call("eng_pool_stats", pool, ctypes.byref(st))
        assert st.bytes_in_use == 256 + 256 + 512 + 8192
        assert st.num_driver_allocs == 1
        for p in ptrs:
            eng.call("eng_pool_deallocate", pool, p, None)
        eng.call("eng_pool_stats", pool, ctypes.byref(st))
        assert st.bytes_in_use == 0 and st.peak_bytes_in_use == 9216
        z = ctypes.c_void_p(1)
        eng.call("eng_pool_allocate", pool, 0, ctypes.byref(z))
        assert z.value is None
        rc = eng.status("eng_pool_deallocate", pool, 0x12345600, None)
        assert rc == 1 and "not allocated by this pool" in eng.last_error()
    finally:
        eng.call("eng_pool_destroy", pool)


def test_unknown_device_kind_is_rejected(eng):
    pool = ctypes.c_void_p()
    assert eng.status("eng_pool_create", ctypes.byref(pool), 7, 1024) == 1
    assert "unsupported device" in eng.last_error()
