"""HIP graph capture of a decode step through the C-ABI (eng_graph_*).

The launchers are meant to be capturable: zero fills are kernels, and the
scratch they pass between their kernels (split-K GEMV and split-KV attention
partials, rmsnorm_linear's normalised rows at M > 1, the FFN's gate / up) is
the stream's arena, sized by an eager call before the capture. The graph is
replayed several times with the program's own eager work and synchronisations
in between -- outputs clobbered, other launches on the same stream, an input
changed in place -- and every replay must equal the eager result bit for bit
(the kernels are deterministic for a given launch configuration).
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
EPS = 1e-5


def f16(gpu, a):
    return gpu.f32_to_f16(np.ascontiguousarray(a, dtype=np.float32))


def test_captured_decode_step_replays_match_eager(gpu):
    rng = np.random.default_rng(5)
    Hd, F = 1024, 2752            # hidden and FFN width
    heads, kv_heads, D, L = 8, 2, 64, 700
    M = 64                        # prefill rows for rmsnorm_linear at M > 1
    up = gpu.upload
    Wq = up(f16(gpu, 0.03 * rng.standard_normal((Hd, Hd))))          # [out x in]
    Wg = up(f16(gpu, 0.03 * rng.standard_normal((F, Hd))))
    Wu = up(f16(gpu, 0.03 * rng.standard_normal((F, Hd))))
    Wd = up(f16(gpu, 0.03 * rng.standard_normal((Hd, F))))
    Wkn = up(f16(gpu, 0.03 * rng.standard_normal((Hd, Hd))))         # [in x out]: split-K
    Wp = up((0.03 * rng.standard_normal((Hd, 512))).astype(np.float32))  # rmsnorm_linear M > 1
    x = up(rng.standard_normal(Hd).astype(np.float32))
    xm = up(rng.standard_normal((M, Hd)).astype(np.float32))
    g = up((1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32))
    q = up(f16(gpu, rng.standard_normal((heads, D))))
    kc = up(f16(gpu, 0.5 * rng.standard_normal((kv_heads, L, D))))
    vc = up(f16(gpu, 0.5 * rng.standard_normal((kv_heads, L, D))))
    outs = {
        "y1": gpu.empty(Hd, np.float32), "act": gpu.empty(F, np.float32),
        "y2": gpu.empty(Hd, np.float32), "ykn": gpu.empty(Hd, np.float32),
        "att": gpu.empty((heads, D), np.uint16), "sum": gpu.empty(Hd, np.float32),
        "norm": gpu.empty(Hd, np.float32), "pre": gpu.empty((M, 512), np.float32),
    }
    o = outs
    s = gpu.stream()
    h = s.handle

    def step():
        gpu.call("eng_gemv_f16w_nk", Wq.ptr, x.ptr, o["y1"].ptr, Hd, Hd, h)
        gpu.call("eng_rmsnorm_linear_swiglu_f16w_nk", o["y1"].ptr, g.ptr, Wg.ptr, Wu.ptr,
                 o["act"].ptr, 1, F, Hd, EPS, h)
        gpu.call("eng_gemv_f16w_nk", Wd.ptr, o["act"].ptr, o["y2"].ptr, Hd, F, h)
        gpu.call("eng_gemv_f16w", Wkn.ptr, x.ptr, o["ykn"].ptr, Hd, Hd, h)
        gpu.call("eng_attention_decode_f16", q.ptr, kc.ptr, vc.ptr, o["att"].ptr, L, heads,
                 kv_heads, D, L * D, 1.0 / np.sqrt(D), 0, h)
        gpu.call("eng_residual_rmsnorm_f32", o["y2"].ptr, o["ykn"].ptr, g.ptr, o["norm"].ptr,
                 o["sum"].ptr, 1, Hd, EPS, h)
        gpu.call("eng_rmsnorm_linear_f32", xm.ptr, g.ptr, Wp.ptr, o["pre"].ptr, M, 512, Hd, EPS, h)

    def results():
        s.sync()
        return {k: v.download().copy() for k, v in outs.items()}

    graph = None
    try:
        step()                                  # eager; sizes the stream's arena
        eager = results()
        graph = gpu.graph(s)
        with graph:
            step()
        for rep in range(3):
            for v in outs.values():              # clobber every output eagerly
                gpu.call("eng_memset", v.ptr, 0xFF, v.nbytes)
            # unrelated eager work on the same stream between replays
            gpu.call("eng_gemv_f16w", Wkn.ptr, o["y2"].ptr, o["sum"].ptr, Hd, Hd, h)
            s.sync()
            graph.launch()
            got = results()
            for k in outs:
                assert np.array_equal(got[k], eager[k]), f"replay {rep}: {k} differs from eager"
        # An input changed in place: the replay reads the new values.
        x.upload(rng.standard_normal(Hd).astype(np.float32))
        step()
        eager2 = results()
        assert not np.array_equal(eager2["y1"], eager["y1"])
        for v in outs.values():
            gpu.call("eng_memset", v.ptr, 0, v.nbytes)
        graph.launch()
        got = results()
        for k in outs:
            assert np.array_equal(got[k], eager2[k]), f"replay after input change: {k}"
    finally:
        if graph is not None:
            graph.destroy()
        s.destroy()


def test_graph_replays_after_the_stream_arena_grows(gpu):
    # A graph captured on a small split-K call keeps addressing the arena block
    # it was captured on after a larger call on the same stream outgrows that
    # block: the outgrown block stays allocated until the stream is destroyed.
    rng = np.random.default_rng(8)
    K, N = 512, 1024
    W = gpu.upload(f16(gpu, 0.03 * rng.standard_normal((K, N))))      # [in x out]: split-K
    x = gpu.upload(rng.standard_normal(K).astype(np.float32))
    y = gpu.empty(N, np.float32)
    # 4 rows of a reference-layout rmsnorm_linear: split-K partials for 4 rows,
    # about 4 MiB, past the 1 MiB the first call sizes the arena to
    Mb, Kb, Nb = 4, 4096, 8192
    Wb = gpu.upload(f16(gpu, 0.01 * rng.standard_normal((Kb, Nb))))
    xb = gpu.upload(rng.standard_normal((Mb, Kb)).astype(np.float32))
    yb = gpu.empty((Mb, Nb), np.float32)
    s = gpu.stream()
    h = s.handle
    graph = None
    try:
        gpu.call("eng_gemv_f16w", W.ptr, x.ptr, y.ptr, N, K, h)       # eager; sizes the arena
        s.sync()
        eager = y.download().copy()
        graph = gpu.graph(s)
        with graph:
            gpu.call("eng_gemv_f16w", W.ptr, x.ptr, y.ptr, N, K, h)
        for rep in range(3):
            gpu.call("eng_rmsnorm_linear_f16w", xb.ptr, None, Wb.ptr, yb.ptr, Mb, Nb, Kb, EPS, h)
            gpu.call("eng_memset", y.ptr, 0xFF, y.nbytes)
            s.sync()
            graph.launch()
            s.sync()
            assert np.array_equal(y.download(), eager), f"replay {rep} after growth"
    finally:
        if graph is not None:
            graph.destroy()
        s.destroy()


def test_capture_on_the_null_stream_is_refused(gpu):
    assert gpu.status("eng_graph_capture_begin", None) == 1
    assert "capture needs a created stream" in gpu.last_error()
