"""HIP graph capture of a decode step through the C-ABI (eng_graph_*).

The launchers are meant to be capturable: zero fills are kernels, and the
scratch they pass between their kernels (split-K GEMV and split-KV attention
partials, the few-row kernel's partial sums, the FFN's gate / up) is
the stream's arena, sized by an eager call before the capture; the graph takes
those blocks over when the capture ends, so replays on other streams never
share scratch with eager calls (checked against the oracle below). The graph is
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
    M = 64                        # rows for rmsnorm_linear at M > 1 (the few-row kernel)
    up = gpu.upload
    Wq = up(f16(gpu, 0.03 * rng.standard_normal((Hd, Hd))))          # [out x in]
    Wg = up(f16(gpu, 0.03 * rng.standard_normal((F, Hd))))
    Wu = up(f16(gpu, 0.03 * rng.standard_normal((F, Hd))))
    Wd = up(f16(gpu, 0.03 * rng.standard_normal((Hd, F))))
    Wkn = up(f16(gpu, 0.03 * rng.standard_normal((Hd, Hd))))         # [in x out]: split-K
    Wp = up((0.03 * rng.standard_normal((Hd, 512))).astype(np.float32))  # rmsnorm_linear, 64 rows
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
    # it was captured on after a larger call on the same stream outgrows the
    # stream's arena: the graph owns the blocks it was captured on.
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


def _kn_case(gpu, orc, rng, K, N, M):
    """Reference-layout fp16 RMSNorm+linear inputs (split-K: scratch partials)."""
    W16 = f16(gpu, 0.02 * rng.standard_normal((K, N)))
    gam = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    return W16, gam, x


def _check_kn(got, x, gam, W16, K, what):
    import helpers

    y64 = helpers.as_f64(helpers.oracle(0).rmsnorm_linear(x, gam, W16, EPS))
    derived, _ = helpers.rmsnorm_linear_bounds(x, gam, W16, y64, K)
    helpers.assert_within(got, y64, derived, what)


def test_graph_replayed_on_another_stream_while_eager_calls_run(gpu, orc):
    # The graph owns the scratch blocks it was captured on; eager calls on the
    # capture stream continue on fresh blocks. Replays on a second stream
    # interleaved with eager calls (different inputs, no synchronisation in
    # between) must each match the oracle for their own inputs.
    rng = np.random.default_rng(21)
    K, N, M = 4096, 4096, 4            # split-K partials for 4 rows: 4 MiB of scratch
    W16, gam, xg = _kn_case(gpu, orc, rng, K, N, M)
    xe = rng.standard_normal((M, K)).astype(np.float32)
    dW, dg = gpu.upload(W16), gpu.upload(gam)
    dxg, dxe = gpu.upload(xg), gpu.upload(xe)
    yg = gpu.empty((M, N), np.float32)
    ye = [gpu.empty((M, N), np.float32) for _ in range(4)]
    a, b = gpu.stream(), gpu.stream()
    graph = None
    try:
        gpu.call("eng_rmsnorm_linear_f16w", dxg.ptr, dg.ptr, dW.ptr, yg.ptr, M, N, K, EPS, a.handle)
        a.sync()
        graph = gpu.graph(a)
        with graph:
            gpu.call("eng_rmsnorm_linear_f16w", dxg.ptr, dg.ptr, dW.ptr, yg.ptr, M, N, K, EPS,
                     a.handle)
        for rep in range(3):
            gpu.call("eng_memset", yg.ptr, 0xFF, yg.nbytes)
            for y in ye:
                gpu.call("eng_memset", y.ptr, 0xFF, y.nbytes)
            for i, y in enumerate(ye):
                gpu.call("eng_rmsnorm_linear_f16w", dxe.ptr, dg.ptr, dW.ptr, y.ptr, M, N, K, EPS,
                         a.handle)
                if i == 1:
                    graph.launch(b)
            a.sync()
            b.sync()
            _check_kn(yg.download(), xg, gam, W16, K, f"graph replay {rep} on a second stream")
            for i, y in enumerate(ye):
                _check_kn(y.download(), xe, gam, W16, K, f"eager call {i} during replay {rep}")
    finally:
        if graph is not None:
            graph.destroy()
        a.destroy()
        b.destroy()


def test_graph_outlives_its_capture_stream(gpu, orc):
    rng = np.random.default_rng(22)
    K, N, M = 2048, 3072, 1
    W16, gam, x = _kn_case(gpu, orc, rng, K, N, M)
    dW, dg, dx = gpu.upload(W16), gpu.upload(gam), gpu.upload(x)
    y = gpu.empty((M, N), np.float32)
    a, b = gpu.stream(), gpu.stream()
    graph = None
    try:
        gpu.call("eng_rmsnorm_linear_f16w", dx.ptr, dg.ptr, dW.ptr, y.ptr, M, N, K, EPS, a.handle)
        a.sync()
        graph = gpu.graph(a)
        with graph:
            gpu.call("eng_rmsnorm_linear_f16w", dx.ptr, dg.ptr, dW.ptr, y.ptr, M, N, K, EPS,
                     a.handle)
        a.destroy()                      # frees the stream's own blocks, not the graph's
        for rep in range(3):
            gpu.call("eng_memset", y.ptr, 0xFF, y.nbytes)
            graph.launch(b)
            b.sync()
            _check_kn(y.download(), x, gam, W16, K, f"replay {rep} after the capture stream died")
    finally:
        if graph is not None:
            graph.destroy()
        a.destroy()
        b.destroy()


def test_capture_that_would_grow_the_arena_is_refused(gpu):
    # A fresh stream has no scratch arena yet: a split-K call captured before
    # any eager call would have to allocate during the capture.
    rng = np.random.default_rng(23)
    K, N = 1024, 1024
    W = gpu.upload(f16(gpu, 0.03 * rng.standard_normal((K, N))))
    x = gpu.upload(rng.standard_normal(K).astype(np.float32))
    y = gpu.empty(N, np.float32)
    s = gpu.stream()
    try:
        gpu.call("eng_graph_capture_begin", s.handle)
        rc = gpu.status("eng_gemv_f16w", W.ptr, x.ptr, y.ptr, N, K, s.handle)
        msg = gpu.last_error()
        import ctypes

        h = ctypes.c_void_p(0)
        if gpu.status("eng_graph_capture_end", s.handle, ctypes.byref(h)) == 0 and h.value:
            gpu.call("eng_graph_destroy", h.value)
        assert rc == 1, f"status {rc}: {msg}"
        assert "run the same work once eagerly on this stream before capturing" in msg
        # after an eager call, the same capture works
        gpu.call("eng_gemv_f16w", W.ptr, x.ptr, y.ptr, N, K, s.handle)
        s.sync()
        eager = y.download().copy()
        g = gpu.graph(s)
        with g:
            gpu.call("eng_gemv_f16w", W.ptr, x.ptr, y.ptr, N, K, s.handle)
        gpu.call("eng_memset", y.ptr, 0, y.nbytes)
        g.launch()
        s.sync()
        g.destroy()
        assert np.array_equal(y.download(), eager)
    finally:
        s.destroy()
