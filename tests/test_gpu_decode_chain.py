"""BASELINE config 5 as a chain: two Llama-7B-shape decode layers back to back
(H = 4096, F = 11008, fp16 weights, fp32 activations), each

    qkv = W_qkv . x            one GEMV over q, k and v stored as one matrix (N = 3H = 12288)
    o   = W_o . v              v = qkv[2H:3H]
    act = SiLU(RMSNorm(o) . W_gate) * (RMSNorm(o) . W_up)      one fused launch
    x'  = W_down . act         the next layer's input

exactly as bench.py's fastest config-5 arrangement issues them, in both weight
layouts (output-major [out x in] through the *_nk entries; the reference layout
[in x out] through eng_gemv_f16w / eng_rmsnorm_linear_swiglu_f16w), eagerly and
as a replayed HIP graph. Checks:

* every launch against the C oracle applied to that launch's own GPU input,
  within the derived bound of one fp32-accumulated dot product (so each launch
  is pinned exactly, whatever the earlier launches' rounding);
* the final output against a float64 chain from the first input, within the
  derived bounds propagated through the chain (first order: each stage's error
  bound is carried through |W| of the next, through the RMSNorm scale's
  sensitivity and SiLU's slope), doubled;
* graph replays bit-equal to the eager token.

The reference composes its transformer-block tests from the same launches
(tests/test_kernels.cu:2867-2915).
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
EPS = 1e-5
U = helpers.U32
H, F = 4096, 11008


def silu64(v):
    return v / (1.0 + np.exp(-v))


def _weights(rng):
    """Layer-1 weights (reference layout [in x out], fp16 bits); layer 2 uses
    their negation, so a launch that read the wrong layer's matrix fails."""
    def w(k, n):
        return (0.02 * rng.standard_normal((k, n), dtype=np.float32)).astype(np.float16).view(np.uint16)
    one = {"qkv": w(H, 3 * H), "o": w(H, H), "gate": w(H, F), "up": w(H, F), "down": w(F, H)}
    two = {k: v ^ np.uint16(0x8000) for k, v in one.items()}
    return [one, two]


def _gv_bound(x, A):
    """Derived bound of one fp16-weight GEMV out = x . A (float64 result, bound)."""
    y64 = helpers.as_f64(x) @ helpers.as_f64(A)
    a = helpers.absdot(x, A)
    return y64, helpers.dot_bounds(a, y64, A.shape[0])[0]


def _glu64(o, g, Wg, Wu):
    xs = helpers.rms_scale64(o[None, :]) * helpers.as_f64(o[None, :]) * helpers.as_f64(g)
    g64 = (xs @ helpers.as_f64(Wg))[0]
    u64 = (xs @ helpers.as_f64(Wu))[0]
    return g64, u64


def _chain64(x, g, layers):
    """float64 chain and its propagated error bound (first order)."""
    x64 = helpers.as_f64(x)
    err = np.zeros_like(x64)
    for L in layers:
        Wqkv, Wo = helpers.as_f64(L["qkv"]), helpers.as_f64(L["o"])
        Wg, Wu, Wd = helpers.as_f64(L["gate"]), helpers.as_f64(L["up"]), helpers.as_f64(L["down"])
        qkv = x64 @ Wqkv
        e_qkv = err @ np.abs(Wqkv) + H * U * (np.abs(x64) @ np.abs(Wqkv)) + U * np.abs(qkv)
        v, e_v = qkv[2 * H:], e_qkv[2 * H:]
        o = v @ Wo
        e_o = e_v @ np.abs(Wo) + H * U * (np.abs(v) @ np.abs(Wo)) + U * np.abs(o)
        # RMSNorm(o) * gamma: scale s = 1/rms(o); ds / s <= sum|o e_o| / sum o^2
        gm = helpers.as_f64(g)
        s = 1.0 / np.sqrt(np.mean(o * o) + EPS)
        xs = s * o * gm
        rel_s = np.sum(np.abs(o) * e_o) / np.sum(o * o)
        e_xs = s * e_o * np.abs(gm) + rel_s * np.abs(xs)
        gt, up = xs @ Wg, xs @ Wu
        # each projection: propagated input error + its own (K + 3) u sum|.| and
        # the fp32 row scale (K / 2 + 4) u |y|
        e_g = e_xs @ np.abs(Wg) + (H + 3) * U * (np.abs(xs) @ np.abs(Wg)) + (H / 2 + 5) * U * np.abs(gt)
        e_u = e_xs @ np.abs(Wu) + (H + 3) * U * (np.abs(xs) @ np.abs(Wu)) + (H / 2 + 5) * U * np.abs(up)
        sg = silu64(gt)
        act = sg * up
        e_act = 1.1 * np.abs(up) * e_g + np.abs(sg) * e_u + e_g * e_u + 8 * U * np.abs(act)
        x64 = act @ Wd
        err = e_act @ np.abs(Wd) + F * U * (np.abs(act) @ np.abs(Wd)) + U * np.abs(x64)
    return x64, err


class Chain:
    def __init__(self, gpu, layers, nk, x, g):
        self.gpu, self.nk = gpu, nk
        up = gpu.upload
        self.dev = []
        for L in layers:
            if nk:  # output-major: [out x in]
                self.dev.append({k: up(np.ascontiguousarray(v.T)) for k, v in L.items()})
            else:
                self.dev.append({k: up(v) for k, v in L.items()})
        self.x = up(x)
        self.g = up(g)
        self.qkv = [gpu.empty(3 * H, np.float32) for _ in layers]
        self.o = [gpu.empty(H, np.float32) for _ in layers]
        self.act = [gpu.empty(F, np.float32) for _ in layers]
        self.out = [gpu.empty(H, np.float32) for _ in layers]

    def token(self, s):
        gpu = self.gpu
        gv = "eng_gemv_f16w_nk" if self.nk else "eng_gemv_f16w"
        glu = "eng_rmsnorm_linear_swiglu_f16w_nk" if self.nk else "eng_rmsnorm_linear_swiglu_f16w"
        xin = self.x.ptr
        for i, W in enumerate(self.dev):
            gpu.call(gv, W["qkv"].ptr, xin, self.qkv[i].ptr, 3 * H, H, s)
            gpu.call(gv, W["o"].ptr, self.qkv[i].ptr + 2 * H * 4, self.o[i].ptr, H, H, s)
            gpu.call(glu, self.o[i].ptr, self.g.ptr, W["gate"].ptr, W["up"].ptr, self.act[i].ptr,
                     1, F, H, EPS, s)
            gpu.call(gv, W["down"].ptr, self.act[i].ptr, self.out[i].ptr, H, F, s)
            xin = self.out[i].ptr

    def results(self):
        return [{"qkv": self.qkv[i].download(), "o": self.o[i].download(),
                 "act": self.act[i].download(), "out": self.out[i].download()}
                for i in range(len(self.dev))]

    def clobber(self):
        for bufs in (self.qkv, self.o, self.act, self.out):
            for b in bufs:
                self.gpu.call("eng_memset", b.ptr, 0xFF, b.nbytes)

    def free(self):
        for W in self.dev:
            for d in W.values():
                d.free()
        for d in [self.x, self.g] + self.qkv + self.o + self.act + self.out:
            d.free()


@pytest.fixture(scope="module")
def chain_inputs():
    rng = np.random.default_rng(4)
    layers = _weights(rng)
    x = rng.standard_normal(H, dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return layers, x, g


@pytest.mark.parametrize("nk", [True, False], ids=["output_major", "reference_layout"])
def test_config5_two_layer_chain_eager_and_graph(gpu, orc, chain_inputs, nk):
    layers, x, g = chain_inputs
    ch = Chain(gpu, layers, nk, x, g)
    s = gpu.stream()
    graph = None
    try:
        ch.token(s.handle)
        s.sync()
        eager = ch.results()
        # each launch against the oracle on its own GPU input
        xin = x
        for i, (L, r) in enumerate(zip(layers, eager)):
            tag = f"{'nk' if nk else 'kn'} layer {i}"
            y64, b = _gv_bound(xin, L["qkv"])
            helpers.assert_within(r["qkv"], y64, b, tag + " qkv (N = 12288) vs float64")
            helpers.assert_within(r["qkv"], orc.gemv_f16w(L["qkv"], xin), 2 * b, tag + " qkv vs oracle")
            v = r["qkv"][2 * H:]
            y64, b = _gv_bound(v, L["o"])
            helpers.assert_within(r["o"], orc.gemv_f16w(L["o"], v), 2 * b, tag + " o vs oracle")
            o = r["o"]
            orc_act = orc.rmsnorm_linear_swiglu(o[None, :], g, L["gate"], L["up"], EPS)[0]
            g64, u64 = _glu64(o, g, L["gate"], L["up"])
            dg = helpers.rmsnorm_linear_bounds(o[None, :], g, L["gate"], g64[None, :], H)[0][0]
            du = helpers.rmsnorm_linear_bounds(o[None, :], g, L["up"], u64[None, :], H)[0][0]
            sg = silu64(g64)
            act64 = sg * u64
            b_act = 1.1 * np.abs(u64) * dg + np.abs(sg) * du + dg * du + 8 * U * np.abs(act64)
            helpers.assert_within(r["act"], act64, b_act, tag + " gate/up + SwiGLU vs float64")
            helpers.assert_within(r["act"], orc_act, 2 * b_act, tag + " gate/up + SwiGLU vs oracle")
            y64, b = _gv_bound(r["act"], L["down"])
            helpers.assert_within(r["out"], orc.gemv_f16w(L["down"], r["act"]), 2 * b,
                                  tag + " down (K = 11008) vs oracle")
            xin = r["out"]
        # end to end from the first input
        x64, err = _chain64(x, g, layers)
        helpers.assert_within(eager[-1]["out"], x64, 2 * err, "two-layer chain end to end")
        # the same token replayed from a HIP graph, bit for bit
        graph = gpu.graph(s)
        with graph:
            ch.token(s.handle)
        for rep in range(2):
            ch.clobber()
            graph.launch()
            s.sync()
            got = ch.results()
            for i in range(len(layers)):
                for k in got[i]:
                    assert np.array_equal(got[i][k].view(np.uint32), eager[i][k].view(np.uint32)), \
                        f"graph replay {rep}: layer {i} {k} differs from the eager token"
    finally:
        if graph is not None:
            graph.destroy()
        s.destroy()
        ch.free()
