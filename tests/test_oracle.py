"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the checker.

Against: the float64 golden fixtures (reference case tables), closed forms,
exact rational brute force on tiny shapes, NumPy's IEEE float16, and planted
mistakes (oracle/liboracle_mut<N>.so) that each check must catch.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import helpers

EPS = 1e-5


def oracle_bound(a, y64, K):
    """Double-accumulated oracle vs float64 golden: output rounding + double sum."""
    return helpers.U32 * np.abs(y64) + 2.0 * K * 2.0**-53 * a + 1e-300


# --------------------------------------------------------------- run helpers
def run_matmul(orc, c):
    x = helpers.inputs(c)
    return orc.matmul(x["A"], x["B"]), x


def check_matmul(orc, c):
    got, x = run_matmul(orc, c)
    exp = helpers.expected(c)
    K = c["params"]["K"]
    # The golden is float32-rounded: allow its rounding as well.
    bound = oracle_bound(helpers.absdot(x["A"], x["B"]), exp, K) + helpers.U32 * np.abs(exp)
    return helpers.assert_within(got, exp, bound, c["stem"])


def check_gemv(orc, c):
    x = helpers.inputs(c)
    got = orc.gemv(x["A"], x["x"])
    exp = helpers.expected(c)
    bound = oracle_bound(helpers.absdot(x["x"], x["A"]), exp, c["params"]["K"]) + helpers.U32 * np.abs(exp)
    return helpers.assert_within(got, exp, bound, c["stem"])


def check_rmsnorm(orc, c):
    x = helpers.inputs(c)
    got = orc.rmsnorm(x["input"], x.get("weight"), EPS)
    exp = helpers.expected(c)
    # scale rounded to float, then two float multiplies, then the golden's rounding
    bound = 5 * helpers.U32 * np.abs(exp) + 1e-30
    return helpers.assert_within(got, exp, bound, c["stem"])


def check_rmsnorm_linear(orc, c):
    x = helpers.inputs(c)
    got = orc.rmsnorm_linear(x["input"], x.get("weight"), x["W"], EPS)
    exp = helpers.expected(c)
    K = c["params"]["K"]
    s = helpers.rms_scale64(x["input"])
    g = 1.0 if "weight" not in x else helpers.as_f64(x["weight"])
    a = s * (np.abs(helpers.as_f64(x["input"]) * g) @ np.abs(helpers.as_f64(x["W"])))
    # temp[k] carries ~3 float roundings (scale, two multiplies): 4u relative per term.
    bound = 4 * helpers.U32 * a + 2 * helpers.U32 * np.abs(exp) + 2.0 * K * 2.0**-53 * a
    return helpers.assert_within(got, exp, bound, c["stem"])


def check_residual_rmsnorm(orc, c):
    x = helpers.inputs(c)
    norm, sm = orc.residual_rmsnorm(x["x"], x["residual"], x.get("weight"), EPS)
    exp = helpers.expected(c)
    # sum rounded to float (u), scale from the rounded sums (u), scale to float,
    # two float multiplies, the golden's rounding: 6u relative.
    helpers.assert_within(norm, exp, 6 * helpers.U32 * np.abs(exp) + 1e-30, c["stem"])
    # sum_out is one float addition: bit-exact with NumPy's float32 add.
    assert np.array_equal(sm, x["x"] + x["residual"]), c["stem"] + " sum_out"


def check_swiglu(orc, c):
    x = helpers.inputs(c)
    got = orc.swiglu(x["gate"], x["up"])
    exp = helpers.expected(c)
    # double evaluation then one float rounding, plus the golden's float32 rounding
    return helpers.assert_within(got, exp, 2 * helpers.U32 * np.abs(exp) + 2.0**-149, c["stem"])


def swiglu_bound(g64, u64, dg, du, act64):
    """|d act| for act = silu(g) u given |d g| <= dg, |d u| <= du (|silu'| < 1.1)."""
    silu = g64 / (1.0 + np.exp(-g64))
    return 1.1 * np.abs(u64) * dg + np.abs(silu) * du + dg * du + 2 * helpers.U32 * np.abs(act64)


def check_rmsnorm_linear_swiglu(orc, c):
    x = helpers.inputs(c)
    got = orc.rmsnorm_linear_swiglu(x["input"], x.get("weight"), x["Wg"], x["Wu"], EPS)
    exp, g64, u64 = (helpers.expected(c, n) for n in ("expected", "gate", "up"))
    K = c["params"]["K"]
    s = helpers.rms_scale64(x["input"])
    gw = 1.0 if "weight" not in x else helpers.as_f64(x["weight"])
    xs = np.abs(helpers.as_f64(x["input"]) * gw)
    ag = s * (xs @ np.abs(helpers.as_f64(x["Wg"])))
    au = s * (xs @ np.abs(helpers.as_f64(x["Wu"])))
    dg = 4 * helpers.U32 * ag + 2 * helpers.U32 * np.abs(g64) + 2.0 * K * 2.0**-53 * ag
    du = 4 * helpers.U32 * au + 2 * helpers.U32 * np.abs(u64) + 2.0 * K * 2.0**-53 * au
    return helpers.assert_within(got, exp, swiglu_bound(g64, u64, dg, du, exp), c["stem"])


def run_attention(orc, c):
    x = helpers.inputs(c)
    P = c["params"]
    D, s_kv = P["head_dim"], P["s_kv"]
    return orc.attention(x["q"], x["k"], x["v"], P["n_heads"], P["n_kv_heads"], D, s_kv, s_kv * D,
                         1.0 / np.sqrt(D), P["q_pos_offset"], P["is_causal"], want_lse=True)


def check_attention(orc, c):
    out, lse = run_attention(orc, c)
    exp = helpers.expected(c).reshape(out.shape)
    # double softmax then half rounding (half an ulp) against the float32-stored golden
    bound = helpers.U16 * np.abs(exp) + 2.0**-25 + 2 * helpers.U32 * np.abs(exp)
    helpers.assert_within(helpers.as_f64(out), exp, bound, c["stem"])
    else_ = helpers.expected(c, "lse")
    helpers.assert_within(lse, else_, 2 * helpers.U32 * np.abs(else_) + 1e-30, c["stem"] + " lse")


# ------------------------------------------------------------------- goldens
@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("attention")])
def test_attention_matches_golden(orc, stem):
    check_attention(orc, helpers.case(stem))


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(14)
    H, Hkv, D, L = 8, 2, 128, 40
    f16 = lambda a: orc.f32_to_f16(np.asarray(a, np.float32))
    q = f16(rng.standard_normal((1, H, D)))
    k = f16(rng.standard_normal((Hkv, L, D)))
    v = f16(rng.standard_normal((Hkv, L, D)))
    sc = 1.0 / np.sqrt(D)
    # one key: the output is that key's value row, exactly
    o1 = orc.attention(q, k, v, H, Hkv, D, 1, L * D, sc)
    for h in range(H):
        assert np.array_equal(o1[0, h], v[h // 4, 0])
    # q = 0: every score is 0, the output is the mean value row
    o0 = orc.attention(np.zeros_like(q), k, v, H, Hkv, D, L, L * D, sc)
    mean = helpers.as_f64(v).mean(axis=1)
    for h in range(H):
        assert np.array_equal(o0[0, h], orc.f32_to_f16(mean[h // 4].astype(np.float32)))
    # a dominant key (score ~ +1e4 above the rest) selects its value row
    kd = k.copy()
    kd[:, 17] = f16(np.sign(helpers.as_f64(q[0, ::4])) * 8.0)
    od = orc.attention(q, kd, v, H, Hkv, D, L, L * D, 1.0)
    for h in range(0, H, 4):
        assert np.array_equal(od[0, h], v[h // 4, 17])
    # key order does not matter (up to one half ulp from the double sums)
    perm = rng.permutation(L)
    op = orc.attention(q, k[:, perm], v[:, perm], H, Hkv, D, L, L * D, sc)
    o = orc.attention(q, k, v, H, Hkv, D, L, L * D, sc)
    helpers.assert_within(helpers.as_f64(op), helpers.as_f64(o),
                          helpers.U16 * np.abs(helpers.as_f64(o)) * 2 + 2.0**-24, "key permutation")
    # strided KV heads and GQA mapping against NumPy float64
    stride = (L + 5) * D
    kp = np.zeros((Hkv, L + 5, D), np.uint16)
    vp = np.zeros((Hkv, L + 5, D), np.uint16)
    kp[:, :L], vp[:, :L] = k, v
    os_ = orc.attention(q, kp, vp, H, Hkv, D, L, stride, sc)
    q64, k64, v64 = (helpers.as_f64(a) for a in (q, k, v))
    for h in range(H):
        s = k64[h // 4] @ q64[0, h] * sc
        w = np.exp(s - s.max())
        ref = (w @ v64[h // 4]) / w.sum()
        helpers.assert_within(helpers.as_f64(os_[0, h]), ref, helpers.U16 * np.abs(ref) + 2.0**-25,
                              f"strided head {h}")
    # the empty sequence writes zeros and -inf lse
    oe, le = orc.attention(q, k, v, H, Hkv, D, 0, 0, sc, want_lse=True)
    assert np.all(oe == 0) and np.all(np.isneginf(le))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("vector_add")])
def test_vector_add_is_float32_addition(orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = orc.vector_add(x["a"], x["b"])
    assert np.array_equal(got, x["a"] + x["b"])
    assert np.array_equal(got.astype(np.float64), helpers.expected(c).astype(np.float32).astype(np.float64))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("residual_rmsnorm")])
def test_residual_rmsnorm_matches_golden(orc, stem):
    check_residual_rmsnorm(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("swiglu")])
def test_swiglu_matches_golden(orc, stem):
    check_swiglu(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("swiglu_fp16")])
def test_swiglu_fp16_matches_golden(orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got16 = orc.swiglu_fp16(x["gate"], x["up"])
    exp = helpers.expected(c)
    bound = helpers.U16 * np.abs(exp) + 2.0**-25 + 2 * helpers.U32 * np.abs(exp)
    helpers.assert_within(helpers.as_f64(got16), exp, bound, stem)
    # the fp32 formula on the decoded halves, rounded to half: bit for bit
    ref = orc.f32_to_f16(orc.swiglu(orc.f16_to_f32(x["gate"]), orc.f16_to_f32(x["up"])))
    assert np.array_equal(got16, ref)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear_swiglu")
                                  + helpers.cases("rmsnorm_linear_swiglu_f16w")])
def test_rmsnorm_linear_swiglu_matches_golden(orc, stem):
    check_rmsnorm_linear_swiglu(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("ffn_subblock")])
def test_ffn_subblock_matches_golden(orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    S, D, F = (c["params"][k] for k in ("S", "D", "F"))
    got = orc.ffn_subblock(x["x"], x["ffn_rms_w"], x["w_gate"], x["w_up"], x["w_down"], EPS)
    # The same numbers as the composition of the individually pinned functions.
    hn = orc.rmsnorm(x["x"], x["ffn_rms_w"], EPS)
    act = orc.swiglu(orc.matmul(hn, x["w_gate"]), orc.matmul(hn, x["w_up"]))
    assert np.array_equal(got, orc.vector_add(x["x"], orc.matmul(act, x["w_down"])))
    # Against the float64 golden: error of act (gate / up as in rmsnorm_linear,
    # propagated through SwiGLU), carried through the down projection.
    exp, act64 = helpers.expected(c), helpers.expected(c, "act")
    h64, w64 = helpers.as_f64(x["x"]), helpers.as_f64(x["ffn_rms_w"])
    s = helpers.rms_scale64(x["x"])
    xs = s * np.abs(h64 * w64)
    g64 = (s * h64 * w64) @ helpers.as_f64(x["w_gate"])
    u64 = (s * h64 * w64) @ helpers.as_f64(x["w_up"])
    ag, au = xs @ np.abs(helpers.as_f64(x["w_gate"])), xs @ np.abs(helpers.as_f64(x["w_up"]))
    dg = 4 * helpers.U32 * ag + 2 * helpers.U32 * np.abs(g64) + 2.0 * D * 2.0**-53 * ag
    du = 4 * helpers.U32 * au + 2 * helpers.U32 * np.abs(u64) + 2.0 * D * 2.0**-53 * au
    dact = swiglu_bound(g64, u64, dg, du, act64)
    wd = np.abs(helpers.as_f64(x["w_down"]))
    down_bound = dact @ wd + (helpers.U32 + 2.0 * F * 2.0**-53) * (np.abs(act64) @ wd)
    bound = down_bound + 2 * helpers.U32 * np.abs(exp)
    helpers.assert_within(got, exp, bound, stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("matmul")])
def test_matmul_matches_golden(orc, stem):
    check_matmul(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv")])
def test_gemv_matches_golden(orc, stem):
    check_gemv(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv_fp16")])
def test_gemv_fp16_matches_golden(orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = helpers.as_f64(orc.gemv_fp16(x["A"], x["x"]))
    exp = helpers.expected(c)
    # half output rounding (half an ulp, 2^-11 relative, 2^-25 absolute near 0)
    bound = helpers.U16 * np.abs(exp) + 2.0**-25 + helpers.U32 * np.abs(exp)
    helpers.assert_within(got, exp, bound, stem)


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("gemv_f16w")])
def test_gemv_f16w_matches_golden(orc, stem):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    got = orc.gemv_f16w(x["A"], x["x"])
    exp = helpers.expected(c)
    bound = oracle_bound(helpers.absdot(x["x"], x["A"]), exp, c["params"]["K"]) + helpers.U32 * np.abs(exp)
    helpers.assert_within(got, exp, bound, stem)
    # Same numbers as the fp32 GEMV over the decoded matrix, bit for bit.
    assert np.array_equal(got, orc.gemv(orc.f16_to_f32(x["A"]), x["x"]))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm")])
def test_rmsnorm_matches_golden(orc, stem):
    check_rmsnorm(orc, helpers.case(stem))


@pytest.mark.parametrize("stem", [c["stem"] for c in helpers.cases("rmsnorm_linear")
                                  + helpers.cases("rmsnorm_linear_f16w")])
def test_rmsnorm_linear_matches_golden(orc, stem):
    check_rmsnorm_linear(orc, helpers.case(stem))


def test_golden_inputs_are_reproducible():
    """Every fixture input regenerates to the recorded SHA-256."""
    for c in helpers.manifest()["cases"]:
        helpers.inputs(c)


# -------------------------------------------------------------- closed forms
def test_matmul_identity_is_a_copy(orc):
    rng = np.random.default_rng(5)
    A = rng.standard_normal((37, 53), dtype=np.float32)
    assert np.array_equal(orc.matmul(A, np.eye(53, dtype=np.float32)), A)


def test_matmul_all_ones_gives_k(orc):
    for K in (1, 7, 1000, 4097):
        C = orc.matmul(np.ones((3, K), np.float32), np.ones((K, 5), np.float32))
        assert np.all(C == K)


def test_matmul_exact_rational_brute_force(orc):
    rng = np.random.default_rng(11)
    for M, N, K in ((1, 1, 1), (3, 4, 5), (2, 7, 3)):
        A = rng.standard_normal((M, K), dtype=np.float32)
        B = rng.standard_normal((K, N), dtype=np.float32)
        C = orc.matmul(A, B)
        for i in range(M):
            for j in range(N):
                exact = sum(Fraction(float(A[i, k])) * Fraction(float(B[k, j])) for k in range(K))
                # products of floats are exact in double; a few double sums then one
                # rounding to float: equal to the correctly rounded value within 1 ulp
                assert abs(Fraction(float(C[i, j])) - exact) <= Fraction(abs(float(exact))) * Fraction(2, 2**24)


def test_gemv_is_matmul_at_m1_bit_exact(orc):
    rng = np.random.default_rng(6)
    A = rng.standard_normal((300, 77), dtype=np.float32)
    x = rng.standard_normal(300, dtype=np.float32)
    assert np.array_equal(orc.gemv(A, x), orc.matmul(x[None, :], A)[0])


def test_gemv_of_zero_input_is_zero(orc):
    out = orc.gemv(np.ones((128, 64), np.float32), np.zeros(128, np.float32))
    assert np.all(out == 0.0)


def test_gemv_fp16_small_integers_are_exact(orc):
    # Sums of small integer products are exact in every format involved.
    A = orc.f32_to_f16(np.arange(12, dtype=np.float32).reshape(4, 3) - 5)
    x = orc.f32_to_f16(np.array([1, -2, 3, 1], np.float32))
    got = orc.f16_to_f32(orc.gemv_fp16(A, x))
    Af = orc.f16_to_f32(A).astype(np.float64)
    assert np.array_equal(got, (np.array([1, -2, 3, 1.0]) @ Af).astype(np.float32))


def test_rmsnorm_zero_row_is_zero_not_nan(orc):
    out = orc.rmsnorm(np.zeros((2, 256), np.float32), None, EPS)
    assert np.all(out == 0.0)


def test_rmsnorm_null_weight_equals_unit_weight(orc):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 300), dtype=np.float32)
    assert np.array_equal(orc.rmsnorm(x, None, EPS), orc.rmsnorm(x, np.ones(300, np.float32), EPS))
    W = rng.standard_normal((300, 40), dtype=np.float32)
    assert np.array_equal(orc.rmsnorm_linear(x, None, W, EPS),
                          orc.rmsnorm_linear(x, np.ones(300, np.float32), W, EPS))


def test_rmsnorm_linear_is_rmsnorm_then_matmul(orc):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((9, 200), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(200)).astype(np.float32)
    W = rng.standard_normal((200, 33), dtype=np.float32)
    assert np.array_equal(orc.rmsnorm_linear(x, g, W, EPS), orc.matmul(orc.rmsnorm(x, g, EPS), W))
    W16 = orc.f32_to_f16(W)
    assert np.array_equal(orc.rmsnorm_linear(x, g, W16, EPS),
                          orc.rmsnorm_linear(x, g, orc.f16_to_f32(W16), EPS))


def test_residual_rmsnorm_closed_forms(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 300), dtype=np.float32)
    r = rng.standard_normal((5, 300), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(300)).astype(np.float32)
    norm, sm = orc.residual_rmsnorm(x, r, g, EPS)
    # == rmsnorm of the float sum, bit for bit; NULL sum_out changes nothing
    assert np.array_equal(norm, orc.rmsnorm(x + r, g, EPS))
    assert np.array_equal(orc.residual_rmsnorm(x, r, g, EPS, want_sum=False)[0], norm)
    # NULL weight == ones; NULL residual == rmsnorm of x
    assert np.array_equal(orc.residual_rmsnorm(x, r, None, EPS)[0],
                          orc.residual_rmsnorm(x, r, np.ones(300, np.float32), EPS)[0])
    assert np.array_equal(orc.residual_rmsnorm(x, None, g, EPS)[0], orc.rmsnorm(x, g, EPS))
    z = np.zeros((2, 64), np.float32)
    nz, sz = orc.residual_rmsnorm(z, z, None, EPS)
    assert np.all(nz == 0.0) and np.all(sz == 0.0)


def test_swiglu_closed_forms(orc):
    rng = np.random.default_rng(12)
    g = rng.standard_normal(1000, dtype=np.float32) * 4
    u = rng.standard_normal(1000, dtype=np.float32)
    assert np.all(orc.swiglu(np.zeros(1000, np.float32), u) == 0.0)
    assert np.all(orc.swiglu(g, np.zeros(1000, np.float32)) == 0.0)
    # silu(g) - silu(-g) == g: sigmoid(g) + sigmoid(-g) == 1
    one = np.ones(1000, np.float32)
    d = orc.swiglu(g, one).astype(np.float64) - orc.swiglu(-g, one).astype(np.float64)
    helpers.assert_within(d, g.astype(np.float64), 2 * helpers.U32 * (np.abs(g) + 1e-30) * 2,
                          "silu(g) - silu(-g)")
    # far tails: silu(50) rounds to 50, silu(-50) is ~ -1e-20
    big = np.full(4, 50.0, np.float32)
    assert np.array_equal(orc.swiglu(big, u[:4]), (big * u[:4]).astype(np.float32))
    assert np.all(np.abs(orc.swiglu(-big, one[:4])) < 1e-19)
    # fp16 form on the same values
    g16, u16 = orc.f32_to_f16(g), orc.f32_to_f16(u)
    assert np.all(orc.swiglu_fp16(np.zeros(1000, np.uint16), u16) & 0x7FFF == 0)


def test_rmsnorm_linear_swiglu_is_the_composition(orc):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((4, 96), dtype=np.float32)
    g = (1 + 0.1 * rng.standard_normal(96)).astype(np.float32)
    Wg = rng.standard_normal((96, 50), dtype=np.float32) / 10
    Wu = rng.standard_normal((96, 50), dtype=np.float32) / 10
    for W1, W2 in ((Wg, Wu), (orc.f32_to_f16(Wg), orc.f32_to_f16(Wu))):
        ref = orc.swiglu(orc.rmsnorm_linear(x, g, W1, EPS), orc.rmsnorm_linear(x, g, W2, EPS))
        assert np.array_equal(orc.rmsnorm_linear_swiglu(x, g, W1, W2, EPS), ref)


# ---------------------------------------------------------------------- half
def test_half_to_float_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def half_probe_floats() -> np.ndarray:
    rng = np.random.default_rng(9)
    sampled = rng.integers(0, 2**32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    # every float next to a half rounding boundary (+-1 ulp around each midpoint)
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32).view(np.uint32)
    edges = np.concatenate([mids - 1, mids, mids + 1, np.array([0x477FF000, 0x477FEFFF, 0x33000000,
                                                                  0x33000001, 0x7F800000, 0x7FC00000], np.uint32)])
    allb = np.concatenate([sampled, edges, edges | 0x80000000]).astype(np.uint32)
    return allb.view(np.float32)


def test_float_to_half_matches_numpy(orc):
    f = half_probe_floats()
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16)
    got = orc.f32_to_f16(f)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], ref[~nan].view(np.uint16))


# ------------------------------------------------------------ planted mistakes
@pytest.mark.parametrize("mutation,check", [
    (1, lambda o: check_matmul(o, helpers.case("matmul__128x64x256"))),
    (2, lambda o: check_gemv(o, helpers.case("gemv__256x4096"))),
    (3, lambda o: check_rmsnorm(o, helpers.case("rmsnorm__1x4096_w"))),
    (4, lambda o: check_rmsnorm_linear(o, helpers.case("rmsnorm_linear__32x256x512_w"))),
    (5, lambda o: test_float_to_half_matches_numpy(o)),
    (6, lambda o: check_swiglu(o, helpers.case("swiglu__n1024"))),
    (7, lambda o: check_residual_rmsnorm(o, helpers.case("residual_rmsnorm__1x4096_w"))),
    (8, lambda o: check_attention(o, helpers.case("attention__s1_kv257_h32_kv4_d64_decode"))),
])
def test_planted_mistakes_are_caught(mutation, check):
    mutant = helpers.oracle(mutation)
    assert mutant.mutation() == mutation
    with pytest.raises(AssertionError):
        check(mutant)
