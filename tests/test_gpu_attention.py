"""GPU parity of decode attention (FlashDecoding over an fp16 KV cache) and
its bridge kernels, called through the C-ABI, against the float64 golden
fixtures (the reference's decode attention cases) and the C oracle.

Two tolerances are checked everywhere:
* the reference's own decode tolerance (tests/test_kernels.cu:292-296):
  |got - exp| <= 1.5 * 2^-10 + 4 * s_kv * 2^-23 + 2 * 2^-10 * |exp|;
* a derived bound (u = 2^-24): with w_j = exp(s_j - max s), the fp32 scores
  carry |ds_j| <= (D + 1) u scale sum_d |q_d k_jd| =: e_j; the kernel forms
  weights as 2^((s_j - m) log2 e) with the scale, the subtraction and the
  hardware exp2 rounding once each (<= 4 u max_j |s_j| + 8 u relative), so the
  weights carry at most 2 max_j e_j + 4 u max_j |s_j| + 8 u relative error;
  the fp32 sums of p_j v_j and p_j add (s_kv + 24) u relative to
  sum_j w_j |v_j|; the matrix-core kernel (GQA groups) multiplies V by each
  weight as two fp16 terms (hi + lo, scaled by 2^7), which adds 4 u relative
  and at most 2^-32 absolute per weight (the max key's weight is >= 1, so
  s_kv 2^-32 max_j |v_j| in all); the output adds half rounding 2^-11 |y| + 2^-25:
      |got - y| <= 2^-11 |y| + 2^-25 + s_kv 2^-32 max_j |v_j|
                   + (2 max e + 4 u max |s| + (s_kv + 36) u) (sum_j w_j |v_j| / sum_j w_j + |y|).
Long sequences (8K / 32K keys) also use the reference's output-scaled
tolerance (test_kernels.cu:2565-2640): rtol = 2^-9, atol = rtol * rms(out).
"""

from __future__ import annotations

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
U = helpers.U32


def decode64(q, k, v, H, Hkv, D, L, stride, scale):
    """float64 decode attention and the derived bound; q [H, D] / k / v flat
    half bits with `stride` elements per KV head."""
    q64 = helpers.as_f64(q).reshape(H, D)
    k64 = helpers.as_f64(k).reshape(Hkv, -1)
    v64 = helpers.as_f64(v).reshape(Hkv, -1)
    group = H // Hkv
    y = np.zeros((H, D))
    bound = np.zeros((H, D))
    for h in range(H):
        kh = k64[h // group, : L * D].reshape(L, D)
        vh = v64[h // group, : L * D].reshape(L, D)
        s = kh @ q64[h] * scale
        w = np.exp(s - s.max())
        y[h] = (w @ vh) / w.sum()
        e = (D + 1) * U * scale * (np.abs(kh) @ np.abs(q64[h]))
        mag = (w @ np.abs(vh)) / w.sum() + np.abs(y[h])
        rel = 2 * e.max() + 4 * U * np.abs(s).max() + (L + 36) * U
        bound[h] = (helpers.U16 * np.abs(y[h]) + 2.0**-25 + L * 2.0**-32 * np.abs(vh).max()
                    + rel * mag)
    return y, bound


def reference_tol(exp, s_kv):
    return 1.5 * 2.0**-10 + 4.0 * s_kv * 2.0**-23 + 2.0 * 2.0**-10 * np.abs(exp)


def gpu_decode(eng, q, k, v, L, H, Hkv, D, stride, scale, split_kv=0, share=None, out_fill=None,
               k_offset=0):
    dq, dk, dv = eng.upload(q), eng.upload(k), eng.upload(v)
    dout = eng.empty((H, D), np.uint16)
    if out_fill is not None:
        dout.upload(np.full((H, D), out_fill, np.uint16))
    if share is None:
        eng.call("eng_attention_decode_f16", dq.ptr, dk.ptr + 2 * k_offset, dv.ptr + 2 * k_offset,
                 dout.ptr, L, H, Hkv, D, stride, scale, split_kv, None)
    else:
        eng.call("eng_attention_decode_with_mode_f16", dq.ptr, dk.ptr + 2 * k_offset,
                 dv.ptr + 2 * k_offset, dout.ptr, L, H, Hkv, D, stride, scale, split_kv,
                 int(share), None)
    eng.sync()
    return dout.download()


def check_decode(got16, q, k, v, H, Hkv, D, L, stride, scale, orc, what):
    got = helpers.as_f64(got16).reshape(H, D)
    y, bound = decode64(q, k, v, H, Hkv, D, L, stride, scale)
    helpers.assert_within(got, y, bound, what + " [derived bound]")
    helpers.assert_within(got, y, reference_tol(y, L), what + " [reference tolerance]")
    ref = helpers.as_f64(orc.attention(q, k, v, H, Hkv, D, L, stride, scale)).reshape(H, D)
    helpers.assert_within(got, ref, bound + helpers.U16 * np.abs(ref) + 2.0**-25, what + " [vs oracle]")
    return got


def rand_half(orc, rng, shape, amp=1.0):
    return orc.f32_to_f16((amp * rng.standard_normal(shape)).astype(np.float32))


# ------------------------------------------------------------------ goldens
DECODE_STEMS = [c["stem"] for c in helpers.cases("attention") if c["params"]["s_q"] == 1]


@pytest.mark.parametrize("stem", DECODE_STEMS)
@pytest.mark.parametrize("split_kv", [0, 1, 8])
def test_attention_decode_matches_golden(gpu, orc, stem, split_kv):
    c = helpers.case(stem)
    x = helpers.inputs(c)
    P = c["params"]
    H, Hkv, D, L = P["n_heads"], P["n_kv_heads"], P["head_dim"], P["s_kv"]
    scale = 1.0 / np.sqrt(D)
    got = gpu_decode(gpu, x["q"], x["k"], x["v"], L, H, Hkv, D, L * D, scale, split_kv)
    exp = helpers.expected(c).reshape(H, D)
    helpers.assert_within(helpers.as_f64(got), exp, reference_tol(exp, L), f"{stem} split={split_kv} golden")
    check_decode(got, x["q"], x["k"], x["v"], H, Hkv, D, L, L * D, scale, orc, f"{stem} split={split_kv}")


def test_attention_decode_splits_and_edges(gpu, orc):
    """Reference attention_decode_splits_and_contracts, GPU part."""
    c = helpers.case("attention__s1_kv513_h8_kv2_d128_decode")
    x = helpers.inputs(c)
    q, k, v = x["q"], x["k"], x["v"]
    H, Hkv, D, L = 8, 2, 128, 513
    sc = 1.0 / np.sqrt(D)
    s1 = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, 1)
    s8 = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, 8)
    _, bound = decode64(q, k, v, H, Hkv, D, L, L * D, sc)
    helpers.assert_within(helpers.as_f64(s1), helpers.as_f64(s8).reshape(s1.shape),
                          2 * bound.reshape(s1.shape), "split 1 vs 8")
    # kv_len = 3 < split_kv = 16 (clamped), kv_len = 1 (exactly the value row)
    got3 = gpu_decode(gpu, q, k, v, 3, H, Hkv, D, L * D, sc, 16)
    check_decode(got3, q, k, v, H, Hkv, D, 3, L * D, sc, orc, "kv_len 3 < split 16")
    got1 = gpu_decode(gpu, q, k, v, 1, H, Hkv, D, L * D, sc, 0)
    vv = v.reshape(Hkv, L, D)
    for h in range(H):
        assert np.array_equal(got1[h], vv[h // 4, 0]), h
    # kv_len = 0 zero-fills (output prefilled with 5.0)
    got0 = gpu_decode(gpu, q, k, v, 0, H, Hkv, D, 0, sc, 4, out_fill=0x4500)
    assert np.all(got0 == 0)
    # one query head per workgroup (no GQA sharing), split 8
    ns = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, 8, share=False)
    check_decode(ns, q, k, v, H, Hkv, D, L, L * D, sc, orc, "per-head split 8")


def test_attention_decode_concurrent_streams_reuse_scratch(gpu, orc):
    c = helpers.case("attention__s1_kv513_h8_kv2_d128_decode")
    x = helpers.inputs(c)
    q, k, v = x["q"], x["k"], x["v"]
    H, Hkv, D, L = 8, 2, 128, 513
    sc = 1.0 / np.sqrt(D)
    dq, dk, dv = gpu.upload(q), gpu.upload(k), gpu.upload(v)
    da, db = gpu.empty((H, D), np.uint16), gpu.empty((H, D), np.uint16)
    sa, sb = gpu.stream(), gpu.stream()
    try:
        for _ in range(4):
            gpu.call("eng_attention_decode_f16", dq.ptr, dk.ptr, dv.ptr, da.ptr, L, H, Hkv, D, L * D,
                     sc, 8, sa.handle)
            gpu.call("eng_attention_decode_f16", dq.ptr, dk.ptr, dv.ptr, db.ptr, 257, H, Hkv, D, L * D,
                     sc, 8, sb.handle)
        sa.sync()
        sb.sync()
    finally:
        sa.destroy()
        sb.destroy()
    check_decode(da.download(), q, k, v, H, Hkv, D, L, L * D, sc, orc, "stream A")
    check_decode(db.download(), q, k, v, H, Hkv, D, 257, L * D, sc, orc, "stream B (kv_len 257)")


def test_attention_decode_repeated_calls_and_streams(gpu, orc):
    """Back-to-back GQA calls (D = 64, the MFMA kernel) with new data on one
    stream, reusing the stream's partial-state scratch at several split
    counts; the same data twice (fixed merge order: equal bits); and two
    streams interleaving calls of different lengths and split counts."""
    H, Hkv, D = 32, 4, 64
    sc = 1.0 / np.sqrt(D)
    rng = np.random.default_rng(77)
    first = None
    for rep, (L, split) in enumerate([(2048, 0), (2048, 0), (1500, 16), (777, 5), (2048, 0)]):
        q = rand_half(orc, rng, (H, D))
        k = rand_half(orc, rng, (Hkv, L, D))
        v = rand_half(orc, rng, (Hkv, L, D))
        got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split)
        check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"call {rep} L={L} split={split}")
        if rep == 0:
            first = (q, k, v, got)
    q, k, v, got0 = first
    again = gpu_decode(gpu, q, k, v, 2048, H, Hkv, D, 2048 * D, sc, 0)
    assert np.array_equal(again, got0), "same inputs, different bits"

    La, Lb = 2048, 1200
    qa, ka, va = (rand_half(orc, rng, sh) for sh in ((H, D), (Hkv, La, D), (Hkv, La, D)))
    qb, kb, vb = (rand_half(orc, rng, sh) for sh in ((H, D), (Hkv, Lb, D), (Hkv, Lb, D)))
    dqa, dka, dva = gpu.upload(qa), gpu.upload(ka), gpu.upload(va)
    dqb, dkb, dvb = gpu.upload(qb), gpu.upload(kb), gpu.upload(vb)
    da, db = gpu.empty((H, D), np.uint16), gpu.empty((H, D), np.uint16)
    sa, sb = gpu.stream(), gpu.stream()
    try:
        for _ in range(4):
            gpu.call("eng_attention_decode_f16", dqa.ptr, dka.ptr, dva.ptr, da.ptr, La, H, Hkv, D,
                     La * D, sc, 0, sa.handle)
            gpu.call("eng_attention_decode_f16", dqb.ptr, dkb.ptr, dvb.ptr, db.ptr, Lb, H, Hkv, D,
                     Lb * D, sc, 24, sb.handle)
        sa.sync()
        sb.sync()
    finally:
        sa.destroy()
        sb.destroy()
    check_decode(da.download(), qa, ka, va, H, Hkv, D, La, La * D, sc, orc, "stream A")
    check_decode(db.download(), qb, kb, vb, H, Hkv, D, Lb, Lb * D, sc, orc, "stream B")


# --------------------------------------------------------- model shapes
@pytest.mark.parametrize("H,Hkv,D,L,split", [
    (32, 32, 128, 2048, 0),   # Llama-2-7B, MHA
    (32, 4, 64, 2048, 0),     # TinyLlama, GQA 8
    (32, 4, 64, 2048, 1),     # one split per head group
    (12, 3, 128, 1000, 0),    # GQA 4, ragged
    (10, 5, 64, 777, 3),      # GQA 2
    (6, 6, 64, 300, 0),       # short sequence: one split
    (8, 2, 64, 96, 3),        # one 32-key block per split: one-wave splits
    (32, 4, 64, 4096, 100),   # more than 64 splits: the 1024-thread merge
    (16, 2, 64, 6000, 200),   # ragged splits of 30 keys, 200 states per head
])
def test_attention_decode_shapes_against_oracle(gpu, orc, H, Hkv, D, L, split):
    rng = np.random.default_rng(H * 1000 + L)
    q = rand_half(orc, rng, (H, D))
    k = rand_half(orc, rng, (Hkv, L, D))
    v = rand_half(orc, rng, (Hkv, L, D))
    sc = 1.0 / np.sqrt(D)
    got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split)
    check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"decode H={H}/{Hkv} D={D} L={L}")


@pytest.mark.parametrize("D", [64, 128])
def test_attention_decode_every_pipeline_depth(gpu, orc, D):
    """One split per head group with 1..12 tiles of 4096 / D keys, the last
    one ragged: the pipelined kernel's prologue, steady loop and every tail
    length (and GQA 4 sharing) against the oracle."""
    rng = np.random.default_rng(D)
    H, Hkv = 8, 2
    T = 4096 // D
    for ntiles in range(1, 13):
        L = T * ntiles - (5 if ntiles > 1 else 0)
        q = rand_half(orc, rng, (H, D))
        k = rand_half(orc, rng, (Hkv, L, D))
        v = rand_half(orc, rng, (Hkv, L, D))
        sc = 1.0 / np.sqrt(D)
        got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, 1)
        check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"D={D} tiles={ntiles} L={L}")


@pytest.mark.parametrize("D", [64, 128])
def test_attention_decode_single_head_every_shape(gpu, orc, D):
    """One query head per KV head, one split, lengths of 1 to 70 32-key blocks:
    the register-fed single-head kernel with 1, 2, 4 and 8 waves, 1, 2 and 4
    blocks in flight per wave and its ring (D = 128 past 16 blocks), and at
    D = 64 the hand-over to the LDS kernel past 32 blocks; ragged last blocks,
    and two splits with ragged ends, against the oracle."""
    rng = np.random.default_rng(300 + D)
    H = Hkv = 4
    sc = 1.0 / np.sqrt(D)
    for L, split in ((1, 1), (31, 1), (33, 1), (64, 1), (100, 1), (250, 1), (256, 1),
                     (290, 1), (512, 1), (530, 1), (1000, 1), (1024, 1), (1060, 1),
                     (2240, 1), (1111, 2), (777, 3)):
        q = rand_half(orc, rng, (H, D))
        k = rand_half(orc, rng, (Hkv, L, D))
        v = rand_half(orc, rng, (Hkv, L, D))
        got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split)
        check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"single head D={D} L={L} split={split}")


@pytest.mark.parametrize("D", [64, 128])
def test_attention_decode_gqa_every_shape(gpu, orc, D):
    """GQA groups (4 query heads per KV head; also 2 and 8) on the matrix-core
    kernel, one split, lengths of 1 to 70 32-key blocks: 1, 2, 4 and 8 waves,
    1, 2 and (D = 64) 4 blocks in flight per wave, and the ring (D = 128 past 16
    blocks, D = 64 past 32); ragged last blocks and splits, against the oracle."""
    rng = np.random.default_rng(500 + D)
    sc = 1.0 / np.sqrt(D)
    cases = [(8, 2, L, split) for L, split in ((1, 1), (31, 1), (33, 1), (64, 1), (100, 1), (250, 1),
                                                (256, 1), (290, 1), (512, 1), (530, 1), (1000, 1),
                                                (1024, 1), (1060, 1), (2240, 1), (1111, 2), (777, 3))]
    cases += [(16, 2, 530, 1), (16, 2, 2240, 0), (4, 2, 290, 1), (4, 2, 1060, 2)]
    for H, Hkv, L, split in cases:
        q = rand_half(orc, rng, (H, D))
        k = rand_half(orc, rng, (Hkv, L, D))
        v = rand_half(orc, rng, (Hkv, L, D))
        got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split)
        check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"GQA H={H}/{Hkv} D={D} L={L} split={split}")


def test_attention_decode_unaligned_cache_takes_scalar_loads(gpu, orc):
    """K / V not 16-byte aligned, and a head stride that is not a multiple of 8."""
    rng = np.random.default_rng(41)
    H, Hkv, D, L = 8, 2, 64, 300
    stride = L * D + 3
    q = rand_half(orc, rng, (H, D))
    k = np.zeros(Hkv * stride + 1, np.uint16)
    v = np.zeros(Hkv * stride + 1, np.uint16)
    kk = rand_half(orc, rng, (Hkv, L, D))
    vv = rand_half(orc, rng, (Hkv, L, D))
    for h in range(Hkv):
        k[1 + h * stride: 1 + h * stride + L * D] = kk[h].ravel()
        v[1 + h * stride: 1 + h * stride + L * D] = vv[h].ravel()
    sc = 1.0 / np.sqrt(D)
    got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, stride, sc, 0, k_offset=1)
    check_decode(got, q, k[1:], v[1:], H, Hkv, D, L, stride, sc, orc, "unaligned cache")


@pytest.mark.parametrize("L,D", [(8192, 64), (32768, 64), (8192, 128), (32768, 128)])
def test_attention_decode_long_sequence(gpu, orc, L, D):
    """Reference attention_decode_long_sequence: GQA 8:1, D = 64 (and the same
    at D = 128), a strided KV cache padded with NaN past kv_len (never read),
    O(1) outputs."""
    rng = np.random.default_rng(L + D)
    H, Hkv = 8, 1
    stride = (L + 17) * D
    nan16 = np.uint16(0x7E00)
    sc = 1.0 / np.sqrt(D)
    q = rand_half(orc, rng, (H, D), 0.5)
    kk = rand_half(orc, rng, (L, D), 0.5)
    pos = np.linspace(-1, 1, L)[:, None]
    vv = orc.f32_to_f16((0.5 + 0.5 * pos + 0.25 * rng.standard_normal((L, D))).astype(np.float32))

    def cache(body):
        c = np.full(Hkv * stride, nan16, np.uint16)
        c[: L * D] = body.ravel()
        return c

    k, v = cache(kk), cache(vv)
    ref = helpers.as_f64(orc.attention(q, k, v, H, Hkv, D, L, stride, sc)).reshape(H, D)
    rtol = 2.0**-9
    atol = rtol * max(1e-3, float(np.sqrt(np.mean(ref**2))))
    for split, share in ((0, True), (1, True), (0, False)):
        got = helpers.as_f64(gpu_decode(gpu, q, k, v, L, H, Hkv, D, stride, sc, split, share=share))
        assert np.isfinite(got).all()
        helpers.assert_within(got, ref, atol + rtol * np.abs(ref), f"L={L} split={split} share={share}")
    # needles: one key far above the rest, at the last position, then two equal
    # needles in different splits (cross-split merge)
    qn = orc.f32_to_f16(np.full((H, D), 0.5, np.float32))
    for js in ((L - 1,), (17, L - 1)):
        kn = np.zeros((L, D), np.float32)
        for j in js:
            kn[j] = 8.0
        vn = orc.f32_to_f16((rng.standard_normal((L, D))).astype(np.float32))
        target = helpers.as_f64(vn[list(js)]).mean(axis=0)
        got = helpers.as_f64(gpu_decode(gpu, qn, cache(orc.f32_to_f16(kn)), cache(vn), L, H, Hkv, D,
                                        stride, sc, 0)).reshape(H, D)
        for h in range(H):
            helpers.assert_within(got[h], target, rtol * (1 + np.abs(target)), f"needle {js} h={h}")


# ------------------------------------------------------- adversarial softmax
def adversarial_case(name, D, L, Hq=8, Hkv=2):
    """The decode cases of the reference's attention_adversarial_softmax
    (tests/test_kernels.cu, kv_len = 260, 8 / 2 heads): q = 2 on dims 0..3 and
    k = s on dims 0..3, so with scale 1 / 8 (D = 64) every score is exactly the
    s below; V is the reference's deterministic code ((17 j + 5 d + 11 g + 3)
    % 31 - 15) / 16. At D = 128 the same q and k give scores s * 8 / sqrt(128)."""
    q = np.zeros((Hq, D), np.float32)
    k = np.zeros((Hkv, L, D), np.float32)
    j = np.arange(L)
    if name == "all_equal":
        for h in range(Hq):
            q[h, :4] = (25.0, 100.0, -30.0, -100.0)[h % 4]
        k[:, :, :4] = 2.0
    else:
        q[:, :4] = 2.0
        for g in range(Hkv):
            if name == "neg_30_100":
                s = (-30.0 if g == 0 else -100.0) - (j % 4)
            elif name == "mixed_30":
                s = np.where(j == 199, 30.0, np.where(j % 2 == 0, 10.0, -30.0))
            else:  # dominant key
                s = np.where(j == 197, 30.0, -20.0)
            k[g, :, :4] = s[:, None]
    g_, j_, d_ = np.meshgrid(np.arange(Hkv), j, np.arange(D), indexing="ij")
    v = (((j_ * 17 + d_ * 5 + g_ * 11 + 3) % 31) - 15).astype(np.float32) * 0.0625
    f16 = lambda a: a.astype(np.float16).view(np.uint16)
    return f16(q), f16(k), f16(v)


@pytest.mark.parametrize("split", [1, 4])
def test_attention_decode_many_small_weights(gpu, orc, split):
    """One dominant key (score 10, V row 0) and 2047 keys at score -2.0254
    (weight ~e^-12 ~ 2^-17.3 each, V = 1): every small weight rounds the same
    way, so their errors add up coherently. The matrix-core kernel multiplies
    V by each weight as fp16 hi + lo; taken unscaled, weights this small fall
    below fp16's normal range, and this score puts the weight near the middle
    of a subnormal step (2^-25 absolute each: 6.0e-5 in the output, against a
    derived bound of about 1.2e-5); scaled by 2^7 they err by 2^-32 each
    (2e-7 in the output)."""
    H, Hkv, D, L = 32, 4, 64, 2048
    q = np.zeros((H, D), np.float32)
    q[:, :4] = 2.0                                   # score = k value on dims 0..3 (scale 1/8)
    k = np.zeros((Hkv, L, D), np.float32)
    k[:, 0, :4] = 10.0
    kval = float(np.float16(-2.025))
    k[:, 1:, :4] = kval
    v = np.ones((Hkv, L, D), np.float32)
    v[:, 0, :] = 0.0
    f16 = lambda a: a.astype(np.float16).view(np.uint16)
    q, k, v = f16(q), f16(k), f16(v)
    sc = 1.0 / np.sqrt(D)
    got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split)
    check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"small weights split={split}")
    w = (L - 1) * np.exp(kval - 10.0)
    helpers.assert_within(helpers.as_f64(got), np.full((H, D), w / (1 + w)), 2.0**-11 * w,
                          "small weights closed form")


@pytest.mark.parametrize("name", ["neg_30_100", "mixed_30", "all_equal", "dominant"])
@pytest.mark.parametrize("D", [64, 128])
def test_attention_decode_adversarial_softmax(gpu, orc, name, D):
    """Scores of -30..-103 (underflow without the max), +10 then +30 in a late
    tile (the lazy rescale must fire across tiles and splits), equal logits up
    to +100 (overflow without the max) and one dominant key, for every kernel:
    automatic splits, one split, 8 splits, one head per workgroup, and the
    unaligned-cache kernels."""
    H, Hkv, L = 8, 2, 260
    q, k, v = adversarial_case(name, D, L, H, Hkv)
    sc = 1.0 / np.sqrt(D)
    for split, share in ((0, None), (1, None), (8, None), (8, False)):
        got = gpu_decode(gpu, q, k, v, L, H, Hkv, D, L * D, sc, split, share=share)
        assert np.isfinite(helpers.as_f64(got)).all()
        check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"{name} D={D} split={split} share={share}")
    # the same cache one element off 16-byte alignment
    ku = np.concatenate([np.zeros(1, np.uint16), k.ravel()])
    vu = np.concatenate([np.zeros(1, np.uint16), v.ravel()])
    got = gpu_decode(gpu, q, ku, vu, L, H, Hkv, D, L * D, sc, 8, k_offset=1)
    check_decode(got, q, k, v, H, Hkv, D, L, L * D, sc, orc, f"{name} D={D} unaligned")
    if name == "dominant" and D == 64:
        # closed form: every head's output is key 197's value row (weight ratio e^-50)
        vv = helpers.as_f64(v).reshape(Hkv, L, D)
        for h in range(H):
            assert np.array_equal(helpers.as_f64(got[h]), vv[h // 4, 197]), h


# ------------------------------------------------------------------- bridge
def test_cast_kernels_are_exact(gpu, orc):
    rng = np.random.default_rng(42)
    f = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1000,
                        np.array([65504.0, 65520.0, 1e-8, -0.0, np.inf], np.float32)])
    d_in, d_h = gpu.upload(f), gpu.empty(f.shape, np.uint16)
    gpu.call("eng_cast_f32_to_f16", d_in.ptr, d_h.ptr, f.size, None)
    gpu.sync()
    with np.errstate(over="ignore"):
        assert np.array_equal(d_h.download(), f.astype(np.float16).view(np.uint16))
    bits = np.arange(0, 0x7C00, dtype=np.uint16)
    d_b, d_f = gpu.upload(bits), gpu.empty(bits.shape, np.float32)
    gpu.call("eng_cast_f16_to_f32", d_b.ptr, d_f.ptr, bits.size, None)
    gpu.sync()
    assert np.array_equal(d_f.download(), bits.view(np.float16).astype(np.float32))


def test_kv_cache_write_scatters_token_major_to_head_major(gpu):
    rng = np.random.default_rng(43)
    s_new, Hkv, D, max_seq, pos = 5, 3, 64, 40, 11
    kn = rng.integers(0, 0x7BFF, (s_new, Hkv, D)).astype(np.uint16)
    vn = rng.integers(0, 0x7BFF, (s_new, Hkv, D)).astype(np.uint16)
    kc = np.full((Hkv, max_seq, D), 7, np.uint16)
    vc = np.full((Hkv, max_seq, D), 9, np.uint16)
    dkn, dvn, dkc, dvc = gpu.upload(kn), gpu.upload(vn), gpu.upload(kc), gpu.upload(vc)
    gpu.call("eng_kv_cache_write_f16", dkn.ptr, dvn.ptr, dkc.ptr, dvc.ptr, s_new, Hkv, D, pos, max_seq, None)
    gpu.sync()
    ek, ev = kc.copy(), vc.copy()
    ek[:, pos:pos + s_new] = kn.transpose(1, 0, 2)
    ev[:, pos:pos + s_new] = vn.transpose(1, 0, 2)
    assert np.array_equal(dkc.download(), ek)
    assert np.array_equal(dvc.download(), ev)
