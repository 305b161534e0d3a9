"""Writes the golden fixtures under tests/golden/data/ and tests/golden/manifest.json.

Run from the repository root:  python tests/golden/gen_golden.py

Case tables follow the reference's generator (reference
tools/gen_reference.py:401-440 for shapes, :668-741 for distributions):
inputs ~ N(0, 1), matrices scaled by 1/sqrt(K), RMSNorm gains ~ 1 + N(0, 0.1^2),
eps = 1e-5. Added cases: BASELINE config 1 (512^3, U[-1, 1], seed 0) and the
fp16-weight variants with fp32 activations (gemv_f16w, rmsnorm_linear_f16w).
The FFN-side ops follow :410-415 (residual_rmsnorm), :451 (swiglu) and
:488-491 / :906-928 (FFN sub-block); the fused gate/up + SwiGLU cases are this
build's own.

Inputs are not stored: each is rebuilt from its generator spec by
tests/golden/detgen.py and checked against the SHA-256 recorded here.
Expected outputs are computed in float64 with NumPy, independently of the C
oracle, and stored as float32 ENGREF01 tensors (the reference's convention).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import detgen  # noqa: E402
import engref  # noqa: E402

EPS = 1e-5

MATMUL_SHAPES = [(1, 1, 1), (32, 32, 32), (128, 64, 256), (17, 23, 31), (512, 512, 512)]
RMSNORM_SHAPES = [(1, 4096, True), (128, 4096, True), (32, 127, True), (32, 4096, False)]
RMSNORM_LINEAR_SHAPES = [
    (1, 256, 4096, True),
    (32, 256, 512, True),
    (1, 768, 256, True),
    (17, 127, 31, True),
    (32, 256, 512, False),
]
GEMV_SHAPES = [(256, 4096), (768, 256), (127, 31), (64, 128)]
GEMV_FP16_SHAPES = [(64, 64), (128, 256), (73, 125), (256, 4096)]
# reference tools/gen_reference.py:410-415, :451, :488-491
RESIDUAL_RMSNORM_SHAPES = [(1, 4096, True), (128, 4096, True), (32, 127, True), (32, 4096, False)]
SWIGLU_SIZES = [1, 65, 1024, 4096, 11008]
FFN_SUBBLOCK_CASES = [("prefill_s16_d512_ffn1408", 16, 512, 1408), ("decode_s1_d512_ffn1408", 1, 512, 1408)]
# Fused gate/up + SwiGLU of the FFN (no reference counterpart): decode, prefill, ragged.
RMSNORM_LINEAR_SWIGLU_SHAPES = [(1, 1408, 512, True), (16, 1408, 512, True), (3, 257, 100, False)]
# reference :379 without its 1 Mi case (tests check large sizes against float32 addition)
VECTOR_ADD_SIZES = [1, 31, 32, 33, 255, 256, 257, 4096]
# reference :466-477 -- the decode rows (s_q = 1) plus two causal prefill rows
# that pin the general oracle: (name, s_q, s_kv, n_heads, n_kv_heads, head_dim, q_pos_offset, causal)
ATTENTION_CASES = [
    ("s1_h1_d64_causal", 1, 1, 1, 1, 64, 0, True),
    ("s1_kv31_h4_d64_nocausal", 1, 31, 4, 4, 64, 0, False),
    ("s1_kv257_h32_kv4_d64_decode", 1, 257, 32, 4, 64, 256, False),
    ("s1_kv513_h8_kv2_d128_decode", 1, 513, 8, 2, 128, 512, False),
    ("s17_h8_kv2_d64_causal", 17, 17, 8, 2, 64, 0, True),
    ("s33_kv65_h8_kv2_d128_off32_causal", 33, 65, 8, 2, 128, 32, True),
]


def f64(a: np.ndarray, dtype: str) -> np.ndarray:
    """Value of a generated input in float64 (f16 inputs are bit patterns)."""
    if dtype == "f16":
        return a.view(np.float16).astype(np.float64)
    return a.astype(np.float64)


def silu64(g: np.ndarray) -> np.ndarray:
    """g * sigmoid(g) with the overflow-safe sigmoid of the reference's generator
    (tools/gen_reference.py:158-163)."""
    e = np.exp(-np.abs(g))
    return g * np.where(g >= 0.0, 1.0 / (1.0 + e), e / (1.0 + e))


def attention64(q, k, v, scale, q_pos_offset, causal):
    """float64 two-pass softmax attention (reference gen_reference.py attention):
    q [s_q, H, D], k / v [H_kv, s_kv, D] -> (out [s_q, H, D], lse [s_q, H])."""
    s_q, H, D = q.shape
    H_kv, s_kv, _ = k.shape
    group = H // H_kv
    out = np.zeros((s_q, H, D))
    lse = np.full((s_q, H), -np.inf)
    for i in range(s_q):
        last = min(s_kv - 1, q_pos_offset + i) if causal else s_kv - 1
        if last < 0:
            continue
        for h in range(H):
            kh, vh = k[h // group, : last + 1], v[h // group, : last + 1]
            s = (kh @ q[i, h]) * scale
            m = s.max()
            w = np.exp(s - m)
            out[i, h] = (w @ vh) / w.sum()
            lse[i, h] = m + np.log(w.sum())
    return out, lse


def rms_rows(x64: np.ndarray, w64) -> np.ndarray:
    out = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + EPS)
    if w64 is not None:
        out = out * w64
    return out


class Builder:
    def __init__(self):
        self.cases = []
        self.next_seed = 1

    def spec(self, gen, shape, dtype="f32", **kw):
        s = {"gen": gen, "shape": list(shape), "dtype": dtype, "seed": self.next_seed, **kw}
        self.next_seed += 1
        return s

    def add(self, stem, op, params, specs, expected, extra=None):
        inputs = {}
        for name, s in specs.items():
            arr = detgen.make(s)
            inputs[name] = dict(s, sha256=detgen.digest(arr))
        tensors = {"expected": expected.astype(np.float32)}
        for name, arr in (extra or {}).items():
            tensors[name] = arr.astype(np.float32)
        engref.write(HERE / "data" / f"{stem}.bin", tensors)
        self.cases.append({"stem": stem, "op": op, "params": params, "inputs": inputs})

    def build(self):
        for m, n, k in MATMUL_SHAPES:
            sc = 1.0 / np.sqrt(max(k, 1))
            specs = {"A": self.spec("normal", (m, k), std=sc), "B": self.spec("normal", (k, n), std=sc)}
            a, b = (f64(detgen.make(specs[x]), "f32") for x in ("A", "B"))
            self.add(f"matmul__{m}x{n}x{k}", "matmul", {"M": m, "N": n, "K": k}, specs, a @ b)

        # U[-1, 1], 512^3 (seed field records the config seed).
        specs = {
            "A": dict(self.spec("uniform", (512, 512), lo=-1.0, hi=1.0), seed=0),
            "B": dict(self.spec("uniform", (512, 512), lo=-1.0, hi=1.0), seed=100),
        }
        a, b = (f64(detgen.make(specs[x]), "f32") for x in ("A", "B"))
        self.add("matmul_cfg1__512x512x512", "matmul", {"M": 512, "N": 512, "K": 512}, specs, a @ b)

        for rows, cols, with_w in RMSNORM_SHAPES:
            specs = {"input": self.spec("normal", (rows, cols))}
            if with_w:
                specs["weight"] = self.spec("normal", (cols,), mean=1.0, std=0.1)
            x = f64(detgen.make(specs["input"]), "f32")
            w = f64(detgen.make(specs["weight"]), "f32") if with_w else None
            sfx = "w" if with_w else "now"
            self.add(f"rmsnorm__{rows}x{cols}_{sfx}", "rmsnorm",
                     {"rows": rows, "cols": cols, "eps": EPS}, specs, rms_rows(x, w))
        specs = {"input": self.spec("zeros", (2, 256))}
        self.add("rmsnorm__zeros", "rmsnorm", {"rows": 2, "cols": 256, "eps": EPS}, specs,
                 np.zeros((2, 256)))

        for wdt, tag in (("f32", "rmsnorm_linear"), ("f16", "rmsnorm_linear_f16w")):
            for m, n, k, with_w in RMSNORM_LINEAR_SHAPES:
                specs = {
                    "input": self.spec("normal", (m, k)),
                    "W": self.spec("normal", (k, n), dtype=wdt, std=1.0 / np.sqrt(max(k, 1))),
                }
                if with_w:
                    specs["weight"] = self.spec("normal", (k,), mean=1.0, std=0.1)
                x = f64(detgen.make(specs["input"]), "f32")
                W = f64(detgen.make(specs["W"]), wdt)
                w = f64(detgen.make(specs["weight"]), "f32") if with_w else None
                sfx = "w" if with_w else "now"
                self.add(f"{tag}__{m}x{n}x{k}_{sfx}", tag,
                         {"M": m, "N": n, "K": k, "eps": EPS}, specs, rms_rows(x, w) @ W)

        for n, k in GEMV_SHAPES:
            specs = {"A": self.spec("normal", (k, n), std=1.0 / np.sqrt(max(k, 1))),
                     "x": self.spec("normal", (k,))}
            A = f64(detgen.make(specs["A"]), "f32")
            x = f64(detgen.make(specs["x"]), "f32")
            self.add(f"gemv__{n}x{k}", "gemv", {"N": n, "K": k}, specs, x @ A)

        for xdt, tag in (("f16", "gemv_fp16"), ("f32", "gemv_f16w")):
            for n, k in GEMV_FP16_SHAPES:
                specs = {"A": self.spec("normal", (k, n), dtype="f16", std=1.0 / np.sqrt(max(k, 1))),
                         "x": self.spec("normal", (k,), dtype=xdt)}
                A = f64(detgen.make(specs["A"]), "f16")
                x = f64(detgen.make(specs["x"]), xdt)
                self.add(f"{tag}__{n}x{k}", tag, {"N": n, "K": k}, specs, x @ A)

        self.build_ffn_ops()

    def build_ffn_ops(self):
        """The ops either side of the linear layers (SwiGLU FFN)."""
        for n in VECTOR_ADD_SIZES:
            specs = {"a": self.spec("normal", (n,)), "b": self.spec("normal", (n,))}
            a, b = (f64(detgen.make(specs[x]), "f32") for x in ("a", "b"))
            self.add(f"vector_add__n{n}", "vector_add", {"n": n}, specs, a + b)

        for rows, cols, with_w in RESIDUAL_RMSNORM_SHAPES:
            specs = {"x": self.spec("normal", (rows, cols)), "residual": self.spec("normal", (rows, cols))}
            if with_w:
                specs["weight"] = self.spec("normal", (cols,), mean=1.0, std=0.1)
            x = f64(detgen.make(specs["x"]), "f32")
            r = f64(detgen.make(specs["residual"]), "f32")
            w = f64(detgen.make(specs["weight"]), "f32") if with_w else None
            sfx = "w" if with_w else "now"
            self.add(f"residual_rmsnorm__{rows}x{cols}_{sfx}", "residual_rmsnorm",
                     {"rows": rows, "cols": cols, "eps": EPS}, specs, rms_rows(x + r, w))
        specs = {"x": self.spec("zeros", (2, 256)), "residual": self.spec("zeros", (2, 256))}
        self.add("residual_rmsnorm__zeros", "residual_rmsnorm", {"rows": 2, "cols": 256, "eps": EPS},
                 specs, np.zeros((2, 256)))

        for dt, tag in (("f32", "swiglu"), ("f16", "swiglu_fp16")):
            for n in SWIGLU_SIZES:
                specs = {"gate": self.spec("normal", (n,), dtype=dt), "up": self.spec("normal", (n,), dtype=dt)}
                g, u = (f64(detgen.make(specs[x]), dt) for x in ("gate", "up"))
                self.add(f"{tag}__n{n}", tag, {"n": n}, specs, silu64(g) * u)

        for wdt, tag in (("f32", "rmsnorm_linear_swiglu"), ("f16", "rmsnorm_linear_swiglu_f16w")):
            for m, n, k, with_w in RMSNORM_LINEAR_SWIGLU_SHAPES:
                sc = 1.0 / np.sqrt(max(k, 1))
                specs = {
                    "input": self.spec("normal", (m, k)),
                    "Wg": self.spec("normal", (k, n), dtype=wdt, std=sc),
                    "Wu": self.spec("normal", (k, n), dtype=wdt, std=sc),
                }
                if with_w:
                    specs["weight"] = self.spec("normal", (k,), mean=1.0, std=0.1)
                x = f64(detgen.make(specs["input"]), "f32")
                Wg = f64(detgen.make(specs["Wg"]), wdt)
                Wu = f64(detgen.make(specs["Wu"]), wdt)
                w = f64(detgen.make(specs["weight"]), "f32") if with_w else None
                xn = rms_rows(x, w)
                gate, up = xn @ Wg, xn @ Wu
                sfx = "w" if with_w else "now"
                self.add(f"{tag}__{m}x{n}x{k}_{sfx}", tag, {"M": m, "N": n, "K": k, "eps": EPS},
                         specs, silu64(gate) * up, extra={"gate": gate, "up": up})

        for name, s_q, d, f in FFN_SUBBLOCK_CASES:
            specs = {
                "x": self.spec("normal", (s_q, d)),
                "ffn_rms_w": self.spec("normal", (d,), mean=1.0, std=0.1),
                "w_gate": self.spec("normal", (d, f), std=1.0 / np.sqrt(d)),
                "w_up": self.spec("normal", (d, f), std=1.0 / np.sqrt(d)),
                "w_down": self.spec("normal", (f, d), std=1.0 / np.sqrt(f)),
            }
            x, w, wg, wu, wd = (f64(detgen.make(specs[k]), "f32")
                                for k in ("x", "ffn_rms_w", "w_gate", "w_up", "w_down"))
            xn = rms_rows(x, w)
            act = silu64(xn @ wg) * (xn @ wu)
            self.add(f"ffn_subblock__{name}", "ffn_subblock", {"S": s_q, "D": d, "F": f, "eps": EPS},
                     specs, x + act @ wd, extra={"act": act})

        for name, s_q, s_kv, H, H_kv, D, off, causal in ATTENTION_CASES:
            specs = {
                "q": self.spec("normal", (s_q, H, D), dtype="f16"),
                "k": self.spec("normal", (H_kv, s_kv, D), dtype="f16"),
                "v": self.spec("normal", (H_kv, s_kv, D), dtype="f16"),
            }
            q, k, v = (f64(detgen.make(specs[x]), "f16") for x in ("q", "k", "v"))
            out, lse = attention64(q, k, v, 1.0 / np.sqrt(D), off, causal)
            self.add(f"attention__{name}", "attention",
                     {"s_q": s_q, "s_kv": s_kv, "n_heads": H, "n_kv_heads": H_kv, "head_dim": D,
                      "q_pos_offset": off, "is_causal": causal}, specs, out, extra={"lse": lse})


def main() -> None:
    b = Builder()
    b.build()
    manifest = {"generator": "tests/golden/detgen.py (SplitMix64, Irwin-Hall normals)",
                "eps": EPS, "cases": b.cases}
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"wrote {len(b.cases)} cases to {HERE / 'data'}")


if __name__ == "__main__":
    main()
