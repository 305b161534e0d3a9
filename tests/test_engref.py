"""ENGREF01 reader of the library (eng_engref_*), on the CPU.

The reader is the reference's golden reader (tests/golden.cpp:104-209) moved
into the engine, extended with dtype 1 (f16 at native size) and 2 (f64), plus
the slab layout of the planned mmap weight loader. Checked here without a
GPU: every committed fixture parses to what tests/golden/engref.py (an
independent Python reader) reads; every validation rule of the reference
reader rejects a file that breaks it, with the reference's message; f16
tensors keep their 2-byte size; the slab layout is aligned, ordered and
disjoint; upload preconditions are refused before any device call.
"""

from __future__ import annotations

import struct
import sys

import numpy as np
import pytest

import helpers

sys.path.insert(0, str(helpers.REPO / "tests" / "golden"))
import engref  # noqa: E402  (the Python reader/writer of the fixtures)

DATA = helpers.REPO / "tests" / "golden" / "data"
P = 0x1000  # dummy non-null device pointer, never dereferenced on these paths


def fixture_files():
    return sorted(DATA.glob("*.bin"))


@pytest.mark.parametrize("path", fixture_files(), ids=lambda p: p.stem)
def test_every_fixture_parses_like_the_python_reader(eng, path):
    ref = engref.read(path)
    with eng.engref(path) as f:
        assert f.size() == len(ref)
        assert f.names() == sorted(ref)
        for name, arr in ref.items():
            t = f.at(name)
            assert t.shape == arr.shape
            assert t.nbytes == arr.nbytes
            assert t.host.dtype.itemsize == arr.dtype.itemsize
            assert np.array_equal(t.host.view(np.uint8), arr.view(np.uint8))


def test_f16_is_stored_at_native_size(eng, tmp_path):
    rng = np.random.default_rng(0)
    w = rng.standard_normal((37, 129)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(129).astype(np.float32)
    d = rng.standard_normal(5)
    path = tmp_path / "mixed.bin"
    engref.write(path, {"W": w, "x": x, "d64": d})
    with eng.engref(path) as f:
        tw, tx, td = f.at("W"), f.at("x"), f.at("d64")
        assert (tw.dtype, tw.nbytes) == (1, 2 * w.size)
        assert (tx.dtype, tx.nbytes) == (0, 4 * x.size)
        assert (td.dtype, td.nbytes) == (2, 8 * d.size)
        assert np.array_equal(tw.host, w)
        assert np.array_equal(tx.host, x)
        assert np.array_equal(td.host, d)
        # file = header + data exactly: nothing padded on disk
        assert path.stat().st_size == 8 + 4 + sum(4 + len(n) + 8 + 8 * a.ndim + 8 + a.nbytes
                                                 for n, a in (("W", w), ("x", x), ("d64", d)))


def test_slab_layout_is_aligned_ordered_and_disjoint(eng, tmp_path):
    tensors = {"a": np.ones(3, np.float32), "b": np.zeros((0, 4), np.float32),
               "c": np.arange(300, dtype=np.uint16), "d": np.ones((2, 2), np.float64),
               "e": np.ones(64, np.float32)}
    path = tmp_path / "layout.bin"
    engref.write(path, tensors)
    with eng.engref(path) as f:
        prev_end = 0
        for t, name in zip(f.tensors, tensors):
            assert t.name == name  # file order
            assert t.slab_offset % 256 == 0
            assert t.slab_offset >= prev_end
            assert t.slab_offset - prev_end < 256  # no more padding than alignment needs
            prev_end = t.slab_offset + t.nbytes
        assert f.slab_bytes() % 256 == 0 and f.slab_bytes() >= prev_end
        assert f.slab_bytes() - prev_end < 256


def test_empty_and_zero_tensor_files(eng, tmp_path):
    path = tmp_path / "none.bin"
    engref.write(path, {})
    with eng.engref(path) as f:
        assert f.size() == 0 and f.slab_bytes() == 0
        assert eng.status("eng_engref_upload", f.handle, None, 0, None) == 0  # nothing to copy
    path = tmp_path / "scalar.bin"  # rank 0: one element
    path.write_bytes(header(1) + tensor_bytes(name=b"s", dims=(), data=struct.pack("<f", 2.5)))
    with eng.engref(path) as f:
        t = f.at("s")
        assert t.shape == () and t.nbytes == 4 and float(t.host) == 2.5
        assert f.slab_bytes() == 256


# ----------------------------------------------------------- malformed files
def header(count):
    return b"ENGREF01" + struct.pack("<i", count)


def tensor_bytes(name=b"t", code=0, dims=(2,), nbytes=None, data=None):
    esz = {0: 4, 1: 2, 2: 8}.get(code, 4)
    n = int(np.prod(dims, dtype=np.int64)) if dims else 1
    nb = n * esz if nbytes is None else nbytes
    data = bytes(max(nb, 0)) if data is None else data
    return (struct.pack("<i", len(name)) + name + struct.pack("<ii", code, len(dims))
            + b"".join(struct.pack("<q", d) for d in dims) + struct.pack("<q", nb) + data)


GOOD = header(1) + tensor_bytes()

MALFORMED = [
    ("empty", b"", "bad magic"),
    ("short_magic", b"ENGR", "bad magic"),
    ("wrong_magic", b"ENGREF02" + GOOD[8:], "bad magic"),
    ("no_count", b"ENGREF01", "unexpected end of file while reading n_tensors"),
    ("negative_count", header(-1), "implausible tensor count -1"),
    ("huge_count", header(4097), "implausible tensor count 4097"),
    ("missing_tensor", header(1), "unexpected end of file while reading name_len"),
    ("zero_name", header(1) + tensor_bytes(name=b""), "implausible name length 0"),
    ("long_name", header(1) + struct.pack("<i", 1025), "implausible name length 1025"),
    ("cut_name", header(1) + struct.pack("<i", 10) + b"abc", "truncated tensor name"),
    ("bad_dtype", header(1) + tensor_bytes(code=3), "has dtype 3"),
    ("bad_ndim", header(1) + tensor_bytes(dims=tuple(range(1, 10))), "implausible ndim 9"),
    ("negative_dim", header(1) + tensor_bytes(dims=(4, -2), nbytes=0), "negative dimension in 't'"),
    ("byte_mismatch", header(1) + tensor_bytes(dims=(3,), nbytes=8), "header says 8 bytes but its shape implies 12"),
    ("f16_as_f32_bytes", header(1) + tensor_bytes(code=1, dims=(3,), nbytes=12), "header says 12 bytes but its shape implies 6"),
    ("cut_data", header(1) + tensor_bytes()[:-3], "truncated data for 't'"),
    ("cut_dims", header(1) + tensor_bytes(dims=(2, 3))[:22], "unexpected end of file while reading dim"),
    ("duplicate", header(2) + tensor_bytes() + tensor_bytes(), "duplicate tensor name 't'"),
    ("trailing", GOOD + b"\x00", "unexpected trailing bytes"),
    ("overflow", header(1) + tensor_bytes(dims=(1 << 40, 1 << 40), nbytes=0, data=b""), "shape is too large"),
]


@pytest.mark.parametrize("name,blob,substr", MALFORMED, ids=[m[0] for m in MALFORMED])
def test_malformed_files_are_rejected_with_the_reference_message(eng, pkg, tmp_path, name, blob, substr):
    path = tmp_path / f"{name}.bin"
    path.write_bytes(blob)
    with pytest.raises(pkg.EngineError) as e:
        eng.engref(path)
    assert e.value.code == pkg.INVALID_ARGUMENT
    assert substr in str(e.value)
    assert str(path) in str(e.value)


def test_good_file_of_the_malformed_family_parses(eng, tmp_path):
    path = tmp_path / "good.bin"
    path.write_bytes(GOOD)
    with eng.engref(path) as f:
        assert f.names() == ["t"] and f.at("t").nbytes == 8


def test_host_views_are_read_only_and_end_with_the_file(eng, tmp_path):
    path = tmp_path / "v.bin"
    engref.write(path, {"a": np.arange(5, dtype=np.float32)})
    f = eng.engref(path)
    t = f.at("a")
    with pytest.raises(ValueError):
        t.host[0] = 1.0
    kept = t.host.copy()
    f.close()
    with pytest.raises(ValueError, match="closed"):
        t.host
    assert np.array_equal(kept, np.arange(5, dtype=np.float32))


def test_missing_file_and_unknown_name(eng, pkg, tmp_path):
    with pytest.raises(pkg.EngineError) as e:
        eng.engref(tmp_path / "absent.bin")
    assert "cannot open" in str(e.value) and "absent.bin" in str(e.value)
    path = tmp_path / "two.bin"
    engref.write(path, {"beta": np.ones(2, np.float32), "alpha": np.ones(1, np.float32)})
    with eng.engref(path) as f:
        with pytest.raises(pkg.EngineError) as e:
            f.at("gamma")
        assert "'gamma' not found. Available: alpha beta" in str(e.value)


def test_null_and_range_preconditions(eng, pkg, tmp_path):
    import ctypes
    n = ctypes.c_int32(0)
    assert eng.status("eng_engref_count", None, ctypes.byref(n)) == 1
    assert "file is null" in eng.last_error()
    assert eng.status("eng_engref_close", None) == 0
    h = ctypes.c_void_p(123)
    assert eng.status("eng_engref_open", None, ctypes.byref(h)) == 1
    assert h.value is None and "path is null" in eng.last_error()
    path = tmp_path / "one.bin"
    engref.write(path, {"a": np.ones(2, np.float32)})
    with eng.engref(path) as f:
        for bad in (-1, 1):
            assert eng.status("eng_engref_tensor", f.handle, bad, None, None, None, None, None,
                              None, None) == 1
            assert "out of range" in eng.last_error()


def test_upload_preconditions_are_checked_before_any_device_call(eng, pkg, tmp_path):
    path = tmp_path / "w.bin"
    engref.write(path, {"a": np.ones(100, np.float32), "b": np.ones(7, np.uint16)})
    with eng.engref(path) as f:
        need = f.slab_bytes()
        assert need == 768  # a: [0, 400), b: [512, 526), rounded up to 256
        cases = [((P, -1), "capacity must be non-negative"),
                 ((P, need - 1), "bytes needed"),
                 ((None, need), "slab is null"),
                 ((P + 4, need), "256-byte aligned")]
        for (slab, cap), substr in cases:
            assert eng.status("eng_engref_upload", f.handle, slab, cap, None) == 1
            assert substr in eng.last_error()
