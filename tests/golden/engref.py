"""Reader/writer of ENGREF01 golden files.

The container layout is the reference's golden format, kept so fixtures can
be exchanged with the reference's tooling (reference tests/golden.hpp:21-33,
tools/gen_reference.py:64-83): the magic ``ENGREF01``, an int32 tensor count,
then per tensor an int32 name length, the UTF-8 name, an int32 dtype code, an
int32 rank, int64 dimensions, an int64 byte count and the little-endian data.

dtype codes: 0 = float32 (the reference's only code), 1 = float16 bit
patterns and 2 = float64 (extensions of this build; the reference reader
rejects them, so files meant for it use code 0 only).
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

MAGIC = b"ENGREF01"
CODES = {0: np.dtype("<f4"), 1: np.dtype("<u2"), 2: np.dtype("<f8")}
_BY_DTYPE = {np.dtype("float32"): 0, np.dtype("uint16"): 1, np.dtype("float64"): 2}


def write(path: Path, tensors: dict) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<i", len(tensors)))
        for name, arr in tensors.items():
            arr = np.ascontiguousarray(arr)
            code = _BY_DTYPE[arr.dtype]
            raw = arr.astype(CODES[code], copy=False).tobytes(order="C")
            nb = name.encode("utf-8")
            f.write(struct.pack("<i", len(nb)))
            f.write(nb)
            f.write(struct.pack("<i", code))
            f.write(struct.pack("<i", arr.ndim))
            for d in arr.shape:
                f.write(struct.pack("<q", int(d)))
            f.write(struct.pack("<q", len(raw)))
            f.write(raw)


def read(path: Path) -> dict:
    data = Path(path).read_bytes()
    if data[:8] != MAGIC:
        raise ValueError(f"{path}: bad magic {data[:8]!r}")
    pos = 8
    (count,) = struct.unpack_from("<i", data, pos)
    pos += 4
    out = {}
    for _ in range(count):
        (nlen,) = struct.unpack_from("<i", data, pos)
        pos += 4
        name = data[pos : pos + nlen].decode("utf-8")
        pos += nlen
        code, ndim = struct.unpack_from("<ii", data, pos)
        pos += 8
        if code not in CODES:
            raise ValueError(f"{path}: tensor {name!r} has unknown dtype code {code}")
        dims = struct.unpack_from("<" + "q" * ndim, data, pos)
        pos += 8 * ndim
        (nbytes,) = struct.unpack_from("<q", data, pos)
        pos += 8
        dt = CODES[code]
        expect = int(np.prod(dims, dtype=np.int64)) * dt.itemsize
        if nbytes != expect:
            raise ValueError(f"{path}: tensor {name!r} holds {nbytes} bytes, shape needs {expect}")
        arr = np.frombuffer(data, dtype=dt, count=expect // dt.itemsize, offset=pos)
        pos += nbytes
        out[name] = arr.reshape(dims).copy()
    if pos != len(data):
        raise ValueError(f"{path}: {len(data) - pos} trailing bytes")
    return out
