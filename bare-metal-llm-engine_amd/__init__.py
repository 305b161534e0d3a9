"""Python binding of the MI355X matrix-multiply engine's C-ABI (libengine_hip.so).

This module is plumbing for the test suite and the benchmark: it loads the
built library with ctypes, declares the signatures of every function in
include/engine_hip.h, turns non-zero status codes into EngineError, and moves
numpy arrays to and from device memory through the library's own allocator
and copy functions. It computes nothing itself and has no fallback: if the
library is not built, loading fails.

The directory name is not a Python identifier; load it with
``importlib.util.spec_from_file_location`` (see tests/conftest.py).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libengine_hip.so")

OK = 0
INVALID_ARGUMENT = 1
DEVICE_ERROR = 2
DEVICE_CPU = 0
DEVICE_GPU = 1
STREAM_NON_BLOCKING = 1
EVENT_DISABLE_TIMING = 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f = ctypes.c_float
_int = ctypes.c_int
_pint = ctypes.POINTER(ctypes.c_int)
_pf = ctypes.POINTER(ctypes.c_float)
_pd = ctypes.POINTER(ctypes.c_double)
_pp = ctypes.POINTER(ctypes.c_void_p)


class AllocStats(ctypes.Structure):
    _fields_ = [
        ("bytes_in_use", ctypes.c_uint64),
        ("bytes_reserved", ctypes.c_uint64),
        ("peak_bytes_in_use", ctypes.c_uint64),
        ("num_allocs", ctypes.c_uint64),
        ("num_driver_allocs", ctypes.c_uint64),
    ]


# name -> argument types; every function returns int status except the two
# string accessors.
SIGNATURES = {
    "eng_device_count": [_pint],
    "eng_device_summary": [ctypes.c_char_p, _sz],
    "eng_peak_bandwidth_gbs": [_pd],
    "eng_driver_version": [ctypes.c_char_p, _sz],
    "eng_clock_rate_khz": [_pint],
    "eng_live_sm_clock_mhz": [_pint],
    "eng_live_mem_clock_mhz": [_pint],
    "eng_live_clock_source": [ctypes.c_char_p, _sz],
    "eng_device_arch": [ctypes.c_char_p, _sz],
    "eng_device_cu_count": [_pint],
    "eng_malloc": [_pp, _sz],
    "eng_free": [_p],
    "eng_memcpy_h2d": [_p, _p, _sz],
    "eng_memcpy_d2h": [_p, _p, _sz],
    "eng_memcpy_d2d": [_p, _p, _sz],
    "eng_memcpy_h2d_async": [_p, _p, _sz, _p],
    "eng_memcpy_d2h_async": [_p, _p, _sz, _p],
    "eng_memset": [_p, _int, _sz],
    "eng_memset_async": [_p, _int, _sz, _p],
    "eng_device_sync": [],
    "eng_check_last_launch": [],
    "eng_stream_create": [_pp, ctypes.c_uint],
    "eng_stream_destroy": [_p],
    "eng_stream_sync": [_p],
    "eng_stream_wait_event": [_p, _p, ctypes.c_uint],
    "eng_stream_delay": [_p, ctypes.c_uint],
    "eng_event_create": [_pp, ctypes.c_uint],
    "eng_event_destroy": [_p],
    "eng_graph_capture_begin": [_p],
    "eng_graph_capture_end": [_p, _p],
    "eng_graph_launch": [_p, _p],
    "eng_graph_destroy": [_p],
    "eng_event_record": [_p, _p],
    "eng_event_query": [_p, _pint],
    "eng_event_sync": [_p],
    "eng_event_elapsed_ms": [_pf, _p, _p],
    "eng_pool_create": [_pp, _int, _sz],
    "eng_pool_destroy": [_p],
    "eng_pool_default": [_pp, _int],
    "eng_pool_allocate": [_p, _sz, _pp],
    "eng_pool_deallocate": [_p, _p, _p],
    "eng_pool_stats": [_p, ctypes.POINTER(AllocStats)],
    "eng_pool_reset": [_p],
    "eng_passthrough_allocate": [_int, _sz, _pp],
    "eng_passthrough_deallocate": [_int, _p],
    "eng_passthrough_stats": [_int, ctypes.POINTER(AllocStats)],
    "eng_f32_to_f16_host": [_p, _p, _sz],
    "eng_f16_to_f32_host": [_p, _p, _sz],
    "eng_matmul_f32": [_p, _p, _p, _i64, _i64, _i64, _p],
    "eng_gemv_f32": [_p, _p, _p, _i64, _i64, _p],
    "eng_gemv_f16": [_p, _p, _p, _i64, _i64, _p],
    "eng_gemv_f16w": [_p, _p, _p, _i64, _i64, _p],
    "eng_rmsnorm_f32": [_p, _p, _p, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_f32": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_f16w": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_f16w_noalloc": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_fused_direct_f32": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_gemv_f16w_nk": [_p, _p, _p, _i64, _i64, _p],
    "eng_gemv_f32_nk": [_p, _p, _p, _i64, _i64, _p],
    "eng_rmsnorm_linear_f16w_nk": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_f32_nk": [_p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_vector_add_f32": [_p, _p, _p, _i64, _p],
    "eng_residual_rmsnorm_f32": [_p, _p, _p, _p, _p, _i64, _i64, _f, _p],
    "eng_swiglu_f32": [_p, _p, _p, _i64, _p],
    "eng_swiglu_f16": [_p, _p, _p, _i64, _p],
    "eng_rmsnorm_linear_swiglu_f16w_nk": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_swiglu_f32_nk": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_swiglu_f16w": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_rmsnorm_linear_swiglu_f32": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p],
    "eng_attention_decode_f16": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, ctypes.c_int, _p],
    "eng_attention_decode_with_mode_f16": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f,
                                           ctypes.c_int, ctypes.c_int, _p],
    "eng_cast_f32_to_f16": [_p, _p, _i64, _p],
    "eng_cast_f16_to_f32": [_p, _p, _i64, _p],
    "eng_kv_cache_write_f16": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "eng_transpose_f16": [_p, _p, _i64, _i64, _p],
    "eng_transpose_f32": [_p, _p, _i64, _i64, _p],
    "eng_engref_open": [ctypes.c_char_p, _pp],
    "eng_engref_close": [_p],
    "eng_engref_count": [_p, ctypes.POINTER(ctypes.c_int32)],
    "eng_engref_find": [_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)],
    "eng_engref_tensor": [_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_char_p),
                          ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                          ctypes.POINTER(ctypes.POINTER(ctypes.c_int64)),
                          ctypes.POINTER(ctypes.c_int64), _pp, ctypes.POINTER(ctypes.c_int64)],
    "eng_engref_slab_bytes": [_p, ctypes.POINTER(ctypes.c_int64)],
    "eng_engref_upload": [_p, _p, _i64, _p],
}

# ENGREF01 dtype codes -> numpy element types (f16 as its bit pattern).
ENGREF_DTYPES = {0: np.dtype("<f4"), 1: np.dtype("<u2"), 2: np.dtype("<f8")}
STRING_FUNCTIONS = ("eng_last_error", "eng_build_info")


class EngineError(RuntimeError):
    """A non-zero status from the C-ABI, with eng_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built; run __graft_entry__.build() (or `make -C "
            f"{HERE}`) first. There is no fallback implementation."
        )
    lib = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    for name in STRING_FUNCTIONS:
        fn = getattr(lib, name)
        fn.argtypes = []
        fn.restype = ctypes.c_char_p
    return lib


class Engine:
    """Status-checked access to the library plus numpy <-> device helpers."""

    def __init__(self, path: str = LIB_PATH):
        self.lib = load_library(path)
        self.path = path

    # -- calls -----------------------------------------------------------
    def status(self, name: str, *args) -> int:
        """Call `name` and return its raw status (for contract tests)."""
        return getattr(self.lib, name)(*args)

    def last_error(self) -> str:
        return self.lib.eng_last_error().decode()

    def call(self, name: str, *args) -> None:
        rc = getattr(self.lib, name)(*args)
        if rc != OK:
            raise EngineError(rc, self.last_error())

    # -- device ----------------------------------------------------------
    def device_count(self) -> int:
        n = ctypes.c_int(0)
        self.call("eng_device_count", ctypes.byref(n))
        return n.value

    def _string(self, name: str) -> str:
        buf = ctypes.create_string_buffer(512)
        self.call(name, buf, 512)
        return buf.value.decode()

    def device_summary(self) -> str:
        return self._string("eng_device_summary")

    def device_arch(self) -> str:
        return self._string("eng_device_arch")

    def peak_bandwidth_gbs(self) -> float:
        v = ctypes.c_double(0)
        self.call("eng_peak_bandwidth_gbs", ctypes.byref(v))
        return v.value

    def cu_count(self) -> int:
        v = ctypes.c_int(0)
        self.call("eng_device_cu_count", ctypes.byref(v))
        return v.value

    def clock_rate_khz(self) -> int:
        v = ctypes.c_int(0)
        self.call("eng_clock_rate_khz", ctypes.byref(v))
        return v.value

    def live_clocks_mhz(self) -> tuple:
        """(engine clock, memory clock) in MHz as the driver reports them now
        (see eng_live_sm_clock_mhz; the memory clock is 0 when unreadable)."""
        sm, mem = ctypes.c_int(0), ctypes.c_int(0)
        self.call("eng_live_sm_clock_mhz", ctypes.byref(sm))
        self.call("eng_live_mem_clock_mhz", ctypes.byref(mem))
        return sm.value, mem.value

    def live_clock_source(self) -> str:
        return self._string("eng_live_clock_source")

    def driver_version(self) -> str:
        return self._string("eng_driver_version")

    def build_info(self) -> str:
        return self.lib.eng_build_info().decode()

    def sync(self) -> None:
        self.call("eng_device_sync")

    # -- memory ----------------------------------------------------------
    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p(0)
        self.call("eng_malloc", ctypes.byref(p), nbytes)
        return p.value or 0

    def free(self, ptr: int) -> None:
        self.call("eng_free", ptr)

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host)
        d = DeviceArray(self, host.shape, host.dtype)
        d.upload(host)
        return d

    # -- streams and events ----------------------------------------------
    def stream(self, flags: int = STREAM_NON_BLOCKING) -> "Stream":
        return Stream(self, flags)

    def event(self, flags: int = 0) -> "Event":
        return Event(self, flags)

    def graph(self, stream: "Stream") -> "Graph":
        return Graph(self, stream)

    # -- ENGREF01 files --------------------------------------------------
    def engref(self, path) -> "EngrefFile":
        return EngrefFile(self, path)

    # -- host fp16 -------------------------------------------------------
    def f32_to_f16(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        out = np.empty(a.shape, dtype=np.uint16)
        self.call("eng_f32_to_f16_host", a.ctypes.data, out.ctypes.data, a.size)
        return out

    def f16_to_f32(self, bits: np.ndarray) -> np.ndarray:
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        out = np.empty(bits.shape, dtype=np.float32)
        self.call("eng_f16_to_f32_host", bits.ctypes.data, out.ctypes.data, bits.size)
        return out


class DeviceArray:
    """Owning device allocation (the DeviceBuffer<T> contract: move-free, freed once)."""

    def __init__(self, eng: Engine, shape, dtype):
        self.eng = eng
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if np.ndim(shape) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = eng.malloc(self.nbytes) if self.nbytes else 0

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def upload(self, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host)
        if host.nbytes != self.nbytes:
            raise ValueError(f"upload: {host.nbytes} host bytes for a {self.nbytes}-byte buffer")
        if self.nbytes:
            self.eng.call("eng_memcpy_h2d", self.ptr, host.ctypes.data, self.nbytes)

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            self.eng.call("eng_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def fill_bytes(self, value: int) -> None:
        if self.nbytes:
            self.eng.call("eng_memset", self.ptr, value, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            ptr, self.ptr = self.ptr, 0
            self.eng.free(ptr)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self, eng: Engine, flags: int = STREAM_NON_BLOCKING):
        self.eng = eng
        h = ctypes.c_void_p(0)
        eng.call("eng_stream_create", ctypes.byref(h), flags)
        self.handle = h.value

    def sync(self) -> None:
        self.eng.call("eng_stream_sync", self.handle)

    def wait(self, event: "Event") -> None:
        self.eng.call("eng_stream_wait_event", self.handle, event.handle, 0)

    def destroy(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            self.eng.call("eng_stream_destroy", h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


class Graph:
    """A HIP graph captured from the work issued on `stream` inside the
    `with` block (see eng_graph_capture_begin): replay it with launch()."""

    def __init__(self, eng: Engine, stream: Stream):
        self.eng = eng
        self.stream = stream
        self.handle = None

    def __enter__(self):
        self.eng.call("eng_graph_capture_begin", self.stream.handle)
        return self

    def __exit__(self, exc_type, *exc):
        h = ctypes.c_void_p(0)
        rc = self.eng.status("eng_graph_capture_end", self.stream.handle, ctypes.byref(h))
        if exc_type is None:
            if rc != OK:
                raise EngineError(rc, self.eng.last_error())
            self.handle = h.value
        return False

    def launch(self, stream: "Stream | None" = None) -> None:
        s = stream or self.stream
        self.eng.call("eng_graph_launch", self.handle, s.handle)

    def destroy(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            self.eng.call("eng_graph_destroy", h)


class Event:
    def __init__(self, eng: Engine, flags: int = 0):
        self.eng = eng
        h = ctypes.c_void_p(0)
        eng.call("eng_event_create", ctypes.byref(h), flags)
        self.handle = h.value

    def record(self, stream=None) -> None:
        self.eng.call("eng_event_record", self.handle, stream.handle if stream else None)

    def sync(self) -> None:
        self.eng.call("eng_event_sync", self.handle)

    def done(self) -> bool:
        d = ctypes.c_int(0)
        self.eng.call("eng_event_query", self.handle, ctypes.byref(d))
        return bool(d.value)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        self.eng.call("eng_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            self.eng.call("eng_event_destroy", h)


class EngrefTensor:
    """One tensor of an ENGREF01 file: name, dtype code, shape, byte count,
    slab offset and `host`, a read-only numpy view of the mapped bytes (f16
    tensors as uint16 bit patterns). The view reads the file's mapping, so it
    is only handed out while the file is open; copy it to keep it longer."""

    def __init__(self, file, name, dtype, shape, nbytes, slab_offset, host):
        self._file = file
        self.name = name
        self.dtype = dtype
        self.shape = shape
        self.nbytes = nbytes
        self.slab_offset = slab_offset
        self._host = host

    @property
    def host(self) -> np.ndarray:
        if not self._file.handle:
            raise ValueError(f"engref tensor '{self.name}': the file is closed")
        return self._host


class EngrefFile:
    """An ENGREF01 file mapped by the library (eng_engref_*), with the
    reference reader's interface (tests/golden.hpp:48-72: at / has / names /
    size) plus the slab layout for uploading every tensor in one allocation."""

    def __init__(self, eng: Engine, path):
        self.eng = eng
        h = ctypes.c_void_p(0)
        eng.call("eng_engref_open", os.fsencode(str(path)), ctypes.byref(h))
        self.handle = h.value
        n = ctypes.c_int32(0)
        eng.call("eng_engref_count", self.handle, ctypes.byref(n))
        self.tensors = [self._tensor(i) for i in range(n.value)]
        self._by_name = {t.name: t for t in self.tensors}

    def _tensor(self, index: int) -> EngrefTensor:
        name = ctypes.c_char_p()
        dtype = ctypes.c_int32(0)
        ndim = ctypes.c_int32(0)
        dims = ctypes.POINTER(ctypes.c_int64)()
        nbytes = ctypes.c_int64(0)
        data = ctypes.c_void_p(0)
        off = ctypes.c_int64(0)
        self.eng.call("eng_engref_tensor", self.handle, index, ctypes.byref(name),
                      ctypes.byref(dtype), ctypes.byref(ndim), ctypes.byref(dims),
                      ctypes.byref(nbytes), ctypes.byref(data), ctypes.byref(off))
        shape = tuple(int(dims[i]) for i in range(ndim.value))
        dt = ENGREF_DTYPES[dtype.value]
        if nbytes.value:
            raw = (ctypes.c_char * nbytes.value).from_address(data.value)
            host = np.frombuffer(raw, dtype=dt).reshape(shape)
        else:
            host = np.empty(shape, dtype=dt)
        host.flags.writeable = False  # the mapping is read-only
        return EngrefTensor(self, name.value.decode(), dtype.value, shape, nbytes.value, off.value,
                            host)

    def size(self) -> int:
        return len(self.tensors)

    def names(self) -> list:
        return sorted(self._by_name)

    def has(self, name: str) -> bool:
        return name in self._by_name

    def index(self, name: str) -> int:
        i = ctypes.c_int32(0)
        self.eng.call("eng_engref_find", self.handle, name.encode(), ctypes.byref(i))
        return i.value

    def at(self, name: str) -> EngrefTensor:
        return self.tensors[self.index(name)]

    def slab_bytes(self) -> int:
        v = ctypes.c_int64(0)
        self.eng.call("eng_engref_slab_bytes", self.handle, ctypes.byref(v))
        return v.value

    def upload(self, slab: DeviceArray, stream: "Stream | None" = None) -> None:
        self.eng.call("eng_engref_upload", self.handle, slab.ptr, slab.nbytes,
                      stream.handle if stream else None)

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            self.tensors = []
            self._by_name = {}
            self.eng.call("eng_engref_close", h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
