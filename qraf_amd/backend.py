"""Host-side mirror of the reference's dispatch layer (include/nn/backend.h)
over the HIP C ABI.

Same names, argument meaning and in-place semantics as backend.h:27-45, with
numpy arrays in place of raw pointers.  One deliberate difference: an unknown
quantized dtype raises HipError (code ERR_DTYPE) where the reference
zero-fills y (backend.cpp:195-198).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import F32, Q4_0, Q8_0, call, fp, lib

__all__ = ["backend_init", "dispatch_matvec_q", "dispatch_matvec_opt", "dispatch_dot_f32", "dispatch_rms_norm",
           "dispatch_softmax", "dispatch_silu", "dispatch_add", "dispatch_mul", "dispatch_scale",
           "register_weights", "unregister_weights", "DeviceBuffer", "Stream", "Event", "Graph", "device_count"]


def _f32(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a.ctypes.data_as(fp)


def device_count() -> int:
    n = C.c_int(0)
    rc = lib.qraf_hip_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def backend_init(device: int = 0) -> None:
    """backend_init() (backend.cpp:18-50) for the HIP backend."""
    call("qraf_hip_init", device)


def register_weights(w: np.ndarray) -> None:
    """Upload an immutable host weight buffer to HBM once (see qraf_hip.h)."""
    call("qraf_hip_register_weights", w.ctypes.data, w.nbytes)


def unregister_weights(w: np.ndarray) -> None:
    call("qraf_hip_unregister_weights", w.ctypes.data)


def dispatch_matvec_q(w_data: np.ndarray, w_size: int, w_dtype: int, block_size: int | None, out_dim: int,
                      in_dim: int, x: np.ndarray, y: np.ndarray) -> None:
    """dispatch_matvec_q (backend.cpp:131-199).  block_size None means no
    QuantScheme, i.e. 32 (backend.cpp:135)."""
    call("qraf_hip_matvec_q", w_data.ctypes.data, w_size, w_dtype, block_size or 0, out_dim, in_dim,
         _f32(x, "x"), _f32(y, "y"))


def dispatch_matvec_opt(W: np.ndarray, x: np.ndarray, y: np.ndarray, out_dim: int, in_dim: int) -> None:
    """dispatch_matvec_opt (backend.cpp:62-105)."""
    call("qraf_hip_matvec_f32", _f32(W, "W"), _f32(x, "x"), _f32(y, "y"), out_dim, in_dim)


def dispatch_dot_f32(a: np.ndarray, b: np.ndarray, n: int) -> float:
    """dispatch_dot_f32 (backend.cpp:109-127)."""
    r = C.c_float()
    call("qraf_hip_dot_f32", _f32(a, "a"), _f32(b, "b"), n, C.byref(r))
    return r.value


def dispatch_rms_norm(x: np.ndarray, weight: np.ndarray, size: int, eps: float) -> None:
    call("qraf_hip_rms_norm", _f32(x, "x"), _f32(weight, "weight"), size, eps)


def dispatch_softmax(x: np.ndarray, size: int) -> None:
    call("qraf_hip_softmax", _f32(x, "x"), size)


def dispatch_silu(x: np.ndarray, size: int) -> None:
    call("qraf_hip_silu", _f32(x, "x"), size)


def dispatch_add(x: np.ndarray, y: np.ndarray, size: int) -> None:
    call("qraf_hip_add", _f32(x, "x"), _f32(y, "y"), size)


def dispatch_mul(x: np.ndarray, y: np.ndarray, size: int) -> None:
    call("qraf_hip_mul", _f32(x, "x"), _f32(y, "y"), size)


def dispatch_scale(x: np.ndarray, scale: float, size: int) -> None:
    call("qraf_hip_scale", _f32(x, "x"), scale, size)


# ------------------------------------------------------------ device plumbing

class DeviceBuffer:
    """A block of HBM owned by the library's allocator."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("qraf_hip_malloc", C.byref(p), self.nbytes)
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        call("qraf_hip_memcpy_h2d", self.ptr + offset, a.ctypes.data, a.nbytes)

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        call("qraf_hip_memcpy_d2h", out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def zero(self) -> None:
        call("qraf_hip_memset", self.ptr, 0, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            call("qraf_hip_free", self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = C.c_void_p()
        call("qraf_hip_stream_create", C.byref(p))
        self.h = p.value

    def synchronize(self):
        call("qraf_hip_stream_synchronize", self.h)

    def destroy(self):
        if self.h:
            call("qraf_hip_stream_destroy", self.h)
            self.h = None


class Event:
    def __init__(self):
        p = C.c_void_p()
        call("qraf_hip_event_create", C.byref(p))
        self.h = p.value

    def record(self, stream: Stream | None = None):
        call("qraf_hip_event_record", self.h, stream.h if stream else None)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("qraf_hip_event_elapsed_ms", self.h, end.h, C.byref(ms))
        return ms.value

    def destroy(self):
        if self.h:
            call("qraf_hip_event_destroy", self.h)
            self.h = None


class Graph:
    """Capture of the stream-ordered calls made inside `with Graph(stream)`."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.h = None

    def __enter__(self):
        call("qraf_hip_graph_begin", self.stream.h)
        return self

    def __exit__(self, et, ev, tb):
        p = C.c_void_p()
        rc = lib.qraf_hip_graph_end(self.stream.h, C.byref(p))
        if et is None:
            if rc != 0:
                raise RuntimeError("graph capture failed: " + lib.qraf_hip_last_error().decode())
            self.h = p.value
        return False

    def launch(self):
        call("qraf_hip_graph_launch", self.h, self.stream.h)

    def destroy(self):
        if self.h:
            call("qraf_hip_graph_destroy", self.h)
            self.h = None
