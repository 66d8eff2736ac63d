"""Device-resident arrays for the HIP backend.

``DeviceArray`` owns (or views) a block from the library's caching allocator.
Host NumPy buffers cross the boundary only through :func:`to_device` and
:meth:`DeviceArray.numpy`.  Kernels are enqueued on the calling thread's
stream, so work on one thread is ordered without explicit synchronisation.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _lib

_DTYPES = {np.dtype(t) for t in (np.float32, np.float16, np.int8, np.uint8, np.int64, np.int32, np.uint32,
                                 np.float64, np.uint16)}


class _Block:
    """One allocation; freed when the last DeviceArray viewing it goes away."""

    __slots__ = ("ptr", "nbytes")

    def __init__(self, nbytes: int):
        _lib.init()
        p = ctypes.c_void_p()
        _lib.call("malloc", ctypes.addressof(p), max(1, int(nbytes)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def __del__(self):
        try:
            if self.ptr and _lib._lib is not None:
                _lib.lib().cv3_free(ctypes.c_void_p(self.ptr))
        except Exception:
            pass
        self.ptr = None


class DeviceArray:
    """A typed, C-contiguous view of device memory."""

    __slots__ = ("shape", "dtype", "_block", "offset", "__weakref__")

    def __init__(self, shape: Sequence[int], dtype=np.float32, block: Optional[_Block] = None,
                 offset: int = 0):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        if self.dtype not in _DTYPES:
            raise TypeError(f"unsupported device dtype {self.dtype}")
        self._block = block if block is not None else _Block(self.nbytes)
        self.offset = int(offset)

    # -- basic properties ------------------------------------------------
    @property
    def size(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def ptr(self) -> int:
        return self._block.ptr + self.offset

    def __len__(self):
        return self.shape[0]

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype})"

    # -- views -----------------------------------------------------------
    def reshape(self, *shape) -> "DeviceArray":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            i = shape.index(-1)
            rest = int(np.prod([s for j, s in enumerate(shape) if j != i])) or 1
            shape[i] = self.size // rest
        if int(np.prod(shape)) != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {tuple(shape)}")
        return DeviceArray(shape, self.dtype, self._block, self.offset)

    def rows(self, r0: int, r1: int) -> "DeviceArray":
        """View of rows [r0, r1) along the first axis."""
        row = self.size // self.shape[0] if self.shape[0] else 0
        return DeviceArray((r1 - r0,) + self.shape[1:], self.dtype, self._block,
                           self.offset + r0 * row * self.dtype.itemsize)

    def view_at(self, elem_offset: int, shape, dtype=None) -> "DeviceArray":
        """Sub-view starting ``elem_offset`` elements in (no bounds growth allowed)."""
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        off = self.offset + elem_offset * self.dtype.itemsize
        n = int(np.prod(shape)) * dt.itemsize
        if off < 0 or off + n > self._block.nbytes:
            raise ValueError("view exceeds the allocation")
        return DeviceArray(shape, dt, self._block, off)

    # -- transfers -------------------------------------------------------
    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            _lib.call("copy_d2h", out.ctypes.data, self.ptr, self.nbytes, None)
        return out

    def copy_from(self, arr: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.size != self.size:
            raise ValueError(f"size mismatch {a.shape} -> {self.shape}")
        if a.nbytes:
            _lib.call("copy_h2d", self.ptr, a.ctypes.data, a.nbytes, None)
        return self

    def record_stream(self, stream) -> "DeviceArray":
        """Declare that work on ``stream`` (a :class:`Stream`) uses this array, so its block
        is not reused before that work is done."""
        if stream is not None:
            _lib.call("record_stream", self._block.ptr, stream.handle)
        return self

    def zero_(self) -> "DeviceArray":
        if self.nbytes:
            _lib.call("fill_zero", self.ptr, self.nbytes, None)
        return self

    def copy(self) -> "DeviceArray":
        out = DeviceArray(self.shape, self.dtype)
        if self.nbytes:
            _lib.call("copy_d2d", out.ptr, self.ptr, self.nbytes, None)
        return out


def empty(shape, dtype=np.float32) -> DeviceArray:
    return DeviceArray(shape, dtype)


def zeros(shape, dtype=np.float32) -> DeviceArray:
    return DeviceArray(shape, dtype).zero_()


def to_device(arr, dtype=None) -> DeviceArray:
    """Upload a host array (C-contiguous copy in ``dtype``, default its own)."""
    if isinstance(arr, DeviceArray):
        return arr
    a = np.asarray(arr)
    if dtype is not None:
        a = a.astype(dtype, copy=False)
    a = np.ascontiguousarray(a)
    return DeviceArray(a.shape, a.dtype).copy_from(a)


def synchronize():
    _lib.call("stream_sync", None)


class Timer:
    """HIP-event timing on the calling thread's stream."""

    def __init__(self):
        _lib.init()
        self._a = ctypes.c_void_p()
        self._b = ctypes.c_void_p()
        _lib.call("event_create", ctypes.addressof(self._a))
        _lib.call("event_create", ctypes.addressof(self._b))

    def start(self):
        _lib.call("event_record", self._a, None)

    def stop(self) -> float:
        """Milliseconds since :meth:`start` (waits for the stop event)."""
        _lib.call("event_record", self._b, None)
        ms = ctypes.c_float()
        _lib.call("event_elapsed_ms", self._a, self._b, ctypes.addressof(ms))
        return ms.value

    def __del__(self):
        try:
            _lib.lib().cv3_event_destroy(self._a)
            _lib.lib().cv3_event_destroy(self._b)
        except Exception:
            pass


class Stream:
    """A non-blocking stream of default priority (work on it runs beside the thread's own)."""

    def __init__(self):
        _lib.init()
        h = ctypes.c_void_p()
        _lib.call("stream_create", ctypes.addressof(h))
        self.handle = h.value

    def wait(self, event: "Event"):
        """Later work on this stream waits for the event's last recorded point."""
        _lib.call("stream_wait_event", self.handle, event.handle)

    def __del__(self):
        try:
            if self.handle:
                _lib.lib().cv3_stream_destroy(ctypes.c_void_p(self.handle))
        except Exception:
            pass


class Event:
    """A HIP event, recorded on a stream (None: the calling thread's)."""

    def __init__(self):
        _lib.init()
        h = ctypes.c_void_p()
        _lib.call("event_create", ctypes.addressof(h))
        self.handle = h.value

    def record(self, stream: "Optional[Stream]" = None) -> "Event":
        _lib.call("event_record", self.handle, stream.handle if stream is not None else None)
        return self

    def __del__(self):
        try:
            if self.handle:
                _lib.lib().cv3_event_destroy(ctypes.c_void_p(self.handle))
        except Exception:
            pass


def wait_event(event: Event):
    """Later work on the calling thread's stream waits for the event."""
    _lib.call("stream_wait_event", None, event.handle)


class Graph:
    """A captured sequence of launches on the calling thread's stream."""

    def __init__(self):
        self.exec = None

    def __enter__(self):
        _lib.init()
        _lib.call("graph_begin", None)
        return self

    def __exit__(self, et, ev, tb):
        x = ctypes.c_void_p()
        rc = _lib.lib().cv3_graph_end(None, ctypes.addressof(x))
        if et is None:
            if rc:
                _lib._raise(rc, "cv3_graph_end")
            self.exec = x.value
        return False

    def launch(self, stream: "Optional[Stream]" = None):
        _lib.call("graph_launch", self.exec, stream.handle if stream is not None else None)

    def __del__(self):
        try:
            if self.exec:
                _lib.lib().cv3_graph_destroy(ctypes.c_void_p(self.exec))
        except Exception:
            pass
