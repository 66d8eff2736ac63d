"""ctypes binding of ``libcv3hip.so``.

The argument types are read from the C header (``include/cv3hip.h``) so the
binding cannot drift from the ABI.  Every entry point returns an int status;
:func:`call` maps non-zero codes onto the exceptions the reference raises
(IndexError, ValueError, AssertionError) or RuntimeError for HIP failures.

There is no CPU fallback: if the library is missing, or no GPU is visible,
:func:`lib` / :func:`init` raise.
"""

from __future__ import annotations

import atexit
import ctypes
import os
import re
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("CV3HIP_LIB", os.path.join(HERE, "libcv3hip.so"))
_ROOT = os.path.dirname(os.path.dirname(HERE))
HEADER = os.path.join(_ROOT, "include", "cv3hip.h")

OK, EINVAL, EINDEX, EASSERT, EHIP, EUNSUPPORTED = 0, 1, 2, 3, 4, 5
F32, F16 = 0, 1
KIND_F32, KIND_F16, KIND_Q8, KIND_Q4 = 0, 1, 2, 3
ACT = {"none": 0, "silu": 1, "sigmoid": 2, "gelu_tanh": 3, "gelu": 4, "mish": 5, "elu": 6,
       "leaky": 7, "tanh": 8}


class Epilogue(ctypes.Structure):
    """``cv3_epilogue``: y = residual + gate * act(acc + bias)."""

    _fields_ = [("act", ctypes.c_int), ("act_param", ctypes.c_float),
                ("residual", ctypes.c_void_p), ("ld_res", ctypes.c_int64),
                ("gate", ctypes.c_void_p), ("gate_stride", ctypes.c_int64),
                ("rows_per_gate", ctypes.c_int64),
                ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p), ("rope_rows", ctypes.c_int64),
                ("rope_period", ctypes.c_int64), ("rope_width", ctypes.c_int64), ("rope_limit", ctypes.c_int64)]


_SCALARS = {
    "int": ctypes.c_int, "int64_t": ctypes.c_int64, "uint64_t": ctypes.c_uint64,
    "size_t": ctypes.c_size_t, "float": ctypes.c_float, "double": ctypes.c_double,
    "cv3_stream_t": ctypes.c_void_p,
}


def parse_header(path: str = HEADER):
    """{name: (restype, [argtypes])} for every function declared in the header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(int|const char\*)\s+(cv3_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        argtypes = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                if "*" in a:
                    argtypes.append(ctypes.c_void_p)
                else:
                    ty = " ".join(a.replace("const ", "").split()[:-1])
                    argtypes.append(_SCALARS[ty])
        decls[name] = (ctypes.c_char_p if ret.startswith("const char") else ctypes.c_int, argtypes)
    return decls


# re-entrant: init() holds it while its call() loads the library through lib()
_lock = threading.RLock()
_lib = None
_inited = False
_shut = False


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                                      "(or python -m cv3amd.build) first")
                h = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in parse_header().items():
                    fn = getattr(h, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = h
    return _lib


class HIPError(RuntimeError):
    pass


def _raise(rc: int, what: str):
    msg = lib().cv3_last_error().decode(errors="replace")
    if rc == EINDEX:
        raise IndexError(msg)
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == EASSERT:
        raise AssertionError(msg)
    if rc == EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise HIPError(f"{what}: {msg}")


def call(name: str, *args):
    """Call ``cv3_<name>`` and raise on a non-zero status (RuntimeError after :func:`shutdown`:
    the library's device objects are gone, and a thread still running past interpreter exit
    must not enqueue work)."""
    if _shut:
        raise RuntimeError(f"cv3_{name}: the library has been shut down")
    fn = getattr(lib(), "cv3_" + name)
    rc = fn(*args)
    if rc:
        _raise(rc, "cv3_" + name)
    return rc


def init(device: int = 0):
    """Select the device once per process (raises if no GPU is visible).  Registers
    :func:`shutdown` to run at interpreter exit."""
    global _inited
    if not _inited:
        with _lock:
            if not _inited:
                call("init", device)
                atexit.register(shutdown)
                _inited = True


def shutdown():
    """Release every device object the library holds (graphs, blocks, per-thread streams,
    and the streams and events it handed out) after synchronising the device.  Runs from
    ``atexit``, i.e. before the interpreter tears down the objects that own those handles
    and before the HIP runtime's own exit handlers; device arrays, streams, events and
    graphs released after it are no-ops, and every other call raises."""
    global _shut
    if _lib is not None and _inited and not _shut:
        _shut = True
        _lib.cv3_shutdown()


def live_handles():
    """{streams, events, graphs, blocks} the library still holds (all 0 after :func:`shutdown`)."""
    vals = [ctypes.c_int64() for _ in range(4)]
    rc = lib().cv3_live_handles(*[ctypes.addressof(v) for v in vals])
    if rc:
        _raise(rc, "cv3_live_handles")
    return dict(zip(("streams", "events", "graphs", "blocks"), (v.value for v in vals)))


def device_info():
    init()
    cu = ctypes.c_int()
    mem = ctypes.c_int64()
    name = ctypes.create_string_buffer(64)
    call("device_info", ctypes.addressof(cu), ctypes.addressof(mem), ctypes.addressof(name), 64)
    return {"cu_count": cu.value, "hbm_bytes": mem.value, "arch": name.value.decode()}


def mem_stats():
    """(bytes held by live allocations, bytes parked in the allocator's cache)."""
    init()
    in_use = ctypes.c_size_t()
    cached = ctypes.c_size_t()
    call("mem_stats", ctypes.addressof(in_use), ctypes.addressof(cached))
    return in_use.value, cached.value


def epilogue(act: str = "none", act_param: float = 0.0, residual=None, ld_res: int = 0,
             gate=None, gate_stride: int = 0, rows_per_gate: int = 0, rope=None):
    """Build a ``cv3_epilogue`` (pointers are ints or None).  ``rope`` is
    ``(cos_ptr, sin_ptr, rows, period, width, limit)`` for the fused DiT rotary."""
    r = rope or (None, None, 0, 1, 0, 0)
    return Epilogue(ACT[act], act_param, residual, ld_res, gate, gate_stride, rows_per_gate, *r)


def ptr(obj) -> int:
    """Address of a ctypes object (for the out-parameter pointers of the ABI)."""
    return ctypes.addressof(obj)
