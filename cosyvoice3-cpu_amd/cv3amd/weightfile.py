"""The reference's on-disk weight file, read straight into the device harnesses.

Format (cv3cpu/io/weights.py:1-21, cv3cpu/io/safetensors_io.py): a ``.safetensors``
file -- u64 little-endian header length, that many bytes of JSON naming each
tensor's dtype, shape and byte range, then the packed data.  Quantised weights
keep their payload under the tensor's own name (``I8`` for q8, ``U8`` for packed
q4 nibbles) and their per-block scales under ``<name>.__scales__`` (``F16``); the
``__metadata__`` entry ``cv3cpu`` is a JSON blob ``{"version", "meta", "quant"}``
whose ``quant`` maps each quantised name to its kind, block, logical shape
(``shape``, a conv's ``(out, in, k)``) and matrix shape (``mshape``).

:class:`DeviceWeightFile` has the read API of the reference's ``WeightFile``
(``get``, ``get_f32``, ``entry``, ``keys``, ``meta``, ``subset``, ``release``,
``evict``), so ``DeviceQwen2`` / ``DeviceDiT`` / ``DeviceHiFT`` take it directly.
Tensors are views of a read-only memory map.  Device copies are made once per
host object by the harnesses (``cv3amd.weights``) and freed when ``release`` /
``evict`` drop the objects, the per-stage lifetime of the reference
(io/weights.py:177-205).  :func:`write_weight_file` writes the same layout.
"""

from __future__ import annotations

import json
import mmap
import os
import struct
from typing import Any, Dict, Iterable, Optional

import numpy as np

SCALES_SUFFIX = ".__scales__"
METADATA_KEY = "cv3cpu"
FORMAT_VERSION = 1

_DTYPES = {"F64": np.dtype("<f8"), "F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "I64": np.dtype("<i8"),
           "I32": np.dtype("<i4"), "I16": np.dtype("<i2"), "I8": np.dtype("i1"), "U8": np.dtype("u1"),
           "BOOL": np.dtype("?")}
_TAGS = {v: k for k, v in _DTYPES.items()}
_RAW_KINDS = {"F32": "f32", "F16": "f16", "I32": "i32", "I64": "i64", "I8": "i8", "U8": "u8"}


def _frozen(arr: np.ndarray) -> np.ndarray:
    """Read-only, like the mapped views: the device cache keys read-only arrays."""
    arr.flags.writeable = False
    return arr


def read_header(fh) -> tuple:
    """(tensor index, metadata, byte offset of the data section) of an open file."""
    fh.seek(0)
    raw = fh.read(8)
    if len(raw) != 8:
        raise ValueError("not a safetensors file: shorter than its length prefix")
    (n,) = struct.unpack("<Q", raw)
    if n <= 0 or n > (1 << 28):
        raise ValueError(f"implausible safetensors header length {n}")
    head = json.loads(fh.read(n).decode("utf-8"))
    meta = head.pop("__metadata__", {}) or {}
    return head, meta, 8 + n


class DeviceWeightFile:
    """Read side of the reference weight file; ``get(name)`` is an ndarray or a QTensor."""

    def __init__(self, path: str, qtensor_cls=None):
        from .quant import QTensor
        self.path = path
        self._qcls = qtensor_cls or QTensor
        self._fh = open(path, "rb")
        self._index, metadata, self._data0 = read_header(self._fh)
        self._size = os.fstat(self._fh.fileno()).st_size
        self._map = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        blob = json.loads(metadata.get(METADATA_KEY, "{}"))
        self.meta: Dict[str, Any] = blob.get("meta", {})
        self._quant: Dict[str, Dict[str, Any]] = blob.get("quant", {})
        for name, info in self._index.items():
            a, b = info["data_offsets"]
            if not (0 <= a <= b and self._data0 + b <= self._size):
                raise ValueError(f"{name}: byte range {a}..{b} outside the file")
        self._names = [k for k in self._index if not k.endswith(SCALES_SUFFIX)]
        self._cache: Dict[str, Any] = {}

    # -- introspection ------------------------------------------------------
    def keys(self) -> Iterable[str]:
        return list(self._names)

    def __contains__(self, name: str) -> bool:
        return name in self._index and not name.endswith(SCALES_SUFFIX)

    def entry(self, name: str) -> Dict[str, Any]:
        if name not in self:
            raise KeyError(name)
        q = self._quant.get(name)
        nbytes = self._nbytes(name)
        if q is not None:
            return {"kind": q["kind"], "shape": list(q["shape"]), "block": q["block"], "mshape": list(q["mshape"]),
                    "nbytes": nbytes + self._nbytes(name + SCALES_SUFFIX)}
        info = self._index[name]
        return {"kind": _RAW_KINDS.get(info["dtype"], info["dtype"].lower()), "shape": list(info["shape"]),
                "nbytes": nbytes}

    def _nbytes(self, name: str) -> int:
        a, b = self._index[name]["data_offsets"]
        return b - a

    def total_bytes(self) -> int:
        return sum(self._nbytes(k) for k in self._index)

    def stage_bytes(self, prefix: str) -> int:
        return sum(self._nbytes(k) for k in self._index if k.startswith(prefix))

    # -- access ---------------------------------------------------------------
    def _array(self, name: str) -> np.ndarray:
        info = self._index[name]
        a, b = info["data_offsets"]
        shape = tuple(int(s) for s in info["shape"])
        if info["dtype"] == "BF16":  # widened to float32: numpy has no bfloat16
            raw = np.frombuffer(self._map, np.dtype("<u2"), (b - a) // 2, self._data0 + a)
            return _frozen((raw.astype(np.uint32) << 16).view(np.float32).reshape(shape))
        dt = _DTYPES.get(info["dtype"])
        if dt is None:
            raise ValueError(f"{name}: unsupported safetensors dtype {info['dtype']}")
        count = (b - a) // dt.itemsize
        if count != int(np.prod(shape)):
            raise ValueError(f"{name}: {b - a} bytes do not hold {shape} x {info['dtype']}")
        arr = np.frombuffer(self._map, dt, count, self._data0 + a).reshape(shape)
        if dt.itemsize > 1 and arr.ctypes.data % dt.itemsize:
            arr = _frozen(np.array(arr, copy=True))  # a misaligned view would take NumPy's slow path
        return arr

    def get(self, name: str):
        hit = self._cache.get(name)
        if hit is not None:
            return hit
        if name not in self:
            raise KeyError(name)
        q = self._quant.get(name)
        if q is None:
            out = self._array(name)
        else:
            out = self._qcls(q["kind"], self._array(name), self._array(name + SCALES_SUFFIX), tuple(q["mshape"]),
                             int(q["block"]), tuple(q["shape"]))
        self._cache[name] = out
        return out

    def get_f32(self, name: str) -> np.ndarray:
        """float32 copy; a quantised entry comes back as its (N, K) matrix (io/weights.py:167-170)."""
        t = self.get(name)
        return t.dequant() if hasattr(t, "dequant") else np.asarray(t, dtype=np.float32)

    def subset(self, prefix: str) -> Dict[str, Any]:
        n = len(prefix)
        return {k[n:]: self.get(k) for k in self._names if k.startswith(prefix)}

    # -- lifetime -------------------------------------------------------------
    def upload(self, prefix: str = "") -> int:
        """Copy every tensor under ``prefix`` into HBM now, one pass per stage, for the
        per-op path (``cv3amd.ops`` finds the copies by host object); returns the bytes
        uploaded.  The copies live as long as the host objects this file caches, i.e.
        until ``release`` / ``evict``.  The model harnesses need no upload: they lay a
        stage's weights out themselves (fused QKV, stacked layers) as they are built."""
        from .weights import device_f32, device_qtensor
        total = 0
        for k in self._names:
            if not k.startswith(prefix):
                continue
            t = self.get(k)
            if hasattr(t, "scales"):
                device_qtensor(t)
                total += t.nbytes
            else:
                total += device_f32(t).nbytes
        return total

    def release(self, prefix: str = "") -> None:
        """Drop the host objects under ``prefix``; their device copies go with them."""
        for k in [k for k in self._cache if k.startswith(prefix)]:
            del self._cache[k]

    def evict(self, prefix: str = "") -> int:
        """``release`` plus MADV_DONTNEED on the mapped pages of every tensor under
        ``prefix`` (io/weights.py:182-205); returns the bytes handed back."""
        lo = hi = None
        for name, info in self._index.items():
            if name.startswith(prefix):
                a, b = info["data_offsets"]
                lo = a if lo is None else min(lo, a)
                hi = b if hi is None else max(hi, b)
        self.release(prefix)
        if lo is None:
            return 0
        page = mmap.PAGESIZE
        start = (self._data0 + lo + page - 1) // page * page
        end = (self._data0 + hi) // page * page
        if end <= start or not hasattr(self._map, "madvise"):
            return 0
        self._map.madvise(mmap.MADV_DONTNEED, start, end - start)
        return end - start

    def close(self) -> None:
        self._cache.clear()
        try:
            self._map.close()
        except BufferError:
            pass  # views still alive: the mapping closes when they go
        self._fh.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def write_weight_file(path: str, tensors: Dict[str, Any], meta: Optional[Dict[str, Any]] = None) -> None:
    """Write ``tensors`` in the reference's layout.  Values are arrays (stored with their
    own dtype) or quantised records ``{"kind", "q", "scales", "shape", "block",
    "orig_shape"}`` (``shape`` is the matrix shape)."""
    index: Dict[str, Dict[str, Any]] = {}
    quant: Dict[str, Dict[str, Any]] = {}
    blobs = []
    pos = 0

    def add(name, arr):
        nonlocal pos
        arr = np.ascontiguousarray(arr)
        dt = arr.dtype.newbyteorder("<") if arr.dtype.byteorder == ">" else arr.dtype
        if np.dtype(dt) not in _TAGS:
            raise ValueError(f"{name}: no safetensors dtype for {arr.dtype}")
        index[name] = {"dtype": _TAGS[np.dtype(dt)], "shape": list(arr.shape), "data_offsets": [pos, pos + arr.nbytes]}
        blobs.append(arr.astype(dt, copy=False).tobytes())
        pos += arr.nbytes

    for name, v in tensors.items():
        if isinstance(v, dict):
            add(name, np.asarray(v["q"]))
            add(name + SCALES_SUFFIX, np.asarray(v["scales"]))
            mshape = [int(s) for s in v["shape"]]
            quant[name] = {"kind": v["kind"], "block": int(v["block"]),
                           "shape": list(v.get("orig_shape") or mshape), "mshape": mshape}
        else:
            add(name, np.asarray(v))
    blob = json.dumps({"version": FORMAT_VERSION, "meta": dict(meta or {}), "quant": quant}, separators=(",", ":"))
    header = dict(index)
    header["__metadata__"] = {METADATA_KEY: blob}
    raw = json.dumps(header, separators=(",", ":")).encode("utf-8")
    raw += b" " * ((8 - (8 + len(raw)) % 8) % 8)  # keep the data section 8-byte aligned
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(raw)))
        fh.write(raw)
        for b in blobs:
            fh.write(b)
