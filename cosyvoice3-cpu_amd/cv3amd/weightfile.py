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


class _Record:
    """One logical tensor of the file: where its bytes are, how to read them, and the
    host object once something asked for it."""

    __slots__ = ("name", "dtype", "shape", "span", "scales", "quant", "obj")

    def __init__(self, name: str, info: Dict[str, Any], data0: int, size: int):
        a, b = info["data_offsets"]
        if not (0 <= a <= b and data0 + b <= size):
            raise ValueError(f"{name}: byte range {a}..{b} outside the file")
        self.name = name
        self.dtype = info["dtype"]
        self.shape = tuple(int(x) for x in info["shape"])
        self.span = (data0 + a, b - a)       # absolute file offset, bytes
        self.scales: Optional["_Record"] = None
        self.quant: Optional[Dict[str, Any]] = None
        self.obj = None

    def spans(self):
        yield self.span
        if self.scales is not None:
            yield self.scales.span

    def nbytes(self) -> int:
        return sum(n for _, n in self.spans())


class DeviceWeightFile:
    """Read side of the reference weight file; ``get(name)`` is an ndarray or a QTensor.

    The header is parsed once into a table of records, one per logical tensor in file
    order, each holding its payload's and (quantised) its scales' byte spans.  Every query
    reads that table; materialised objects live on their records, so dropping a stage is
    clearing its records, and evicting it advises exactly the stage's own byte runs."""

    def __init__(self, path: str, qtensor_cls=None):
        from .quant import QTensor
        self.path = path
        self._qcls = qtensor_cls or QTensor
        self._fh = open(path, "rb")
        index, metadata, data0 = read_header(self._fh)
        size = os.fstat(self._fh.fileno()).st_size
        self._map = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        blob = json.loads(metadata.get(METADATA_KEY, "{}"))
        self.meta: Dict[str, Any] = blob.get("meta", {})
        quant: Dict[str, Dict[str, Any]] = blob.get("quant", {})
        all_records = {k: _Record(k, v, data0, size) for k, v in index.items()}
        # a scales entry belongs to the tensor it is named after; it is not a tensor of its own
        self._rec: Dict[str, _Record] = {}
        for name, r in all_records.items():
            if name.endswith(SCALES_SUFFIX):
                continue
            r.quant = quant.get(name)
            if r.quant is not None:
                r.scales = all_records.get(name + SCALES_SUFFIX)
                if r.scales is None:
                    raise ValueError(f"{name}: quantised, but the file has no {name + SCALES_SUFFIX}")
            self._rec[name] = r
        # orphan scales entries still count towards the file's bytes
        owned = {id(r.scales) for r in self._rec.values() if r.scales is not None}
        self._orphans = [r for k, r in all_records.items() if k.endswith(SCALES_SUFFIX) and id(r) not in owned]

    def _under(self, prefix: str):
        return (r for k, r in self._rec.items() if k.startswith(prefix))

    def _record(self, name: str) -> _Record:
        r = self._rec.get(name)
        if r is None:
            raise KeyError(name)
        return r

    # -- introspection ------------------------------------------------------
    def keys(self) -> Iterable[str]:
        return list(self._rec)

    def __contains__(self, name: str) -> bool:
        return name in self._rec

    def entry(self, name: str) -> Dict[str, Any]:
        """Storage kind, logical shape and bytes on disk (payload plus scales)."""
        r = self._record(name)
        if r.quant is None:
            return {"kind": _RAW_KINDS.get(r.dtype, r.dtype.lower()), "shape": list(r.shape), "nbytes": r.nbytes()}
        q = r.quant
        return {"kind": q["kind"], "shape": list(q["shape"]), "block": q["block"], "mshape": list(q["mshape"]),
                "nbytes": r.nbytes()}

    def total_bytes(self) -> int:
        return sum(r.nbytes() for r in self._rec.values()) + sum(r.nbytes() for r in self._orphans)

    def stage_bytes(self, prefix: str) -> int:
        return sum(r.nbytes() for r in self._under(prefix)) + sum(
            r.nbytes() for r in self._orphans if r.name.startswith(prefix))

    # -- access ---------------------------------------------------------------
    def _view(self, r: _Record) -> np.ndarray:
        off, n = r.span
        if r.dtype == "BF16":  # widened to float32: numpy has no bfloat16
            raw = np.frombuffer(self._map, np.dtype("<u2"), n // 2, off)
            return _frozen((raw.astype(np.uint32) << 16).view(np.float32).reshape(r.shape))
        dt = _DTYPES.get(r.dtype)
        if dt is None:
            raise ValueError(f"{r.name}: unsupported safetensors dtype {r.dtype}")
        if n != int(np.prod(r.shape)) * dt.itemsize:
            raise ValueError(f"{r.name}: {n} bytes do not hold {r.shape} x {r.dtype}")
        arr = np.frombuffer(self._map, dt, n // dt.itemsize, off).reshape(r.shape)
        if dt.itemsize > 1 and arr.ctypes.data % dt.itemsize:
            arr = _frozen(np.array(arr, copy=True))  # a misaligned view would take NumPy's slow path
        return arr

    def get(self, name: str):
        r = self._record(name)
        if r.obj is None:
            if r.quant is None:
                r.obj = self._view(r)
            else:
                q = r.quant
                r.obj = self._qcls(q["kind"], self._view(r), self._view(r.scales), tuple(q["mshape"]),
                                   int(q["block"]), tuple(q["shape"]))
        return r.obj

    def get_f32(self, name: str) -> np.ndarray:
        """float32 copy; a quantised entry comes back as its (N, K) matrix (io/weights.py:167-170)."""
        t = self.get(name)
        return t.dequant() if hasattr(t, "dequant") else np.asarray(t, dtype=np.float32)

    def subset(self, prefix: str) -> Dict[str, Any]:
        """The tensors under ``prefix``, keyed by the rest of their names."""
        cut = len(prefix)
        return {r.name[cut:]: self.get(r.name) for r in list(self._under(prefix))}

    # -- lifetime -------------------------------------------------------------
    def upload(self, prefix: str = "") -> int:
        """Copy every tensor under ``prefix`` into HBM now, one pass per stage, for the
        per-op path (``cv3amd.ops`` finds the copies by host object); returns the bytes
        uploaded.  The copies live as long as the host objects this file holds, i.e.
        until ``release`` / ``evict``.  The model harnesses need no upload: they lay a
        stage's weights out themselves (fused QKV, stacked layers) as they are built."""
        from .weights import device_f32, device_qtensor
        total = 0
        for r in list(self._under(prefix)):
            t = self.get(r.name)
            if r.quant is not None:
                device_qtensor(t)
                total += t.nbytes
            else:
                total += device_f32(t).nbytes
        return total

    def release(self, prefix: str = "") -> None:
        """Drop the host objects under ``prefix``; their device copies go with them."""
        for r in self._under(prefix):
            r.obj = None

    def evict(self, prefix: str = "") -> int:
        """``release``, then hand back to the kernel (MADV_DONTNEED) the whole pages that
        only the stage's own bytes cover (io/weights.py:182-205: the per-stage lifetime).
        The stage's payload and scales spans are merged into maximal contiguous runs and
        each run's page-aligned interior is advised, so a tensor of another stage stored
        between two of this stage's keeps its pages.  Returns the bytes handed back."""
        spans = [sp for r in self._under(prefix) for sp in r.spans()]
        spans += [r.span for r in self._orphans if r.name.startswith(prefix)]
        spans.sort()
        self.release(prefix)
        runs = []
        for off, n in spans:
            if runs and off <= runs[-1][1]:
                runs[-1][1] = max(runs[-1][1], off + n)
            else:
                runs.append([off, off + n])
        page = mmap.PAGESIZE
        freed = 0
        for lo, hi in runs:
            first = -(-lo // page) * page
            last = hi - hi % page
            if last > first and hasattr(self._map, "madvise"):
                self._map.madvise(mmap.MADV_DONTNEED, first, last - first)
                freed += last - first
        return freed

    def close(self) -> None:
        self.release()
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
