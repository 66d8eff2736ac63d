"""Weight containers and the device weight cache.

``WeightStore`` mirrors the subset of the reference's ``WeightFile``
(cv3cpu/io/weights.py:94-215) the models use: ``get``, ``get_f32``, ``entry``,
``__contains__``, ``keys`` and ``meta``.  Quantised entries are built with a
configurable QTensor class so one store can feed either this package or a
NumPy restatement.

Device copies of weights are cached per host object (the reference's
``WeightFile.get`` returns the same object for a name, io/weights.py:153-165)
and released by ``weakref.finalize`` when the host object goes away, the
analogue of ``WeightFile.evict`` (io/weights.py:182-205).  Only read-only
arrays (mmap views, or arrays a store has frozen) and QTensors are cached; a
writeable array is re-uploaded on every call because it may change.
"""

from __future__ import annotations

import threading
import weakref
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from . import _lib
from .device import DeviceArray, to_device


@dataclass
class DeviceQ:
    kind_code: int
    q: DeviceArray
    scales: DeviceArray
    scale_code: int
    kp: int
    block: int
    n: int
    k: int


_CACHE: Dict[int, object] = {}
_UPLOAD = threading.Lock()   # one upload per weight object when several threads miss at once


def _remember(obj, value):
    key = id(obj)
    _CACHE[key] = value
    weakref.finalize(obj, _CACHE.pop, key, None)
    return value


def device_qtensor(qt) -> DeviceQ:
    """Device copy of a QTensor's payload and scales (cached per object)."""
    hit = _CACHE.get(id(qt))
    if hit is not None:
        return hit
    with _UPLOAD:
        hit = _CACHE.get(id(qt))
        return hit if hit is not None else _upload_qtensor(qt)


def _upload_qtensor(qt) -> DeviceQ:
    kind = {"q8": _lib.KIND_Q8, "q4": _lib.KIND_Q4}[qt.kind]
    sdt = np.dtype(qt.scales.dtype)
    sc_code = _lib.F16 if sdt == np.float16 else _lib.F32
    q = qt.q if isinstance(qt.q, DeviceArray) else to_device(np.ascontiguousarray(qt.q))
    s = qt.scales if isinstance(qt.scales, DeviceArray) else to_device(np.ascontiguousarray(qt.scales))
    kp = int(qt.scales.shape[1]) * int(qt.block)
    d = DeviceQ(kind, q, s, sc_code, kp, int(qt.block), int(qt.shape[0]), int(qt.shape[1]))
    return _remember(qt, d)


def device_f32(arr) -> DeviceArray:
    """Device float32 copy of a host weight (cached if the array is read-only)."""
    if isinstance(arr, DeviceArray):
        return arr
    if isinstance(arr, np.ndarray) and not arr.flags.writeable:
        hit = _CACHE.get(id(arr))
        if hit is not None:
            return hit
        with _UPLOAD:
            hit = _CACHE.get(id(arr))
            return hit if hit is not None else _remember(arr, to_device(arr, np.float32))
    return to_device(np.asarray(arr), np.float32)


class WeightStore:
    """In-memory weight container with the reference WeightFile's read API.

    ``tensors`` maps names to float arrays or to quantised records
    ``{"kind", "q", "scales", "shape", "block", "orig_shape"}``.
    """

    def __init__(self, tensors: Dict[str, object], meta: Optional[dict] = None, qtensor_cls=None):
        from .quant import QTensor
        self._t = {}
        for name, v in tensors.items():
            if isinstance(v, np.ndarray):
                v = np.ascontiguousarray(v)
                v.flags.writeable = False
            self._t[name] = v
        self.meta = dict(meta or {})
        self._qcls = qtensor_cls or QTensor
        self._objs: Dict[str, object] = {}

    def keys(self):
        return self._t.keys()

    def __contains__(self, name):
        return name in self._t

    def raw(self, name):
        return self._t[name]

    def get(self, name):
        if name in self._objs:
            return self._objs[name]
        v = self._t[name]
        if isinstance(v, dict):
            v = self._qcls(v["kind"], v["q"], v["scales"], tuple(v["shape"]), int(v["block"]),
                           tuple(v["orig_shape"]) if v.get("orig_shape") is not None else None)
        self._objs[name] = v
        return v

    def get_f32(self, name):
        v = self.get(name)
        if hasattr(v, "dequant"):
            out = v.dequant()
            if v.orig_shape is not None:
                out = out.reshape(v.orig_shape)
            return np.asarray(out, dtype=np.float32)
        return np.asarray(v, dtype=np.float32)

    def entry(self, name):
        v = self._t[name]
        if isinstance(v, dict):
            shape = v.get("orig_shape") or v["shape"]
            return {"shape": list(shape), "kind": v["kind"]}
        return {"shape": list(np.shape(v)), "kind": str(np.asarray(v).dtype)}

    def with_qtensor(self, qtensor_cls) -> "WeightStore":
        """Same tensors, QTensors built from ``qtensor_cls``."""
        return WeightStore(self._t, self.meta, qtensor_cls)
