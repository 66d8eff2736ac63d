"""Drop-in replacement for ``cv3cpu.quant`` on the HIP backend.

Same names, signatures and results as cv3cpu/quant.py:31-204.  Quantisation,
row dequantisation and the quantised matmul run on the GPU; host arrays are
copied in and out, ``DeviceArray`` inputs stay resident.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from .device import DeviceArray, to_device
from . import weights as _w

Q8_BLOCK = 64              # quant.py:31
Q4_BLOCK = 32              # quant.py:32
TILE_BYTES = 1 << 20       # quant.py:39 (accepted, unused: the GPU does not tile by bytes)
BIG_TILE_BYTES = 8 << 20   # quant.py:40
THREAD_ROW_LIMIT = 4       # quant.py:43 (GEMV below, MFMA GEMM above)


def _kp(k: int, block: int) -> int:
    return -(-k // block) * block


def quantize_q8(w, block: int = Q8_BLOCK, scale_dtype=np.float16):
    """``(int8 codes [N, Kp], scales [N, Kp/block], Kp)``, bit-exact with quant.py:56-67.

    ``scale_dtype=np.float32`` keeps the fp32 scales (the per-output-channel
    layout uses ``block = K``).
    """
    dev = isinstance(w, DeviceArray)
    wd = to_device(w, np.float32) if not dev else w
    n = wd.shape[0]
    k = wd.size // n if n else 0
    kp = _kp(k, block)
    sdt = np.dtype(scale_dtype)
    if sdt not in (np.dtype(np.float16), np.dtype(np.float32)):
        raise ValueError("scale dtype must be float16 or float32")
    q = DeviceArray((n, kp), np.int8)
    sc = DeviceArray((n, kp // block), sdt)
    _lib.call("quantize_q8", wd.ptr, n, k, block, _lib.F16 if sdt == np.float16 else _lib.F32,
              q.ptr, sc.ptr, None)
    if dev:
        return q, sc, kp
    return q.numpy(), sc.numpy(), kp


def quantize_q4(w, block: int = Q4_BLOCK):
    """``(packed uint8 [N, Kp/2], float16 scales, Kp)`` (quant.py:70-86)."""
    dev = isinstance(w, DeviceArray)
    wd = to_device(w, np.float32) if not dev else w
    n = wd.shape[0]
    k = wd.size // n if n else 0
    kp = _kp(k, block)
    q = DeviceArray((n, kp // 2), np.uint8)
    sc = DeviceArray((n, kp // block), np.float16)
    _lib.call("quantize_q4", wd.ptr, n, k, block, q.ptr, sc.ptr, None)
    if dev:
        return q, sc, kp
    return q.numpy(), sc.numpy(), kp


@dataclass
class QTensor:
    """A quantised 2-D weight (quant.py:89-136).  ``q``/``scales`` may be host
    arrays (e.g. mmap views) or DeviceArrays."""

    kind: str
    q: object
    scales: object
    shape: tuple
    block: int
    orig_shape: Optional[tuple] = None

    def __hash__(self):
        return id(self)

    def __eq__(self, other):
        return self is other

    @property
    def kernel_size(self) -> Optional[int]:
        if self.orig_shape is not None and len(self.orig_shape) == 3:
            return int(self.orig_shape[2])
        return None

    @property
    def nbytes(self) -> int:
        return int(self.q.nbytes + self.scales.nbytes)

    def dequant_rows(self, r0: int, r1: int, out: Optional[np.ndarray] = None):
        """float32 rows [r0, r1) sliced to K, dequantised on the device (quant.py:110-133)."""
        k = self.shape[1]
        nb = self.scales.shape[1]
        width = nb * self.block
        if out is not None and out.shape[1] < width:
            raise ValueError("scratch buffer is narrower than the padded row")
        dq = _w.device_qtensor(self)
        rows = r1 - r0
        res = DeviceArray((rows, k), np.float32)
        _lib.call("dequant_rows", dq.kind_code, dq.q.ptr, dq.scales.ptr, dq.scale_code, dq.kp, self.block,
                  k, r0, r1, res.ptr, k, None)
        host = res.numpy()
        if out is not None:
            out[:rows, :k] = host
            return out[:rows, :k]
        return host

    def dequant(self):
        return self.dequant_rows(0, self.shape[0])


def qmatmul(x, w, bias=None, tile_bytes: Optional[int] = None, threads: Optional[int] = None):
    """``x @ w.T (+ bias)`` for a QTensor or a plain (N, K) array (quant.py:156-204).

    ``tile_bytes`` and ``threads`` are accepted for signature compatibility;
    the device kernels do not depend on them.
    """
    from .ops import linear
    return linear(x, w, bias)
