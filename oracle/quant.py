"""Oracle restatement of block quantisation and the dequantising matmul.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/quant.py.  Layout for a logical ``(N, K)`` weight:
  * K is zero-padded up to a multiple of ``block`` (quant.py:46-53);
  * q8: ``int8[N, Kp]`` codes and ``float16[N, Kp/block]`` scales (quant.py:56-67);
  * q4: ``uint8[N, Kp/2]``; byte j of a block holds code j (low nibble) and
    code j+block/2 (high nibble), both biased by +8 (quant.py:70-86).

The per-output-channel variant used by the decode benchmark is the same
algorithm with ``block = K`` and the scales kept in float32
(``quantize_q8(w, block=K, scale_dtype=np.float32)``).
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from typing import Optional

import numpy as np

Q8_BLOCK = 64          # quant.py:31
Q4_BLOCK = 32          # quant.py:32
TILE_BYTES = 1 << 20   # quant.py:39
BIG_TILE_BYTES = 8 << 20   # quant.py:40
THREAD_ROW_LIMIT = 4   # quant.py:43


def pad_k(w: np.ndarray, block: int) -> np.ndarray:
    """Zero-pad the last axis to a multiple of ``block`` (quant.py:46-53)."""
    extra = (-w.shape[-1]) % block
    if not extra:
        return w
    widths = [(0, 0)] * (w.ndim - 1) + [(0, extra)]
    return np.pad(w, widths)


def quantize_q8(w: np.ndarray, block: int = Q8_BLOCK, scale_dtype=np.float16):
    """``(codes int8[N,Kp], scales[N,Kp/block], Kp)`` (quant.py:56-67).

    amax per block; scale = float32(amax / 127) with 0 -> 1; codes are
    round-half-even of the *true* float32 quotient, clipped to +-127; the
    stored scale is the float32 scale cast (RNE) to ``scale_dtype``.
    """
    w32 = np.ascontiguousarray(w, dtype=np.float32)
    rows = w32.shape[0]
    wp = pad_k(w32, block)
    kp = wp.shape[1]
    blk = wp.reshape(rows, kp // block, block)
    amax = np.max(np.abs(blk), axis=2)
    scale = np.divide(amax, np.float32(127.0), dtype=np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    codes = np.rint(blk / scale[:, :, None])
    codes = np.clip(codes, -127, 127).astype(np.int8)
    return codes.reshape(rows, kp), scale.astype(scale_dtype), kp


def quantize_q4(w: np.ndarray, block: int = Q4_BLOCK):
    """``(packed uint8[N,Kp/2], float16 scales, Kp)`` (quant.py:70-86).

    The scale anchors on the signed extreme of the block (first index of the
    largest magnitude) so that value maps exactly to code 0 (-8 after bias).
    """
    w32 = np.ascontiguousarray(w, dtype=np.float32)
    rows = w32.shape[0]
    wp = pad_k(w32, block)
    kp = wp.shape[1]
    nb = kp // block
    blk = wp.reshape(rows, nb, block)
    pick = np.argmax(np.abs(blk), axis=2)
    extreme = np.take_along_axis(blk, pick[:, :, None], axis=2)[:, :, 0]
    scale = np.divide(extreme, np.float32(-8.0), dtype=np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    codes = np.clip(np.rint(blk / scale[:, :, None] + np.float32(8.0)), 0, 15).astype(np.uint8)
    h = block // 2
    packed = (codes[:, :, :h] | (codes[:, :, h:] << 4)).astype(np.uint8)
    return packed.reshape(rows, kp // 2), scale.astype(np.float16), kp


@dataclass
class QTensor:
    """Quantised 2-D weight (quant.py:89-136)."""

    kind: str
    q: np.ndarray
    scales: np.ndarray
    shape: tuple
    block: int
    orig_shape: Optional[tuple] = None

    @property
    def kernel_size(self) -> Optional[int]:
        if self.orig_shape is not None and len(self.orig_shape) == 3:
            return int(self.orig_shape[2])
        return None

    @property
    def nbytes(self) -> int:
        return self.q.nbytes + self.scales.nbytes

    def dequant_rows(self, r0: int, r1: int, out: Optional[np.ndarray] = None) -> np.ndarray:
        """float32 rows [r0, r1): code * float32(scale), sliced to K (quant.py:110-133)."""
        nb = self.scales.shape[1]
        width = nb * self.block
        n = r1 - r0
        if out is None:
            out = np.empty((n, width), dtype=np.float32)
        elif out.shape[1] < width:
            raise ValueError("scratch buffer is narrower than the padded row")
        view = out[:n, :width].reshape(n, nb, self.block)
        if self.kind == "q8":
            view[...] = self.q[r0:r1].reshape(n, nb, self.block)
        else:
            h = self.block // 2
            b = self.q[r0:r1].reshape(n, nb, h)
            view[:, :, :h] = (b & 0x0F).astype(np.float32) - np.float32(8.0)
            view[:, :, h:] = (b >> 4).astype(np.float32) - np.float32(8.0)
        view *= self.scales[r0:r1].astype(np.float32)[:, :, None]
        return out[:n, :self.shape[1]]

    def dequant(self) -> np.ndarray:
        return self.dequant_rows(0, self.shape[0])


def default_threads() -> int:
    """``min(4, cpus)`` or ``CV3_MATMUL_THREADS`` (quant.py:139-143)."""
    env = os.environ.get("CV3_MATMUL_THREADS")
    if env:
        return max(1, int(env))
    return max(1, min(4, os.cpu_count() or 1))


_POOLS = {}


def _pool(n: int) -> ThreadPoolExecutor:
    if n not in _POOLS:
        _POOLS[n] = ThreadPoolExecutor(max_workers=n)
    return _POOLS[n]


def qmatmul(x: np.ndarray, w, bias: Optional[np.ndarray] = None,
            tile_bytes: Optional[int] = None, threads: Optional[int] = None) -> np.ndarray:
    """``x @ w.T (+ bias)`` (quant.py:156-204).

    Plain arrays go straight to BLAS.  QTensors are expanded one row tile at a
    time (1 MB tiles for <=4 activation rows, 8 MB otherwise) and the tiles are
    spread over a thread pool for the decode case, as the reference does, so the
    CPU timing of this restatement is representative.
    """
    if not isinstance(w, QTensor):
        y = x.astype(np.float32, copy=False) @ np.asarray(w, dtype=np.float32).T
        if bias is not None:
            y += bias
        return y
    n = w.shape[0]
    lead = x.shape[:-1]
    xf = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    m = xf.shape[0]
    width = w.scales.shape[1] * w.block
    if tile_bytes is None:
        tile_bytes = TILE_BYTES if m <= THREAD_ROW_LIMIT else BIG_TILE_BYTES
    step = max(1, min(n, tile_bytes // max(1, width * 4)))
    yt = np.empty((n, m), dtype=np.float32)
    starts = list(range(0, n, step))

    def run(rows):
        buf = np.empty((step, width), dtype=np.float32)
        for r0 in rows:
            r1 = min(n, r0 + step)
            np.dot(w.dequant_rows(r0, r1, buf), xf.T, out=yt[r0:r1])

    nt = default_threads() if threads is None else threads
    if nt > 1 and m <= THREAD_ROW_LIMIT and len(starts) >= 2 * nt:
        list(_pool(nt).map(run, [starts[i::nt] for i in range(nt)]))
    else:
        run(starts)
    y = np.ascontiguousarray(yt.T)
    if bias is not None:
        y += bias
    return y.reshape(*lead, n)
