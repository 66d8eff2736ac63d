"""Drop-in replacement for ``cv3cpu.ops`` on the HIP backend.

Same function names and signatures as cv3cpu/ops.py:21-377.  Each function
accepts NumPy arrays (copied to the device, computed, copied back) or
``DeviceArray``s (computed in place on the device, result left resident, no
synchronisation).  Rebinding ``cv3cpu.ops.<name>`` to these functions
redirects every model, since the models resolve ``ops.<name>`` at call time.

There is no CPU fallback: every op runs a HIP kernel from ``libcv3hip.so``.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple, Union

import numpy as np

from . import _lib
from . import weights as _w
from .device import DeviceArray, to_device
from .quant import QTensor

Weight = Union[np.ndarray, QTensor]
TILE_BYTES = 8 << 20  # ops.py:23 (accepted, unused)


def _dev(x) -> Tuple[DeviceArray, bool]:
    if isinstance(x, DeviceArray):
        return x, True
    return to_device(np.asarray(x), np.float32), False


def _ret(d: DeviceArray, resident: bool):
    return d if resident else d.numpy()


# ----------------------------------------------------------------------------
# elementwise
# ----------------------------------------------------------------------------

def _act(x, name, param=0.0):
    xd, res = _dev(x)
    y = DeviceArray(xd.shape, np.float32)
    _lib.call("act", _lib.ACT[name], float(param), xd.ptr, y.ptr, xd.size, None)
    return _ret(y, res)


def silu(x):
    """ops.py:30-31"""
    return _act(x, "silu")


def sigmoid(x):
    """ops.py:34-35"""
    return _act(x, "sigmoid")


def gelu_tanh(x):
    """ops.py:41-43"""
    return _act(x, "gelu_tanh")


def gelu(x):
    """ops.py:46-60 (A&S 7.1.26 erf)"""
    return _act(x, "gelu")


def mish(x):
    """ops.py:63-66"""
    return _act(x, "mish")


def elu(x, alpha: float = 1.0):
    """ops.py:69-70"""
    return _act(x, "elu", alpha)


def leaky_relu(x, slope: float = 0.01):
    """ops.py:73-74"""
    return _act(x, "leaky", slope)


def snake(x, alpha, eps: float = 1e-9):
    """ops.py:77-81: x + sin^2(alpha x) / (alpha + eps) over (C, T)."""
    xd, res = _dev(x)
    ad = _w.device_f32(alpha) if not isinstance(alpha, DeviceArray) else alpha
    c = xd.shape[0]
    t = xd.size // c if c else 0
    y = DeviceArray(xd.shape, np.float32)
    _lib.call("snake", xd.ptr, ad.ptr, y.ptr, c, t, float(eps), None)
    return _ret(y, res)


def _last_axis(x, axis):
    nd = x.ndim
    ax = axis % nd if nd else 0
    return ax == nd - 1


def softmax(x, axis: int = -1):
    """ops.py:84-87"""
    return _softmax(x, axis, 0)


def log_softmax(x, axis: int = -1):
    """ops.py:90-93"""
    return _softmax(x, axis, 1)


def _softmax(x, axis, logmode):
    if isinstance(x, DeviceArray):
        if not _last_axis(x, axis):
            raise ValueError("device-resident softmax runs over the last axis")
        xd, res = x, True
    else:
        xa = np.asarray(x, dtype=np.float32)
        if not _last_axis(xa, axis):
            moved = np.moveaxis(xa, axis, -1)
            return np.moveaxis(_softmax(np.ascontiguousarray(moved), -1, logmode), -1, axis)
        xd, res = to_device(xa), False
    cols = xd.shape[-1] if xd.ndim else 1
    rows = xd.size // cols if cols else 0
    y = DeviceArray(xd.shape, np.float32)
    _lib.call("softmax_rows", xd.ptr, y.ptr, rows, cols, logmode, None)
    return _ret(y, res)


# ----------------------------------------------------------------------------
# norms, linear, embedding
# ----------------------------------------------------------------------------

def rms_norm(x, weight, eps: float = 1e-6):
    """ops.py:101-104"""
    xd, res = _dev(x)
    wd = _w.device_f32(weight)
    cols = xd.shape[-1]
    y = DeviceArray(xd.shape, np.float32)
    _lib.call("rms_norm", xd.ptr, wd.ptr, y.ptr, xd.size // cols, cols, float(eps), None)
    return _ret(y, res)


def layer_norm(x, weight=None, bias=None, eps: float = 1e-5):
    """ops.py:107-118"""
    xd, res = _dev(x)
    cols = xd.shape[-1]
    wd = _w.device_f32(weight) if weight is not None else None
    bd = _w.device_f32(bias) if bias is not None else None
    y = DeviceArray(xd.shape, np.float32)
    _lib.call("layer_norm", xd.ptr, y.ptr, xd.size // cols, cols, float(eps),
              wd.ptr if wd is not None else None, bd.ptr if bd is not None else None,
              None, None, 0, 0, None)
    return _ret(y, res)


def linear(x, weight: Weight, bias=None):
    """x @ weight.T + bias, weight (out, in) or QTensor (ops.py:121-123, quant.py:156-204)."""
    xd, res = _dev(x)
    k = xd.shape[-1]
    m = xd.size // k if k else 0
    bd = _w.device_f32(bias) if bias is not None else None
    if isinstance(weight, QTensor) or (hasattr(weight, "kind") and hasattr(weight, "scales")):
        dq = _w.device_qtensor(weight)
        n = dq.n
        if dq.k != k:
            raise ValueError(f"linear: x has {k} features but the weight expects {dq.k}")
        y = DeviceArray(xd.shape[:-1] + (n,), np.float32)
        _lib.call("linear_q", dq.kind_code, xd.ptr, m, k, k, dq.q.ptr, dq.scales.ptr, dq.scale_code,
                  dq.kp, dq.block, n, bd.ptr if bd is not None else None, y.ptr, n, None, None)
    else:
        wd = _w.device_f32(weight)
        n = wd.shape[0]
        if wd.size // max(n, 1) != k:
            raise ValueError(f"linear: x has {k} features but the weight is {wd.shape}")
        y = DeviceArray(xd.shape[:-1] + (n,), np.float32)
        _lib.call("linear_f32", xd.ptr, m, k, k, wd.ptr, k, n, bd.ptr if bd is not None else None,
                  y.ptr, n, None, None)
    return _ret(y, res)


def embedding(table: Weight, ids):
    """Bounds-checked row gather (ops.py:126-144); out-of-range ids raise IndexError."""
    ids_h = np.asarray(ids.numpy() if isinstance(ids, DeviceArray) else ids)
    resident = isinstance(ids, DeviceArray)
    flat = np.ascontiguousarray(ids_h.reshape(-1), dtype=np.int64)
    if isinstance(table, QTensor) or (hasattr(table, "kind") and hasattr(table, "scales")):
        dq = _w.device_qtensor(table)
        rows, cols = dq.n, dq.k
        args = (dq.kind_code, dq.q.ptr, dq.scales.ptr, dq.scale_code, rows, cols, dq.kp, dq.block)
    else:
        arr = table if isinstance(table, DeviceArray) else np.asarray(table)
        rows, cols = arr.shape[0], int(np.prod(arr.shape[1:]))
        if isinstance(arr, DeviceArray):
            td, kind = arr, (_lib.KIND_F16 if arr.dtype == np.float16 else _lib.KIND_F32)
        elif arr.dtype == np.float16:
            td, kind = _cached_raw(arr), _lib.KIND_F16
        else:
            td, kind = _w.device_f32(arr), _lib.KIND_F32
        args = (kind, td.ptr, None, _lib.F32, rows, cols, cols, 1)
    if flat.size and (int(flat.min()) < 0 or int(flat.max()) >= rows):
        raise IndexError(f"token id {int(flat.max())} is outside the {rows}-row embedding table")
    out = DeviceArray((flat.size, cols), np.float32)
    if flat.size:
        idd = to_device(flat)
        _lib.call("embedding", *args, idd.ptr, flat.size, out.ptr, None)
    out = out.reshape(ids_h.shape + (cols,))
    return _ret(out, resident)


def _cached_raw(arr: np.ndarray) -> DeviceArray:
    if not arr.flags.writeable:
        hit = _w._CACHE.get(id(arr))
        if hit is not None:
            return hit
        return _w._remember(arr, to_device(arr))
    return to_device(arr)


# ----------------------------------------------------------------------------
# convolution
# ----------------------------------------------------------------------------

def conv1d(x, weight: Weight, bias=None, stride: int = 1, dilation: int = 1, groups: int = 1,
           pad: Tuple[int, int] = (0, 0), kernel_size: Optional[int] = None,
           tile_bytes: int = TILE_BYTES):
    """(C_in, T) -> (C_out, T_out) 1-D convolution (ops.py:165-219)."""
    xd, res = _dev(x)
    if isinstance(weight, QTensor) or (hasattr(weight, "kind") and hasattr(weight, "scales")):
        k = kernel_size or weight.kernel_size
        if k is None:
            raise ValueError("kernel_size is required for a quantised conv weight "
                             "that does not record its original 3-D shape")
        assert groups == 1, "quantised grouped convs are not supported"
        cout = weight.shape[0]
        wd = _dequant_conv_weight(weight)
    else:
        wd = _w.device_f32(weight)
        cout, _, k = wd.shape if isinstance(weight, DeviceArray) else np.shape(weight)
    cin, t_in = xd.shape[0], (xd.size // xd.shape[0] if xd.shape[0] else 0)
    cin_g = wd.size // (cout * k)
    assert cin == cin_g * groups, (cin, cin_g, groups)
    bd = _w.device_f32(bias) if bias is not None else None
    t_out = ctypes.c_int64()
    _lib.call("conv1d", xd.ptr, cin, t_in, t_in, 1, wd.ptr, cout, k, None, stride, dilation, groups,
              pad[0], pad[1], 1, None, 0, 0, _lib.ptr(t_out), 0, 0.0, None, 0.0, None, 0, 0, None)
    n_out = max(0, t_out.value)
    y = DeviceArray((cout, n_out), np.float32)
    if n_out:
        _lib.call("conv1d", xd.ptr, cin, t_in, t_in, 1, wd.ptr, cout, k,
                  bd.ptr if bd is not None else None, stride, dilation, groups, pad[0], pad[1], 1,
                  y.ptr, n_out, 1, None, 0, 0.0, None, 0.0, None, 0, 0, None)
    return _ret(y, res)


def _dequant_conv_weight(qt) -> DeviceArray:
    hit = _w._CACHE.get(("conv", id(qt)))
    if hit is not None:
        return hit
    dq = _w.device_qtensor(qt)
    full = DeviceArray((dq.n, dq.k), np.float32)
    _lib.call("dequant_rows", dq.kind_code, dq.q.ptr, dq.scales.ptr, dq.scale_code, dq.kp, dq.block,
              dq.k, 0, dq.n, full.ptr, dq.k, None)
    return full


def depthwise_conv1d(x, weight, bias=None, dilation: int = 1, pad=(0, 0)):
    """groups == C convolution (ops.py:222-237)."""
    xd, res = _dev(x)
    wd = _w.device_f32(weight)
    c, one, k = wd.shape if isinstance(weight, DeviceArray) else np.shape(weight)
    assert one == 1
    bd = _w.device_f32(bias) if bias is not None else None
    t_in = xd.size // c
    t_out = t_in + pad[0] + pad[1] - dilation * (k - 1)
    y = DeviceArray((c, max(0, t_out)), np.float32)
    if t_out > 0:
        _lib.call("depthwise_conv1d", xd.ptr, c, t_in, wd.ptr, k, bd.ptr if bd is not None else None,
                  dilation, pad[0], pad[1], y.ptr, None, None)
    return _ret(y, res)


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------

def _mask_args(spec):
    if spec is None:
        return 0, 0, 0
    if spec[0] == "causal":
        return 1, int(spec[1]) if len(spec) > 1 else 0, 0
    if spec[0] == "chunk":
        return 2, int(spec[1]), int(spec[2])
    raise ValueError(f"unknown mask spec {spec}")


def sdpa(q, k, v, mask_spec=None, scale: Optional[float] = None, tile_bytes: int = TILE_BYTES):
    """Attention over (H, N, D) with GQA and causal/chunk masks (ops.py:267-300)."""
    mk, ma, mb = _mask_args(mask_spec)
    qd, res = _dev(q)
    kd, _ = _dev(k)
    vd, _ = _dev(v)
    h, n, d = qd.shape
    hk, m, _ = kd.shape
    if hk != h and h % hk:
        raise ValueError(f"{h} query heads is not a multiple of {hk} kv heads")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = DeviceArray((h, n, d), np.float32)
    S = ctypes.c_int64 * 3
    _lib.call("attention", qd.ptr, kd.ptr, vd.ptr, out.ptr, 1, h, hk, n, m, d,
              S(0, n * d, d), S(0, m * d, d), S(0, m * d, d), S(0, n * d, d),
              float(np.float32(scale)), mk, ma, mb, None)
    return _ret(out, res)


# ----------------------------------------------------------------------------
# resampling / STFT
# ----------------------------------------------------------------------------

def interpolate_linear(x, size: int, align_corners: bool = False):
    """ops.py:318-332"""
    xd, res = _dev(x)
    c, t = xd.shape
    if t == size:
        return _ret(xd.copy(), res)
    y = DeviceArray((c, size), np.float32)
    _lib.call("interp_linear", xd.ptr, y.ptr, c, t, size, int(bool(align_corners)), None)
    return _ret(y, res)


def interpolate_nearest(x, scale: int):
    """ops.py:335-336 (repeat along the last axis)."""
    xd, res = _dev(x)
    t = xd.shape[-1]
    c = xd.size // t if t else 0
    y = DeviceArray(xd.shape[:-1] + (t * scale,), np.float32)
    _lib.call("interp_nearest", xd.ptr, y.ptr, c, t, int(scale), None)
    return _ret(y, res)


def hann_window(n: int, periodic: bool = True):
    """ops.py:339-343"""
    y = DeviceArray((n,), np.float32)
    _lib.call("hann_window", int(n), int(bool(periodic)), y.ptr, None)
    return y.numpy()


def stft(x, n_fft: int, hop: int, win, center: bool = True, pad_mode: str = "reflect"):
    """One-sided STFT (F, frames) complex64 (ops.py:346-355).  Device input -> (re, im) DeviceArrays."""
    if pad_mode != "reflect" and center:
        raise ValueError("only reflect padding is implemented")
    xd, res = _dev(x)
    wd = _w.device_f32(win) if not isinstance(win, DeviceArray) else win
    frames = ctypes.c_int64()
    _lib.call("stft", xd.ptr, xd.size, n_fft, hop, wd.ptr, int(center), None, None, _lib.ptr(frames), None)
    f = n_fft // 2 + 1
    re = DeviceArray((f, frames.value), np.float32)
    im = DeviceArray((f, frames.value), np.float32)
    _lib.call("stft", xd.ptr, xd.size, n_fft, hop, wd.ptr, int(center), re.ptr, im.ptr, None, None)
    if res:
        return re, im
    return (re.numpy() + 1j * im.numpy()).astype(np.complex64)


def istft(spec, n_fft: int, hop: int, win, center: bool = True, length: Optional[int] = None):
    """Inverse STFT (ops.py:358-377).  ``spec`` is complex (F, N) or a (re, im) DeviceArray pair."""
    if isinstance(spec, tuple):
        red, imd = spec
        res = True
    else:
        sp = np.asarray(spec)
        red = to_device(np.ascontiguousarray(sp.real, dtype=np.float32))
        imd = to_device(np.ascontiguousarray(sp.imag, dtype=np.float32))
        res = False
    frames = red.shape[1]
    wd = _w.device_f32(win) if not isinstance(win, DeviceArray) else win
    buf = DeviceArray((frames, n_fft), np.float32)
    n_out = ctypes.c_int64()
    ln = -1 if length is None else int(length)
    _lib.call("istft", 0, red.ptr, imd.ptr, frames, n_fft, hop, wd.ptr, int(center), ln, 0.0, buf.ptr,
              None, _lib.ptr(n_out), None)
    y = DeviceArray((n_out.value,), np.float32)
    _lib.call("istft", 0, red.ptr, imd.ptr, frames, n_fft, hop, wd.ptr, int(center), ln, 0.0, buf.ptr,
              y.ptr, None, None)
    return _ret(y, res)
