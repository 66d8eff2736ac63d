"""Oracle restatement of the reference kernel library.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function restates the float32 semantics of the same-named function in
cv3cpu/ops.py (line numbers cited per function).  Tiling knobs
(``tile_bytes``) are kept so that the CPU timing baseline does the same
amount of work in the same blocking as the reference.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import numpy as np

from .quant import QTensor, qmatmul

Weight = Union[np.ndarray, QTensor]
TILE_BYTES = 8 << 20   # ops.py:23

_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)   # ops.py:38


# ----------------------------------------------------------------------------
# elementwise (ops.py:30-93)
# ----------------------------------------------------------------------------

def silu(x):
    """x / (1 + exp(-x)) in float32 (ops.py:30-31)."""
    return x / (1.0 + np.exp(-x, dtype=np.float32))


def sigmoid(x):
    """1 / (1 + exp(-x)) (ops.py:34-35)."""
    return 1.0 / (1.0 + np.exp(-x, dtype=np.float32))


def gelu_tanh(x):
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (ops.py:41-43)."""
    return 0.5 * x * (1.0 + np.tanh(_SQRT_2_OVER_PI * (x + 0.044715 * x * x * x)))


def _erf_as7126(x):
    """Abramowitz & Stegun 7.1.26 rational erf approximation (ops.py:51-60)."""
    s = np.sign(x)
    a = np.abs(x)
    t = 1.0 / (1.0 + 0.3275911 * a)
    poly = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t
             - 0.284496736) * t + 0.254829592) * t
    return s * (1.0 - poly * np.exp(-a * a))


def gelu(x):
    """Exact-erf GELU via the A&S erf (ops.py:46-48)."""
    return 0.5 * x * (1.0 + _erf_as7126(x / math.sqrt(2.0)))


def mish(x):
    """x tanh(softplus(x)), softplus = x above 20 (ops.py:63-66)."""
    sp = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    return x * np.tanh(sp)


def elu(x, alpha: float = 1.0):
    """x if x > 0 else alpha expm1(x) (ops.py:69-70)."""
    return np.where(x > 0, x, alpha * np.expm1(np.minimum(x, 0.0)))


def leaky_relu(x, slope: float = 0.01):
    """x if x >= 0 else slope x (ops.py:73-74)."""
    return np.where(x >= 0, x, x * slope)


def snake(x, alpha, eps: float = 1e-9):
    """x + sin^2(alpha x) / (alpha + eps), alpha per row of (C, T) (ops.py:77-81)."""
    a = alpha.reshape(-1, 1)
    s = np.sin(a * x)
    return x + (1.0 / (a + eps)) * (s * s)


def softmax(x, axis: int = -1):
    """Max-subtracted softmax (ops.py:84-87)."""
    e = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return e / np.sum(e, axis=axis, keepdims=True)


def log_softmax(x, axis: int = -1):
    """z - log(sum(exp(z))), z = x - max (ops.py:90-93)."""
    z = x - np.max(x, axis=axis, keepdims=True)
    return z - np.log(np.sum(np.exp(z), axis=axis, keepdims=True))


# ----------------------------------------------------------------------------
# norms, linear, embedding (ops.py:101-144)
# ----------------------------------------------------------------------------

def rms_norm(x, weight, eps: float = 1e-6):
    """x * (1/sqrt(mean(x^2) + eps)) * w (ops.py:101-104)."""
    x32 = x.astype(np.float32, copy=False)
    ms = np.mean(x32 * x32, axis=-1, keepdims=True)
    return (x32 * (1.0 / np.sqrt(ms + eps))) * weight


def layer_norm(x, weight=None, bias=None, eps: float = 1e-5):
    """Two-pass centred LayerNorm, optional affine (ops.py:107-118)."""
    x32 = x.astype(np.float32, copy=False)
    xc = x32 - np.mean(x32, axis=-1, keepdims=True)
    y = xc / np.sqrt(np.mean(xc * xc, axis=-1, keepdims=True) + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def linear(x, weight: Weight, bias=None):
    """x @ W.T + b, W is (out, in) (ops.py:121-123)."""
    return qmatmul(x, weight, bias)


def embedding(table: Weight, ids):
    """Bounds-checked row gather; QTensor rows are dequantised once each (ops.py:126-144)."""
    ids = np.asarray(ids)
    nrows = table.shape[0] if isinstance(table, QTensor) else np.shape(table)[0]
    if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= nrows):
        raise IndexError(f"token id {int(ids.max())} is outside the {nrows}-row embedding table")
    if isinstance(table, QTensor):
        flat = ids.reshape(-1)
        uniq, inv = np.unique(flat, return_inverse=True)
        rows = np.stack([table.dequant_rows(int(r), int(r) + 1)[0] for r in uniq]) \
            if uniq.size else np.zeros((0, table.shape[1]), np.float32)
        return rows[inv].reshape(*ids.shape, table.shape[1])
    return np.asarray(table[ids], dtype=np.float32)


# ----------------------------------------------------------------------------
# convolution (ops.py:152-237)
# ----------------------------------------------------------------------------

def _patches(xp, k, stride, dilation, t0, t1):
    """(C, k, t1-t0) strided patch view for output frames [t0, t1) (ops.py:152-162)."""
    c = xp.shape[0]
    s_c, s_t = xp.strides
    return np.lib.stride_tricks.as_strided(
        xp[:, t0 * stride:], shape=(c, k, t1 - t0),
        strides=(s_c, s_t * dilation, s_t * stride), writeable=False)


def conv1d(x, weight: Weight, bias=None, stride: int = 1, dilation: int = 1,
           groups: int = 1, pad: Tuple[int, int] = (0, 0),
           kernel_size: Optional[int] = None, tile_bytes: int = TILE_BYTES):
    """(C_in, T) -> (C_out, T_out) convolution via time-tiled im2col (ops.py:165-219).

    ``weight`` is (C_out, C_in/groups, k) or a QTensor of the flattened
    (C_out, C_in*k) weight (groups == 1 only).  Inputs and weights are cast to
    float32 whatever their dtype (ops.py:182,190), so the F0 network's
    "float64" convolutions also run in float32.
    """
    quant = isinstance(weight, QTensor)
    if quant:
        cout = weight.shape[0]
        k = kernel_size or weight.kernel_size
        if k is None:
            raise ValueError("kernel_size is required for a quantised conv weight "
                             "that does not record its original 3-D shape")
        cin_g = weight.shape[1] // k
    else:
        weight = np.asarray(weight, dtype=np.float32)
        cout, cin_g, k = weight.shape
    assert x.shape[0] == cin_g * groups, (x.shape[0], cin_g, groups)
    dt = np.float32
    xp = np.pad(x, ((0, 0), pad)) if (pad[0] or pad[1]) else x
    xp = np.ascontiguousarray(xp, dtype=dt)
    span = dilation * (k - 1) + 1
    t_out = (xp.shape[1] - span) // stride + 1
    if t_out <= 0:
        return np.zeros((cout, 0), dtype=np.float32)
    out = np.empty((cout, t_out), dtype=dt)
    tile = max(1, min(t_out, tile_bytes // max(1, cin_g * k * 4)))
    cout_g = cout // groups
    for g in range(groups):
        xg = xp[g * cin_g:(g + 1) * cin_g]
        if quant:
            assert groups == 1, "quantised grouped convs are not supported"
        else:
            wg = weight[g * cout_g:(g + 1) * cout_g].reshape(cout_g, cin_g * k)
        for t0 in range(0, t_out, tile):
            t1 = min(t_out, t0 + tile)
            cols = np.ascontiguousarray(_patches(xg, k, stride, dilation, t0, t1))
            cols = cols.reshape(cin_g * k, t1 - t0)
            if quant:
                out[:, t0:t1] = qmatmul(cols.T, weight).T
            else:
                out[g * cout_g:(g + 1) * cout_g, t0:t1] = np.dot(wg, cols)
    if bias is not None:
        out += np.asarray(bias, dtype=dt).reshape(-1, 1)
    return out


def depthwise_conv1d(x, weight, bias=None, dilation: int = 1, pad=(0, 0)):
    """groups == C conv as k shifted multiply-accumulates (ops.py:222-237)."""
    weight = np.asarray(weight, dtype=np.float32)
    c, one, k = weight.shape
    assert one == 1
    xp = np.pad(x, ((0, 0), pad)) if (pad[0] or pad[1]) else x
    t_out = xp.shape[1] - dilation * (k - 1)
    out = np.zeros((c, t_out), dtype=np.float32)
    for j in range(k):
        out += weight[:, 0, j:j + 1] * xp[:, j * dilation:j * dilation + t_out]
    if bias is not None:
        out += np.asarray(bias, dtype=np.float32).reshape(-1, 1)
    return out


# ----------------------------------------------------------------------------
# attention (ops.py:244-310)
# ----------------------------------------------------------------------------

def block_mask(q0, q1, k0, k1, spec):
    """Boolean (q1-q0, k1-k0) mask block; None = all allowed (ops.py:244-264)."""
    if spec is None:
        return None
    qi = np.arange(q0, q1)[:, None]
    ki = np.arange(k0, k1)[None, :]
    if spec[0] == "causal":
        off = spec[1] if len(spec) > 1 else 0
        return ki <= qi + off
    if spec[0] == "chunk":
        size, left = spec[1], spec[2]
        end = (qi // size + 1) * size
        start = np.zeros_like(qi) if left < 0 else np.maximum((qi // size - left) * size, 0)
        return (ki < end) & (ki >= start)
    raise ValueError(f"unknown mask spec {spec}")


def additive_mask(q0, q1, m, spec):
    """(1, q1-q0, m) float mask, -inf where forbidden (ops.py:303-310)."""
    if spec is None:
        return None
    allowed = block_mask(q0, q1, 0, m, spec)
    add = np.zeros((1, q1 - q0, m), dtype=np.float32)
    add[0][~allowed] = -np.inf
    return add


def sdpa(q, k, v, mask_spec=None, scale: Optional[float] = None, tile_bytes: int = TILE_BYTES):
    """Query-tiled softmax attention over (H, N, D) with GQA (ops.py:267-300).

    The scale multiplies q before q@k^T (scale defaults to 1/sqrt(D)); each
    query tile takes one ordinary max-subtracted softmax over all keys.
    kv head of query head i is i // (H/Hk).
    """
    h, n, d = q.shape
    hk, m, _ = k.shape
    if hk != h:
        if h % hk:
            raise ValueError(f"{h} query heads is not a multiple of {hk} kv heads")
        k = np.repeat(k, h // hk, axis=0)
        v = np.repeat(v, h // hk, axis=0)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    tq = max(1, min(n, tile_bytes // max(1, h * m * 4)))
    kt = np.ascontiguousarray(np.swapaxes(k, 1, 2))
    out = np.empty((h, n, d), dtype=np.float32)
    for q0 in range(0, n, tq):
        q1 = min(n, q0 + tq)
        s = (q[:, q0:q1] * np.float32(scale)) @ kt
        add = additive_mask(q0, q1, m, mask_spec)
        if add is not None:
            s += add
        s -= s.max(axis=-1, keepdims=True)
        np.exp(s, out=s)
        s /= s.sum(axis=-1, keepdims=True)
        out[:, q0:q1] = s @ v
    return out


# ----------------------------------------------------------------------------
# resampling / STFT (ops.py:318-377)
# ----------------------------------------------------------------------------

def interpolate_linear(x, size: int, align_corners: bool = False):
    """F.interpolate(mode='linear') over the last axis of (C, T) (ops.py:318-332)."""
    c, t = x.shape
    if t == size:
        return x.astype(np.float32, copy=True)
    if align_corners:
        pos = np.linspace(0.0, t - 1.0, size, dtype=np.float64)
    else:
        pos = np.clip((np.arange(size, dtype=np.float64) + 0.5) * (t / size) - 0.5, 0.0, t - 1.0)
    i0 = np.floor(pos).astype(np.int64)
    i1 = np.minimum(i0 + 1, t - 1)
    f = (pos - i0).astype(np.float32)
    return x[:, i0] * (1.0 - f) + x[:, i1] * f


def interpolate_nearest(x, scale: int):
    """Repeat each frame ``scale`` times (ops.py:335-336)."""
    return np.repeat(x, scale, axis=-1)


def hann_window(n: int, periodic: bool = True):
    """Periodic (fftbins) or symmetric Hann in float32 (ops.py:339-343)."""
    denom = n if periodic else (n - 1)
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n) / denom)).astype(np.float32)


def stft(x, n_fft: int, hop: int, win, center: bool = True, pad_mode: str = "reflect"):
    """One-sided complex STFT (F, frames), torch.stft conventions (ops.py:346-355)."""
    x = np.asarray(x, dtype=np.float32)
    if center:
        x = np.pad(x, (n_fft // 2, n_fft // 2), mode=pad_mode)
    nfr = 1 + (len(x) - n_fft) // hop
    fr = np.lib.stride_tricks.as_strided(x, shape=(nfr, n_fft),
                                         strides=(x.strides[0] * hop, x.strides[0]),
                                         writeable=False)
    return np.fft.rfft(fr * win, n=n_fft, axis=1).T


def istft(spec, n_fft: int, hop: int, win, center: bool = True, length: Optional[int] = None):
    """Inverse STFT: irfft, window, overlap-add, divide by sum(w^2) where > 1e-11,
    trim n_fft/2 each side (ops.py:358-377)."""
    fr = np.fft.irfft(spec, n=n_fft, axis=0).astype(np.float32) * win[:, None]
    nfr = fr.shape[1]
    total = (nfr - 1) * hop + n_fft
    y = np.zeros(total, dtype=np.float32)
    env = np.zeros(total, dtype=np.float32)
    w2 = (win * win).astype(np.float32)
    for j in range(n_fft):
        y[j:j + (nfr - 1) * hop + 1:hop] += fr[j]
        env[j:j + (nfr - 1) * hop + 1:hop] += w2[j]
    ok = np.abs(env) > 1e-11
    y[ok] /= env[ok]
    if center:
        y = y[n_fft // 2:total - n_fft // 2]
    if length is not None:
        y = y[:length] if len(y) >= length else np.pad(y, (0, length - len(y)))
    return y
