"""Pin the oracle's kernels against textbook definitions written here.

Each reference below is the plain definition (scalar math, direct loops, a
materialised fp64 softmax, a direct DFT), so agreement means the oracle's
tiling, masking and conventions are right.  These restate the checks of the
reference's tests/test_ops.py against the oracle.
"""

import math

import numpy as np
import pytest

from conftest import rel_err as rel
import oracle.ops as ops


@pytest.fixture
def rng():
    return np.random.default_rng(0)


def _scalar(fn, x):
    return np.array([fn(float(v)) for v in np.asarray(x).reshape(-1)]).reshape(np.shape(x))


def test_activations_match_scalar_definitions(rng):
    x = rng.normal(size=(5, 17)).astype(np.float32) * 3.0
    assert rel(ops.silu(x), _scalar(lambda v: v / (1 + math.exp(-v)), x)) < 1e-6
    assert rel(ops.sigmoid(x), _scalar(lambda v: 1 / (1 + math.exp(-v)), x)) < 1e-6
    assert rel(ops.gelu(x), _scalar(lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2))), x)) < 1e-6
    assert rel(ops.gelu_tanh(x), _scalar(
        lambda v: 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))), x)) < 1e-6
    assert rel(ops.mish(x), _scalar(lambda v: v * math.tanh(math.log1p(math.exp(v))), x)) < 1e-5
    assert rel(ops.elu(x), _scalar(lambda v: v if v > 0 else math.expm1(v), x)) < 1e-6
    assert rel(ops.leaky_relu(x, 0.1), _scalar(lambda v: v if v >= 0 else 0.1 * v, x)) < 1e-6


def test_mish_guard():
    x = np.array([-50.0, 0.0, 20.0, 100.0, 1e4], dtype=np.float32)
    got = ops.mish(x)
    assert np.isfinite(got).all()
    assert rel(got[-2:], x[-2:]) < 1e-6


def test_snake(rng):
    a = np.abs(rng.normal(size=5)).astype(np.float32) + 0.5
    x = rng.normal(size=(5, 13)).astype(np.float32)
    ref = x + (1.0 / (a[:, None] + 1e-9)) * np.sin(a[:, None] * x) ** 2
    assert rel(ops.snake(x, a), ref) < 1e-6


def test_norms(rng):
    x = rng.normal(size=(5, 17)).astype(np.float32)
    w = rng.normal(size=17).astype(np.float32)
    b = rng.normal(size=17).astype(np.float32)
    ln = np.stack([(r - r.mean()) / np.sqrt(r.var() + 1e-6) for r in x.astype(np.float64)])
    assert rel(ops.layer_norm(x, None, None, 1e-6), ln) < 1e-5
    assert rel(ops.layer_norm(x, w, b, 1e-6), ln * w + b) < 1e-5
    rms = np.stack([r / np.sqrt((r ** 2).mean() + 1e-6) for r in x.astype(np.float64)])
    assert rel(ops.rms_norm(x, w, 1e-6), rms * w) < 1e-5


def test_softmax_stable(rng):
    x = rng.normal(size=(4, 9)).astype(np.float32) * 50
    p = ops.softmax(x)
    assert np.isfinite(p).all() and np.allclose(p.sum(-1), 1.0, atol=1e-6)
    x64 = x.astype(np.float64)
    m = x64.max(-1, keepdims=True)
    ref = x64 - (m + np.log(np.exp(x64 - m).sum(-1, keepdims=True)))
    assert np.abs(ops.log_softmax(x) - ref).max() < 1e-3


def naive_conv1d(x, w, b, stride, dilation, groups, pad):
    xp = np.pad(np.asarray(x, np.float64), ((0, 0), pad))
    cout, cin_g, k = w.shape
    cout_g = cout // groups
    t_out = (xp.shape[1] - (dilation * (k - 1) + 1)) // stride + 1
    out = np.zeros((cout, t_out))
    for o in range(cout):
        g = o // cout_g
        for t in range(t_out):
            acc = 0.0
            for c in range(cin_g):
                for j in range(k):
                    acc += w[o, c, j] * xp[g * cin_g + c, t * stride + j * dilation]
            out[o, t] = acc + (b[o] if b is not None else 0.0)
    return out


CONV_CASES = [
    (4, 6, 3, 1, 1, 1, 12, (1, 1)),
    (4, 6, 5, 1, 2, 1, 16, (4, 0)),          # causal, dilated
    (8, 8, 3, 1, 1, 4, 13, (2, 2)),          # grouped
    (3, 6, 4, 2, 1, 1, 17, (0, 0)),          # strided
    (18, 8, 30, 15, 1, 1, 61, (14, 0)),      # HiFT source downsample
    (16, 16, 7, 1, 1, 4, 20, (6, 0)),        # DiT-style grouped causal
]


@pytest.mark.parametrize("cin,cout,k,stride,dil,groups,T,pad", CONV_CASES)
def test_conv1d(rng, cin, cout, k, stride, dil, groups, T, pad):
    w = rng.normal(size=(cout, cin // groups, k)).astype(np.float32) * 0.1
    b = rng.normal(size=cout).astype(np.float32)
    x = rng.normal(size=(cin, T)).astype(np.float32)
    ref = naive_conv1d(x, w, b, stride, dil, groups, pad)
    for tile in (1 << 8, 1 << 20):
        got = ops.conv1d(x, w, b, stride=stride, dilation=dil, groups=groups, pad=pad, tile_bytes=tile)
        assert got.shape == ref.shape and rel(got, ref) < 1e-5


def test_depthwise(rng):
    c, k, t = 12, 7, 20
    w = rng.normal(size=(c, 1, k)).astype(np.float32)
    b = rng.normal(size=c).astype(np.float32)
    x = rng.normal(size=(c, t)).astype(np.float32)
    assert rel(ops.depthwise_conv1d(x, w, b, pad=(3, 3)), naive_conv1d(x, w, b, 1, 1, c, (3, 3))) < 1e-5


def naive_attention(q, k, v, mask=None):
    h, n, d = q.shape
    kk = np.repeat(k, h // k.shape[0], axis=0)
    vv = np.repeat(v, h // v.shape[0], axis=0)
    out = np.zeros((h, n, d))
    for i in range(h):
        s = q[i].astype(np.float64) @ kk[i].astype(np.float64).T / np.sqrt(d)
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        out[i] = (p / p.sum(-1, keepdims=True)) @ vv[i].astype(np.float64)
    return out


def chunk_mask(n, chunk, left=-1, m=None):
    m = n if m is None else m
    out = np.zeros((n, m), dtype=bool)
    for i in range(n):
        start = 0 if left < 0 else max((i // chunk - left) * chunk, 0)
        out[i, start:min((i // chunk + 1) * chunk, m)] = True
    return out


def test_attention_full_causal(rng):
    h, n, d = 4, 23, 16
    q, k, v = (rng.normal(size=(h, n, d)).astype(np.float32) for _ in range(3))
    for tile in (1 << 10, 1 << 22):
        assert rel(ops.sdpa(q, k, v, tile_bytes=tile), naive_attention(q, k, v)) < 1e-5
        assert rel(ops.sdpa(q, k, v, ("causal",), tile_bytes=tile),
                   naive_attention(q, k, v, np.tril(np.ones((n, n), bool)))) < 1e-5


@pytest.mark.parametrize("chunk,left", [(8, -1), (8, 1), (5, 0)])
def test_attention_chunk(rng, chunk, left):
    h, n, d = 4, 23, 16
    q, k, v = (rng.normal(size=(h, n, d)).astype(np.float32) for _ in range(3))
    assert rel(ops.sdpa(q, k, v, ("chunk", chunk, left), tile_bytes=1 << 10),
               naive_attention(q, k, v, chunk_mask(n, chunk, left))) < 1e-5


def test_attention_gqa_and_offset(rng):
    q = rng.normal(size=(4, 19, 16)).astype(np.float32)
    k = rng.normal(size=(2, 19, 16)).astype(np.float32)
    v = rng.normal(size=(2, 19, 16)).astype(np.float32)
    assert rel(ops.sdpa(q, k, v), naive_attention(q, k, v)) < 1e-5
    q1 = rng.normal(size=(4, 1, 16)).astype(np.float32)
    k1 = rng.normal(size=(4, 10, 16)).astype(np.float32)
    v1 = rng.normal(size=(4, 10, 16)).astype(np.float32)
    assert rel(ops.sdpa(q1, k1, v1, ("causal", 9)), naive_attention(q1, k1, v1)) < 1e-5
    with pytest.raises(ValueError):
        ops.sdpa(q, k[:1].repeat(3, 0), v[:1].repeat(3, 0))


def naive_stft(x, n_fft, hop, win):
    xp = np.pad(np.asarray(x, np.float64), (n_fft // 2, n_fft // 2), mode="reflect")
    n = 1 + (len(xp) - n_fft) // hop
    out = np.zeros((n_fft // 2 + 1, n), dtype=np.complex128)
    idx = np.arange(n_fft)
    for t in range(n):
        fr = xp[t * hop:t * hop + n_fft] * win
        for f in range(n_fft // 2 + 1):
            out[f, t] = (fr * np.exp(-2j * np.pi * f * idx / n_fft)).sum()
    return out


def test_stft_istft(rng):
    win = ops.hann_window(16)
    sig = rng.normal(size=200).astype(np.float32)
    got, ref = ops.stft(sig, 16, 4, win), naive_stft(sig, 16, 4, win)
    assert got.shape == ref.shape
    assert rel(np.stack([got.real, got.imag]), np.stack([ref.real, ref.imag])) < 1e-5
    sig2 = rng.normal(size=2000).astype(np.float32)
    back = ops.istft(ops.stft(sig2, 16, 4, win), 16, 4, win, length=len(sig2))
    assert rel(back[16:-16], sig2[16:-16]) < 1e-5
    spec = (rng.normal(size=(9, 51)) + 1j * rng.normal(size=(9, 51))).astype(np.complex64)
    assert len(ops.istft(spec, 16, 4, win)) == 50 * 4


def test_hann_and_interp(rng):
    assert rel(ops.hann_window(8), [0, 0.1464466, 0.5, 0.8535534, 1, 0.8535534, 0.5, 0.1464466]) < 1e-6
    x = np.arange(10, dtype=np.float32)[None, :]
    assert rel(ops.interpolate_linear(x, 5)[0], [0.5, 2.5, 4.5, 6.5, 8.5]) < 1e-6
    y = rng.normal(size=(3, 5)).astype(np.float32)
    up = ops.interpolate_nearest(y, 4)
    assert up.shape == (3, 20) and np.array_equal(up[:, 3::4], y)


def test_embedding_bounds():
    table = np.zeros((10, 4), dtype=np.float32)
    assert ops.embedding(table, np.array([0, 9])).shape == (2, 4)
    with pytest.raises(IndexError, match="outside"):
        ops.embedding(table, np.array([10]))
