"""The oracle's kernel semantics (oracle/ops.py) pinned by mathematics alone.

Each check is built so that a plausible slip in the restatement (a dropped term,
a wrong sign, an off-by-one in a pad or a mask edge, a transposed operand) fails:

* closed forms evaluated in float64 with NumPy's own vectorised math;
* algebraic identities the operation must obey (shift invariance of softmax,
  scale invariance of RMSNorm, linearity and the impulse response of a conv,
  Parseval for the STFT, permutation equivariance of attention);
* independent float64 references written differently from the oracle: a conv
  as an einsum over sliding windows, attention as one materialised einsum with a
  broadcast mask, the STFT as a product with an explicit DFT matrix.

Error norm: max|got - ref| / max|ref| (``conftest.rel_err``).
"""

import numpy as np
import pytest

from conftest import rel_err
import oracle.ops as ops


def _draw(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# ----------------------------------------------------------------------------
# elementwise (cv3cpu/ops.py:30-81)
# ----------------------------------------------------------------------------

def _f64(x):
    return np.asarray(x, np.float64)


def test_logistic_family_closed_forms():
    x = np.linspace(-30.0, 30.0, 1201, dtype=np.float32)
    d = _f64(x)
    sig = 0.5 * (1.0 + np.tanh(0.5 * d))          # logistic written through tanh
    assert rel_err(ops.sigmoid(x), sig) < 1e-6
    assert rel_err(ops.silu(x), d * sig) < 1e-6
    # softplus through log-add-exp, then the mish identity x * tanh(softplus(x))
    assert rel_err(ops.mish(x), d * np.tanh(np.logaddexp(0.0, d))) < 1e-5


def test_gelu_variants():
    x = np.linspace(-8.0, 8.0, 801, dtype=np.float32)
    d = _f64(x)
    from scipy.special import erf
    exact = 0.5 * d * (1.0 + erf(d / np.sqrt(2.0)))
    # the erf-based GELU follows a polynomial erf of absolute error ~1.5e-7
    assert np.abs(ops.gelu(x) - exact).max() < 2e-6 * max(1.0, np.abs(exact).max())
    cubic = d + 0.044715 * d ** 3
    tanh_form = 0.5 * d * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * cubic))
    assert rel_err(ops.gelu_tanh(x), tanh_form) < 1e-6
    # and the two agree to the tanh approximation's known accuracy
    assert np.abs(tanh_form - exact).max() < 1e-3


def test_piecewise_activations():
    x = np.concatenate([np.linspace(-6, 6, 97, dtype=np.float32), np.float32([0.0, -0.0, 1e-30, -1e-30])])
    d = _f64(x)
    assert rel_err(ops.elu(x), np.where(d > 0, d, np.expm1(d))) < 1e-6
    assert rel_err(ops.elu(x, 0.5), np.where(d > 0, d, 0.5 * np.expm1(d))) < 1e-6
    for slope in (0.1, 0.01, 0.2):
        assert rel_err(ops.leaky_relu(x, slope), np.where(d >= 0, d, slope * d)) < 1e-7
    # continuity at 0 and the asymptotes
    assert ops.elu(np.float32([-40.0]))[0] == pytest.approx(-1.0, abs=1e-6)
    assert ops.mish(np.float32([0.0]))[0] == 0.0


def test_mish_large_inputs_take_the_guard():
    big = np.float32([20.5, 50.0, 100.0, 3e4])
    got = ops.mish(big)
    assert np.isfinite(got).all() and np.array_equal(got, big)   # tanh(x) == 1 in float32 there
    assert np.isfinite(ops.mish(np.float32([-200.0, -1e4]))).all()


def test_snake_zeros_and_periodicity():
    alpha = np.float32([0.5, 1.0, 2.5])
    # at x = k pi / alpha, sin(alpha x) vanishes and snake is the identity
    k = np.arange(-3, 4, dtype=np.float64)
    x = (k[None, :] * np.pi / _f64(alpha)[:, None]).astype(np.float32)
    assert np.abs(ops.snake(x, alpha) - x).max() < 1e-5
    # float64 definition elsewhere
    y = _draw(3, 3, 40, scale=2.0)
    ref = _f64(y) + np.sin(_f64(alpha)[:, None] * _f64(y)) ** 2 / (_f64(alpha)[:, None] + 1e-9)
    assert rel_err(ops.snake(y, alpha), ref) < 1e-6


# ----------------------------------------------------------------------------
# softmax and norms (cv3cpu/ops.py:84-118)
# ----------------------------------------------------------------------------

def test_softmax_identities():
    x = _draw(4, 6, 33, scale=8.0)
    p = ops.softmax(x)
    assert np.allclose(p.sum(-1), 1.0, atol=1e-6) and (p >= 0).all()
    # invariant under a per-row shift, including shifts that would overflow exp
    assert rel_err(ops.softmax(x + np.float32(1e3)), p) < 1e-5
    d = _f64(x)
    ref = np.exp(d - d.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    assert rel_err(p, ref) < 1e-6
    assert np.abs(ops.log_softmax(x) - np.log(ref)).max() < 1e-4
    # the other axis
    assert rel_err(ops.softmax(x, axis=0), np.exp(d - d.max(0)) / np.exp(d - d.max(0)).sum(0)) < 1e-6


def test_rms_norm_scale_invariance_and_definition():
    x = _draw(5, 4, 96)
    w = _draw(6, 96)
    y = ops.rms_norm(x, w, 1e-6)
    d = _f64(x)
    assert rel_err(y, d / np.sqrt(np.mean(d * d, -1, keepdims=True) + 1e-6) * _f64(w)) < 1e-6
    assert rel_err(ops.rms_norm(np.float32(7.0) * x, w, 1e-6), y) < 1e-5   # rows far above eps


def test_layer_norm_moments_and_affine():
    x = _draw(7, 5, 130, scale=3.0) + np.float32(4.0)
    y = _f64(ops.layer_norm(x, None, None, 1e-6))
    assert np.abs(y.mean(-1)).max() < 1e-5 and np.abs(y.var(-1) - 1.0).max() < 1e-4
    g, b = _draw(8, 130), _draw(9, 130)
    # rows whose variance is comparable to eps: eps sits inside the square root, once
    small = _draw(10, 3, 130, scale=2e-3)
    d = _f64(small) - _f64(small).mean(-1, keepdims=True)
    ref = d / np.sqrt((d * d).mean(-1, keepdims=True) + 1e-6)
    assert rel_err(ops.layer_norm(small, g, b, 1e-6), ref * _f64(g) + _f64(b)) < 1e-5
    assert rel_err(ops.layer_norm(x, g, b, 1e-6), y * _f64(g) + _f64(b)) < 1e-5
    # a constant row normalises to exactly zero (centred variance, not E[x^2] - E[x]^2)
    const = np.full((1, 64), 3.25, np.float32)
    assert np.abs(ops.layer_norm(const, None, None, 1e-6)).max() == 0.0


# ----------------------------------------------------------------------------
# convolution (cv3cpu/ops.py:152-237)
# ----------------------------------------------------------------------------

def conv_ref(x, w, b, stride, dilation, groups, pad):
    """float64 conv via sliding windows and one einsum per group."""
    xp = np.pad(_f64(x), ((0, 0), pad))
    cout, cig, k = w.shape
    span = dilation * (k - 1) + 1
    win = np.lib.stride_tricks.sliding_window_view(xp, span, axis=1)[:, ::stride, ::dilation]   # (C, T_out, k)
    cog = cout // groups
    out = np.concatenate([np.einsum("ctk,ock->ot", win[g * cig:(g + 1) * cig], _f64(w[g * cog:(g + 1) * cog]))
                          for g in range(groups)], axis=0)
    return out if b is None else out + _f64(b)[:, None]


# (cin, cout, k, stride, dilation, groups, T, (pad_l, pad_r))
GEOMETRIES = [
    (3, 5, 1, 1, 1, 1, 9, (0, 0)),            # pointwise
    (6, 4, 2, 1, 3, 2, 15, (3, 0)),           # even kernel, dilated, grouped
    (10, 10, 9, 1, 1, 10, 30, (8, 0)),        # depthwise, causal
    (4, 12, 6, 3, 1, 1, 25, (2, 3)),          # strided, asymmetric pad
    (9, 9, 21, 7, 1, 3, 70, (10, 0)),         # long strided kernel in groups
    (32, 8, 5, 1, 4, 8, 40, (16, 0)),         # wide input, many groups
]


@pytest.mark.parametrize("cin,cout,k,stride,dil,groups,T,pad", GEOMETRIES)
def test_conv1d_against_windows(cin, cout, k, stride, dil, groups, T, pad):
    w = _draw(10 + k, cout, cin // groups, k, scale=0.3)
    b = _draw(11, cout)
    x = _draw(12 + T, cin, T)
    ref = conv_ref(x, w, b, stride, dil, groups, pad)
    for tile in (64, 1 << 24):      # one output frame per tile, and the whole signal in one
        got = ops.conv1d(x, w, b, stride=stride, dilation=dil, groups=groups, pad=pad, tile_bytes=tile)
        assert got.shape == ref.shape
        assert rel_err(got, ref) < 1e-5


def test_conv1d_impulse_response():
    """A unit impulse at input position p of channel c lands w[o, c, j] at every output t
    with t * stride + j * dilation == p + pad_l: the kernel is not flipped, and the
    stride, dilation and pad offsets all enter where they should."""
    cin, cout, k, stride, dil, pad = 2, 3, 4, 2, 3, (5, 1)
    w = _draw(13, cout, cin, k)
    T = 20
    for c in range(cin):
        for p in (0, 7, T - 1):
            x = np.zeros((cin, T), np.float32)
            x[c, p] = 1.0
            y = ops.conv1d(x, w, None, stride=stride, dilation=dil, pad=pad)
            want = np.zeros_like(y)
            for j in range(k):
                q = p + pad[0] - j * dil
                if q >= 0 and q % stride == 0 and q // stride < y.shape[1]:
                    want[:, q // stride] += w[:, c, j]
            assert np.array_equal(y, want)


def test_conv1d_linearity_and_bias():
    w = _draw(14, 6, 6, 3)
    a, b = _draw(15, 6, 31), _draw(16, 6, 31)
    bias = _draw(17, 6)
    f = lambda x, bb=None: _f64(ops.conv1d(x, w, bb, dilation=2, pad=(4, 0)))
    assert rel_err(f(np.float32(2.0) * a - b), 2.0 * f(a) - f(b)) < 1e-5
    assert rel_err(f(a, bias) - f(a), np.broadcast_to(_f64(bias)[:, None], f(a).shape)) < 1e-5


def test_conv1d_empty_output_and_errors():
    w = _draw(18, 2, 2, 9)
    assert ops.conv1d(_draw(19, 2, 4), w).shape == (2, 0)
    with pytest.raises(AssertionError):
        ops.conv1d(_draw(19, 3, 20), w)          # channels do not match the weight


def test_depthwise_is_grouped_conv():
    c = 7
    w = _draw(20, c, 1, 5)
    b = _draw(21, c)
    x = _draw(22, c, 26)
    assert rel_err(ops.depthwise_conv1d(x, w, b, dilation=2, pad=(8, 0)),
                   conv_ref(x, w, b, 1, 2, c, (8, 0))) < 1e-5


# ----------------------------------------------------------------------------
# attention (cv3cpu/ops.py:244-310)
# ----------------------------------------------------------------------------

def allowed_ref(n, m, spec):
    """Boolean (n, m) visibility from the mask spec, by broadcast comparisons."""
    i = np.arange(n)[:, None]
    j = np.arange(m)[None, :]
    if spec is None:
        return np.ones((n, m), bool)
    if spec[0] == "causal":
        return j - i <= (spec[1] if len(spec) > 1 else 0)
    size, left = spec[1], spec[2]
    blk_i, blk_j = i // size, j // size
    lo = np.full_like(blk_i, -1 << 40) if left < 0 else blk_i - left
    return (blk_j <= blk_i) & (blk_j >= lo)


def attention_ref(q, k, v, spec=None, scale=None):
    h, n, d = q.shape
    rep = h // k.shape[0]
    kk, vv = _f64(np.repeat(k, rep, 0)), _f64(np.repeat(v, rep, 0))
    s = np.einsum("hnd,hmd->hnm", _f64(q), kk) * (1.0 / np.sqrt(d) if scale is None else scale)
    s = np.where(allowed_ref(n, k.shape[1], spec)[None], s, -np.inf)
    s = np.exp(s - s.max(-1, keepdims=True))
    return np.einsum("hnm,hmd->hnd", s / s.sum(-1, keepdims=True), vv)


@pytest.mark.parametrize("spec", [None, ("causal",), ("causal", 3), ("chunk", 6, -1), ("chunk", 6, 0),
                                  ("chunk", 4, 2)])
@pytest.mark.parametrize("tile", [256, 1 << 24])
def test_sdpa_masks(spec, tile):
    q, k, v = _draw(23, 3, 29, 8), _draw(24, 3, 29, 8), _draw(25, 3, 29, 8)
    assert rel_err(ops.sdpa(q, k, v, spec, tile_bytes=tile), attention_ref(q, k, v, spec)) < 1e-5


def test_sdpa_gqa_explicit_scale_and_decode_row():
    q = _draw(26, 6, 11, 16)
    k, v = _draw(27, 2, 11, 16), _draw(28, 2, 11, 16)
    assert rel_err(ops.sdpa(q, k, v, scale=0.3), attention_ref(q, k, v, scale=0.3)) < 1e-5
    # query heads 0-2 see kv head 0 and 3-5 kv head 1
    assert rel_err(ops.sdpa(q[3:], k[1:], v[1:]), attention_ref(q, k, v)[3:]) < 1e-5
    # one new query against a longer cache, causal with the cache offset: sees everything
    q1 = _draw(29, 6, 1, 16)
    assert rel_err(ops.sdpa(q1, k, v, ("causal", 10)), attention_ref(q1, k, v)) < 1e-5
    with pytest.raises(ValueError):
        ops.sdpa(q[:5], k, v)                    # 5 query heads over 2 kv heads
    with pytest.raises(ValueError):
        ops.sdpa(q, k, v, ("window", 3))


def test_sdpa_key_permutation_and_uniform_keys():
    """Without a mask the output does not depend on key order; identical keys average v."""
    q, k, v = _draw(30, 2, 7, 8), _draw(31, 2, 13, 8), _draw(32, 2, 13, 8)
    perm = np.random.default_rng(33).permutation(13)
    assert rel_err(ops.sdpa(q, k[:, perm], v[:, perm]), ops.sdpa(q, k, v)) < 1e-5
    same = np.repeat(k[:, :1], 13, axis=1)
    assert rel_err(ops.sdpa(q, same, v), np.broadcast_to(_f64(v).mean(1, keepdims=True), q.shape)) < 1e-5


# ----------------------------------------------------------------------------
# resampling and STFT (cv3cpu/ops.py:318-377)
# ----------------------------------------------------------------------------

def test_hann_closed_form():
    for n in (4, 16, 31):
        i = np.arange(n)
        assert rel_err(ops.hann_window(n), np.sin(np.pi * i / n) ** 2) < 1e-6
        assert rel_err(ops.hann_window(n, periodic=False), np.sin(np.pi * i / (n - 1)) ** 2) < 1e-6


def test_interpolation():
    y = _draw(34, 4, 6)
    assert np.array_equal(ops.interpolate_nearest(y, 5), np.kron(y, np.ones((1, 5), np.float32)))
    ramp = np.arange(12, dtype=np.float32)[None] * np.float32(2.0)
    # half-pixel centres on a linear ramp reproduce the ramp at the new centres (clamped at the ends)
    got = ops.interpolate_linear(ramp, 4)
    centres = np.clip((np.arange(4) + 0.5) * 3.0 - 0.5, 0, 11) * 2.0
    assert rel_err(got[0], centres) < 1e-6
    assert rel_err(ops.interpolate_linear(ramp, 23, align_corners=True)[0], np.linspace(0, 22, 23)) < 1e-6


def _dft_stft(x, n_fft, hop, win):
    xp = np.pad(_f64(x), n_fft // 2, mode="reflect")
    frames = np.lib.stride_tricks.sliding_window_view(xp, n_fft)[::hop] * _f64(win)
    f = np.arange(n_fft // 2 + 1)[:, None]
    dft = np.exp(-2j * np.pi * f * np.arange(n_fft)[None, :] / n_fft)
    return dft @ frames.T


@pytest.mark.parametrize("n_fft,hop,length", [(16, 4, 301), (8, 2, 64), (32, 8, 129)])
def test_stft_against_dft_matrix(n_fft, hop, length):
    win = ops.hann_window(n_fft)
    sig = _draw(35 + n_fft, length)
    got, ref = ops.stft(sig, n_fft, hop, win), _dft_stft(sig, n_fft, hop, win)
    assert got.shape == ref.shape
    assert rel_err(np.concatenate([got.real, got.imag]), np.concatenate([ref.real, ref.imag])) < 1e-5


def test_stft_parseval_per_frame():
    """With a rectangular window each frame's one-sided spectrum carries its energy."""
    n_fft, hop = 16, 4
    sig = _draw(36, 200)
    spec = _f64(np.abs(ops.stft(sig, n_fft, hop, np.ones(n_fft, np.float32)))) ** 2
    wts = np.full(n_fft // 2 + 1, 2.0)
    wts[0] = wts[-1] = 1.0
    frames = np.lib.stride_tricks.sliding_window_view(np.pad(_f64(sig), 8, mode="reflect"), n_fft)[::hop]
    assert rel_err((wts[:, None] * spec).sum(0) / n_fft, (frames ** 2).sum(1)) < 1e-5


def test_istft_inverts_stft_and_frame_count():
    win = ops.hann_window(16)
    sig = _draw(37, 1500)
    back = ops.istft(ops.stft(sig, 16, 4, win), 16, 4, win, length=len(sig))
    assert back.shape == sig.shape
    # the reflect-padded ends are covered too: hop 4 with a periodic Hann window is COLA
    assert rel_err(back, sig) < 1e-5
    spec = (_draw(38, 9, 40) + 1j * _draw(39, 9, 40)).astype(np.complex64)
    assert ops.istft(spec, 16, 4, win).shape == (39 * 4,)
    assert ops.istft(spec, 16, 4, win, length=200).shape == (200,)


def test_embedding_bounds():
    table = np.arange(20, dtype=np.float32).reshape(5, 4)
    assert np.array_equal(ops.embedding(table, np.array([4, 0, 4])), table[[4, 0, 4]])
    for bad in (5, -1):
        with pytest.raises(IndexError, match="outside"):
            ops.embedding(table, np.array([bad]))
