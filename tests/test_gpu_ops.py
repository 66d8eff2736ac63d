"""GPU parity of every drop-in op (cv3amd.ops / cv3amd.quant) against the oracle.

Tolerances: int8 codes and scales bit-exact; fp32 outputs within 1e-5 of the
oracle in the reference's max-norm relative error (rel_err).
"""

import ctypes

import numpy as np
import pytest

from conftest import rel_err
import oracle.ops as ref
import oracle.quant as refq

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def dev(gpu):
    import cv3amd.ops as ops
    import cv3amd.quant as quant
    return ops, quant


@pytest.fixture
def rng():
    return np.random.default_rng(0)


@pytest.mark.parametrize("name,args", [("silu", ()), ("sigmoid", ()), ("gelu_tanh", ()), ("gelu", ()),
                                       ("mish", ()), ("elu", (1.0,)), ("leaky_relu", (0.1,))])
def test_activations(dev, rng, name, args):
    ops, _ = dev
    x = (rng.normal(size=(7, 333)) * 4).astype(np.float32)
    x[0, :6] = [0.0, -0.0, 30.0, -30.0, 1e-20, -1e-20]
    assert rel_err(getattr(ops, name)(x, *args), getattr(ref, name)(x, *args)) < TOL


def test_mish_large_inputs(dev):
    ops, _ = dev
    x = np.array([-50.0, 0.0, 20.0, 100.0, 1e4], dtype=np.float32)
    got = ops.mish(x)
    assert np.isfinite(got).all() and rel_err(got, ref.mish(x)) < TOL


def test_snake(dev, rng):
    ops, _ = dev
    a = (np.abs(rng.normal(size=64)) + 0.5).astype(np.float32)
    x = (rng.normal(size=(64, 1001)) * 3).astype(np.float32)
    assert rel_err(ops.snake(x, a), ref.snake(x, a)) < TOL


@pytest.mark.parametrize("shape", [(4, 9), (1, 6761), (3, 5, 17)])
def test_softmax(dev, rng, shape):
    ops, _ = dev
    x = (rng.normal(size=shape) * 20).astype(np.float32)
    assert rel_err(ops.softmax(x), ref.softmax(x)) < TOL
    assert rel_err(ops.log_softmax(x), ref.log_softmax(x)) < TOL
    assert rel_err(ops.softmax(x, axis=0), ref.softmax(x, axis=0)) < TOL


def test_norms(dev, rng):
    ops, _ = dev
    x = rng.normal(size=(6, 1024)).astype(np.float32) * 3 + 1
    w = rng.normal(size=1024).astype(np.float32)
    b = rng.normal(size=1024).astype(np.float32)
    assert rel_err(ops.rms_norm(x[:, :896], w[:896]), ref.rms_norm(x[:, :896], w[:896])) < TOL
    assert rel_err(ops.layer_norm(x, None, None, 1e-6), ref.layer_norm(x, None, None, 1e-6)) < TOL
    assert rel_err(ops.layer_norm(x, w, b), ref.layer_norm(x, w, b)) < TOL


@pytest.mark.parametrize("cols", [4, 200, 256, 260, 512, 1020, 1024, 2048])
def test_layer_norm_widths(dev, rng, cols):
    """Row widths on both sides of the one-wave-per-row kernel's 256 / 512 / 1024 limits,
    with an odd row count (a partly filled last workgroup)."""
    ops, _ = dev
    x = (rng.normal(size=(7, cols)) * 2 - 0.5).astype(np.float32)
    w = rng.normal(size=cols).astype(np.float32)
    b = rng.normal(size=cols).astype(np.float32)
    assert rel_err(ops.layer_norm(x, w, b, 1e-6), ref.layer_norm(x, w, b, 1e-6)) < TOL
    assert rel_err(ops.layer_norm(x, None, None), ref.layer_norm(x, None, None)) < TOL


@pytest.mark.parametrize("n,k,block", [(896, 896, 64), (128, 896, 64), (4864, 896, 64), (896, 4864, 64),
                                       (37, 200, 64), (9, 100, 64), (6144, 1024, 64)])
def test_quantize_q8_bit_exact(dev, n, k, block):
    _, quant = dev
    w = (np.random.default_rng(n + k).normal(size=(n, k)) * 0.02).astype(np.float32)
    w[0, :3] = [1e-40, -3e-39, 0.0]       # fp32 denormals in a block
    w[1 % n, :] = 0.0                      # an all-zero row
    q, s, kp = quant.quantize_q8(w, block)
    rq, rs, rkp = refq.quantize_q8(w, block)
    assert kp == rkp
    assert np.array_equal(q, rq)
    assert s.dtype == np.float16 and np.array_equal(s.view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("n,k", [(896, 896), (4864, 896), (896, 4864), (1024, 2048)])
def test_quantize_q8_per_channel_bit_exact(dev, n, k):
    _, quant = dev
    w = (np.random.default_rng(k).normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, _ = quant.quantize_q8(w, k, np.float32)
    rq, rs, _ = refq.quantize_q8(w, k, np.float32)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_quantize_q8_tiny_scales_are_fp16_subnormals(dev):
    """amax below 127 * 2^-14 gives fp16-subnormal scales; they must round like numpy."""
    _, quant = dev
    w = (np.random.default_rng(5).normal(size=(16, 128)) * 1e-4).astype(np.float32)
    q, s, _ = quant.quantize_q8(w)
    rq, rs, _ = refq.quantize_q8(w)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("n,k", [(896, 896), (33, 100), (4864, 896)])
def test_quantize_q4_bit_exact(dev, n, k):
    _, quant = dev
    w = (np.random.default_rng(n).normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, _ = quant.quantize_q4(w)
    rq, rs, _ = refq.quantize_q4(w)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint16), rs.view(np.uint16))


def test_dequant_rows(dev):
    _, quant = dev
    w = (np.random.default_rng(2).normal(size=(70, 150)) * 0.02).astype(np.float32)
    for kind, fn, blk in (("q8", refq.quantize_q8, 64), ("q4", refq.quantize_q4, 32)):
        q, s, _ = fn(w)
        mine = quant.QTensor(kind, q, s, (70, 150), blk)
        theirs = refq.QTensor(kind, q, s, (70, 150), blk)
        assert np.array_equal(mine.dequant_rows(5, 40), theirs.dequant_rows(5, 40))
        assert np.array_equal(mine.dequant(), theirs.dequant())


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 64, 1000])
@pytest.mark.parametrize("k,n", [(896, 1152), (1024, 6144), (257, 130), (320, 1024), (9, 1), (2048, 80),
                                 (64, 96), (128, 200)])
def test_linear_f32(dev, rng, m, k, n):
    ops, _ = dev
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    assert rel_err(ops.linear(x, w, b), ref.linear(x, w, b)) < TOL
    assert rel_err(ops.linear(x, w), ref.linear(x, w)) < TOL


@pytest.mark.parametrize("m", [1, 3, 4, 7, 300])
@pytest.mark.parametrize("k,n,block,sdt", [(896, 896, 64, np.float16), (896, 4864, 64, np.float16),
                                           (4864, 896, 64, np.float16), (896, 896, 896, np.float32),
                                           (4864, 896, 4864, np.float32), (100, 9, 64, np.float16)])
def test_linear_q8(dev, rng, m, k, n, block, sdt):
    ops, quant = dev
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, _ = refq.quantize_q8(w, block, sdt)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    mine = quant.QTensor("q8", q, s, (n, k), block)
    theirs = refq.QTensor("q8", q, s, (n, k), block)
    assert rel_err(ops.linear(x, mine, b), ref.linear(x, theirs, b)) < TOL


@pytest.mark.parametrize("kind,m,k,n", [("f32", 1100, 1024, 2000), ("f32", 1100, 1030, 2000),
                                        ("q8", 1100, 1024, 1000), ("q8", 3000, 1024, 520)])
def test_linear_large_activation(dev, rng, kind, m, k, n):
    """Activations beyond one XCD's L2 (over 4 MB) take the grouped tile order, whose
    last group is ragged here (18 or 47 M-tiles in groups of 8)."""
    ops, quant = dev
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    if kind == "f32":
        assert rel_err(ops.linear(x, w, b), ref.linear(x, w, b)) < TOL
    else:
        q, s, _ = refq.quantize_q8(w, 64, np.float16)
        mine = quant.QTensor("q8", q, s, (n, k), 64)
        theirs = refq.QTensor("q8", q, s, (n, k), 64)
        assert rel_err(ops.linear(x, mine, b), ref.linear(x, theirs, b)) < TOL


@pytest.mark.parametrize("m", [1, 4, 9, 64, 300])
@pytest.mark.parametrize("k,n", [(896, 300), (896, 4864), (4864, 896), (100, 9), (1024, 1024), (130, 70)])
def test_linear_q4(dev, rng, m, k, n):
    """q4 weights: the GEMV up to 4 rows, the MFMA GEMM (nibbles dequantised on their way
    into LDS) above: branch-free (K % 64 == 0) and guarded (ragged K) stages, the
    8-wave kernel (at most 256 tiles) and the 4-wave one."""
    ops, quant = dev
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, _ = refq.quantize_q4(w)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    assert rel_err(ops.linear(x, quant.QTensor("q4", q, s, (n, k), 32), b),
                   ref.linear(x, refq.QTensor("q4", q, s, (n, k), 32), b)) < TOL


def test_linear_q4_large(dev, rng):
    """1000 activation rows through [2048, 1024] q4 weights: the DiT ff1 shape."""
    ops, quant = dev
    w = (rng.normal(size=(2048, 1024)) * 0.02).astype(np.float32)
    q, s, _ = refq.quantize_q4(w)
    x = rng.normal(size=(1000, 1024)).astype(np.float32)
    assert rel_err(ops.linear(x, quant.QTensor("q4", q, s, (2048, 1024), 32)),
                   ref.linear(x, refq.QTensor("q4", q, s, (2048, 1024), 32))) < TOL


def test_embedding(dev, rng):
    ops, quant = dev
    table = rng.normal(size=(50, 80)).astype(np.float32)
    ids = np.array([[3, 7, 3], [49, 0, 12]])
    assert np.array_equal(ops.embedding(table, ids), ref.embedding(table, ids))
    t16 = table.astype(np.float16)
    assert np.array_equal(ops.embedding(t16, ids), ref.embedding(t16, ids))
    q, s, _ = refq.quantize_q8(table)
    assert np.array_equal(ops.embedding(quant.QTensor("q8", q, s, (50, 80), 64), ids),
                          ref.embedding(refq.QTensor("q8", q, s, (50, 80), 64), ids))
    with pytest.raises(IndexError, match="outside"):
        ops.embedding(table, np.array([50]))


CONV_CASES = [
    (4, 6, 3, 1, 1, 1, 12, (1, 1)),
    (4, 6, 5, 1, 2, 1, 16, (4, 0)),
    (8, 8, 3, 1, 1, 4, 13, (2, 2)),
    (3, 6, 4, 2, 1, 1, 17, (0, 0)),
    (18, 8, 30, 15, 1, 1, 61, (14, 0)),
    (16, 16, 7, 1, 1, 4, 20, (6, 0)),
    (256, 256, 11, 1, 5, 1, 700, (50, 0)),     # HiFT resblock, dilation 5
    (1024, 1024, 31, 1, 1, 16, 130, (30, 0)),  # DiT conv_pos
    (80, 512, 5, 1, 1, 1, 77, (0, 4)),         # HiFT conv_pre (lookahead)
]


@pytest.mark.parametrize("cin,cout,k,stride,dil,groups,T,pad", CONV_CASES)
def test_conv1d(dev, rng, cin, cout, k, stride, dil, groups, T, pad):
    ops, _ = dev
    w = (rng.normal(size=(cout, cin // groups, k)) * 0.1).astype(np.float32)
    b = rng.normal(size=cout).astype(np.float32)
    x = rng.normal(size=(cin, T)).astype(np.float32)
    got = ops.conv1d(x, w, b, stride=stride, dilation=dil, groups=groups, pad=pad)
    want = ref.conv1d(x, w, b, stride=stride, dilation=dil, groups=groups, pad=pad)
    assert got.shape == want.shape and rel_err(got, want) < TOL


def test_conv1d_quantised_weight(dev, rng):
    ops, quant = dev
    w = (rng.normal(size=(6, 4, 3)) * 0.1).astype(np.float32)
    x = rng.normal(size=(4, 15)).astype(np.float32)
    q, s, _ = refq.quantize_q8(w.reshape(6, -1))
    got = ops.conv1d(x, quant.QTensor("q8", q, s, (6, 12), 64, orig_shape=(6, 4, 3)), None, pad=(2, 0))
    want = ref.conv1d(x, refq.QTensor("q8", q, s, (6, 12), 64, orig_shape=(6, 4, 3)), None, pad=(2, 0))
    assert rel_err(got, want) < TOL
    with pytest.raises(ValueError):
        ops.conv1d(x, quant.QTensor("q8", q, s, (6, 12), 64), None)


def test_depthwise(dev, rng):
    ops, _ = dev
    w = rng.normal(size=(12, 1, 7)).astype(np.float32)
    b = rng.normal(size=12).astype(np.float32)
    x = rng.normal(size=(12, 20)).astype(np.float32)
    assert rel_err(ops.depthwise_conv1d(x, w, b, pad=(3, 3)), ref.depthwise_conv1d(x, w, b, pad=(3, 3))) < TOL


@pytest.mark.parametrize("h,hk,n,m,d", [(4, 4, 23, 23, 16), (4, 2, 19, 19, 16), (16, 16, 500, 500, 64),
                                        (14, 2, 1, 513, 64), (2, 1, 37, 37, 64), (3, 3, 70, 130, 32),
                                        (4, 2, 65, 1100, 64)])
@pytest.mark.parametrize("mask", [None, ("causal",), ("chunk", 8, 1), ("chunk", 50, -1), ("chunk", 5, 0)])
def test_sdpa(dev, rng, h, hk, n, m, d, mask):
    ops, _ = dev
    if mask is not None and mask[0] == "causal" and n != m:
        mask = ("causal", m - n)
    q = rng.normal(size=(h, n, d)).astype(np.float32)
    k = rng.normal(size=(hk, m, d)).astype(np.float32)
    v = rng.normal(size=(hk, m, d)).astype(np.float32)
    assert rel_err(ops.sdpa(q, k, v, mask), ref.sdpa(q, k, v, mask)) < TOL


def test_sdpa_errors(dev, rng):
    ops, _ = dev
    q = rng.normal(size=(4, 3, 16)).astype(np.float32)
    k = rng.normal(size=(3, 3, 16)).astype(np.float32)
    with pytest.raises(ValueError):
        ops.sdpa(q, k, k)
    with pytest.raises(ValueError):
        ops.sdpa(q, q, q, ("sliding", 3))


def test_stft_istft(dev, rng):
    ops, _ = dev
    win = ref.hann_window(16)
    assert np.abs(ops.hann_window(16) - win).max() < 1e-7
    sig = rng.normal(size=4001).astype(np.float32)
    got, want = ops.stft(sig, 16, 4, win), ref.stft(sig, 16, 4, win)
    assert got.shape == want.shape
    assert rel_err(np.stack([got.real, got.imag]), np.stack([want.real, want.imag])) < TOL
    spec = (rng.normal(size=(9, 301)) + 1j * rng.normal(size=(9, 301))).astype(np.complex64)
    assert rel_err(ops.istft(spec, 16, 4, win), ref.istft(spec, 16, 4, win)) < TOL
    assert rel_err(ops.istft(spec, 16, 4, win, length=1500), ref.istft(spec, 16, 4, win, length=1500)) < TOL


def test_interpolation(dev, rng):
    ops, _ = dev
    x = rng.normal(size=(5, 37)).astype(np.float32)
    for size, ac in ((100, False), (20, False), (100, True)):
        assert rel_err(ops.interpolate_linear(x, size, ac), ref.interpolate_linear(x, size, ac)) < TOL
    assert np.array_equal(ops.interpolate_nearest(x, 3), ref.interpolate_nearest(x, 3))


@pytest.mark.parametrize("T,k,cin,groups", [(500, 31, 1024, 16), (37, 31, 1024, 16), (70, 5, 256, 4),
                                            (100, 4, 512, 8), (3, 2, 128, 2)])
def test_conv1d_channels_last(dev, rng, T, k, cin, groups):
    """The DiT conv_pos path: grouped causal conv on [batch, time, channel] activations
    against the oracle's (channel, time) conv1d, per batch row, with the Mish + residual epilogue."""
    import ctypes
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, to_device
    B, cout = 2, cin
    x = rng.normal(size=(B, T, cin)).astype(np.float32)
    w = (rng.normal(size=(cout, cin // groups, k)) * 0.02).astype(np.float32)
    b = (rng.normal(size=cout) * 0.02).astype(np.float32)
    res = rng.normal(size=(B, T, cout)).astype(np.float32)
    want = np.stack([ref.mish(ref.conv1d(np.ascontiguousarray(x[i].T), w, b, groups=groups, pad=(k - 1, 0))).T
                     + res[i] for i in range(B)])
    xd = to_device(x)
    wd = to_device(np.ascontiguousarray(w.transpose(0, 2, 1)))
    bd = to_device(b)
    yd = to_device(res)
    epi = _lib.epilogue("mish", residual=yd.ptr, ld_res=cout)
    _lib.call("conv1d_cl", xd.ptr, B, T, cin, cin, wd.ptr, cout, k, groups, k - 1, bd.ptr, yd.ptr, cout,
              ctypes.byref(epi), None)
    assert rel_err(yd.numpy(), want) < TOL
    # the same conv with the weight as bfloat16 planes in fragment order (cv3_conv1d_cl_x3f)
    kk = k * (cin // groups)
    if kk % 64 == 0:
        ne = ctypes.c_int64()
        _lib.call("x3_frag_elems", cout, kk, ctypes.byref(ne))
        fr = DeviceArray((ne.value,), np.uint16)
        _lib.call("split_x3_frag", wd.ptr, cout, kk, kk, fr.ptr, None)
        y3 = to_device(res)
        epi3 = _lib.epilogue("mish", residual=y3.ptr, ld_res=cout)
        _lib.call("conv1d_cl_x3f", xd.ptr, B, T, cin, cin, fr.ptr, cout, k, groups, k - 1, bd.ptr, y3.ptr, cout,
                  ctypes.byref(epi3), None)
        assert rel_err(y3.numpy(), want) < TOL


PACKED_CASES = [
    # cin, cout, k, dil, up, T, pad, epilogue, K slices
    (64, 64, 11, 5, 1, 300, (50, 0), "snake", 1),       # HiFT stage-2 resblock conv1 + Snake
    (64, 64, 11, 1, 1, 301, (10, 0), "residual", 1),    # resblock conv2 + residual
    (128, 64, 7, 1, 3, 150, (6, 0), "none", 1),         # last upsampling conv (nearest x3 fused)
    (512, 256, 16, 1, 8, 40, (15, 0), "none", 1),       # first upsampling conv (nearest x8 fused)
    (256, 256, 3, 3, 1, 70, (6, 0), "leaky", 1),
    (64, 18, 7, 1, 1, 200, (6, 0), "none", 1),          # conv_post, 18 outputs
    (192, 100, 5, 2, 2, 33, (3, 4), "residual", 1),     # ragged tiles, left and right padding
    (256, 256, 11, 1, 1, 944, (10, 0), "snake", 4),     # 1 s-chunk stage-0 conv, split 4 ways
    (512, 256, 16, 1, 8, 14, (15, 0), "none", 8),       # 1 s-chunk first upsampling conv, 8 ways
    (256, 256, 11, 3, 1, 300, (30, 0), "residual", 4),  # split-K with an in-place residual
    (128, 128, 7, 5, 1, 99, (30, 0), "leaky", 2),
]


@pytest.mark.parametrize("cin,cout,k,dil,up,T,pad,epi,ks", PACKED_CASES)
def test_conv1d_packed(dev, rng, cin, cout, k, dil, up, T, pad, epi, ks):
    """The stride-1 fast path with the weight repacked (out, k, in), against the oracle's
    upsample + conv1d + epilogue on (channel, time) data."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, to_device
    x = rng.normal(size=(cin, T)).astype(np.float32)
    w = (rng.normal(size=(cout, cin, k)) * 0.05).astype(np.float32)
    b = (rng.normal(size=cout) * 0.05).astype(np.float32)
    alpha = (np.abs(rng.normal(size=cout)) + 0.5).astype(np.float32)
    xin = ref.interpolate_nearest(x, up) if up > 1 else x
    y = ref.conv1d(xin, w, b, dilation=dil, pad=pad)
    t_out = y.shape[1]
    res = rng.normal(size=(cout, t_out)).astype(np.float32)
    if epi == "snake":
        want = ref.snake(y, alpha)
    elif epi == "leaky":
        want = ref.leaky_relu(y, 0.1)
    elif epi == "residual":
        want = y + res
    else:
        want = y
    xd = to_device(x)
    wd = to_device(np.ascontiguousarray(w.transpose(0, 2, 1)))
    bd = to_device(b)
    ad = to_device(alpha)
    yd = to_device(res) if epi == "residual" else DeviceArray((cout, t_out))
    ws = DeviceArray((ks * cout * t_out,)) if ks > 1 else None
    for _ in range(2):  # the second call sees the first call's partials in the workspace
        if epi == "residual":
            _lib.call("copy_h2d", yd.ptr, res.ctypes.data, res.nbytes, None)
        _lib.call("conv1d_packed", xd.ptr, cin, T, T, wd.ptr, cout, k, bd.ptr, dil, pad[0], pad[1], up, yd.ptr,
                  t_out, 1, _lib.ACT["leaky" if epi == "leaky" else "none"], 0.1 if epi == "leaky" else 0.0,
                  ad.ptr if epi == "snake" else None, 1e-9, yd.ptr if epi == "residual" else None, t_out, 1,
                  ks, ws.ptr if ws else None, ws.size if ws else 0, None)
        assert rel_err(yd.numpy(), want) < TOL


def test_conv1d_packed_rejects_unaligned_channels(dev):
    from cv3amd import _lib
    from cv3amd.device import DeviceArray
    x, w, y = DeviceArray((80, 16)), DeviceArray((8, 5, 80)), DeviceArray((8, 16))
    with pytest.raises(NotImplementedError):
        _lib.call("conv1d_packed", x.ptr, 80, 16, 16, w.ptr, 8, 5, None, 1, 4, 0, 1, y.ptr, 16, 1, 0, 0.0,
                  None, 1e-9, None, 0, 0, 1, None, 0, None)


def test_conv1d_packed_rejects_odd_split(dev):
    from cv3amd import _lib
    from cv3amd.device import DeviceArray
    x, w, y = DeviceArray((64, 16)), DeviceArray((8, 3, 64)), DeviceArray((8, 16))
    ws = DeviceArray((2 * 8 * 16,))
    with pytest.raises(ValueError):   # 3 taps x 2 stages = 6 stages: not 2 even slices
        _lib.call("conv1d_packed", x.ptr, 64, 16, 16, w.ptr, 8, 3, None, 1, 2, 0, 1, y.ptr, 16, 1, 0, 0.0,
                  None, 1e-9, None, 0, 0, 2, ws.ptr, ws.size, None)


CL_CASES = [
    # cin, cout, k, dil, up, T, pad, epilogue, K slices, channels-first output
    (64, 64, 11, 5, 1, 300, (50, 0), "snake", 1, False),
    (64, 64, 11, 1, 1, 301, (10, 0), "residual", 1, False),
    (128, 64, 7, 1, 3, 150, (6, 0), "none", 1, False),
    (512, 256, 16, 1, 8, 40, (15, 0), "none", 2, False),
    (256, 256, 3, 3, 1, 70, (6, 0), "leaky", 3, False),
    (64, 18, 7, 1, 1, 200, (6, 0), "none", 1, True),         # conv_post, written (channel, time)
    (96, 100, 5, 2, 2, 33, (3, 4), "residual", 5, False),    # ragged tiles, both pads, odd split
    (32, 40, 1, 1, 1, 17, (0, 0), "none", 1, False),         # one stage
    # 32, 64 and 128 channels in at the resblocks' spans (split K, a right pad, spans of 64 and 80)
    (128, 128, 11, 5, 1, 257, (50, 0), "snake", 2, False),
    (128, 64, 3, 3, 1, 130, (6, 0), "residual", 1, False),
    (32, 64, 6, 3, 1, 95, (15, 3), "leaky", 1, False),
    (64, 64, 3, 32, 1, 200, (64, 0), "none", 1, False),
    (64, 64, 3, 40, 1, 200, (80, 0), "none", 1, False),
]


@pytest.mark.parametrize("x3", [False, True])
@pytest.mark.parametrize("cin,cout,k,dil,up,T,pad,epi,ks,cf", CL_CASES)
def test_conv1d_cl_packed(dev, rng, cin, cout, k, dil, up, T, pad, epi, ks, cf, x3):
    """Channels-last stride-1 conv through the DMA implicit GEMM (and, ``x3``, its
    bfloat16-plane forms, cv3_conv1d_cl_packed_x3 and, with the planes in fragment order,
    cv3_conv1d_cl_packed_x3f, where a K slice has an even number of 32-channel stages),
    against the oracle's upsample + conv1d + epilogue on (channel, time) data; the two plane
    forms give the same bits."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, to_device
    if x3 and (k * cin // 32 // ks) % 2:
        pytest.skip("the bfloat16-plane conv needs an even number of stages per K slice")
    x = rng.normal(size=(cin, T)).astype(np.float32)
    w = (rng.normal(size=(cout, cin, k)) * 0.05).astype(np.float32)
    b = (rng.normal(size=cout) * 0.05).astype(np.float32)
    alpha = (np.abs(rng.normal(size=cout)) + 0.5).astype(np.float32)
    xin = ref.interpolate_nearest(x, up) if up > 1 else x
    y = ref.conv1d(xin, w, b, dilation=dil, pad=pad)
    t_out = y.shape[1]
    res = rng.normal(size=(cout, t_out)).astype(np.float32)
    want = {"snake": lambda: ref.snake(y, alpha), "leaky": lambda: ref.leaky_relu(y, 0.1),
            "residual": lambda: y + res, "none": lambda: y}[epi]()
    xd = to_device(np.ascontiguousarray(x.T))                       # (T, cin)
    wd = to_device(np.ascontiguousarray(w.transpose(0, 2, 1)))
    bd, ad = to_device(b), to_device(alpha)
    res_cl = np.ascontiguousarray(res.T)                             # (t_out, cout)
    if cf:
        yd, y_ts, y_cs = DeviceArray((cout, t_out)), 1, t_out
    else:
        yd, y_ts, y_cs = (to_device(res_cl) if epi == "residual" else DeviceArray((t_out, cout))), cout, 1
    ws = DeviceArray((ks * cout * t_out,)) if ks > 1 else None
    forms = [(wd.ptr, "conv1d_cl_packed")]
    if x3:
        planes = DeviceArray((3, cout, k * cin), np.uint16)
        _lib.call("split_x3", wd.ptr, cout, k * cin, k * cin, planes.ptr, k * cin, None)
        ne = ctypes.c_int64()
        _lib.call("x3_frag_elems", cout, k * cin, ctypes.byref(ne))
        frag = DeviceArray((ne.value,), np.uint16)
        _lib.call("split_x3_frag", wd.ptr, cout, k * cin, k * cin, frag.ptr, None)
        forms = [(planes.ptr, "conv1d_cl_packed_x3"), (frag.ptr, "conv1d_cl_packed_x3f")]
    outs = []
    for wptr, fn in forms:
        for _ in range(2):  # the second call sees the first call's partials in the workspace
            if epi == "residual":
                _lib.call("copy_h2d", yd.ptr, res_cl.ctypes.data, res_cl.nbytes, None)
            _lib.call(fn, xd.ptr, T, cin, cin, wptr, cout, k, bd.ptr, dil, pad[0], pad[1], up,
                      yd.ptr, y_ts, y_cs, _lib.ACT["leaky" if epi == "leaky" else "none"],
                      0.1 if epi == "leaky" else 0.0, ad.ptr if epi == "snake" else None, 1e-9,
                      yd.ptr if epi == "residual" else None, cout, 1, ks, ws.ptr if ws else None,
                      ws.size if ws else 0, None)
            got = yd.numpy() if cf else yd.numpy().T
            assert rel_err(got, want) < TOL, fn
        outs.append(got)
    if x3:
        assert np.array_equal(outs[0], outs[1])


def test_empty_inputs_match_the_reference(dev, rng):
    """Zero rows, zero-length convolutions and zero queries give the reference's empty shapes."""
    ops, quant = dev
    w = (rng.normal(size=(7, 12)) * 0.1).astype(np.float32)
    x0 = np.zeros((0, 12), np.float32)
    got, want = ops.linear(x0, w), ref.linear(x0, w)
    assert got.shape == want.shape == (0, 7)
    q, s, _ = refq.quantize_q8(w)
    got = quant.qmatmul(x0, quant.QTensor("q8", q, s, (7, 12), 64))
    assert got.shape == (0, 7)
    xc = rng.normal(size=(4, 3)).astype(np.float32)
    wc = rng.normal(size=(5, 4, 7)).astype(np.float32)
    got, want = ops.conv1d(xc, wc), ref.conv1d(xc, wc)     # kernel longer than the input: t_out <= 0
    assert got.shape == want.shape
    assert ops.softmax(np.zeros((0, 5), np.float32)).shape == (0, 5)
    assert ops.layer_norm(np.zeros((0, 8), np.float32)).shape == (0, 8)
    qs = np.zeros((2, 0, 16), np.float32)
    kv = rng.normal(size=(2, 5, 16)).astype(np.float32)
    got, want = ops.sdpa(qs, kv, kv), ref.sdpa(qs, kv, kv)
    assert got.shape == want.shape


def test_dropin_accepts_the_reference_tuning_keywords(dev, rng):
    """Callers pass tile_bytes / threads (qwen2.py:169, the reference's own tests); the result
    does not depend on them."""
    ops, quant = dev
    x = rng.normal(size=(3, 64)).astype(np.float32)
    w = (rng.normal(size=(40, 64)) * 0.1).astype(np.float32)
    q, s, _ = refq.quantize_q8(w)
    qt = quant.QTensor("q8", q, s, (40, 64), 64)
    base = quant.qmatmul(x, qt)
    for tb, th in ((1 << 10, 1), (1 << 22, 4)):
        assert np.array_equal(quant.qmatmul(x, qt, tile_bytes=tb, threads=th), base)
    xc = rng.normal(size=(4, 30)).astype(np.float32)
    wc = rng.normal(size=(6, 4, 3)).astype(np.float32)
    assert np.array_equal(ops.conv1d(xc, wc, tile_bytes=1 << 10), ops.conv1d(xc, wc))
    qa = rng.normal(size=(2, 9, 16)).astype(np.float32)
    assert np.array_equal(ops.sdpa(qa, qa, qa, tile_bytes=1 << 10), ops.sdpa(qa, qa, qa))
