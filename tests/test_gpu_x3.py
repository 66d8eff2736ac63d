"""The float32 linear on the bfloat16 matrix cores (cv3_split_x3 / cv3_linear_x3).

The weight is held as three bfloat16 planes (hi, mid, lo), each the round-to-nearest-even
bfloat16 of what the planes before it leave, and each product runs as the six plane
products of weight >= 2^-16.  No reference function corresponds to the planes; they are
pinned here by what the arithmetic fixes:

* the planes equal an independent NumPy restatement of the rounding (bit-exact), and
  hi + mid + lo reproduces every float32 weight to 2^-24 of its magnitude;
* the linear matches the oracle's float32 ``x @ W.T + b`` (ops.py:121-123) within the
  same 1e-5 as every other linear, and its error against float64 is no larger than the
  float32 matrix-core GEMM's (cv3_linear_f32) on the same inputs;
* each epilogue (activation, gated residual, DiT rotary) gives what the float32 GEMM,
  itself pinned to the oracle with these epilogues, gives.
"""

import ctypes

import numpy as np
import pytest

from conftest import rel_err
import oracle.ops as ref

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def lib(gpu):
    from cv3amd import _lib
    from cv3amd.device import to_device, empty
    return _lib, to_device, empty


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return ((u >> 16) & 0xFFFF).astype(np.uint16)


def bf16_value(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def planes_numpy(w: np.ndarray):
    w = np.asarray(w, np.float32)
    hi = bf16_rne(w)
    r1 = (w - bf16_value(hi)).astype(np.float32)
    mid = bf16_rne(r1)
    r2 = (r1 - bf16_value(mid)).astype(np.float32)
    return hi, mid, bf16_rne(r2)


def split(lib, w):
    _lib, to_device, empty = lib
    n, k = w.shape
    dw = to_device(np.ascontiguousarray(w, np.float32))
    planes = empty((3, n, k), np.uint16)
    _lib.call("split_x3", dw.ptr, n, k, k, planes.ptr, k, None)
    return planes


def linear(lib, planes, x, n, bias=None, epi=None, out=None):
    _lib, to_device, empty = lib
    m, k = x.shape
    dx = to_device(np.ascontiguousarray(x, np.float32))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = out if out is not None else empty((m, n))
    _lib.call("linear_x3", dx.ptr, m, k, k, planes.ptr, k, n, db.ptr if db is not None else None, y.ptr, n,
              ctypes.byref(epi) if epi is not None else None, None)
    return y.numpy()


def linear_f32(lib, w, x, bias=None, epi=None, out=None):
    _lib, to_device, empty = lib
    m, k = x.shape
    n = w.shape[0]
    dx = to_device(np.ascontiguousarray(x, np.float32))
    dw = to_device(np.ascontiguousarray(w, np.float32))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = out if out is not None else empty((m, n))
    _lib.call("linear_f32", dx.ptr, m, k, k, dw.ptr, k, n, db.ptr if db is not None else None, y.ptr, n,
              ctypes.byref(epi) if epi is not None else None, None)
    return y.numpy()


def test_planes_are_the_rounding_chain(lib):
    rng = np.random.default_rng(1)
    w = (rng.normal(size=(37, 1024)) * np.exp(rng.uniform(-30, 30, size=(37, 1))).astype(np.float32)).astype(np.float32)
    w[0, :8] = [0.0, -0.0, 1.0, -1.0, 3.0e38, -1.17549435e-38, 1.0 + 2.0 ** -23, 65504.0]
    w[1, :] = np.float32(1.0) + np.arange(1024, dtype=np.float32) * np.float32(2.0 ** -23)  # every low bit
    got = split(lib, w).numpy()
    hi, mid, lo = planes_numpy(w)
    np.testing.assert_array_equal(got[0], hi)
    np.testing.assert_array_equal(got[1], mid)
    np.testing.assert_array_equal(got[2], lo)
    total = bf16_value(got[0]).astype(np.float64) + bf16_value(got[1]) + bf16_value(got[2])
    assert np.all(np.abs(total - w.astype(np.float64)) <= 2.0 ** -24 * np.abs(w.astype(np.float64)))


SHAPES = [(1, 64, 64), (7, 128, 64), (65, 192, 130), (300, 1024, 1024), (1000, 1024, 3072),
          (1000, 2048, 1024), (3000, 1024, 1024),
          # wide outputs: a ragged last column tile, one row, n a multiple of 128
          (65, 128, 2100), (1, 64, 4096), (130, 256, 2048)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_linear_x3_matches_oracle(lib, m, k, n):
    rng = np.random.default_rng(m * 7 + k + n)
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.normal(size=n).astype(np.float32)
    print(f"[x3] m={m} k={k} n={n}", flush=True)
    got = linear(lib, split(lib, w), x, n, b)
    want = ref.linear(x, w, b)
    assert rel_err(got, want) < TOL
    # error against float64: no larger than the float32 matrix cores' own
    exact = x.astype(np.float64) @ w.astype(np.float64).T + b
    e_x3 = np.abs(got - exact).max()
    e_f32 = np.abs(linear_f32(lib, w, x, b) - exact).max()
    print(f"[x3]   max err vs float64: split-bf16 {e_x3:.3e}, float32 MFMA {e_f32:.3e}", flush=True)
    assert e_x3 <= e_f32 * 1.25 + 1e-30


def test_linear_x3_wide_range(lib):
    """Activations and weights spanning 2^-30 .. 2^30: the planes keep float32's range."""
    rng = np.random.default_rng(5)
    m, k, n = 128, 256, 128
    x = (rng.normal(size=(m, k)) * np.exp2(rng.integers(-30, 30, size=(m, 1)))).astype(np.float32)
    w = (rng.normal(size=(n, k)) * np.exp2(rng.integers(-30, 30, size=(n, 1)))).astype(np.float32)
    got = linear(lib, split(lib, w), x, n)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    assert np.all(np.abs(got - exact) <= 1e-6 * scale)


def test_linear_x3_epilogues(lib):
    _lib, to_device, empty = lib
    rng = np.random.default_rng(3)
    m, k, n = 1000, 1024, 3072
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) / 32).astype(np.float32)
    b = rng.normal(size=n).astype(np.float32)
    planes = split(lib, w)
    # activation
    for act in ("gelu_tanh", "silu", "mish"):
        e = _lib.epilogue(act)
        assert rel_err(linear(lib, planes, x, n, b, e), linear_f32(lib, w, x, b, e)) < TOL
    # gated residual, one gate row per 500 output rows (the DiT's per-batch AdaLN gate)
    res = rng.normal(size=(m, n)).astype(np.float32)
    gate = rng.normal(size=(2, n)).astype(np.float32)
    dres, dgate = to_device(res), to_device(gate)
    e = _lib.epilogue(residual=dres.ptr, ld_res=n, gate=dgate.ptr, gate_stride=n, rows_per_gate=500)
    assert rel_err(linear(lib, planes, x, n, b, e), linear_f32(lib, w, x, b, e)) < TOL
    # DiT partial rotary on q and k (64 channels per head, period 1024, limit 2048), T = 500
    from cv3amd.dit import dit_rope_tables
    c, s = dit_rope_tables(500, 64)
    dc, ds = to_device(c), to_device(s)
    e = _lib.epilogue(rope=(dc.ptr, ds.ptr, 500, 1024, 64, 2048))
    assert rel_err(linear(lib, planes, x, n, b, e), linear_f32(lib, w, x, b, e)) < TOL


def test_linear_x3_in_place_residual(lib):
    """y = y + gate * (x . W^T): C is the residual itself, as in the DiT's out / ff2 linears."""
    _lib, to_device, empty = lib
    rng = np.random.default_rng(4)
    m, k, n = 1000, 2048, 1024
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) / 45).astype(np.float32)
    h0 = rng.normal(size=(m, n)).astype(np.float32)
    gate = rng.normal(size=(1, n)).astype(np.float32)
    dgate = to_device(gate)
    outs = []
    for fn in (lambda e, y: linear(lib, split(lib, w), x, n, None, e, out=y),
               lambda e, y: linear_f32(lib, w, x, None, e, out=y)):
        y = to_device(h0)
        e = _lib.epilogue(residual=y.ptr, ld_res=n, gate=dgate.ptr, gate_stride=0, rows_per_gate=1)
        outs.append(fn(e, y))
    assert rel_err(outs[0], outs[1]) < TOL
    assert rel_err(outs[0], h0 + gate * (x @ w.T)) < TOL


def test_linear_x3_rejects_ragged_k(lib):
    _lib, to_device, empty = lib
    w = np.ones((64, 96), np.float32)
    planes = split(lib, w)
    with pytest.raises(NotImplementedError):
        linear(lib, planes, np.ones((64, 96), np.float32), 64)


# ---- q8 weights: the activation's planes times the codes, exact in bfloat16 ----

import oracle.quant as refq


def linear_q8_x3(lib, q, s, kp, block, x, n, bias=None, epi=None):
    _lib, to_device, empty = lib
    m, k = x.shape
    dx = to_device(np.ascontiguousarray(x, np.float32))
    dq = to_device(np.ascontiguousarray(q))
    ds = to_device(np.ascontiguousarray(s))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = empty((m, n))
    _lib.call("linear_q8_x3", dx.ptr, m, k, k, dq.ptr, ds.ptr, _lib.F16 if s.dtype == np.float16 else _lib.F32,
              kp, block, n, db.ptr if db is not None else None, y.ptr, n,
              ctypes.byref(epi) if epi is not None else None, None)
    return y.numpy()


def linear_q8_f32(lib, q, s, kp, block, x, n, bias=None):
    """The same q8 linear on the float32 matrix cores (codes dequantised into LDS)."""
    _lib, to_device, empty = lib
    m, k = x.shape
    dx, dq, ds = to_device(np.ascontiguousarray(x, np.float32)), to_device(q), to_device(s)
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = empty((m, n))
    _lib.call("linear_q", _lib.KIND_Q8, dx.ptr, m, k, k, dq.ptr, ds.ptr,
              _lib.F16 if s.dtype == np.float16 else _lib.F32, kp, block, n,
              db.ptr if db is not None else None, y.ptr, n, None, None)
    return y.numpy()


Q8_CASES = [(1000, 1024, 3072, 64, np.float16), (1000, 1024, 1024, 1024, np.float32),
            (3000, 2048, 1024, 64, np.float16), (3000, 2048, 1024, 2048, np.float32),
            (65, 128, 130, 128, np.float32), (7, 64, 64, 64, np.float16)]


@pytest.mark.parametrize("m,k,n,block,sdt", Q8_CASES)
def test_linear_q8_x3_matches_oracle(lib, m, k, n, block, sdt):
    """Block-64 float16 scales (the converter's balanced profile) and per-output-channel float32
    scales (block = K), at the 10 s and 30 s DiT shapes."""
    rng = np.random.default_rng(m + k + n + block)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, kp = refq.quantize_q8(w, block, sdt)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    print(f"[x3q] m={m} k={k} n={n} block={block} {np.dtype(sdt).name}", flush=True)
    got = linear_q8_x3(lib, q, s, kp, block, x, n, b)
    want = refq.qmatmul(x, refq.QTensor("q8", q, s, (n, k), block), b)
    assert rel_err(got, want) < TOL
    # against float64 over the dequantised weight: no larger than the float32 matrix cores' error
    wd = refq.QTensor("q8", q, s, (n, k), block).dequant().astype(np.float64)
    exact = x.astype(np.float64) @ wd.T + b
    e_x3 = np.abs(got - exact).max()
    e_f32 = np.abs(linear_q8_f32(lib, q, s, kp, block, x, n, b) - exact).max()
    print(f"[x3q]   max err vs float64: split-bf16 {e_x3:.3e}, float32 MFMA {e_f32:.3e}", flush=True)
    assert e_x3 <= e_f32 * 1.25 + 1e-30


def test_linear_q8_x3_epilogue(lib):
    """The gated in-place residual of the DiT's out / ff2 linears, against the float32 path."""
    _lib, to_device, empty = lib
    rng = np.random.default_rng(9)
    m, k, n = 1000, 2048, 1024
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, kp = refq.quantize_q8(w, 64, np.float16)
    x = rng.normal(size=(m, k)).astype(np.float32)
    res = rng.normal(size=(m, n)).astype(np.float32)
    gate = rng.normal(size=(2, n)).astype(np.float32)
    dres, dgate = to_device(res), to_device(gate)
    e = _lib.epilogue("gelu_tanh", residual=dres.ptr, ld_res=n, gate=dgate.ptr, gate_stride=n, rows_per_gate=500)
    got = linear_q8_x3(lib, q, s, kp, 64, x, n, None, e)
    want = ref.gelu_tanh(refq.qmatmul(x, refq.QTensor("q8", q, s, (n, k), 64)))
    want = res + np.repeat(gate, 500, axis=0) * want
    assert rel_err(got, want) < TOL


def test_linear_q8_x3_rejects_small_blocks(lib):
    _lib, to_device, empty = lib
    w = np.ones((64, 128), np.float32)
    q, s, kp = refq.quantize_q8(w, 32, np.float16)
    with pytest.raises(NotImplementedError):
        linear_q8_x3(lib, q, s, kp, 32, np.ones((64, 128), np.float32), 64)


# ---- attention with head dim 64 on the bfloat16 matrix cores ----

def attention(lib, name, q, k, v, mask=None):
    """(H, N, 64) queries over (Hk, M, 64) keys/values through cv3_attention[_x3]."""
    _lib, to_device, empty = lib
    from cv3amd.ops import _mask_args
    mk, ma, mb = _mask_args(mask)
    h, n, d = q.shape
    hk, m, _ = k.shape
    dq, dk, dv = to_device(q), to_device(k), to_device(v)
    out = empty((h, n, d))
    S = ctypes.c_int64 * 3
    _lib.call(name, dq.ptr, dk.ptr, dv.ptr, out.ptr, 1, h, hk, n, m, d, S(0, n * d, d), S(0, m * d, d),
              S(0, m * d, d), S(0, n * d, d), float(np.float32(1.0 / np.sqrt(d))), mk, ma, mb, None)
    return out.numpy()


def sdpa64(q, k, v, mask=None):
    """float64 attention, the same masks (oracle's mask semantics, in float64)."""
    h, n, d = q.shape
    hk, m, _ = k.shape
    rep = h // hk
    kk = np.repeat(k.astype(np.float64), rep, axis=0)
    vv = np.repeat(v.astype(np.float64), rep, axis=0)
    s = (q.astype(np.float64) * np.float64(np.float32(1.0 / np.sqrt(d)))) @ kk.transpose(0, 2, 1)
    add = ref.additive_mask(0, n, m, mask)
    if add is not None:
        s = s + add.astype(np.float64)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(axis=-1, keepdims=True)) @ vv


ATT_CASES = [(16, 16, 500, 500, None), (16, 16, 1500, 1500, None), (14, 2, 200, 200, ("causal", 0)),
             (8, 8, 130, 390, ("causal", 260)), (4, 4, 300, 300, ("chunk", 25, 1)), (2, 1, 1, 77, None),
             (3, 3, 65, 64, None)]


@pytest.mark.parametrize("h,hk,n,m,mask", ATT_CASES)
def test_attention_x3_matches_oracle(lib, h, hk, n, m, mask):
    rng = np.random.default_rng(h * 131 + n + m)
    q = rng.normal(size=(h, n, 64)).astype(np.float32)
    k = rng.normal(size=(hk, m, 64)).astype(np.float32)
    v = rng.normal(size=(hk, m, 64)).astype(np.float32)
    print(f"[att] h={h} hk={hk} n={n} m={m} mask={mask}", flush=True)
    got = attention(lib, "attention_x3", q, k, v, mask)
    assert rel_err(got, ref.sdpa(q, k, v, mask)) < TOL
    exact = sdpa64(q, k, v, mask)
    e_x3 = np.abs(got - exact).max()
    e_f32 = np.abs(attention(lib, "attention", q, k, v, mask) - exact).max()
    print(f"[att]   max err vs float64: split-bf16 {e_x3:.3e}, float32 MFMA {e_f32:.3e}", flush=True)
    assert e_x3 <= e_f32 * 1.25 + 1e-30


# ---- the weight planes in fragment order (cv3_split_x3_frag / cv3_linear_x3_frag) ----

def split_frag(lib, w):
    _lib, to_device, empty = lib
    n, k = w.shape
    dw = to_device(np.ascontiguousarray(w, np.float32))
    ne = ctypes.c_int64()
    _lib.call("x3_frag_elems", n, k, ctypes.byref(ne))
    frag = empty((ne.value,), np.uint16)
    _lib.call("split_x3_frag", dw.ptr, n, k, k, frag.ptr, None)
    return frag


def linear_frag(lib, frag, x, n, bias=None, epi=None, out=None):
    _lib, to_device, empty = lib
    m, k = x.shape
    dx = to_device(np.ascontiguousarray(x, np.float32))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = out if out is not None else empty((m, n))
    _lib.call("linear_x3_frag", dx.ptr, m, k, k, frag.ptr, n, db.ptr if db is not None else None, y.ptr, n,
              ctypes.byref(epi) if epi is not None else None, None)
    return y.numpy()


@pytest.mark.parametrize("n,k", [(130, 128), (3072, 1024), (32, 64), (1, 64)])
def test_frag_planes_are_the_planes_in_fragment_order(lib, n, k):
    """frag[p][nb][t][l] = plane p of w[32 nb + l % 32][16 t + 8 (l / 32) .. + 7], rows past n zero:
    the NumPy rounding chain's planes, reordered."""
    rng = np.random.default_rng(n + k)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    got = split_frag(lib, w).numpy()
    nb = -(-n // 32)
    planes = np.zeros((3, nb * 32, k), np.uint16)
    planes[:, :n] = np.stack(planes_numpy(w))
    # [p][nb][32 rows][T][2 halves][8] -> [p][nb][T][2 halves][32 rows][8] = [p][nb][T][lane][8]
    want = planes.reshape(3, nb, 32, k // 16, 2, 8).transpose(0, 1, 3, 4, 2, 5).reshape(-1)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_linear_x3_frag_is_linear_x3(lib, m, k, n):
    """The same MFMA operands in the same order: bit-identical to the LDS-staged kernel, at the DiT's
    shapes and ragged ones (rows and columns past a tile)."""
    if k % 64:
        pytest.skip("the split GEMMs take K % 64 == 0")
    rng = np.random.default_rng(m + 3 * k + n)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    got = linear_frag(lib, split_frag(lib, w), x, n, b)
    np.testing.assert_array_equal(got, linear(lib, split(lib, w), x, n, b))
    assert rel_err(got, ref.linear(x, w, b)) < TOL


def test_linear_x3_frag_epilogues(lib):
    """GELU, the DiT's partial rotary and the gated in-place residual, bit-identical to cv3_linear_x3."""
    _lib, to_device, empty = lib
    rng = np.random.default_rng(31)
    m, k, n = 1000, 1024, 3072
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    fr, pl = split_frag(lib, w), split(lib, w)
    np.testing.assert_array_equal(linear_frag(lib, fr, x, n, b, _lib.epilogue("gelu_tanh")),
                                  linear(lib, pl, x, n, b, _lib.epilogue("gelu_tanh")))
    T = 500
    ang = np.arange(T, dtype=np.float64)[:, None] * (1.0 / 10000 ** (np.arange(0, 64, 2) / 64))[None, :]
    ang = np.repeat(ang, 2, axis=1).astype(np.float32)
    cos, sin = to_device(np.cos(ang)), to_device(np.sin(ang))
    rope = _lib.epilogue(rope=(cos.ptr, sin.ptr, T, 1024, 64, 2048))
    np.testing.assert_array_equal(linear_frag(lib, fr, x, n, b, rope), linear(lib, pl, x, n, b, rope))
    h0 = rng.normal(size=(m, n)).astype(np.float32)
    gate = to_device(rng.normal(size=n).astype(np.float32))
    outs = []
    for fn, wts in ((linear_frag, fr), (linear, pl)):
        y = to_device(h0)
        e = _lib.epilogue(residual=y.ptr, ld_res=n, gate=gate.ptr, gate_stride=0, rows_per_gate=1)
        outs.append(fn(lib, wts, x, n, b, e, out=y))
    np.testing.assert_array_equal(outs[0], outs[1])


def linear_q8_frag(lib, q, s, kp, block, x, n, bias=None, epi=None):
    _lib, to_device, empty = lib
    m, k = x.shape
    dx = to_device(np.ascontiguousarray(x, np.float32))
    dq = to_device(np.ascontiguousarray(q))
    qf = empty((-(-n // 32) * 32 * k,), np.int8)
    _lib.call("pack_q8_frag", dq.ptr, n, k, kp, qf.ptr, None)
    ds = to_device(np.ascontiguousarray(s))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = empty((m, n))
    _lib.call("linear_q8_x3_frag", dx.ptr, m, k, k, qf.ptr, ds.ptr, _lib.F16 if s.dtype == np.float16 else _lib.F32,
              kp, block, n, db.ptr if db is not None else None, y.ptr, n,
              ctypes.byref(epi) if epi is not None else None, None)
    return y.numpy(), qf.numpy()


@pytest.mark.parametrize("m,k,n,block,sdt", Q8_CASES)
def test_linear_q8_x3_frag_is_linear_q8_x3(lib, m, k, n, block, sdt):
    """Codes in fragment order (rows past n zero) and the q8 product from them: bit-identical to the
    LDS-staged kernel, block-64 float16 and per-channel float32 scales, ragged shapes."""
    rng = np.random.default_rng(3 * m + k + n + block)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, kp = refq.quantize_q8(w, block, sdt)
    x = rng.normal(size=(m, k)).astype(np.float32)
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    got, qf = linear_q8_frag(lib, q, s, kp, block, x, n, b)
    nb = -(-n // 32)
    qp = np.zeros((nb * 32, k), np.int8)
    qp[:n] = q[:, :k]
    want_qf = qp.reshape(nb, 32, k // 16, 2, 8).transpose(0, 2, 3, 1, 4).reshape(-1)
    np.testing.assert_array_equal(qf, want_qf)
    np.testing.assert_array_equal(got, linear_q8_x3(lib, q, s, kp, block, x, n, b))


# ---- per-channel q8 linears on the int8 matrix cores (four int8 digit planes of the activation) ----

def linear_q8_digits(lib, q, s, x, n, bias=None, epi=None, rexp_in=None):
    """cv3_linear_q8_digits; returns the output, the packed codes and the row exponents (``rexp_in``:
    exponents handed in with row_exp_given = 1 instead of computed)."""
    _lib, to_device, empty = lib
    m, k = x.shape
    dx = to_device(np.ascontiguousarray(x, np.float32))
    dq = to_device(np.ascontiguousarray(q))
    npad = -(-n // 32) * 32
    qf = empty((npad * (k + 4),), np.int8)
    _lib.call("pack_q8_frag32", dq.ptr, n, k, q.shape[1], qf.ptr, None)
    ds = to_device(np.ascontiguousarray(s))
    db = to_device(np.asarray(bias, np.float32)) if bias is not None else None
    y = empty((m, n))
    rexp = empty((max(m, 1),), np.int32) if rexp_in is None else to_device(np.asarray(rexp_in, np.int32))
    _lib.call("linear_q8_digits", dx.ptr, m, k, k, qf.ptr, ds.ptr, _lib.F16 if s.dtype == np.float16 else _lib.F32,
              n, db.ptr if db is not None else None, y.ptr, n, ctypes.byref(epi) if epi is not None else None,
              rexp.ptr, int(rexp_in is not None), None)
    return y.numpy(), qf.numpy(), rexp.numpy()[:m]


def digits_numpy(x, q, s):
    """The digit-plane product restated: each row rounded to X = rint(x 2^(30 - E)) (E: frexp of the
    row's largest |x|, at least -96), the int8 codes times X exactly, times 2^(E - 30) and the scale."""
    mx = np.abs(x).max(axis=1)
    e = np.where(mx > 0, np.frexp(mx)[1], 0).astype(np.int64)
    e = np.maximum(e, -96)
    X = np.rint(x.astype(np.float64) * np.exp2(30 - e)[:, None]).astype(np.int64)
    t = X @ q.astype(np.int64).T                       # exact integers
    return t.astype(np.float64) * np.exp2(e - 30)[:, None] * s.astype(np.float64).reshape(1, -1), e


DIGIT_CASES = [(3000, 1024, 3072, np.float32), (3000, 2048, 1024, np.float32), (1000, 320, 1024, np.float32),
               (77, 128, 80, np.float32), (65, 64, 130, np.float16), (1, 2048, 32, np.float32)]


@pytest.mark.parametrize("m,k,n,sdt", DIGIT_CASES)
def test_linear_q8_digits_matches_oracle(lib, m, k, n, sdt):
    """Per-channel scales at the 30 s DiT shapes, proj_in's K = 320, ragged m and n: the codes in
    fragment order followed by each row's code sum; the row exponents; the output against the oracle
    within 1e-5 and against float64 no worse than the bfloat16-plane kernel on the same inputs; every
    output within 1e-6 of a float64 restatement of the digit-plane arithmetic (its only rounding is
    the final float32 one)."""
    rng = np.random.default_rng(m + 3 * k + n)
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, kp = refq.quantize_q8(w, k, sdt)
    x = rng.normal(size=(m, k)).astype(np.float32)
    x[0, :] = 0.0                                    # a zero row
    if m > 2:
        x[1] *= np.float32(1e-30)                    # a tiny row (exponent clamped at -96)
        x[2, 0] = np.float32(3e4)                    # a wide row: one large element
    b = (rng.normal(size=n) * 0.02).astype(np.float32)
    print(f"[q8d] m={m} k={k} n={n} {np.dtype(sdt).name}", flush=True)
    got, qf, rexp = linear_q8_digits(lib, q, s, x, n, b)
    npad = -(-n // 32) * 32
    qp = np.zeros((npad, k), np.int8)
    qp[:n] = q[:, :k]
    want_qf = qp.reshape(npad // 32, 32, k // 32, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    np.testing.assert_array_equal(qf[:npad * k], want_qf)
    np.testing.assert_array_equal(qf[npad * k:].view(np.int32), qp.astype(np.int32).sum(axis=1))
    want_dig, e = digits_numpy(x, q[:, :k], s[:, 0])
    np.testing.assert_array_equal(rexp, e)
    want_dig = want_dig + b.astype(np.float64)
    assert np.abs(got - want_dig).max() <= 1e-6 * np.abs(want_dig).max() + 1e-30
    want = refq.qmatmul(x, refq.QTensor("q8", q, s, (n, k), k), b)
    assert rel_err(got, want) < TOL
    wd = refq.QTensor("q8", q, s, (n, k), k).dequant().astype(np.float64)
    exact = x.astype(np.float64) @ wd.T + b
    e_dig = np.abs(got - exact).max()
    e_x3 = np.abs(linear_q8_x3(lib, q, s, kp, k, x, n, b) - exact).max()
    print(f"[q8d]   max err vs float64: digit planes {e_dig:.3e}, bfloat16 planes {e_x3:.3e}", flush=True)
    assert e_dig <= e_x3 * 1.25 + 1e-30


def test_linear_q8_digits_epilogues(lib):
    """The DiT's epilogues on the digit-plane kernel: GELU, the gated in-place residual and the
    rotary of the QKV projection, against the bfloat16-plane kernel with the same epilogue."""
    _lib, to_device, empty = lib
    rng = np.random.default_rng(11)
    m, k, n = 1000, 1024, 1024
    w = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
    q, s, kp = refq.quantize_q8(w, k, np.float32)
    x = rng.normal(size=(m, k)).astype(np.float32)
    res = rng.normal(size=(m, n)).astype(np.float32)
    gate = rng.normal(size=(2, n)).astype(np.float32)
    dres, dgate = to_device(res), to_device(gate)
    e = _lib.epilogue("gelu_tanh", residual=dres.ptr, ld_res=n, gate=dgate.ptr, gate_stride=n, rows_per_gate=500)
    got, _, _ = linear_q8_digits(lib, q, s, x, n, None, e)
    want = linear_q8_x3(lib, q, s, kp, k, x, n, None, e)
    assert rel_err(got, want) < TOL
    cs = rng.normal(size=(500, 64)).astype(np.float32)
    sn = rng.normal(size=(500, 64)).astype(np.float32)
    dcs, dsn = to_device(cs), to_device(sn)
    er = _lib.epilogue("none")
    er.rope_cos, er.rope_sin = dcs.ptr, dsn.ptr
    er.rope_rows, er.rope_width, er.rope_period, er.rope_limit = 500, 64, 64, 128
    got, _, _ = linear_q8_digits(lib, q, s, x, n, None, er)
    want = linear_q8_x3(lib, q, s, kp, k, x, n, None, er)
    assert rel_err(got, want) < TOL


def test_linear_q8_digits_rejects_long_or_ragged_k(lib):
    """K above 2048 could overflow a plane's int32 sum: the product is refused; codes whose K is not
    a multiple of 64 are refused at packing."""
    q, s, _ = refq.quantize_q8(np.ones((32, 4096), np.float32), 4096, np.float32)
    with pytest.raises(NotImplementedError):
        linear_q8_digits(lib, q, s, np.ones((4, 4096), np.float32), 32)
    q, s, _ = refq.quantize_q8(np.ones((32, 96), np.float32), 96, np.float32)
    with pytest.raises(ValueError):
        linear_q8_digits(lib, q, s, np.ones((4, 96), np.float32), 32)


@pytest.mark.parametrize("modulate", [True, False])
def test_layer_norm_rexp_feeds_digits(lib, modulate):
    """cv3_layer_norm_rexp at the DiT's 30 s shape: the same output as cv3_layer_norm, bit for bit;
    each row's exponent that of the row's largest |y| (an all-zero row 0); and the digit-plane linear
    given those exponents equal, bit for bit, to the one that computes them itself."""
    _lib, to_device, empty = lib
    rng = np.random.default_rng(5 + modulate)
    m, d, n = 3000, 1024, 1024
    h = rng.normal(size=(m, d)).astype(np.float32)
    h[7] = 2.5                                       # a constant row: LN gives 0 (then the shift)
    h[8] *= np.float32(1e-3)
    sh = (rng.normal(size=d) * 0.1).astype(np.float32)
    sc = (rng.normal(size=d) * 0.1).astype(np.float32)
    dh, dsh, dsc = to_device(h), to_device(sh), to_device(sc)
    shp, scp = (dsh.ptr, dsc.ptr) if modulate else (None, None)
    y0, y1 = empty((m, d)), empty((m, d))
    rexp = empty((m,), np.int32)
    print(f"[lnrexp] m={m} d={d} modulate={modulate}", flush=True)
    _lib.call("layer_norm", dh.ptr, y0.ptr, m, d, 1e-6, None, None, shp, scp, 0, 0, None)
    _lib.call("layer_norm_rexp", dh.ptr, y1.ptr, m, d, 1e-6, None, None, shp, scp, 0, 0, rexp.ptr, None)
    y = y1.numpy()
    np.testing.assert_array_equal(y, y0.numpy())
    mx = np.abs(y).max(axis=1)
    want = np.maximum(np.where(mx > 0, np.frexp(mx)[1], 0), -96).astype(np.int32)
    if not modulate:
        assert want[7] == 0
    got_e = rexp.numpy()
    np.testing.assert_array_equal(got_e, want)
    w = (rng.normal(size=(n, d)) * 0.02).astype(np.float32)
    q, s, _ = refq.quantize_q8(w, d, np.float32)
    a, _, e_self = linear_q8_digits(lib, q, s, y, n)
    b, _, _ = linear_q8_digits(lib, q, s, y, n, rexp_in=got_e)
    np.testing.assert_array_equal(e_self, got_e)
    np.testing.assert_array_equal(a, b)


def test_layer_norm_rexp_refuses_wide_rows(lib):
    """Row exponents come from the one-wave-per-row norm: rows wider than 1024 are refused."""
    _lib, to_device, empty = lib
    x = to_device(np.ones((4, 2048), np.float32))
    y, e = empty((4, 2048)), empty((4,), np.int32)
    with pytest.raises(NotImplementedError):
        _lib.call("layer_norm_rexp", x.ptr, y.ptr, 4, 2048, 1e-6, None, None, None, None, 0, 0, e.ptr, None)


def test_dit_digits_switch(lib, monkeypatch):
    """The DiT with its per-channel q8 QKV and ff1 linears on the digit planes (row exponents from
    the layer norm) against the same DiT on the bfloat16 planes: two blocks, 256 frames, two Euler
    steps, outputs within 1e-5."""
    import cv3amd.dit as dit
    import cv3amd.quant as quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    rng = np.random.default_rng(21)
    T = 256
    t2, meta = synth.dit_tensors(depth=2), synth.dit_meta(depth=2)
    qt = synth.quantize_store(t2, "per_channel", quant.quantize_q8)
    mu, cond, x0 = (rng.standard_normal((1, 80, T), dtype=np.float32) for _ in range(3))
    spks = rng.standard_normal((1, 80), dtype=np.float32)
    outs = []
    for digits in (False, True):
        monkeypatch.setattr(dit, "DIGITS", digits)
        d = dit.DeviceDiT(WeightStore(qt, meta, quant.QTensor), steps=2)
        assert d.qkv[0].q8_digits == digits and d.ff1[1].q8_digits == digits
        assert not d.out[0].q8_digits and not d.ff2[0].q8_digits
        d.prepare(mu, spks, cond)
        print(f"[dit-digits] digits={digits} T={T}", flush=True)
        outs.append(d.solve(x0).numpy().copy())
    assert rel_err(outs[1], outs[0]) < 1e-5
