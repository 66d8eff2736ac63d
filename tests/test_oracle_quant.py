"""Pin the oracle's quantisation and quantised matmul.

quantize_q8's codes are fixed by a closed form; the invariants below each fail
on a plausible slip (dividing by 128, reciprocal-multiply rounding, rounding
half away from zero, forgetting the zero-scale guard, leaking the K padding,
storing the scale unrounded).
"""

import numpy as np
import pytest

from oracle.quant import Q4_BLOCK, Q8_BLOCK, QTensor, qmatmul, quantize_q4, quantize_q8


def test_q8_closed_form_invariants():
    rng = np.random.default_rng(0)
    w = (rng.normal(size=(37, 200)) * 0.02).astype(np.float32)
    q, s, kp = quantize_q8(w)
    assert kp == 256 and q.shape == (37, 256) and s.shape == (37, 4) and s.dtype == np.float16
    assert np.abs(q).max() <= 127
    blk = np.pad(w, ((0, 0), (0, 56))).reshape(37, 4, 64)
    amax = np.abs(blk).max(-1)
    # the block's extreme maps to +-127 exactly
    qb = q.reshape(37, 4, 64).astype(np.int32)
    assert (np.abs(qb).max(-1)[amax > 0] == 127).all()
    # codes are round-half-even of the true fp32 quotient by the fp32 scale
    sc32 = (amax / np.float32(127)).astype(np.float32)
    exact = np.rint(blk / sc32[..., None])
    assert np.array_equal(qb, np.clip(exact, -127, 127))
    # stored scale = RNE fp16 of the fp32 scale
    assert np.array_equal(s, sc32.astype(np.float16))
    # padding quantises to zero
    assert (q[:, 200:] == 0).all()


def test_q8_half_even_and_zero_rows():
    # block [127, 0.5, 1.5, 2.5, -0.5, ...]: scale exactly 1, codes of x.5 go to even
    w = np.zeros((2, 64), dtype=np.float32)
    w[0, :5] = [127.0, 0.5, 1.5, 2.5, -0.5]
    q, s, _ = quantize_q8(w)
    assert list(q[0, :5]) == [127, 0, 2, 2, 0]
    assert float(s[0, 0]) == 1.0
    assert (q[1] == 0).all() and float(s[1, 0]) == 1.0   # zero block -> scale 1, codes 0


def test_q8_per_channel_layout():
    rng = np.random.default_rng(3)
    w = (rng.normal(size=(8, 96)) * 0.02).astype(np.float32)
    q, s, kp = quantize_q8(w, block=96, scale_dtype=np.float32)
    assert kp == 96 and s.shape == (8, 1) and s.dtype == np.float32
    assert np.array_equal(s[:, 0], (np.abs(w).max(1) / np.float32(127)).astype(np.float32))


def test_q4_closed_form():
    w = np.zeros((1, 32), dtype=np.float32)
    w[0, :4] = [-8.0, 4.0, 1.0, 0.0]
    q, s, kp = quantize_q4(w)
    assert kp == 32 and float(s[0, 0]) == 1.0     # scale = extreme / -8 = 1
    codes = np.concatenate([q[0] & 15, q[0] >> 4]).astype(int)
    assert list(codes[:4]) == [0, 12, 9, 8]        # rint(w / 1 + 8)
    assert (codes[4:] == 8).all()


@pytest.mark.parametrize("kind,tol", [("q8", 0.02), ("q4", 0.15)])
@pytest.mark.parametrize("shape", [(128, 257), (896, 4864), (64, 64)])
def test_quantised_matmul_error(kind, tol, shape):
    rng = np.random.default_rng(0)
    n, k = shape
    w = rng.normal(size=(n, k)).astype(np.float32)
    q, sc, _ = quantize_q8(w) if kind == "q8" else quantize_q4(w)
    t = QTensor(kind, q, sc, (n, k), Q8_BLOCK if kind == "q8" else Q4_BLOCK)
    for m in (1, 7):
        x = rng.normal(size=(m, k)).astype(np.float32)
        ref = x @ w.T
        assert np.abs(qmatmul(x, t) - ref).mean() / np.abs(ref).mean() < tol


def test_qmatmul_dequant_is_exact_product():
    """Dequantisation is code * fp16 scale, exact in fp32; the matmul equals a
    float64 brute force of that product to fp32 accumulation error."""
    rng = np.random.default_rng(1)
    w = rng.normal(size=(50, 130)).astype(np.float32)
    q, sc, _ = quantize_q8(w)
    t = QTensor("q8", q, sc, (50, 130), Q8_BLOCK)
    deq = t.dequant()
    brute = (q.astype(np.float64).reshape(50, 3, 64) * sc.astype(np.float64)[..., None]).reshape(50, 192)[:, :130]
    assert np.array_equal(deq.astype(np.float64), brute)
    x = rng.normal(size=(3, 130)).astype(np.float32)
    assert np.abs(qmatmul(x, t) - x.astype(np.float64) @ brute.T).max() < 1e-4


def test_qmatmul_tile_and_thread_invariant():
    rng = np.random.default_rng(1)
    w = rng.normal(size=(1000, 640)).astype(np.float32)
    q, sc, _ = quantize_q8(w)
    t = QTensor("q8", q, sc, (1000, 640), Q8_BLOCK)
    x = rng.normal(size=(3, 640)).astype(np.float32)
    base = qmatmul(x, t, tile_bytes=1 << 23, threads=1)
    for tb in (1 << 14, 1 << 20):
        for th in (1, 4):
            assert np.abs(qmatmul(x, t, tile_bytes=tb, threads=th) - base).max() < 1e-4


def test_plain_weight_and_bias():
    rng = np.random.default_rng(2)
    w = rng.normal(size=(5, 7)).astype(np.float32)
    b = rng.normal(size=5).astype(np.float32)
    x = rng.normal(size=(2, 7)).astype(np.float32)
    assert np.abs(qmatmul(x, w, b) - (x @ w.T + b)).max() < 1e-5
