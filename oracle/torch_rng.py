"""Oracle restatement of the PyTorch CPU generator replica.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/torch_rng.py: MT19937 with ``init_genrand`` seeding
(torch_rng.py:27-37), the standard twist and tempering (torch_rng.py:39-86),
float32 uniforms from the low 24 bits (torch_rng.py:88-91), float64 uniforms
from a 64-bit draw whose first word is the high half (torch_rng.py:93-102),
and ``normal_fill``'s 16-wide Box-Muller pairing j with j+8
(torch_rng.py:105-114, 117-142).
"""

from __future__ import annotations

import numpy as np

N = 624
M = 397
MATRIX_A = 0x9908B0DF
UPPER_MASK = 0x80000000
LOWER_MASK = 0x7FFFFFFF


class TorchMT19937:
    def __init__(self, seed: int = 0):
        s = np.zeros(N, dtype=np.uint64)
        s[0] = seed & 0xFFFFFFFF
        for i in range(1, N):
            p = int(s[i - 1])
            s[i] = (1812433253 * (p ^ (p >> 30)) + i) & 0xFFFFFFFF
        self.state = s.astype(np.uint32)
        self.pos = N

    @staticmethod
    def _mix(hi_word, lo_word, src):
        y = (hi_word & np.uint32(UPPER_MASK)) | (lo_word & np.uint32(LOWER_MASK))
        odd = (y & np.uint32(1)).astype(bool)
        return src ^ (y >> np.uint32(1)) ^ np.where(odd, np.uint32(MATRIX_A), np.uint32(0))

    def _regenerate(self):
        old = self.state
        new = np.empty_like(old)
        lag = N - M            # 227: how far behind the new words the source runs
        # words [0, lag) take their source from old words [M, N)
        new[:lag] = self._mix(old[:lag], old[1:lag + 1], old[M:N])
        # words [lag, N-1) take their source from new words already produced
        i = lag
        while i < N - 1:
            j = min(i + lag, N - 1)
            new[i:j] = self._mix(old[i:j], old[i + 1:j + 1], new[i - lag:j - lag])
            i = j
        # the last word wraps: its low bits come from the *new* word 0
        new[N - 1] = self._mix(old[N - 1:N], new[0:1], new[M - 1:M])[0]
        self.state = new
        self.pos = 0

    def next_u32(self, n: int) -> np.ndarray:
        raw = np.empty(n, dtype=np.uint32)
        got = 0
        while got < n:
            if self.pos >= N:
                self._regenerate()
            take = min(n - got, N - self.pos)
            raw[got:got + take] = self.state[self.pos:self.pos + take]
            self.pos += take
            got += take
        y = raw
        y = y ^ (y >> np.uint32(11))
        y = y ^ ((y << np.uint32(7)) & np.uint32(0x9D2C5680))
        y = y ^ ((y << np.uint32(15)) & np.uint32(0xEFC60000))
        y = y ^ (y >> np.uint32(18))
        return y

    def random_float32(self, n: int) -> np.ndarray:
        low24 = self.next_u32(n) & np.uint32(0xFFFFFF)
        return low24.astype(np.float32) * np.float32(1.0 / 16777216.0)

    def random_float64(self, n: int) -> np.ndarray:
        w = self.next_u32(2 * n).astype(np.uint64)
        v = (w[0::2] << np.uint64(32)) | w[1::2]
        return (v & np.uint64((1 << 53) - 1)).astype(np.float64) * (1.0 / float(1 << 53))


def _box_muller16(u: np.ndarray) -> np.ndarray:
    """(..., 16) float32 uniforms -> (..., 16) normals; fp64 arithmetic, float32 result."""
    d = u.astype(np.float64)
    r = np.sqrt(-2.0 * np.log(1.0 - d[..., :8]))
    th = 2.0 * np.pi * d[..., 8:]
    return np.concatenate([r * np.cos(th), r * np.sin(th)], axis=-1).astype(np.float32)


def randn(shape, seed: int = 0, gen: "TorchMT19937 | None" = None) -> np.ndarray:
    """torch.manual_seed(seed); torch.randn(shape) on CPU (torch_rng.py:117-142)."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape)) if shape else 1
    g = gen if gen is not None else TorchMT19937(seed)
    if n < 16:
        # scalar normal_distribution<double>: theta from the first double uniform,
        # radius from the second, both outputs of a pair used.
        npairs = (n + 1) // 2
        u = g.random_float64(2 * npairs).reshape(npairs, 2)
        r = np.sqrt(-2.0 * np.log1p(-u[:, 1]))
        th = 2.0 * np.pi * u[:, 0]
        out = np.stack([r * np.cos(th), r * np.sin(th)], axis=1).astype(np.float32).reshape(-1)
        return out[:n].reshape(shape)
    u = g.random_float32(n)
    full = (n // 16) * 16
    out = np.empty(n, dtype=np.float32)
    out[:full] = _box_muller16(u[:full].reshape(-1, 16)).reshape(-1)
    if n % 16:
        out[n - 16:] = _box_muller16(g.random_float32(16))
    return out.reshape(shape)


def rand(shape, seed: int = 0, gen: "TorchMT19937 | None" = None) -> np.ndarray:
    """torch.manual_seed(seed); torch.rand(shape) on CPU (torch_rng.py:145-150)."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape)) if shape else 1
    g = gen if gen is not None else TorchMT19937(seed)
    return g.random_float32(n).reshape(shape)
