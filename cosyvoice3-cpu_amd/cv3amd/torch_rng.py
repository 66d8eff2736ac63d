"""Host-side PyTorch CPU-generator replica (cv3cpu/torch_rng.py:27-150).

The ODE initial noise (cv3cpu/models/flow.py:16-17,36-43) and the vocoder's
NSF dither (cv3cpu/models/hift.py:75-81) must be bit-identical to
``torch.randn`` / ``torch.rand`` under a fixed seed.  The generator runs on the
host, in the C++ half of ``libcv3hip.so`` (``cv3_mt_*``): MT19937 with torch's
seeding, 24-bit float32 uniforms, and ATen's 16-wide Box-Muller ``normal_fill``.
It needs no GPU.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class TorchMT19937:
    """A torch CPU generator seeded like ``torch.manual_seed(seed)`` (torch_rng.py:27-37)."""

    def __init__(self, seed: int = 0):
        self._g = ctypes.c_void_p()
        _lib.call("mt_create", int(seed), ctypes.addressof(self._g))

    def random_float32(self, n: int) -> np.ndarray:
        """``torch.rand(n)`` draws: 24-bit uniforms in [0, 1) (torch_rng.py:88-91)."""
        out = np.empty(int(n), np.float32)
        _lib.call("mt_uniform_f32", self._g, int(n), out.ctypes.data)
        return out

    def randn(self, n: int) -> np.ndarray:
        """``torch.randn(n)`` draws (torch_rng.py:105-142)."""
        out = np.empty(int(n), np.float32)
        _lib.call("mt_normal_f32", self._g, int(n), out.ctypes.data)
        return out

    def __del__(self):
        try:
            if self._g:
                _lib.lib().cv3_mt_destroy(self._g)
        except Exception:
            pass


def randn(shape, seed: int = 0) -> np.ndarray:
    """``torch.manual_seed(seed); torch.randn(shape)`` (torch_rng.py:117-142)."""
    n = int(np.prod(shape))
    return TorchMT19937(seed).randn(n).reshape(shape)


def rand(shape, seed: int = 0) -> np.ndarray:
    """``torch.manual_seed(seed); torch.rand(shape)`` (torch_rng.py:145-150)."""
    n = int(np.prod(shape))
    return TorchMT19937(seed).random_float32(n).reshape(shape)
