"""Shared test setup.

* ``gpu`` marker: tests that need an MI355X.  The CPU suite runs with
  ``-m "not gpu"``; the GPU suite with ``-m gpu``.  A gpu test fails (not
  skips) when the HIP library is missing, so a GPU run can never pass on a
  silent fallback.
* The package lives in ``cosyvoice3-cpu_amd/`` and the oracle in ``oracle/``.
"""

import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cosyvoice3-cpu_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built libcv3hip.so")


def rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| (the reference's norm, tests/conftest.py:13-16)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(float(np.abs(ref).max()), 1e-9))


@pytest.fixture(scope="session")
def reference_io():
    with np.load(os.path.join(GOLDEN, "reference_io.npz")) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def torch_rng_golden():
    with open(os.path.join(GOLDEN, "torch_rng.json")) as fh:
        return json.load(fh)


def load_toy(qtensor_cls=None):
    """The toy checkpoint as a WeightStore (float32 'f32' profile)."""
    from cv3amd.weights import WeightStore
    with np.load(os.path.join(GOLDEN, "toy_weights.npz")) as z:
        meta = json.loads(str(z["__meta__"]))
        tensors = {k: z[k] for k in z.files if k != "__meta__"}
    return WeightStore(tensors, meta, qtensor_cls)


@pytest.fixture(scope="session")
def toy_oracle_store():
    import oracle.quant
    return load_toy(oracle.quant.QTensor)


@pytest.fixture(scope="session")
def gpu():
    """Initialise the device; fails loudly if the library or the GPU is missing."""
    from cv3amd import _lib
    print("\n[gpu] loading libcv3hip.so", flush=True)
    _lib.lib()
    print("[gpu] initialising device 0", flush=True)
    _lib.init(0)
    info = _lib.device_info()
    print(f"[gpu] {info}", flush=True)
    return info
