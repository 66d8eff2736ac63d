"""Re-entrancy of the drop-in ops and stream safety of the caching allocator.

* The reference calls the quantised GEMV from a pool of min(4, cpu) threads
  (cv3cpu/quant.py:139-153,192-197).  Here four host threads call
  ``cv3amd.ops.linear`` at once, each on its own stream, on weights they share
  (one device upload per weight object); every result meets the oracle.
* A block freed while its thread's stream is being captured belongs to the
  graph: it is not handed out again until the graph is destroyed.
"""

import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def test_linear_from_four_threads(gpu):
    import oracle.ops as rops
    import oracle.quant as rquant
    import cv3amd.ops as ops
    import cv3amd.quant as quant
    rng = np.random.default_rng(11)
    w8 = rng.standard_normal((4864, 896), dtype=np.float32) * np.float32(0.02)
    q, s, _ = rquant.quantize_q8(w8, 896, np.float32)
    qb, sb, _ = rquant.quantize_q8(w8, 64, np.float16)
    dev_w = {"pc": quant.QTensor("q8", q, s, (4864, 896), 896), "blk": quant.QTensor("q8", qb, sb, (4864, 896), 64)}
    ref_w = {"pc": rquant.QTensor("q8", q, s, (4864, 896), 896), "blk": rquant.QTensor("q8", qb, sb, (4864, 896), 64)}
    wf = rng.standard_normal((1024, 1024), dtype=np.float32) * np.float32(0.02)
    wf.flags.writeable = False
    bias = rng.standard_normal(1024, dtype=np.float32) * np.float32(0.02)
    # (weight key, rows): the GEMV regime (m <= 4) and the MFMA GEMM
    jobs = [(key, m, seed) for seed in range(6) for key, m in (("pc", 1), ("blk", 3), ("f32", 200), ("pc", 64))]
    barrier = threading.Barrier(4)
    threads = set()

    def run(job):
        key, m, seed = job
        if seed == 0:
            barrier.wait(timeout=60)    # the first four jobs start together, one per thread
        threads.add(threading.get_ident())
        x = np.random.default_rng(100 + seed).standard_normal((m, 896 if key != "f32" else 1024), dtype=np.float32)
        if key == "f32":
            got, want = ops.linear(x, wf, bias), rops.linear(x, wf, bias)
        else:
            got, want = ops.linear(x, dev_w[key]), rops.linear(x, ref_w[key])
        return key, m, seed, rel_err(got, want)

    print(f"[threads] {len(jobs)} linear calls from 4 host threads", flush=True)
    with ThreadPoolExecutor(4) as ex:
        results = list(ex.map(run, jobs))
    assert len(threads) == 4      # four threads, hence four per-thread streams
    for key, m, seed, e in results:
        assert e < 1e-5, f"{key} m={m} seed={seed}: rel err {e:.2e}"
    print(f"[threads] worst rel err {max(r[3] for r in results):.2e}", flush=True)


def test_block_freed_during_capture_belongs_to_the_graph(gpu):
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Graph, synchronize
    nbytes = 3 << 20
    a = DeviceArray((nbytes // 4,)).zero_()
    pa = a.ptr
    g = Graph()
    with g:
        _lib.call("fill_zero", a.ptr, a.nbytes, None)   # the graph writes a ...
        del a                                           # ... and a is dropped while capturing
    synchronize()
    b = DeviceArray((nbytes // 4,))
    assert b.ptr != pa, "a block the graph refers to was handed out again"
    g.launch()
    g.launch()
    synchronize()
    in_use0, cached0 = _lib.mem_stats()
    del g                                               # the graph goes: its block returns to the cache
    synchronize()
    in_use1, cached1 = _lib.mem_stats()
    assert in_use0 - in_use1 == nbytes and cached1 - cached0 == nbytes
    del b


def test_record_stream_orders_reuse(gpu):
    """A block written on a side stream and freed from the thread's stream is reused only
    behind the side stream's work: the value written there is never overwritten early."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Stream, synchronize
    n = 1 << 22
    src = DeviceArray((n,)).copy_from(np.full(n, 7.0, np.float32))
    side = Stream()
    for _ in range(5):
        tmp = DeviceArray((n,))
        tmp.record_stream(side)
        dst = DeviceArray((n,))
        dst.record_stream(side)
        _lib.call("copy_d2d", tmp.ptr, src.ptr, tmp.nbytes, side.handle)
        _lib.call("copy_d2d", dst.ptr, tmp.ptr, tmp.nbytes, side.handle)
        del tmp                        # its block may be reused below, behind the side stream
        over = DeviceArray((n,)).zero_()
        _lib.call("stream_sync", side.handle)
        synchronize()
        assert float(dst.numpy().min()) == 7.0
        del over, dst
