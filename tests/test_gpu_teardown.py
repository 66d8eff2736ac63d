"""Lifetime of the library's HIP objects.

* ``cv3_shutdown`` releases every stream and event the library handed out
  (``Stream``, ``Event``, ``Timer``), every per-thread stream, graph and allocator
  block, so nothing the library made is left for the HIP runtime's own exit handlers.
  ``cv3_live_handles`` counts what is held; after shutdown every count is 0, every
  further call raises, and releases from the host's own teardown are no-ops.  Runs in a
  child process, since shutdown ends the library for the rest of that process.
* A block recorded on a stream that is destroyed before the block is freed: the
  destroy drains the stream and removes it from the block, so the later free neither
  records onto a destroyed stream nor leaves the block out of the allocator's books.
"""

import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = textwrap.dedent("""
    import sys
    sys.path[:0] = [{root!r}, {pkg!r}]
    import numpy as np
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Event, Graph, Stream, Timer, synchronize
    _lib.init(0)
    streams = [Stream() for _ in range(3)]
    events = [Event() for _ in range(4)]
    timers = [Timer() for _ in range(2)]
    a = DeviceArray((1 << 20,)).copy_from(np.ones(1 << 20, np.float32))
    b = DeviceArray((1 << 20,))
    for s in streams:
        b.record_stream(s)
        _lib.call("copy_d2d", b.ptr, a.ptr, a.nbytes, s.handle)
        events[0].record(s)
    g = Graph()
    with g:
        _lib.call("fill_zero", a.ptr, a.nbytes, None)
    g.launch()
    timers[0].start()
    g.launch()
    ms = timers[0].stop()
    synchronize()
    before = _lib.live_handles()
    print("before", before, flush=True)
    assert before["streams"] >= 4 and before["events"] >= 8 and before["graphs"] == 1 and before["blocks"] >= 2
    _lib.shutdown()
    after = _lib.live_handles()
    print("after", after, flush=True)
    assert after == {{"streams": 0, "events": 0, "graphs": 0, "blocks": 0}}, after
    try:
        DeviceArray((16,))
    except (RuntimeError, ValueError) as e:
        print("refused:", e, flush=True)
    else:
        raise AssertionError("an allocation after shutdown was accepted")
    # the C ABI refuses too, below the binding
    rc = _lib.lib().cv3_fill_zero(None, 16, None)
    assert rc != 0, rc
    # the host's own teardown releases everything again: no-ops
    del streams, events, timers, a, b, g
    print("child done", flush=True)
""")


def test_shutdown_releases_every_handle(gpu):
    code = _CHILD.format(root=ROOT, pkg=os.path.join(ROOT, "cosyvoice3-cpu_amd"))
    print("[teardown] child: streams, events, timers, a graph, then shutdown", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"child exited with {r.returncode}"
    assert "child done" in r.stdout


def test_block_outlives_its_recorded_stream(gpu):
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Stream, synchronize
    n = 1 << 20
    src = DeviceArray((n,)).copy_from(np.full(n, 3.0, np.float32))
    synchronize()
    in0, cached0 = _lib.mem_stats()
    h0 = _lib.live_handles()
    side = Stream()
    arr = DeviceArray((n,))
    arr.record_stream(side)
    _lib.call("copy_d2d", arr.ptr, src.ptr, arr.nbytes, side.handle)
    del side                              # destroyed while arr is still recorded on it
    assert float(arr.numpy().min()) == 3.0  # the destroy drained the stream's copy
    del arr                               # the free records only on live streams
    synchronize()
    in1, cached1 = _lib.mem_stats()
    assert in1 == in0, (in0, in1)          # the block left the in-use count ...
    assert cached1 - cached0 in (0, n * 4), (cached0, cached1)   # ... and sits in the cache (reused or new)
    h1 = _lib.live_handles()
    assert h1["streams"] == h0["streams"], (h0, h1)   # the side stream is gone
    again = DeviceArray((n,)).zero_()     # the cached block is handed out again without error
    synchronize()
    assert float(np.abs(again.numpy()).max()) == 0.0
