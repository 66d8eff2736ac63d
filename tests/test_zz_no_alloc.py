"""cv3_qwen2_decode_step_noalloc (the decode step on the library's fixed scratch)
against cv3_qwen2_decode_step (the same step on a caller workspace), through the
C ABI: logits, tokens and cache rows identical after every step.  Two calls in a
row: the Qwen2-0.5B geometry at 2 layers with 300 cached positions, then a
smaller model (hidden 512, 8 / 2 heads, intermediate 1024) with 40 cached
positions, so the second call reads a scratch the first left full.  Geometries
beyond the scratch are refused with an error, before anything is launched.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(layers, hidden, heads, kv_heads, inter, n, seed):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    t = synth.qwen2_tensors(layers=layers, hidden=hidden, heads=heads, kv_heads=kv_heads, inter=inter, seed=seed)
    t = synth.quantize_store(t, "per_channel", oracle.quant.quantize_q8)
    meta = synth.qwen2_meta(layers=layers, hidden=hidden, heads=heads, kv_heads=kv_heads, inter=inter)
    store = WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(300 + seed)
    hd = hidden // heads
    k = rng.standard_normal((layers, kv_heads, n, hd), dtype=np.float32)
    v = rng.standard_normal((layers, kv_heads, n, hd), dtype=np.float32)
    a, b = DeviceQwen2(store, cap=512), DeviceQwen2(store, cap=512)
    for d in (a, b):
        d.fill_cache(k, v)
        d.begin(int(meta["speech_token_size"]), n)
    return a, b


@pytest.mark.parametrize("case", [
    dict(layers=2, hidden=896, heads=14, kv_heads=2, inter=4864, n=300, seed=0, steps=6),
    dict(layers=1, hidden=512, heads=8, kv_heads=2, inter=1024, n=40, seed=1, steps=6),
])
def test_noalloc_step_matches_the_workspace_step(gpu, case):
    from cv3amd import _lib
    from cv3amd.device import synchronize
    steps = case.pop("steps")
    n = case["n"]
    print(f"[noalloc] {case}, {steps} steps", flush=True)
    ref, got = _pair(**case)
    in_use0 = _lib.mem_stats()
    for s in range(steps):
        _lib.call("qwen2_decode_step", ctypes.byref(ref.model), ctypes.byref(ref.state), None)
        _lib.call("qwen2_decode_step_noalloc", ctypes.byref(got.model), ctypes.byref(got.state), None)
        synchronize()
        assert np.array_equal(got.logits.numpy(), ref.logits.numpy()), f"step {s}"
        assert np.array_equal(got.x.numpy(), ref.x.numpy()), f"step {s}"
    assert _lib.mem_stats() == in_use0          # the allocator was not touched
    ints_r, ints_g = ref.ints.numpy(), got.ints.numpy()
    assert np.array_equal(ints_g[:2 + n + 1 + steps], ints_r[:2 + n + 1 + steps])
    assert np.array_equal(got.k_cache.numpy(), ref.k_cache.numpy())
    assert np.array_equal(got.v_cache.numpy(), ref.v_cache.numpy())


def test_noalloc_step_refuses_geometries_beyond_its_scratch(gpu):
    from cv3amd.qwen2 import Model, State
    from cv3amd import _lib
    m = Model()
    m.layers, m.hidden, m.heads, m.kv_heads, m.head_dim, m.inter = 1, 896, 14, 2, 64, 40000
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("qwen2_decode_step_noalloc", ctypes.byref(m), ctypes.byref(State()), None)


def test_noalloc_calls_from_two_streams_run_one_after_another(gpu):
    """Calls on two streams share the device's scratch: the library orders them (each waits for the
    previous call's end on the other stream), so two decoders stepped alternately on their own
    streams, with no host synchronisation between calls, match the workspace step."""
    from cv3amd import _lib
    from cv3amd.device import Stream, synchronize
    case = dict(layers=2, hidden=896, heads=14, kv_heads=2, inter=4864, n=300, seed=0)
    ref, got = _pair(**case)
    ref2, got2 = _pair(**case)
    sa, sb = Stream(), Stream()
    synchronize()                                 # the caches and states are filled on this thread's stream
    for s in range(4):
        for r in (ref, ref2):
            _lib.call("qwen2_decode_step", ctypes.byref(r.model), ctypes.byref(r.state), None)
        _lib.call("qwen2_decode_step_noalloc", ctypes.byref(got.model), ctypes.byref(got.state), sa.handle)
        _lib.call("qwen2_decode_step_noalloc", ctypes.byref(got2.model), ctypes.byref(got2.state), sb.handle)
    synchronize()
    _lib.call("stream_sync", sa.handle)
    _lib.call("stream_sync", sb.handle)
    for r, g in ((ref, got), (ref2, got2)):
        assert np.array_equal(g.logits.numpy(), r.logits.numpy())
        assert np.array_equal(g.k_cache.numpy(), r.k_cache.numpy())
