"""The device harnesses fed from the reference's weight file (cv3cpu/io/weights.py).

The same synthetic weights go through ``write_weight_file`` and back through
``DeviceWeightFile``; the harness built from the file must give exactly what the
in-memory store gives (same bytes, same kernels: bit-identical), and the stage
lifetime must hold: ``upload`` puts a stage in HBM, ``evict`` hands it back once no
harness holds it, while a live harness keeps working on its own device copies.
"""

import gc

import numpy as np
import pytest

from conftest import load_toy, rel_err

pytestmark = pytest.mark.gpu

PREFILL = 64


def _qwen2_file(tmp_path, layers=2):
    import oracle.quant
    from cv3amd import synth
    from cv3amd.weightfile import write_weight_file
    t = synth.quantize_store(synth.qwen2_tensors(layers=layers), "balanced", oracle.quant.quantize_q8)
    meta = synth.qwen2_meta(layers=layers)
    path = str(tmp_path / "llm.safetensors")
    write_weight_file(path, t, meta)
    return t, meta, path


def _logits(d, k, v, steps):
    d.fill_cache(k, v)
    d.begin(0, PREFILL)
    out = []
    for _ in range(steps):
        d.step(graph=False)
        out.append(d.logits.numpy().copy())
    return out


def test_decode_from_the_weight_file(gpu, tmp_path):
    """DeviceQwen2 lays the file's q8 weights out in one pass (fused QKV, stacked layers);
    after that the file's pages can go, and dropping the harness frees its HBM."""
    from cv3amd import _lib
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weightfile import DeviceWeightFile
    from cv3amd.weights import WeightStore
    layers, steps = 2, 6
    t, meta, path = _qwen2_file(tmp_path, layers)
    rng = np.random.default_rng(7)
    k = rng.standard_normal((layers, 2, PREFILL, 64), dtype=np.float32)
    v = rng.standard_normal((layers, 2, PREFILL, 64), dtype=np.float32)
    print(f"[weightfile] qwen2 {layers} layers balanced q8 from {path}", flush=True)
    want = _logits(DeviceQwen2(WeightStore(t, meta), cap=256), k, v, steps)
    gc.collect()
    base, _ = _lib.mem_stats()
    f = DeviceWeightFile(path)
    assert f.meta == meta
    d = DeviceQwen2(f, cap=256)
    held, _ = _lib.mem_stats()
    body = sum(d.bytes_per_token(0)[x] for x in ("body", "head"))
    print(f"[weightfile] in use {base} -> {held} ({body} bytes of q8 weights)", flush=True)
    assert held - base >= body
    f.evict("llm.")
    got = _logits(d, k, v, steps)
    for s, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(g, w), f"step {s}: rel err {rel_err(g, w):.2e}"
    del d
    gc.collect()
    after, _ = _lib.mem_stats()
    print(f"[weightfile] harness dropped: in use {after}", flush=True)
    assert after <= base
    f.close()


def test_stage_upload_and_evict_for_the_dropin_ops(gpu, tmp_path):
    """``upload`` puts one stage's tensors in HBM for the per-op drop-in path
    (cv3amd.ops); ``evict`` hands them back; results match the in-memory store's."""
    from cv3amd import _lib, ops
    from cv3amd.weightfile import DeviceWeightFile
    from cv3amd.weights import WeightStore
    t, meta, path = _qwen2_file(tmp_path, 1)
    name = "llm.model.layers.0.mlp.up_proj.weight"
    bias = "llm.model.layers.0.self_attn.q_proj.bias"
    x = np.random.default_rng(8).standard_normal((3, 896), dtype=np.float32)
    mem = WeightStore(t, meta)
    want = ops.linear(x, mem.get(name))
    gc.collect()
    base, _ = _lib.mem_stats()
    f = DeviceWeightFile(path)
    up = f.upload("llm.model.layers.0.")
    held, _ = _lib.mem_stats()
    print(f"[weightfile] stage upload {up} bytes; in use {base} -> {held}", flush=True)
    assert up >= f.stage_bytes("llm.model.layers.0.") and held - base >= up
    assert np.array_equal(ops.linear(x, f.get(name)), want)
    assert np.array_equal(f.get(bias), mem.get(bias))
    assert f.evict("llm.model.layers.0.") > 0
    gc.collect()
    after, _ = _lib.mem_stats()
    print(f"[weightfile] evicted: in use {after}", flush=True)
    assert after - base < up // 8
    f.close()


def test_vocoder_from_the_weight_file(gpu, tmp_path, reference_io):
    """The reference's toy checkpoint written out and decoded by DeviceHiFT from the file."""
    import oracle.quant
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weightfile import DeviceWeightFile, write_weight_file
    from oracle.hift import HiFTGenerator
    from oracle.torch_rng import TorchMT19937
    store = load_toy(oracle.quant.QTensor)
    path = str(tmp_path / "toy.safetensors")
    write_weight_file(path, {k: np.asarray(store.raw(k)) for k in store.keys()}, store.meta)
    mel = reference_io["mel"]
    n_mel = mel.shape[1]
    h = HiFTGenerator(store, "hift.")
    h.set_source_noise(TorchMT19937(0).random_float32(480 * n_mel * 9).reshape(480 * n_mel, 9))
    source = h.excitation(h.f0_predict(mel).astype(np.float32))
    print(f"[weightfile] toy hift from {path}, {n_mel} frames", flush=True)
    want = DeviceHiFT(load_toy()).decode(mel, source).numpy()
    with DeviceWeightFile(path) as f:
        got = DeviceHiFT(f).decode(mel, source).numpy()
    assert np.array_equal(got, want)
    assert rel_err(got, h.decode(mel, source)) < 1e-4
