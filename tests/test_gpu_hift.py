"""Device-resident HiFTNet decode (source STFT -> conv stack -> iSTFT head) against the oracle.

The source signal (F0 prediction + NSF excitation, float64 host code in the
reference) comes from the oracle; the device decodes it.  Bars:
* the reference's toy checkpoint: the frozen upstream waveform within the
  reference's 2e-3, the oracle within 1e-4, chunked == full within 1e-5;
* the 512-channel geometry of config 4 on 1 s of mel: the oracle within 1e-4, whole
  and in chunks (the reference's 1 s windows with 64 frames of context), launched
  directly and by replaying the captured per-window graphs (replayed twice: identical).
"""

import numpy as np
import pytest

from conftest import load_toy, rel_err

pytestmark = pytest.mark.gpu


def _oracle_hift(store, n_mel):
    from oracle.hift import HiFTGenerator
    from oracle.torch_rng import TorchMT19937
    h = HiFTGenerator(store, "hift.")
    n = 480 * n_mel
    h.set_source_noise(TorchMT19937(0).random_float32(n * 9).reshape(n, 9))
    return h


def test_toy_checkpoint(gpu, reference_io):
    import oracle.quant
    from cv3amd.hift import DeviceHiFT
    store = load_toy(oracle.quant.QTensor)
    mel = reference_io["mel"]
    n_mel = mel.shape[1]
    h = _oracle_hift(store, n_mel)
    source = h.excitation(h.f0_predict(mel).astype(np.float32))
    want = h.decode(mel, source)
    print(f"[hift] toy checkpoint, {n_mel} mel frames", flush=True)
    d = DeviceHiFT(store)
    got = d.decode(mel, source).numpy()
    assert got.shape == reference_io["hift_wav"].shape
    e_up, e_or = rel_err(got, reference_io["hift_wav"]), rel_err(got, want)
    print(f"[hift] vs upstream {e_up:.2e}, vs oracle {e_or:.2e}", flush=True)
    assert e_up < 2e-3
    assert e_or < 1e-4
    chunked = d.decode(mel, source, chunk=8, context=64).numpy()
    assert rel_err(chunked, got) < 1e-5


@pytest.mark.parametrize("chunk,graph", [(None, True), (None, False), (20, True), (20, False)])
def test_full_width_one_second(gpu, chunk, graph):
    import oracle.quant
    from cv3amd import synth
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weights import WeightStore
    T = 50
    t = synth.hift_tensors(base=512)
    meta = synth.hift_meta()
    cpu = WeightStore(t, meta, oracle.quant.QTensor)
    rng = np.random.default_rng(4)
    mel = (rng.standard_normal((80, T), dtype=np.float32) * 2.0 - 5.0).astype(np.float32)
    source = np.tanh(rng.standard_normal(480 * T, dtype=np.float32) * 0.1).astype(np.float32)
    print(f"[hift] base 512, {T} mel frames, chunk={chunk}, graph={graph}", flush=True)
    h = _oracle_hift(cpu, T)
    want = h.decode(mel, source, chunk=chunk, context=64)
    d = DeviceHiFT(WeightStore(t, meta))
    got = d.decode(mel, source, chunk=chunk, context=64, graph=graph).numpy()
    e = rel_err(got, want)
    if graph:  # a second replay of the captured stacks gives the same samples
        again = d.decode(mel, source, chunk=chunk, context=64, graph=graph).numpy()
        assert np.array_equal(again, got)
    print(f"[hift] rel err {e:.2e}", flush=True)
    assert e < 1e-4
