"""Device-resident HiFTNet (F0 -> NSF source -> source STFT -> conv stack -> iSTFT head)
against the oracle.

``decode`` tests take the source signal from the oracle; ``inference`` tests run the
F0 predictor and the excitation on the device too.  Bars:
* the reference's toy checkpoint: the frozen upstream waveform within the
  reference's 2e-3, the oracle within 1e-4, chunked == full within 1e-5;
* the 512-channel geometry of config 4 on 1 s of mel: the oracle within 1e-4, whole
  and in chunks (the reference's 1 s windows with 64 frames of context), launched
  directly and by replaying the captured per-window graphs (replayed twice: identical);
* device F0 and source against the oracle's within 1e-5, the float64 phase path
  exercised on voiced and unvoiced frames alike; the whole device inference within
  the same waveform bars.
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


def test_whole_stack_branches_change_nothing(gpu, monkeypatch):
    """The whole-input stack captured with its branches on forked streams (each stage's source
    branch beside the upsampling conv, the resblocks side by side) gives the same samples as
    the stack captured on one stream and as the direct launches: the same kernels on the same
    buffers, only their order differs.  Replayed three times, with host reads in between."""
    from cv3amd import synth
    import cv3amd.hift as hift
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weights import WeightStore
    T = 50
    t = synth.hift_tensors(base=512)
    meta = synth.hift_meta()
    rng = np.random.default_rng(5)
    mel = (rng.standard_normal((80, T), dtype=np.float32) * 2.0 - 5.0).astype(np.float32)
    source = np.tanh(rng.standard_normal(480 * T, dtype=np.float32) * 0.1).astype(np.float32)
    print(f"[hift] base 512, {T} mel frames, whole stack with and without branches", flush=True)
    direct = DeviceHiFT(WeightStore(t, meta)).decode(mel, source, graph=False).numpy()
    monkeypatch.setattr(hift, "BRANCHES", False)
    one = DeviceHiFT(WeightStore(t, meta)).decode(mel, source, graph=True).numpy()
    monkeypatch.setattr(hift, "BRANCHES", True)
    d = DeviceHiFT(WeightStore(t, meta))
    for _ in range(3):
        got = d.decode(mel, source, graph=True).numpy()
        assert np.array_equal(got, one)
    assert np.array_equal(one, direct)


def test_toy_inference_on_the_device(gpu, reference_io):
    """mel -> waveform with nothing on the host: the frozen upstream waveform within 2e-3."""
    import oracle.quant
    from cv3amd.hift import DeviceHiFT
    store = load_toy(oracle.quant.QTensor)
    mel = reference_io["mel"]
    n_mel = mel.shape[1]
    h = _oracle_hift(store, n_mel)
    f0_want = h.f0_predict(mel).astype(np.float32)
    src_want = h.excitation(f0_want)
    print(f"[hift] toy inference on the device, {n_mel} mel frames", flush=True)
    d = DeviceHiFT(load_toy())
    f0 = d.f0_predict(mel).numpy()
    src = d.excitation(f0).numpy()
    e_f0, e_src = rel_err(f0, f0_want), rel_err(src, src_want)
    print(f"[hift] f0 rel err {e_f0:.2e}, source rel err {e_src:.2e}", flush=True)
    assert e_f0 < 1e-5 and e_src < 1e-5
    wav = d.inference(mel, chunk=None).numpy()
    e_up, e_or = rel_err(wav, reference_io["hift_wav"]), rel_err(wav, h.decode(mel, src_want))
    print(f"[hift] inference vs upstream {e_up:.2e}, vs oracle {e_or:.2e}", flush=True)
    assert e_up < 2e-3 and e_or < 1e-4
    assert rel_err(d.inference(mel, chunk=8, context=64).numpy(), wav) < 1e-5


def test_source_on_voiced_and_unvoiced_frames(gpu):
    """Full-width F0 net with a classifier scaled so |f0| straddles the voiced threshold:
    the float64 phase, the sines and the dither all contribute."""
    import oracle.quant
    from cv3amd import synth
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weights import WeightStore
    T = 60
    t = synth.hift_tensors(base=512)
    t["hift.f0_predictor.classifier.weight"] = t["hift.f0_predictor.classifier.weight"] * 60.0
    meta = synth.hift_meta()
    rng = np.random.default_rng(5)
    mel = (rng.standard_normal((80, T), dtype=np.float32) * 2.0 - 5.0).astype(np.float32)
    h = _oracle_hift(WeightStore(t, meta, oracle.quant.QTensor), T)
    f0_want = h.f0_predict(mel).astype(np.float32)
    voiced = float((f0_want > 10.0).mean())
    print(f"[hift] base 512, {T} frames, voiced fraction {voiced:.2f}, f0 max {f0_want.max():.1f}", flush=True)
    assert 0.2 < voiced < 0.9
    src_want = h.excitation(f0_want)
    d = DeviceHiFT(WeightStore(t, meta))
    f0 = d.f0_predict(mel).numpy()
    e_f0 = rel_err(f0, f0_want)
    src = d.excitation(f0_want).numpy()
    e_src = rel_err(src, src_want)
    print(f"[hift] f0 rel err {e_f0:.2e}, source rel err {e_src:.2e}", flush=True)
    assert e_f0 < 1e-5 and e_src < 1e-5
    wav = d.inference(mel, chunk=20, context=64).numpy()
    e = rel_err(wav, h.decode(mel, src_want, chunk=20, context=64))
    print(f"[hift] chunked inference rel err {e:.2e}", flush=True)
    assert e < 1e-4


def test_inference_of_an_empty_mel(gpu):
    """Zero frames in, zero samples out (the reference's shapes)."""
    from cv3amd.hift import DeviceHiFT
    d = DeviceHiFT(load_toy())
    assert d.f0_predict(np.zeros((80, 0), np.float32)).shape == (0,)
    assert d.excitation(np.zeros(0, np.float32)).shape == (0,)
