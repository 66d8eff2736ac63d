"""Every benchmarked workload at its own size against the oracle.

* Qwen2-0.5B greedy decode: 24 layers, per-output-channel int8 with float32
  scales, KV cache pre-filled to 512 positions of N(0, 1), 256 tokens from
  speech_embedding[sos] (cv3cpu/models/qwen2.py:139-179, llm.py:112-123).  Both
  device steps (the whole step as one launch, and five kernels per layer) choose
  the oracle's 256 tokens; logits within 1e-5 on a sample of steps.
* DiT flow solve, 10 s: 22 blocks x 10 Euler steps at T = 500 with CFG, the ODE
  noise from the host torch.randn replica (flow.py:36-43,58-93), within 1e-4.
* DiT flow solve, 30 s (T = 1500) with q8 linears dequantised in the GEMM:
  per-output-channel int8 + float32 scales for all 10 steps, and the converter's
  block-64 / float16 profile for 3 steps (the oracle spends ~3.5 s per 30 s
  estimator evaluation, so the second profile is bounded), within 1e-4.
* HiFTNet, 10 s: mel [80, 500] ~ N(-5, 2) through F0 net, NSF excitation and
  decode, whole and in the reference's 1 s windows with 64 frames of context
  (hift.py:170-218), within 1e-4.

Weights: seeded N(0, 0.02) synthetic weights at the real geometries (cv3amd/synth.py),
quantised by the oracle's quantisers (bit-exact with the device's, test_gpu_ops.py).
"""

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

PREFILL, TOKENS = 512, 256


# ----------------------------------------------------------------------------
# Qwen2-0.5B decode
# ----------------------------------------------------------------------------

@pytest.mark.timeout(300)
def test_decode_24_layers_256_tokens_from_kv_512(gpu):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    from oracle.llm import CosyVoice3LM

    t = synth.quantize_store(synth.qwen2_tensors(layers=24), "per_channel", oracle.quant.quantize_q8)
    meta = synth.qwen2_meta(layers=24)
    rng = np.random.default_rng(0)
    k = rng.standard_normal((24, 2, PREFILL, 64), dtype=np.float32)
    v = rng.standard_normal((24, 2, PREFILL, 64), dtype=np.float32)

    lm = CosyVoice3LM(WeightStore(t, meta, oracle.quant.QTensor), "llm.")
    cache = lm.body.new_cache()
    cache._reserve(PREFILL + TOKENS + 1)
    for i in range(24):
        cache.k[i][:, :PREFILL], cache.v[i][:, :PREFILL] = k[i], v[i]
    cache.length = PREFILL
    print(f"[config1] oracle: {TOKENS} greedy tokens from KV {PREFILL}", flush=True)
    x = lm.speech_emb([lm.sos])
    want_tokens, want_logits = [], {}
    sample = {0, 1, 2, 63, 127, 128, 191, 254, 255}
    for s in range(TOKENS):
        logits = lm.head(lm.body.forward(x, cache)[-1:])[0]
        top = int(np.argmax(logits))
        want_tokens.append(top)
        if s in sample:
            want_logits[s] = logits
        x = lm.speech_emb([top])

    d = DeviceQwen2(WeightStore(t, meta, cv3amd.quant.QTensor), cap=1024)
    d.fill_cache(k, v)
    d.begin(lm.sos, PREFILL)
    for s in range(TOKENS):
        d.step_persistent()
        if s in sample:
            e = rel_err(d.logits.numpy(), want_logits[s])
            print(f"[config1] one-launch step {s}: logits rel err {e:.2e}", flush=True)
            assert e < 1e-5, f"step {s}"
    assert not d.persistent_error()
    got = [int(z) for z in d.ints.numpy()[2 + PREFILL + 1: 2 + PREFILL + 1 + TOKENS]]
    first = next((i for i, (a, b) in enumerate(zip(got, want_tokens)) if a != b), None)
    print(f"[config1] one-launch tokens: first mismatch {first}", flush=True)
    assert got == want_tokens
    # the appended cache rows of the last token, every layer
    kc, vc = d.k_cache.numpy(), d.v_cache.numpy()
    end = PREFILL + TOKENS
    for i in (0, 11, 23):
        assert rel_err(kc[i][:, PREFILL:end], cache.k[i][:, PREFILL:end]) < 1e-5
        assert rel_err(vc[i][:, PREFILL:end], cache.v[i][:, PREFILL:end]) < 1e-5

    # the five-kernel step from the same start, replayed from its captured graph
    d.fill_cache(k, v)
    assert d.generate(lm.sos, PREFILL, TOKENS, graph=True) == want_tokens


# ----------------------------------------------------------------------------
# DiT flow solve
# ----------------------------------------------------------------------------

@pytest.fixture(scope="module")
def dit22():
    from cv3amd import synth
    print("[flow] synthesising the 22-block DiT", flush=True)
    return synth.dit_tensors(depth=22), synth.dit_meta(depth=22)


def _flow_inputs(T):
    """The benchmark's inputs: mu, cond, spks ~ N(0, 1) from default_rng(0); the ODE noise
    is the first T columns of torch.randn((1, 80, 15000)) with seed 0 (flow.py:16,36-43)."""
    from cv3amd.torch_rng import randn
    rng = np.random.default_rng(0)
    mu = rng.standard_normal((1, 80, T), dtype=np.float32)
    cond = rng.standard_normal((1, 80, T), dtype=np.float32)
    spks = rng.standard_normal((1, 80), dtype=np.float32)
    x0 = np.ascontiguousarray(randn((1, 80, 15000), 0)[:, :, :T])
    return mu, cond, spks, x0


def _solve_pair(tensors, meta, T, steps):
    import oracle.quant
    import cv3amd.quant
    from cv3amd.dit import DeviceDiT
    from cv3amd.weights import WeightStore
    from oracle.flow import Flow
    mu, cond, spks, x0 = _flow_inputs(T)
    f = Flow(WeightStore(tensors, meta, oracle.quant.QTensor), "flow.")
    f.n_timesteps = steps
    print(f"[flow] oracle: 22 blocks x {steps} steps, T={T}", flush=True)
    want = f.solve_euler(mu, spks, cond, x0=x0)
    d = DeviceDiT(WeightStore(tensors, meta, cv3amd.quant.QTensor), steps=steps)
    d.prepare(mu, spks, cond)
    got = d.solve(x0, graph=True).numpy()
    again = d.solve(x0, graph=True).numpy()      # a second replay of the captured solve
    return got, again, want[0]


@pytest.mark.timeout(300)
def test_flow_10s_22_blocks_10_steps(gpu, dit22):
    got, again, want = _solve_pair(*dit22, 500, 10)
    e = rel_err(got, want)
    print(f"[flow] 10 s solve rel err {e:.2e}", flush=True)
    assert e < 1e-4
    assert np.array_equal(again, got)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("profile,steps", [("per_channel", 10), ("balanced", 10)])
def test_flow_30s_q8_22_blocks(gpu, dit22, profile, steps):
    import oracle.quant
    from cv3amd import synth
    tensors, meta = dit22
    qt = synth.quantize_store(tensors, profile, oracle.quant.quantize_q8)
    got, again, want = _solve_pair(qt, meta, 1500, steps)
    e = rel_err(got, want)
    print(f"[flow] 30 s q8 ({profile}) solve, {steps} steps: rel err {e:.2e}", flush=True)
    assert e < 1e-4
    assert np.array_equal(again, got)


# ----------------------------------------------------------------------------
# HiFTNet vocoder
# ----------------------------------------------------------------------------

def test_vocoder_10s_whole_and_1s_windows(gpu):
    import oracle.quant
    from cv3amd import synth
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weights import WeightStore
    from oracle.hift import HiFTGenerator
    from oracle.torch_rng import TorchMT19937
    T = 500
    t = synth.hift_tensors(base=512)
    meta = synth.hift_meta()
    rng = np.random.default_rng(0)
    mel = (rng.standard_normal((80, T), dtype=np.float32) * np.float32(2.0) - np.float32(5.0)).astype(np.float32)
    h = HiFTGenerator(WeightStore(t, meta, oracle.quant.QTensor), "hift.")
    n = 480 * T
    h.set_source_noise(TorchMT19937(0).random_float32(n * 9).reshape(n, 9))
    print(f"[config4] oracle: F0, excitation, decode of {T} mel frames", flush=True)
    source = h.excitation(h.f0_predict(mel).astype(np.float32))
    d = DeviceHiFT(WeightStore(t, meta))
    for chunk in (None, 50):
        want = h.decode(mel, source, chunk=chunk, context=64)
        for graph in (True, False):
            got = d.inference(mel, chunk=chunk, context=64, graph=graph).numpy()
            assert got.shape == want.shape == (480 * T,)
            e = rel_err(got, want)
            print(f"[config4] chunk={chunk} graph={graph}: rel err {e:.2e}", flush=True)
            assert e < 1e-4
