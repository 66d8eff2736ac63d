"""Device-resident greedy Qwen2 decode against the oracle.

Both sides load the same seeded synthetic Qwen2-0.5B weights (cv3amd/synth.py),
quantised by the oracle's quantize_q8 / quantize_q4 (bit-exact with the device
quantisers, see test_gpu_ops.py) under the per-channel, balanced (q8) and tiny
(q4 body) profiles, with the KV cache pre-filled to 512 positions of N(0, 1).
The oracle runs cv3cpu's Qwen2Model.forward / llm_decoder / speech_embedding
restatement (oracle/qwen2.py, oracle/llm.py) with greedy selection.
Bars: per-step logits within 1e-5 (max abs error over max |logit|), identical
token sequences.
"""

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

PREFILL = 512


def _setup(layers, profile, seed=0):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    t = synth.qwen2_tensors(layers=layers, seed=seed)
    t = synth.quantize_store(t, profile, oracle.quant.quantize_q8, oracle.quant.quantize_q4)
    meta = synth.qwen2_meta(layers=layers)
    cpu = WeightStore(t, meta, oracle.quant.QTensor)
    dev = WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(100 + seed)
    k = rng.standard_normal((layers, 2, PREFILL, 64), dtype=np.float32)
    v = rng.standard_normal((layers, 2, PREFILL, 64), dtype=np.float32)
    return cpu, dev, k, v


def _oracle_lm(cpu, k, v, steps):
    from oracle.llm import CosyVoice3LM
    lm = CosyVoice3LM(cpu, "llm.")
    cache = lm.body.new_cache()
    cache._reserve(PREFILL + steps + 1)
    for i in range(lm.cfg.num_hidden_layers):
        cache.k[i][:, :PREFILL] = k[i]
        cache.v[i][:, :PREFILL] = v[i]
    cache.length = PREFILL
    return lm, cache


@pytest.mark.parametrize("profile", ["per_channel", "balanced", "tiny"])
def test_decode_two_layers_logits_and_tokens(gpu, profile):
    from cv3amd.qwen2 import DeviceQwen2
    steps = 12
    cpu, dev, k, v = _setup(2, profile)
    print(f"[decode] 2 layers, profile={profile}, {steps} steps", flush=True)
    lm, cache = _oracle_lm(cpu, k, v, steps)
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    d.begin(lm.sos, PREFILL)
    x = lm.speech_emb([lm.sos])
    for s in range(steps):
        want = lm.head(lm.body.forward(x, cache)[-1:])[0]
        top = int(np.argmax(want))
        x = lm.speech_emb([top])
        d.step(graph=False)
        got = d.logits.numpy()
        e = rel_err(got, want)
        print(f"[decode] step {s} token {top} logits rel err {e:.2e}", flush=True)
        assert e < 1e-5, f"step {s}"
        assert int(d.ints.numpy()[2 + PREFILL + 1 + s]) == top
    # caches agree too (rotary k and raw v appended at positions 512..)
    kc = d.k_cache.numpy()
    for i in range(2):
        assert rel_err(kc[i][:, :PREFILL + steps], cache.k[i][:, :PREFILL + steps]) < 1e-5


@pytest.mark.parametrize("profile", ["per_channel", "tiny"])
def test_decode_full_depth_graph_replay(gpu, profile):
    """24 layers, 8 greedy tokens replayed from one captured step graph."""
    from cv3amd.qwen2 import DeviceQwen2
    steps = 8
    cpu, dev, k, v = _setup(24, profile)
    print(f"[decode] 24 layers {profile}, {steps} steps, graph", flush=True)
    lm, cache = _oracle_lm(cpu, k, v, steps)
    want = lm.greedy(lm.speech_emb([lm.sos]), cache, steps)
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    got = d.generate(lm.sos, PREFILL, steps, graph=True)
    print(f"[decode] oracle {want}\n[decode] device {got}", flush=True)
    assert got == want
    # a second run from the same state replays the same graph and the same tokens
    d.fill_cache(k, v)
    assert d.generate(lm.sos, PREFILL, steps, graph=True) == want
