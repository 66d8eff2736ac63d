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
    """profile "tiny:packed" is the tiny profile held as packed nibbles on the device
    (``DeviceQwen2(widen_q4=False)``); plain "tiny" widens its codes to int8."""
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    t = synth.qwen2_tensors(layers=layers, seed=seed)
    t = synth.quantize_store(t, profile.split(":")[0], oracle.quant.quantize_q8, oracle.quant.quantize_q4)
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


@pytest.mark.parametrize("profile", ["per_channel", "balanced", "tiny", "tiny:packed"])
def test_decode_two_layers_logits_and_tokens(gpu, profile):
    from cv3amd.qwen2 import DeviceQwen2
    steps = 12
    cpu, dev, k, v = _setup(2, profile)
    print(f"[decode] 2 layers, profile={profile}, {steps} steps", flush=True)
    lm, cache = _oracle_lm(cpu, k, v, steps)
    d = DeviceQwen2(dev, cap=1024, widen_q4=not profile.endswith(":packed"))
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


@pytest.mark.parametrize("profile", ["per_channel", "tiny", "tiny:packed"])
def test_decode_full_depth_graph_replay(gpu, profile):
    """24 layers, 8 greedy tokens replayed from one captured step graph."""
    from cv3amd.qwen2 import DeviceQwen2
    steps = 8
    cpu, dev, k, v = _setup(24, profile)
    print(f"[decode] 24 layers {profile}, {steps} steps, graph", flush=True)
    lm, cache = _oracle_lm(cpu, k, v, steps)
    want = lm.greedy(lm.speech_emb([lm.sos]), cache, steps)
    d = DeviceQwen2(dev, cap=1024, widen_q4=not profile.endswith(":packed"))
    d.fill_cache(k, v)
    got = d.generate(lm.sos, PREFILL, steps, graph=True)
    print(f"[decode] oracle {want}\n[decode] device {got}", flush=True)
    assert got == want
    # a second run from the same state replays the same graph and the same tokens
    d.fill_cache(k, v)
    assert d.generate(lm.sos, PREFILL, steps, graph=True) == want


def test_pcg64_stream_matches_numpy(gpu):
    """cv3_pcg64_random against Generator.random() from the same PCG64 state, and the
    state it leaves behind."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray
    g = np.random.default_rng(20241201)
    st = g.bit_generator.state["state"]
    m = (1 << 64) - 1
    pcg = DeviceArray((4,), np.int64)
    pcg.copy_from(np.array([st["state"] >> 64, st["state"] & m, st["inc"] >> 64, st["inc"] & m],
                           np.uint64).view(np.int64))
    out = DeviceArray((1000,), np.float64)
    _lib.call("pcg64_random", pcg.ptr, 1000, out.ptr, None)
    assert np.array_equal(out.numpy(), g.random(1000))
    c = pcg.numpy().view(np.uint64)
    assert (int(c[0]) << 64 | int(c[1])) == g.bit_generator.state["state"]["state"]


SAMPLING = {
    "default": dict(top_p=0.8, top_k=25, win_size=10, tau_r=0.1),   # SamplingConfig's defaults
    "always_resample": dict(top_p=0.8, top_k=25, win_size=10, tau_r=0.0),
    "top1": dict(top_p=0.8, top_k=1, win_size=10, tau_r=0.1),
    "wide": dict(top_p=0.95, top_k=64, win_size=3, tau_r=0.5),
}


@pytest.mark.parametrize("name", sorted(SAMPLING))
def test_decode_sampled_tokens_and_generator_state(gpu, name):
    """The reference's sampler (llm.py:37-49,125-149) on the device: the same tokens as
    the oracle's loop on the same seeded Generator, which ends in the same state."""
    from cv3amd.qwen2 import DeviceQwen2
    from oracle.llm import Sampling
    max_len, min_len = 40, 4
    cpu, dev, k, v = _setup(2, "per_channel")
    print(f"[decode] sampled, 2 layers, {name}, {max_len} tokens", flush=True)
    lm, cache = _oracle_lm(cpu, k, v, max_len)
    ref = Sampling(seed=1234, **SAMPLING[name])
    want = lm.sampled(lm.speech_emb([lm.sos]), cache, max_len, min_len, ref)
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    got_cfg = Sampling(seed=1234, **SAMPLING[name])
    got = d.generate_sampled(lm.sos, PREFILL, max_len, min_len, got_cfg, lm.speech_token_size, graph=True)
    print(f"[decode] oracle {want[:12]}...\n[decode] device {got[:12]}...", flush=True)
    assert got == want
    assert got_cfg.rng.bit_generator.state == ref.rng.bit_generator.state


@pytest.mark.parametrize("strict", [False, True])
def test_decode_sampled_stops_on_a_control_id(gpu, strict):
    """A head bias that makes two stop ids likely: masked below min_len (only the eos id,
    or every stop id with strict_min_len), then the generation ends on the step the
    oracle's does, direct launches and graph replay alike."""
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    from oracle.llm import Sampling
    t = synth.quantize_store(synth.qwen2_tensors(layers=2), "per_channel", oracle.quant.quantize_q8)
    sts = synth.SPEECH_TOKEN_SIZE
    bias = np.array(t["llm.llm_decoder.bias"], np.float32)
    bias[sts] += 9.0        # eos, the id the reference masks below min_len
    bias[sts + 5] += 4.0    # another control id: masked only with strict_min_len
    t["llm.llm_decoder.bias"] = bias
    meta = synth.qwen2_meta(layers=2)
    cpu, dev = WeightStore(t, meta, oracle.quant.QTensor), WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(100)
    k = rng.standard_normal((2, 2, PREFILL, 64), dtype=np.float32)
    v = rng.standard_normal((2, 2, PREFILL, 64), dtype=np.float32)
    max_len, min_len = 48, 6
    lm, cache = _oracle_lm(cpu, k, v, max_len)
    ref = Sampling(seed=77, strict_min_len=strict)
    want = lm.sampled(lm.speech_emb([lm.sos]), cache, max_len, min_len, ref)
    print(f"[decode] stop test strict={strict}: oracle stops after {len(want)} tokens", flush=True)
    # below min_len only strict_min_len holds the second control id back
    assert (min_len <= len(want) < max_len) if strict else (0 < len(want) < min_len)
    for graph in (False, True):
        d = DeviceQwen2(dev, cap=1024)
        d.fill_cache(k, v)
        cfg = Sampling(seed=77, strict_min_len=strict)
        got = d.generate_sampled(lm.sos, PREFILL, max_len, min_len, cfg, sts, graph=graph, check_every=5)
        assert got == want
        assert cfg.rng.bit_generator.state == ref.rng.bit_generator.state


@pytest.mark.parametrize("profile", ["balanced", "tiny"])
def test_prompt_prefill_cache_logits_and_greedy_continuation(gpu, profile):
    """DeviceQwen2.prefill against Qwen2Model.forward over a prompt (qwen2.py:139-179): the
    cache rows it appends and the last position's logits, for a 37-token prompt and a
    5-token continuation on top of it (causal mask offset by the cache), then greedy
    tokens from there."""
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    from oracle.llm import CosyVoice3LM
    layers = 2
    t = synth.quantize_store(synth.qwen2_tensors(layers=layers), profile, oracle.quant.quantize_q8,
                             oracle.quant.quantize_q4)
    meta = synth.qwen2_meta(layers=layers)
    cpu, dev = WeightStore(t, meta, oracle.quant.QTensor), WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(11)
    x1 = (rng.standard_normal((37, 896), dtype=np.float32) * 0.02).astype(np.float32)
    x2 = (rng.standard_normal((5, 896), dtype=np.float32) * 0.02).astype(np.float32)
    lm = CosyVoice3LM(cpu, "llm.")
    cache = lm.body.new_cache()
    d = DeviceQwen2(dev, cap=256)
    print(f"[decode] prefill {profile}: 37 + 5 prompt positions", flush=True)
    for x, pos0 in ((x1, 0), (x2, 37)):
        want = lm.head(lm.body.forward(x, cache)[-1:])[0]
        d.prefill(x, pos0)
        e = rel_err(d.logits.numpy(), want)
        print(f"[decode] prefill at {pos0}: logits rel err {e:.2e}", flush=True)
        assert e < 1e-5
    n = len(cache)
    kc, vc = d.k_cache.numpy(), d.v_cache.numpy()
    for i in range(layers):
        assert rel_err(kc[i][:, :n], cache.k[i][:, :n]) < 1e-5
        assert rel_err(vc[i][:, :n], cache.v[i][:, :n]) < 1e-5
    # greedy continuation: the argmax of the prompt's logits, then decode steps
    top = int(np.argmax(want))
    ref = [top] + lm.greedy(lm.speech_emb([top]), cache, 7)
    got = d.generate_after_prefill(8, graph=False)
    print(f"[decode] oracle {ref}\n[decode] device {got}", flush=True)
    assert got == ref


def test_prompt_prefill_then_sampled_generation(gpu):
    """generate() end to end (llm.py:80-123) from a prompt: the oracle's loop prefills the
    prompt in its first forward; the device prefills, draws the first token from the
    prompt's logits and decodes the rest, on the same seeded Generator."""
    import oracle.quant
    from cv3amd.qwen2 import DeviceQwen2
    from oracle.llm import Sampling
    max_len, min_len = 30, 24   # stop ids held back (strict) for 24 draws, then allowed
    cpu, dev, _, _ = _setup(2, "balanced")
    rng = np.random.default_rng(12)
    prompt = (rng.standard_normal((61, 896), dtype=np.float32) * 0.02).astype(np.float32)
    from oracle.llm import CosyVoice3LM
    lm = CosyVoice3LM(cpu, "llm.")
    ref = Sampling(seed=99, strict_min_len=True)
    want = lm.sampled(prompt, lm.body.new_cache(), max_len, min_len, ref)
    assert len(want) >= min_len
    d = DeviceQwen2(dev, cap=256)
    d.prefill(prompt, 0)
    cfg = Sampling(seed=99, strict_min_len=True)
    got = d.generate_sampled_after_prefill(max_len, min_len, cfg, lm.speech_token_size, graph=True)
    print(f"[decode] prompt 61: oracle {want[:10]}...\n[decode] device {got[:10]}...", flush=True)
    assert got == want
    assert cfg.rng.bit_generator.state == ref.rng.bit_generator.state
