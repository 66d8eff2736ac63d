"""The one-launch decode step (cv3_qwen2_decode_step_persistent) against the oracle.

Same seeded synthetic Qwen2-0.5B weights as test_gpu_decode.py, q8 under the
per-channel (float32 scales, and float16 scales for the matrix-core phase D's
float16 variant) and balanced (block 64, float16 scales) profiles, and
the tiny profile's q4 body (head and embedding q8).
Bars: per-step logits within 1e-5 (max abs error over max |logit|) of the
oracle, identical greedy tokens, the appended cache rows within 1e-5; at 24
layers the tokens equal the five-kernel step's and the logits agree within 1e-5.
Positions cover an empty cache (one attention chunk), a start just below the
128-key chunk boundary, 512 cached positions (five chunks) and the last chunks of a
1024-position cache; ordinary and cooperative launches.  Failure handling is forced from the host: a preset error
flag (every wait gives up within its bounded polls, the host raises) and the
launch counter's wrap.
"""

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _setup(layers, profile, n, seed=0):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    t = synth.qwen2_tensors(layers=layers, seed=seed)
    t = synth.quantize_store(t, profile.split(":")[0], oracle.quant.quantize_q8, oracle.quant.quantize_q4)
    meta = synth.qwen2_meta(layers=layers)
    cpu = WeightStore(t, meta, oracle.quant.QTensor)
    dev = WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(200 + seed)
    k = rng.standard_normal((layers, 2, n, 64), dtype=np.float32)
    v = rng.standard_normal((layers, 2, n, 64), dtype=np.float32)
    return cpu, dev, k, v


def _oracle_lm(cpu, k, v, n, steps):
    from oracle.llm import CosyVoice3LM
    lm = CosyVoice3LM(cpu, "llm.")
    cache = lm.body.new_cache()
    cache._reserve(n + steps + 1)
    for i in range(lm.cfg.num_hidden_layers):
        cache.k[i][:, :n] = k[i]
        cache.v[i][:, :n] = v[i]
    cache.length = n
    return lm, cache


@pytest.mark.parametrize("profile,n,steps,cooperative", [
    ("per_channel", 512, 10, False), ("balanced", 0, 6, False), ("per_channel", 0, 6, False),
    ("balanced", 122, 10, False), ("per_channel", 122, 10, False), ("per_channel", 300, 6, True),
    ("per_channel", 1000, 4, False), ("balanced", 897, 4, False), ("per_channel", 895, 4, False),
    ("tiny", 300, 8, False), ("tiny:packed", 300, 8, False), ("per_channel_f16", 300, 6, False)])
def test_persistent_step_logits_and_tokens(gpu, profile, n, steps, cooperative):
    from cv3amd.qwen2 import DeviceQwen2
    cpu, dev, k, v = _setup(2, profile, n)
    print(f"[persist] 2 layers, profile={profile}, {n} cached, {steps} steps, cooperative={cooperative}",
          flush=True)
    lm, cache = _oracle_lm(cpu, k, v, n, steps)
    d = DeviceQwen2(dev, cap=1024, widen_q4=not profile.endswith(":packed"))
    d.cooperative = cooperative
    if n:
        d.fill_cache(k, v)
    d.begin(lm.sos, n)
    x = lm.speech_emb([lm.sos])
    for s in range(steps):
        want = lm.head(lm.body.forward(x, cache)[-1:])[0]
        top = int(np.argmax(want))
        x = lm.speech_emb([top])
        d.step_persistent()
        got = d.logits.numpy()
        assert not d.persistent_error(), f"step {s}: a wait gave up"
        e = rel_err(got, want)
        print(f"[persist] step {s} token {top} logits rel err {e:.2e}", flush=True)
        assert e < 1e-5, f"step {s}"
        assert int(d.ints.numpy()[2 + n + 1 + s]) == top
        assert int(d.ints.numpy()[0]) == n + 1 + s
    kc, vc = d.k_cache.numpy(), d.v_cache.numpy()
    for i in range(2):
        assert rel_err(kc[i][:, :n + steps], cache.k[i][:, :n + steps]) < 1e-5
        assert rel_err(vc[i][:, :n + steps], cache.v[i][:, :n + steps]) < 1e-5


@pytest.mark.parametrize("profile", ["balanced", "tiny", "tiny:packed", "per_channel_f16"])
def test_persistent_full_depth_matches_five_kernel_step(gpu, profile):
    """24 layers: the one-launch step and the five-kernel step give the same tokens."""
    from cv3amd.qwen2 import DeviceQwen2
    n, steps = 300, 16
    _, dev, k, v = _setup(24, profile, n)
    print(f"[persist] 24 layers, profile={profile}, {n} cached, {steps} steps", flush=True)
    widen = not profile.endswith(":packed")
    a = DeviceQwen2(dev, cap=1024, widen_q4=widen)
    a.fill_cache(k, v)
    want = []
    a.begin(1, n)
    for _ in range(steps):
        a.step(graph=False)
        want.append(a.logits.numpy())
    want_tok = [int(t) for t in a.ints.numpy()[2 + n + 1: 2 + n + 1 + steps]]
    b = DeviceQwen2(dev, cap=1024, widen_q4=widen)
    b.fill_cache(k, v)
    b.begin(1, n)
    for s in range(steps):
        b.step_persistent()
        e = rel_err(b.logits.numpy(), want[s])
        print(f"[persist] step {s} logits rel err vs five-kernel step {e:.2e}", flush=True)
        assert e < 1e-5, f"step {s}"
    assert not b.persistent_error()
    got_tok = [int(t) for t in b.ints.numpy()[2 + n + 1: 2 + n + 1 + steps]]
    assert got_tok == want_tok
    assert rel_err(b.k_cache.numpy(), a.k_cache.numpy()) < 1e-5
    # and generate_persistent replays the same sequence from the same start
    b.fill_cache(k, v)
    assert b.generate_persistent(1, n, steps) == want_tok


def test_persistent_step_rejects_too_few_workgroups(gpu):
    """The host checks the launch before it is made: 64 workgroups cannot hold the
    step's phases (it needs at least 128 workgroups, and 112 attention items at this cache)."""
    from cv3amd.qwen2 import DeviceQwen2
    _, dev, _, _ = _setup(2, "per_channel", 0)
    d = DeviceQwen2(dev, cap=1024)
    d.begin(1, 0)
    d.step_persistent()
    d._persist.workgroups = 64
    with pytest.raises(NotImplementedError):
        d.step_persistent()


@pytest.mark.parametrize("strict", [False, True])
def test_persistent_sampled_generation(gpu, strict):
    """The one-launch step followed by the device sampler: the oracle's sampled tokens and
    Generator state (llm.py:104-149), including a stop on a control id (a head bias makes
    the eos id and another stop id likely; min_len holds back the eos id, or every stop
    id with strict_min_len)."""
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    from oracle.llm import Sampling
    n, max_len, min_len = 512, 48, 6
    t = synth.quantize_store(synth.qwen2_tensors(layers=2), "per_channel", oracle.quant.quantize_q8)
    sts = synth.SPEECH_TOKEN_SIZE
    bias = np.array(t["llm.llm_decoder.bias"], np.float32)
    bias[sts] += 9.0
    bias[sts + 5] += 4.0
    t["llm.llm_decoder.bias"] = bias
    meta = synth.qwen2_meta(layers=2)
    cpu, dev = WeightStore(t, meta, oracle.quant.QTensor), WeightStore(t, meta, cv3amd.quant.QTensor)
    rng = np.random.default_rng(100)
    k = rng.standard_normal((2, 2, n, 64), dtype=np.float32)
    v = rng.standard_normal((2, 2, n, 64), dtype=np.float32)
    lm, cache = _oracle_lm(cpu, k, v, n, max_len)
    ref = Sampling(seed=77, strict_min_len=strict)
    want = lm.sampled(lm.speech_emb([lm.sos]), cache, max_len, min_len, ref)
    print(f"[persist] sampled, strict={strict}: oracle stops after {len(want)} tokens", flush=True)
    assert (min_len <= len(want) < max_len) if strict else (0 < len(want) < min_len)
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    cfg = Sampling(seed=77, strict_min_len=strict)
    got = d.generate_sampled(lm.sos, n, max_len, min_len, cfg, sts, check_every=5, persistent=True)
    assert got == want
    assert cfg.rng.bit_generator.state == ref.rng.bit_generator.state


@pytest.mark.parametrize("profile", ["balanced", "per_channel"])
def test_persistent_sampled_long_run_matches_five_kernel_step(gpu, profile):
    """40 draws with SamplingConfig's defaults over 24 layers: the same tokens and
    Generator state as the five-kernel sampled step (per-channel: phase D on the matrix cores)."""
    from cv3amd.qwen2 import DeviceQwen2
    from oracle.llm import Sampling
    n, max_len = 200, 40
    _, dev, k, v = _setup(24, profile, n)
    out = []
    for persistent in (False, True):
        d = DeviceQwen2(dev, cap=1024)
        d.fill_cache(k, v)
        cfg = Sampling(seed=5)
        toks = d.generate_sampled(1, n, max_len, 0, cfg, 6561, persistent=persistent)
        out.append((toks, cfg.rng.bit_generator.state))
    print(f"[persist] sampled 24 layers: {out[0][0][:10]}...", flush=True)
    assert out[0][0] == out[1][0]
    assert out[0][1] == out[1][1]


def test_persistent_error_flag_ends_the_launch_and_raises(gpu):
    """A flag already set (as after a wait that gave up) makes every wait of the next launch
    give up within 256 polls: the launch ends normally, and the host raises."""
    from cv3amd.qwen2 import DeviceQwen2
    _, dev, k, v = _setup(2, "per_channel", 64)
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    d.begin(1, 64)
    d.step_persistent()                      # allocates the exchange words and the flag
    assert not d.persistent_error()
    d._perr.copy_from(np.ones(1, np.int64))  # the host sets the flag
    d.step_persistent()
    assert d.persistent_error()
    with pytest.raises(RuntimeError):
        d.generate_persistent(1, 64, 2)


def test_persistent_epoch_counter_wrap(gpu):
    """The launch counter wraps at 2^32 / 256 launches: the host clears the words and starts
    again at 256; the tokens stay the oracle's."""
    from cv3amd.qwen2 import DeviceQwen2
    n, steps = 200, 6
    cpu, dev, k, v = _setup(2, "per_channel", n)
    lm, cache = _oracle_lm(cpu, k, v, n, steps)
    x = lm.speech_emb([lm.sos])
    want = []
    for _ in range(steps):
        top = int(np.argmax(lm.head(lm.body.forward(x, cache)[-1:])[0]))
        want.append(top)
        x = lm.speech_emb([top])
    d = DeviceQwen2(dev, cap=1024)
    d.fill_cache(k, v)
    d.begin(lm.sos, n)
    d.step_persistent()
    d._persist.epoch_base = 0xFFFFFF00 - 256   # the next launch takes the last base, the one after wraps
    for _ in range(steps - 1):
        d.step_persistent()
    assert d._persist.epoch_base == 256 * (steps - 2)
    assert not d.persistent_error()
    assert [int(t) for t in d.ints.numpy()[2 + n + 1: 2 + n + 1 + steps]] == want
