"""Pin the oracle's model call sequences against frozen upstream PyTorch outputs.

The toy checkpoint and ``reference_io.npz`` are the reference's own fixtures
(tests/fixtures), converted by tests/golden/make_golden.py.  Tolerances are the
reference's (tests/test_reference.py:99-169).
"""

import numpy as np
import pytest

from conftest import rel_err
from oracle.flow import Flow
from oracle.hift import HiFTGenerator
from oracle.llm import CosyVoice3LM
from oracle.torch_rng import TorchMT19937


def test_flow_matches_frozen_upstream(toy_oracle_store, reference_io):
    got = Flow(toy_oracle_store, "flow.").inference(
        reference_io["token"], reference_io["prompt_token"], reference_io["prompt_feat"],
        reference_io["embedding"])
    ref = reference_io["flow_mel"]
    assert got.shape == ref.shape
    assert rel_err(got, ref) < 5e-4


def _hift(store, n_mel):
    h = HiFTGenerator(store, "hift.")
    n = 480 * n_mel
    h.set_source_noise(TorchMT19937(0).random_float32(n * 9).reshape(n, 9))
    return h


def test_vocoder_matches_frozen_upstream(toy_oracle_store, reference_io):
    n_mel = toy_oracle_store.meta["fixture_config"]["n_mel"]
    got = _hift(toy_oracle_store, n_mel).inference(reference_io["mel"], chunk=None)
    ref = reference_io["hift_wav"]
    assert got.shape == ref.shape
    assert rel_err(got, ref) < 2e-3


def test_vocoder_chunked_equals_full(toy_oracle_store, reference_io):
    n_mel = toy_oracle_store.meta["fixture_config"]["n_mel"]
    h = _hift(toy_oracle_store, n_mel)
    full = h.inference(reference_io["mel"], chunk=None)
    chunked = h.inference(reference_io["mel"], chunk=8, context=64)
    assert rel_err(chunked, full) < 1e-5


def test_llm_logits_match_frozen_upstream(toy_oracle_store, reference_io):
    lm = CosyVoice3LM(toy_oracle_store, "llm.")
    emb = np.concatenate([lm.speech_emb([lm.sos]), lm.text_emb(reference_io["text"]),
                          lm.speech_emb([lm.task_id]), lm.speech_emb(reference_io["prompt_speech"])], axis=0)
    cache = lm.body.new_cache()
    forced = list(reference_io["forced"])
    step_in = emb
    for i, ref in enumerate(reference_io["llm_logits"]):
        got = lm.head(lm.body.forward(step_in, cache)[-1:])[0]
        assert rel_err(got, ref) < 1e-3, f"decode step {i}"
        if i < len(forced):
            step_in = lm.speech_emb([int(forced[i])])


def test_incremental_equals_full_pass(toy_oracle_store):
    lm = CosyVoice3LM(toy_oracle_store, "llm.")
    x = np.random.default_rng(0).normal(size=(17, lm.cfg.hidden_size)).astype(np.float32) * 0.2
    full = lm.body.forward(x)
    cache = lm.body.new_cache()
    parts = [lm.body.forward(x[:5], cache)] + [lm.body.forward(x[i:i + 1], cache) for i in range(5, 17)]
    assert rel_err(np.concatenate(parts), full) < 5e-5


def test_flow_rejects_overlong_utterance(toy_oracle_store):
    with pytest.raises(ValueError, match="noise"):
        Flow(toy_oracle_store, "flow.").rand_noise(15001)


# -- the sampler (llm.py:37-49,125-149) -------------------------------------------

def _logp(logits):
    import oracle.ops as ops
    return ops.log_softmax(np.asarray(logits, np.float32)[None], axis=-1)[0]


def test_sampler_top_k_one_is_the_stable_argmax():
    from oracle.llm import Sampling, sample
    logits = np.zeros(300, np.float32)
    logits[[17, 40, 41]] = 3.0   # a three-way tie: the stable order puts 17 first
    cfg = Sampling(top_k=1, seed=7)
    fresh = np.random.default_rng(7)
    assert sample(_logp(logits), [], cfg, False, False, 250) == 17
    fresh.random()               # exactly one draw was taken
    assert cfg.rng.bit_generator.state == fresh.bit_generator.state


def test_nucleus_cut_by_hand():
    """probs 0.5 / 0.3 / 0.15 / 0.05: top_p 0.8 keeps two entries (the sum reaches 0.8
    after the second), top_p 0.5 keeps one; the draw is u < cdf by hand."""
    from oracle.llm import nucleus_sampling
    probs = np.array([0.5, 0.3, 0.15, 0.05], np.float32)
    idx = np.array([9, 4, 7, 1])
    for seed in range(40):
        u = np.random.default_rng(seed).random()
        p = probs[:2].astype(np.float64)
        want = 9 if u < (p[0] / p.sum()) / ((p[0] / p.sum()) + (p[1] / p.sum())) else 4
        assert nucleus_sampling(probs, idx, np.random.default_rng(seed), 0.8, 25) == want
        assert nucleus_sampling(probs, idx, np.random.default_rng(seed), 0.5, 25) == 9
        assert nucleus_sampling(probs, idx, np.random.default_rng(seed), 0.99, 3) in (9, 4, 7)


def test_sampler_draws_match_numpy_choice():
    """The nucleus draw is Generator.choice over the renormalised head of the stable order."""
    import oracle.ops as ops
    from oracle.llm import Sampling, sample
    rng = np.random.default_rng(3)
    for seed in range(20):
        logits = (rng.standard_normal(500) * 2).astype(np.float32)
        logp = _logp(logits)
        cfg = Sampling(top_p=0.8, top_k=25, seed=seed)
        probs = ops.softmax(logp.copy())
        order = np.argsort(-probs, kind="stable")
        cum, n = 0.0, 0
        while n < 25 and cum < 0.8:
            cum += float(probs[order[n]])
            n += 1
        p = probs[order[:n]].astype(np.float64)
        want = int(order[np.random.default_rng(seed).choice(n, p=p / p.sum())])
        assert sample(logp, [], cfg, False, False, 450) == want


def test_resample_never_returns_the_repeated_pick():
    from oracle.llm import Sampling, sample
    logits = np.full(300, -30.0, np.float32)
    logits[5] = 0.0
    logits[6] = -1.0
    cfg = Sampling(top_k=1, win_size=10, tau_r=0.1, seed=1)
    picks = [sample(_logp(logits), [5, 3], cfg, False, False, 250) for _ in range(50)]
    assert 5 not in picks and picks.count(6) > 40     # 6 dominates once 5 is masked
    cfg = Sampling(top_k=1, win_size=10, tau_r=0.1, seed=1)
    assert sample(_logp(logits), [3, 4], cfg, False, False, 250) == 5   # no repeat: no resample


def test_eos_masks_below_min_len():
    from oracle.llm import Sampling, sample
    logits = np.full(460, -5.0, np.float32)
    logits[250] = 10.0     # speech_token_size: the eos the reference masks
    logits[251] = 9.0      # another stop id
    logits[3] = 0.0
    cfg = Sampling(top_k=1, seed=2)
    assert sample(_logp(logits), [], cfg, False, False, 250) == 250
    assert sample(_logp(logits), [], cfg, True, False, 250) == 251
    assert sample(_logp(logits), [], cfg, True, True, 250) == 3
