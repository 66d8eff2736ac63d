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
