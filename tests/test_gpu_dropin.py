"""Drop-in proof: the model call sequences with ``ops.*`` rebound to the HIP backend.

The reference's models resolve ``ops.<name>`` on the module object at call time
(cv3cpu/models/dit.py:9 etc.), so rebinding the module attributes redirects
every kernel call.  Here the restated call sequences (oracle/dit.py, flow.py,
qwen2.py, llm.py, hift.py) run with ``oracle.ops`` rebound to ``cv3amd.ops``
on the reference's toy checkpoint, and must reproduce both the frozen upstream
PyTorch outputs (the reference's own tolerances) and the all-CPU oracle run
(1e-4, the flow/vocoder parity bar).
"""

import contextlib

import numpy as np
import pytest

from conftest import load_toy, rel_err

pytestmark = pytest.mark.gpu

NAMES = ["silu", "sigmoid", "gelu_tanh", "gelu", "mish", "elu", "leaky_relu", "snake", "softmax",
         "log_softmax", "rms_norm", "layer_norm", "linear", "embedding", "conv1d", "depthwise_conv1d",
         "sdpa", "interpolate_linear", "interpolate_nearest", "stft", "istft"]


@contextlib.contextmanager
def hip_ops():
    import oracle.ops as target
    import cv3amd.ops as hip
    saved = {n: getattr(target, n) for n in NAMES}
    try:
        for n in NAMES:
            setattr(target, n, getattr(hip, n))
        yield
    finally:
        for n, f in saved.items():
            setattr(target, n, f)


@pytest.fixture(scope="module")
def stores(gpu):
    import oracle.quant
    import cv3amd.quant
    return load_toy(oracle.quant.QTensor), load_toy(cv3amd.quant.QTensor)


def test_flow_dropin(stores, reference_io):
    from oracle.flow import Flow
    cpu_store, hip_store = stores
    args = (reference_io["token"], reference_io["prompt_token"], reference_io["prompt_feat"],
            reference_io["embedding"])
    want = Flow(cpu_store, "flow.").inference(*args)
    with hip_ops():
        got = Flow(hip_store, "flow.").inference(*args)
    assert rel_err(got, reference_io["flow_mel"]) < 5e-4
    assert rel_err(got, want) < 1e-4


def test_vocoder_dropin(stores, reference_io):
    from oracle.hift import HiFTGenerator
    from oracle.torch_rng import TorchMT19937
    cpu_store, hip_store = stores
    n = 480 * cpu_store.meta["fixture_config"]["n_mel"]
    noise = TorchMT19937(0).random_float32(n * 9).reshape(n, 9)

    def run(store, chunk):
        h = HiFTGenerator(store, "hift.")
        h.set_source_noise(noise)
        return h.inference(reference_io["mel"], chunk=chunk)

    want = run(cpu_store, None)
    with hip_ops():
        got = run(hip_store, None)
        got_chunked = run(hip_store, 8)
    assert rel_err(got, reference_io["hift_wav"]) < 2e-3
    assert rel_err(got, want) < 1e-4
    assert rel_err(got_chunked, got) < 1e-5


def test_llm_dropin(stores, reference_io):
    from oracle.llm import CosyVoice3LM
    _, hip_store = stores
    with hip_ops():
        lm = CosyVoice3LM(hip_store, "llm.")
        emb = np.concatenate([lm.speech_emb([lm.sos]), lm.text_emb(reference_io["text"]),
                              lm.speech_emb([lm.task_id]), lm.speech_emb(reference_io["prompt_speech"])])
        cache = lm.body.new_cache()
        forced = list(reference_io["forced"])
        step = emb
        for i, ref in enumerate(reference_io["llm_logits"]):
            got = lm.head(lm.body.forward(step, cache)[-1:])[0]
            assert rel_err(got, ref) < 1e-3, f"decode step {i}"
            if i < len(forced):
                step = lm.speech_emb([int(forced[i])])
