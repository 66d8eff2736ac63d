"""CPU oracle: a NumPy restatement of the reference's tensor-kernel layer.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and there only as the
checker (or the CPU timing baseline), never as the thing being measured.

Every function cites the reference file:line whose semantics it restates
(paths relative to the reference repository root, ``cv3cpu/...``).

Modules
-------
``ops``        the elementwise / norm / linear / conv / attention / STFT kernels
               (cv3cpu/ops.py)
``quant``      block int8 / int4 quantisation, ``QTensor``, ``qmatmul``
               (cv3cpu/quant.py)
``torch_rng``  PyTorch CPU MT19937 replica (cv3cpu/torch_rng.py)
``dit``        DiT estimator call sequence (cv3cpu/models/dit.py)
``flow``       Euler CFM solver + token front (cv3cpu/models/flow.py)
``qwen2``      Qwen2 body with KV cache (cv3cpu/models/qwen2.py)
``llm``        LM head, speech embedding, sampler, greedy / sampled decode
               (cv3cpu/models/llm.py)
``hift``       HiFTNet vocoder (cv3cpu/models/hift.py)

How each function is pinned (golden vector, closed form, invariant or brute
force) is listed in ``PINNING`` below; the tests under ``tests/`` enforce it.
"""

# function -> how the tests pin it.  Every entry names the test that fails on
# a plausible mistake (dropped term, wrong sign/index, transposed operand).
PINNING = {
    "ops.silu/sigmoid/gelu_tanh/gelu/mish/elu/leaky_relu": "scalar math definitions (test_oracle_ops)",
    "ops.snake": "closed form with per-channel alpha (test_oracle_ops)",
    "ops.softmax/log_softmax": "fp64 log-sum-exp, normalisation (test_oracle_ops)",
    "ops.rms_norm/layer_norm": "fp64 per-row definitions (test_oracle_ops)",
    "ops.linear/quant.qmatmul": "fp64 brute-force x@W.T; tile/thread invariance (test_oracle_quant)",
    "ops.embedding": "row gather equality + IndexError bounds (test_oracle_ops)",
    "ops.conv1d/depthwise_conv1d": "direct fp64 quadruple loop over 6 geometries x 2 tile sizes (test_oracle_ops)",
    "ops.sdpa": "materialised fp64 softmax attention, causal/chunk/GQA/offset (test_oracle_ops)",
    "ops.stft/istft/hann_window": "direct DFT, COLA round trip, length rule, Hann values (test_oracle_ops)",
    "ops.interpolate_linear/nearest": "half-pixel closed form, repeat equality (test_oracle_ops)",
    "quant.quantize_q8/q4": "closed-form invariants: |q|<=127, extreme->+-127, zero rows, padding, f16 RNE (test_oracle_quant)",
    "torch_rng": "frozen torch.randn/rand samples from the reference's reference_values.json (test_oracle_rng)",
    "dit+flow": "frozen upstream flow_mel at toy geometry, <5e-4 (test_oracle_models)",
    "hift": "frozen upstream hift_wav at toy geometry, <2e-3; chunked==full (test_oracle_models)",
    "qwen2+llm": "frozen upstream per-step logits, <1e-3; incremental==full (test_oracle_models)",
    "llm.sample/nucleus_sampling": "top_k=1 is the stable argmax; the nucleus cut by hand on a fixed "
                                   "distribution; draws against numpy's own Generator.choice on the same "
                                   "PCG64 stream; the resample never returns the masked pick; eos masks "
                                   "(test_oracle_models)",
}
