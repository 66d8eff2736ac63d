"""Host-side logic of the device harnesses, checked against the oracle on the CPU
(no GPU calls): the Euler t-schedule, sinusoidal time features, rotary tables and
the synthetic-weight profiles."""

import numpy as np
import pytest


def test_euler_schedule_matches_oracle_solver():
    """The (t, dt) sequence the device solve bakes into its kernels is the one the
    oracle's solve_euler loop produces (flow.py:78-90), float32 drift included."""
    import oracle.flow as of
    from cv3amd.dit import euler_schedule
    from cv3amd import synth
    from cv3amd.weights import WeightStore

    seen = []

    class Probe:
        def forward(self, x, mu, t, spks, cond, **kw):
            seen.append(np.asarray(t).copy())
            return np.zeros_like(np.asarray(x))

    f = of.Flow(WeightStore({}, synth.dit_meta(depth=0)), "flow.")
    f.estimator = Probe()
    T = 4
    f.solve_euler(np.zeros((1, 80, T), np.float32), np.zeros((1, 80), np.float32),
                  np.zeros((1, 80, T), np.float32), x0=np.zeros((1, 80, T), np.float32))
    ts, dts = euler_schedule(10)
    assert len(seen) == 10
    for s in range(10):
        assert seen[s].dtype == np.float32 and np.all(seen[s] == ts[s])
    # dt is what moves t: t_{s+1} = t_s + dt_s, and the last dt ends at t_span[-1]
    assert np.all(ts[1:] == (ts[:-1] + dts[:-1]).astype(np.float32))
    assert np.isclose(float(ts[-1] + dts[-1]), 1.0, atol=1e-6)


def test_sinus_features_match_oracle():
    from oracle.dit import sinus_position_embedding
    from cv3amd.dit import euler_schedule, sinus_features
    ts, _ = euler_schedule(10)
    assert np.array_equal(sinus_features(ts), sinus_position_embedding(ts, 256, 1000.0))


def test_dit_rope_tables_match_oracle():
    from oracle.dit import rope_freqs
    from cv3amd.dit import dit_rope_tables
    c, s = dit_rope_tables(1500, 64)
    f = rope_freqs(1500, 64)
    assert np.array_equal(c, np.cos(f)) and np.array_equal(s, np.sin(f))


def test_balanced_profile_kinds():
    """Which DiT tensors are q8 / f16 / f32 under balanced (cv3cpu/convert.py:36-49,255-265)."""
    from cv3amd.synth import choose_kind
    p = "flow.decoder.estimator."
    w = np.zeros((1024, 1024), np.float32)
    assert choose_kind(p + "transformer_blocks.0.attn.to_q.weight", w, "balanced") == "q8"
    assert choose_kind(p + "transformer_blocks.0.attn.to_q.bias", w[0], "balanced") == "f32"
    assert choose_kind(p + "time_embed.time_mlp.2.weight", w, "balanced") == "f16"
    assert choose_kind(p + "proj_out.weight", np.zeros((80, 1024), np.float32), "balanced") == "f16"
    assert choose_kind(p + "input_embed.conv_pos_embed.conv1.0.weight", np.zeros((1024, 64, 31), np.float32),
                       "balanced") == "f32"
    assert choose_kind("llm.model.layers.0.input_layernorm", np.ones(896, np.float32), "balanced") == "f32"
    assert choose_kind("llm.model.layers.0.mlp.up_proj.weight", np.zeros((4864, 896), np.float32),
                       "per_channel") == "q8"


def test_tiny_profile_kinds():
    """tiny = balanced with the Qwen2 body layers in q4 (cv3cpu/convert.py:26-27,254-264)."""
    from cv3amd.synth import choose_kind
    w = np.zeros((4864, 896), np.float32)
    assert choose_kind("llm.model.layers.3.mlp.up_proj.weight", w, "tiny") == "q4"
    assert choose_kind("llm.model.layers.3.self_attn.k_proj.weight", np.zeros((128, 896), np.float32), "tiny") == "q4"
    assert choose_kind("llm.model.layers.3.self_attn.k_proj.bias", np.zeros(128, np.float32), "tiny") == "f32"
    assert choose_kind("llm.model.layers.3.post_attention_layernorm", np.ones(896, np.float32), "tiny") == "f32"
    assert choose_kind("llm.llm_decoder.weight", np.zeros((6761, 896), np.float32), "tiny") == "q8"
    assert choose_kind("llm.speech_embedding", np.zeros((6761, 896), np.float32), "tiny") == "q8"
    assert choose_kind("flow.decoder.estimator.transformer_blocks.0.ff.ff.0.0.weight", w, "tiny") == "q8"


def test_synthetic_tensors_are_seeded_per_name():
    from cv3amd.synth import dit_tensors, tensor
    a = dit_tensors(depth=1)
    b = dit_tensors(depth=2)
    k = "flow.decoder.estimator.transformer_blocks.0.attn.to_q.weight"
    assert np.array_equal(a[k], b[k])
    assert a[k].dtype == np.float32 and abs(float(a[k].std()) - 0.02) < 1e-3
    assert not np.array_equal(tensor("x", (4,)), tensor("y", (4,)))


def test_widened_q4_codes_dequantise_like_the_packed_ones():
    """The decode harness may hold a q4 body as int8 codes n - 8 with the same 32-code
    blocks and float16 scales: code x scale must equal the q4 dequantisation bit for bit
    (quant.py:70-86), including padded K."""
    import numpy as np
    import oracle.quant as oq
    from cv3amd.qwen2 import widen_q4_codes
    rng = np.random.default_rng(11)
    for rows, k in ((7, 896), (3, 100), (1, 4864)):
        w = (rng.normal(size=(rows, k)) * 0.05).astype(np.float32)
        q, s, kp = oq.quantize_q4(w)
        codes = widen_q4_codes(q)
        assert codes.dtype == np.int8 and codes.shape == (rows, kp)
        assert codes.min() >= -8 and codes.max() <= 7
        mine = codes.astype(np.float32) * np.repeat(s.astype(np.float32), 32, axis=1)
        want = oq.QTensor("q4", q, s, (rows, k), 32).dequant()
        assert np.array_equal(mine[:, :k], want)
