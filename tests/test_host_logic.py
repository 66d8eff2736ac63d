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


def _vocoder_receptive_case():
    import oracle.quant
    from oracle.hift import HiFTGenerator
    from cv3amd import synth
    from cv3amd.hift import receptive_frames
    from cv3amd.weights import WeightStore
    m = synth.hift_meta()["hift"]
    t = synth.hift_tensors(base=64, f0_ch=64)
    h = HiFTGenerator(WeightStore(t, synth.hift_meta(), oracle.quant.QTensor), "hift.")
    rates = m["upsample_rates"]
    R = receptive_frames(rates, m["upsample_kernel_sizes"], m["resblock_kernel_sizes"], m["resblock_dilation_sizes"],
                         m["source_resblock_kernel_sizes"], m["source_resblock_dilation_sizes"],
                         [t[f"hift.source_downs.{i}.weight"].shape[2] for i in range(len(rates))],
                         t["hift.conv_post.weight"].shape[2])
    return h, R


def test_vocoder_receptive_field_bounds_what_a_frame_reads():
    """The windowed vocoder's history is cut to the stack's receptive field (receptive_frames):
    on the oracle's stack, a large change to every mel frame and source-STFT frame before that
    field leaves the samples of the frame after it unchanged, bit for bit; the field is not far
    too large (the mel 19 frames back and the source STFT 28 frames back still reach the frame,
    so a bound that dropped the source branch or a resblock fails)."""
    h, R = _vocoder_receptive_case()
    assert R == 29   # for this geometry: the source branch of the first stage reaches furthest
    rng = np.random.default_rng(1)
    T, m0, up = 80, 50, 120
    mel = (rng.standard_normal((80, T), dtype=np.float32) * 2 - 5).astype(np.float32)
    src = np.tanh(rng.standard_normal(480 * T, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    s = h.source_stft(src)
    base = h.spectral(mel, s)
    r0 = 1 + m0 * up               # the frame's first output row

    def changed(mel2, s2):
        return np.abs(h.spectral(mel2, s2)[:, r0:] - base[:, r0:]).max() > 0

    m2 = mel.copy()
    m2[:, :m0 - R] += 1e5
    s2 = s.copy()
    s2[:, :(m0 - R) * up] += 1e5
    assert not changed(m2, s)
    assert not changed(mel, s2)
    m3 = mel.copy()
    m3[:, m0 - 19] += 1e5
    assert changed(m3, s)
    s3 = s.copy()
    s3[:, (m0 - 28) * up:(m0 - 27) * up] += 1e5
    assert changed(mel, s3)


def test_vocoder_windows_with_receptive_history_equal_the_full_context():
    """The reference's windowed decode (hift.py:170-194) with the receptive field as its history
    gives the samples it gives with 64 frames, and the full-utterance samples."""
    h, R = _vocoder_receptive_case()
    rng = np.random.default_rng(2)
    T = 200
    mel = (rng.standard_normal((80, T), dtype=np.float32) * 2 - 5).astype(np.float32)
    src = np.tanh(rng.standard_normal(480 * T, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    s = h.source_stft(src)
    full = h.spectral_chunked(mel, s, 50, 64)
    assert np.array_equal(h.spectral_chunked(mel, s, 50, R), full)
    assert np.array_equal(h.spectral(mel, s), full)
