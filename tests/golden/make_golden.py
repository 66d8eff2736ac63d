"""Write the golden fixtures under tests/golden/ from the reference's own data files.

Run once in a container that has the reference checkout (it is not needed at
test time):  python tests/golden/make_golden.py [/root/reference]

Outputs (all data, no code):
  reference_io.npz   copied verbatim from the reference's tests/fixtures: the frozen
                     upstream-PyTorch outputs (flow_mel, hift_wav, llm_logits) and
                     their inputs at toy geometry.
  torch_rng.json     the "torch_rng" section of tests/reference_values.json: frozen
                     torch.randn / torch.rand samples (indices, values, sums).
  toy_weights.npz    the toy checkpoint (tests/fixtures/checkpoint/{llm,flow,hift}.pt)
                     as float32 arrays under the runtime's tensor names, weight-norm
                     folded (w = g v / ||v|| over all but the output axis, computed in
                     fp32, ||v|| floored at 1e-12 like the converter at
                     cv3cpu/convert.py:52-76), plus a "__meta__" JSON string with the
                     model geometry.

The checkpoints are read with torch.load(weights_only=True), which executes
nothing from the file.  Only this generator uses torch.
"""

from __future__ import annotations

import json
import os
import re
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _fold(sd):
    out, used = {}, set()
    for k in list(sd):
        if k.endswith(".weight_g"):
            base, gk, vk = k[:-len(".weight_g")], k, k[:-2] + "_v"
        elif k.endswith(".parametrizations.weight.original0"):
            base = k[:-len(".parametrizations.weight.original0")]
            gk, vk = k, base + ".parametrizations.weight.original1"
        else:
            continue
        g = np.asarray(sd[gk], dtype=np.float32)
        v = np.asarray(sd[vk], dtype=np.float32)
        nrm = np.sqrt((v * v).sum(axis=tuple(range(1, v.ndim)), keepdims=True))
        out[base + ".weight"] = (g / np.maximum(nrm, 1e-12)) * v
        used |= {gk, vk}
    for k, v in sd.items():
        if k not in used:
            out.setdefault(k, v)
    return out


def _llm_names(sd):
    out = {}
    for k, v in sd.items():
        if k.startswith("llm.model.model."):
            t = k[len("llm.model.model."):]
            if t.endswith("layernorm.weight") or t == "norm.weight":
                t = t[:-len(".weight")]
            if t == "embed_tokens.weight":
                t = "embed_tokens"
            out["llm.model." + t] = v
        elif k.startswith("llm.model.lm_head.") or k.startswith("criterion_ce."):
            continue
        elif k == "speech_embedding.weight":
            out["llm.speech_embedding"] = v
        elif k == "llm_embedding.weight":
            out["llm.llm_embedding"] = v
        else:
            out["llm." + k] = v
    return out


def _flow_names(sd):
    return {("flow.input_embedding" if k == "input_embedding.weight" else "flow." + k): v
            for k, v in sd.items()}


def _hift_names(sd):
    out = {}
    skip = {"stft_window", "m_source.uv", "m_source.l_sin_gen.sine_waves", "m_source.l_sin_gen.rand_ini"}
    for k, v in sd.items():
        k = k[len("generator."):] if k.startswith("generator.") else k
        if k.split(".")[0] in ("discriminator", "mpd", "mrd") or k in skip:
            continue
        m = re.match(r"^f0_predictor\.condnet\.(\d+)\.(weight|bias)$", k)
        if m:
            k = f"f0_predictor.condnet.{int(m.group(1)) // 2}.{m.group(2)}"
        out["hift." + k] = v
    return out


def main(ref: str = "/root/reference"):
    import torch  # only this generator needs it

    fx = os.path.join(ref, "tests", "fixtures")
    shutil.copyfile(os.path.join(fx, "reference_io.npz"), os.path.join(HERE, "reference_io.npz"))
    with open(os.path.join(ref, "tests", "reference_values.json")) as fh:
        rv = json.load(fh)
    with open(os.path.join(HERE, "torch_rng.json"), "w") as fh:
        json.dump(rv["torch_rng"], fh, indent=0, sort_keys=True)
    with open(os.path.join(fx, "config.json")) as fh:
        fcfg = json.load(fh)

    def load(name):
        sd = torch.load(os.path.join(fx, "checkpoint", name), map_location="cpu", weights_only=True)
        return {k: v.detach().to(torch.float32).numpy() for k, v in sd.items()}

    tensors = {}
    tensors.update(_llm_names(_fold(load("llm.pt"))))
    tensors.update(_flow_names(_fold(load("flow.pt"))))
    tensors.update(_hift_names(_fold(load("hift.pt"))))
    with open(os.path.join(fx, "checkpoint", "CosyVoice-BlankEN", "config.json")) as fh:
        qcfg = json.load(fh)
    hid = tensors["llm.model.embed_tokens"].shape[1]
    meta = {
        "qwen2": {"hidden_size": hid, "num_hidden_layers": qcfg["num_hidden_layers"],
                  "num_attention_heads": qcfg["num_attention_heads"],
                  "num_key_value_heads": qcfg["num_key_value_heads"],
                  "intermediate_size": qcfg["intermediate_size"], "rms_norm_eps": qcfg["rms_norm_eps"],
                  "rope_theta": qcfg["rope_theta"], "vocab_size": qcfg["vocab_size"]},
        "speech_token_size": int(tensors["flow.input_embedding"].shape[0]),
        "flow": {"token_mel_ratio": 2, "pre_lookahead_len": 3, "output_size": 80,
                 "inference_cfg_rate": 0.7, "n_timesteps": 10},
        "dit": {"dim": fcfg["dim"], "depth": fcfg["depth"], "heads": fcfg["nhead"], "dim_head": fcfg["dhead"],
                "static_chunk_size": 50, "num_decoding_left_chunks": -1, "conv_pos_kernel": 31,
                "conv_pos_groups": 16},
        "hift": {"upsample_rates": [8, 5, 3], "upsample_kernel_sizes": [16, 11, 7],
                 "resblock_kernel_sizes": [3, 7, 11], "resblock_dilation_sizes": [[1, 3, 5]] * 3,
                 "source_resblock_kernel_sizes": [7, 7, 11],
                 "source_resblock_dilation_sizes": [[1, 3, 5]] * 3, "istft_n_fft": 16, "istft_hop_len": 4,
                 "lrelu_slope": 0.1, "audio_limit": 0.99, "sampling_rate": 24000, "nb_harmonics": 8,
                 "nsf_alpha": 0.1, "nsf_sigma": 0.003, "nsf_voiced_threshold": 10.0,
                 "conv_pre_look_right": 4},
        "fixture_config": fcfg,
    }
    arrays = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in tensors.items()
              if not k.endswith("rotary_embed.inv_freq")}
    np.savez_compressed(os.path.join(HERE, "toy_weights.npz"), __meta__=np.array(json.dumps(meta)), **arrays)
    print(f"wrote {len(arrays)} tensors")


if __name__ == "__main__":
    main(*sys.argv[1:])
