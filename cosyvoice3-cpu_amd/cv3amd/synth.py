"""Synthetic, seeded weights and inputs at the reference's model geometries.

There is no checkpoint on the measurement machines, so the benchmarks and the
full-size parity tests run on random weights of the real architecture.  The
conventions follow the reference's dummy-model generator
(tools/make_dummy_model.py:35-56): every tensor has its own generator seeded
from the tensor's name (crc32, so any subset -- a few DiT blocks, one Qwen2
layer -- is reproducible on its own), weights and biases are
``standard_normal * 0.02`` in float32, and normalisation scales are ones
(tools/make_dummy_model.py:88-90,179-180).

Tensor names are the reference's (cv3cpu/models/dit.py:86-180,
cv3cpu/models/qwen2.py:139-179, cv3cpu/models/llm.py:68-77).  Quantised
profiles follow cv3cpu/convert.py:25-49,255-265: under ``balanced`` every large
matrix is q8 (block 64, float16 scales) except time_embed / proj_out, which are
narrowed to float16, and conv_pos / biases / norms, which stay float32.  The
``per_channel`` profile is the same q8 algorithm with one float32 scale per
output row (block = K).  ``tiny`` is ``balanced`` with the Qwen2 body layers in
q4 (block 32, float16 scales), as the reference's tiny profile stores them.
"""

from __future__ import annotations

import re
import zlib
from typing import Dict

import numpy as np

QWEN2_05B = dict(hidden_size=896, num_hidden_layers=24, num_attention_heads=14, num_key_value_heads=2,
                 intermediate_size=4864, rms_norm_eps=1e-6, rope_theta=1000000.0, vocab_size=151936)
SPEECH_TOKEN_SIZE = 6561
LM_HEAD_ROWS = SPEECH_TOKEN_SIZE + 200          # tools/make_dummy_model.py:26
DIT_META = dict(dim=1024, depth=22, heads=16, dim_head=64, static_chunk_size=50,
                num_decoding_left_chunks=-1, conv_pos_kernel=31, conv_pos_groups=16)
FLOW_META = dict(token_mel_ratio=2, pre_lookahead_len=3, output_size=80, inference_cfg_rate=0.7,
                 n_timesteps=10)

_KEEP_F32 = re.compile(r"(\.bias$)|(layernorm)|(\.norm$)|(alpha)|(conv_pos_embed)|(spk_embed_affine)")
_KEEP_F16 = re.compile(r"(proj_out)|(time_embed)")


def tensor(name: str, shape, seed: int = 0, scale: float = 0.02, ones: bool = False) -> np.ndarray:
    """float32 N(0, scale^2) tensor seeded by (seed, crc32(name)); ones for norms."""
    if ones:
        return np.ones(shape, np.float32)
    rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
    return rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)


def dit_tensors(depth: int = 22, dim: int = 1024, ff_mult: int = 2, mel: int = 80, seed: int = 0,
                prefix: str = "flow.decoder.estimator.", conv_k: int = 31, conv_groups: int = 16
                ) -> Dict[str, np.ndarray]:
    """float32 DiT estimator weights (cv3cpu/models/dit.py:86-180)."""
    shapes = {
        "time_embed.time_mlp.0.weight": (dim, 256), "time_embed.time_mlp.0.bias": (dim,),
        "time_embed.time_mlp.2.weight": (dim, dim), "time_embed.time_mlp.2.bias": (dim,),
        "input_embed.proj.weight": (dim, 4 * mel), "input_embed.proj.bias": (dim,),
        "norm_out.linear.weight": (2 * dim, dim), "norm_out.linear.bias": (2 * dim,),
        "proj_out.weight": (mel, dim), "proj_out.bias": (mel,),
    }
    for c in ("conv1", "conv2"):
        shapes[f"input_embed.conv_pos_embed.{c}.0.weight"] = (dim, dim // conv_groups, conv_k)
        shapes[f"input_embed.conv_pos_embed.{c}.0.bias"] = (dim,)
    for i in range(depth):
        b = f"transformer_blocks.{i}."
        shapes[b + "attn_norm.linear.weight"] = (6 * dim, dim)
        shapes[b + "attn_norm.linear.bias"] = (6 * dim,)
        for p in ("to_q", "to_k", "to_v", "to_out.0"):
            shapes[b + f"attn.{p}.weight"] = (dim, dim)
            shapes[b + f"attn.{p}.bias"] = (dim,)
        shapes[b + "ff.ff.0.0.weight"] = (ff_mult * dim, dim)
        shapes[b + "ff.ff.0.0.bias"] = (ff_mult * dim,)
        shapes[b + "ff.ff.2.weight"] = (dim, ff_mult * dim)
        shapes[b + "ff.ff.2.bias"] = (dim,)
    return {prefix + k: tensor(prefix + k, s, seed) for k, s in shapes.items()}


def dit_meta(depth: int = 22, dim: int = 1024, heads: int = 16, dim_head: int = 64) -> dict:
    return {"dit": dict(DIT_META, depth=depth, dim=dim, heads=heads, dim_head=dim_head),
            "flow": dict(FLOW_META)}


HIFT_META = dict(upsample_rates=[8, 5, 3], upsample_kernel_sizes=[16, 11, 7], resblock_kernel_sizes=[3, 7, 11],
                 resblock_dilation_sizes=[[1, 3, 5]] * 3, source_resblock_kernel_sizes=[7, 7, 11],
                 source_resblock_dilation_sizes=[[1, 3, 5]] * 3, istft_n_fft=16, istft_hop_len=4,
                 lrelu_slope=0.1, audio_limit=0.99, sampling_rate=24000, nb_harmonics=8, nsf_alpha=0.1,
                 nsf_sigma=0.003, nsf_voiced_threshold=10.0, conv_pre_look_right=4)


def hift_tensors(base: int = 512, f0_ch: int = 512, mel: int = 80, seed: int = 0,
                 prefix: str = "hift.") -> Dict[str, np.ndarray]:
    """float32 HiFTNet weights, weight-norm already folded (cv3cpu/convert.py:52-76),
    Snake alphas ones (cv3cpu/models/hift.py:19-218, tools/make_dummy_model.py:88-90)."""
    m = HIFT_META
    n_fft = m["istft_n_fft"]
    shapes = {"conv_pre.weight": (base, mel, 5), "conv_pre.bias": (base,),
              "conv_post.weight": (n_fft + 2, base // 8, 7), "conv_post.bias": (n_fft + 2,),
              "m_source.l_linear.weight": (1, m["nb_harmonics"] + 1), "m_source.l_linear.bias": (1,),
              "f0_predictor.classifier.weight": (1, f0_ch), "f0_predictor.classifier.bias": (1,)}
    for i in range(5):
        shapes[f"f0_predictor.condnet.{i}.weight"] = (f0_ch, mel if i == 0 else f0_ch, 4 if i == 0 else 3)
        shapes[f"f0_predictor.condnet.{i}.bias"] = (f0_ch,)
    downs = [1] + m["upsample_rates"][::-1][:-1]
    down_cum = list(np.cumprod(downs))[::-1]
    ones = []
    for i, (r, k) in enumerate(zip(m["upsample_rates"], m["upsample_kernel_sizes"])):
        cin, cout = base // (2 ** i), base // (2 ** (i + 1))
        shapes[f"ups.{i}.weight"] = (cout, cin, k)
        shapes[f"ups.{i}.bias"] = (cout,)
        u = int(down_cum[i])
        shapes[f"source_downs.{i}.weight"] = (cout, n_fft + 2, 2 * u if u > 1 else 1)
        shapes[f"source_downs.{i}.bias"] = (cout,)
        groups = [("source_resblocks", i, m["source_resblock_kernel_sizes"][i])]
        groups += [("resblocks", i * 3 + j, kj) for j, kj in enumerate(m["resblock_kernel_sizes"])]
        for g, idx, kk in groups:
            for j in range(3):
                for c in ("convs1", "convs2"):
                    shapes[f"{g}.{idx}.{c}.{j}.weight"] = (cout, cout, kk)
                    shapes[f"{g}.{idx}.{c}.{j}.bias"] = (cout,)
                for a in ("activations1", "activations2"):
                    shapes[f"{g}.{idx}.{a}.{j}.alpha"] = (cout,)
                    ones.append(f"{g}.{idx}.{a}.{j}.alpha")
    return {prefix + k: tensor(prefix + k, sh, seed, ones=k in ones) for k, sh in shapes.items()}


def hift_meta() -> dict:
    return {"hift": dict(HIFT_META)}


def qwen2_tensors(layers: int = 24, hidden: int = 896, heads: int = 14, kv_heads: int = 2,
                  inter: int = 4864, head_rows: int = LM_HEAD_ROWS, seed: int = 0,
                  prefix: str = "llm.") -> Dict[str, np.ndarray]:
    """float32 Qwen2 body + LM head / speech embedding (cv3cpu/models/qwen2.py:139-179,
    cv3cpu/models/llm.py:68-77).  Norm weights are ones."""
    hd = hidden // heads
    out = {}
    body = prefix + "model."
    for i in range(layers):
        p = f"{body}layers.{i}."
        shapes = {
            "self_attn.q_proj.weight": (heads * hd, hidden), "self_attn.q_proj.bias": (heads * hd,),
            "self_attn.k_proj.weight": (kv_heads * hd, hidden), "self_attn.k_proj.bias": (kv_heads * hd,),
            "self_attn.v_proj.weight": (kv_heads * hd, hidden), "self_attn.v_proj.bias": (kv_heads * hd,),
            "self_attn.o_proj.weight": (hidden, heads * hd),
            "mlp.gate_proj.weight": (inter, hidden), "mlp.up_proj.weight": (inter, hidden),
            "mlp.down_proj.weight": (hidden, inter),
        }
        for k, s in shapes.items():
            out[p + k] = tensor(p + k, s, seed)
        out[p + "input_layernorm"] = tensor(p + "input_layernorm", (hidden,), ones=True)
        out[p + "post_attention_layernorm"] = tensor(p + "post_attention_layernorm", (hidden,), ones=True)
    out[body + "norm"] = tensor(body + "norm", (hidden,), ones=True)
    out[prefix + "llm_decoder.weight"] = tensor(prefix + "llm_decoder.weight", (head_rows, hidden), seed)
    out[prefix + "llm_decoder.bias"] = tensor(prefix + "llm_decoder.bias", (head_rows,), seed)
    out[prefix + "speech_embedding"] = tensor(prefix + "speech_embedding", (head_rows, hidden), seed)
    return out


def qwen2_meta(layers: int = 24, hidden: int = 896, heads: int = 14, kv_heads: int = 2,
               inter: int = 4864) -> dict:
    return {"qwen2": dict(QWEN2_05B, hidden_size=hidden, num_hidden_layers=layers, num_attention_heads=heads,
                          num_key_value_heads=kv_heads, intermediate_size=inter),
            "speech_token_size": SPEECH_TOKEN_SIZE}


def choose_kind(name: str, arr: np.ndarray, profile: str) -> str:
    """Storage kind of one tensor under a profile (cv3cpu/convert.py:255-265).

    ``f32``: everything float32.  ``balanced``: q8 block 64 / float16 scales for
    large matrices, float16 for time_embed / proj_out.  ``per_channel``: like
    balanced, with one float32 scale per output row (``per_channel_f16``: one float16
    scale per row, the reference's scale dtype at block = K).  ``tiny``: like balanced, with
    q4 for the matrices of ``llm.model.layers.*`` (convert.py:26-27,262-263).
    """
    if profile == "f32" or arr.ndim == 1 or _KEEP_F32.search(name) or arr.size < (1 << 16):
        return "f32"
    if _KEEP_F16.search(name):
        return "f16"
    if arr.ndim == 3:
        return "f32"   # grouped / conv weights stay float32 on this path
    if profile == "tiny" and (name.startswith("llm.model.layers.") or name == "llm.model.embed_tokens"):
        return "q4"
    return "q8"


def quantize_store(tensors: Dict[str, np.ndarray], profile: str, quantize_q8, quantize_q4=None) -> Dict[str, object]:
    """Apply a profile: q8 / q4 entries become ``{"kind","q","scales","shape","block"}``
    records, float16 entries are narrowed.  ``quantize_q8(w, block, scale_dtype)`` and
    ``quantize_q4(w)`` do the work, so the same inputs can be quantised by the device
    kernels or by a restatement."""
    out: Dict[str, object] = {}
    for name, arr in tensors.items():
        kind = choose_kind(name, arr, profile)
        if kind == "q4":
            if quantize_q4 is None:
                raise ValueError(f"profile {profile!r} needs a q4 quantiser")
            q, s, kp = quantize_q4(arr)
            out[name] = {"kind": "q4", "q": np.asarray(q), "scales": np.asarray(s), "shape": arr.shape,
                         "block": 32, "orig_shape": None}
        elif kind == "q8":
            k = arr.shape[1]
            if profile in ("per_channel", "per_channel_f16"):
                q, s, kp = quantize_q8(arr, k, np.float32 if profile == "per_channel" else np.float16)
                block = k
            else:
                q, s, kp = quantize_q8(arr, 64, np.float16)
                block = 64
            out[name] = {"kind": "q8", "q": np.asarray(q), "scales": np.asarray(s), "shape": arr.shape,
                         "block": block, "orig_shape": None}
        elif kind == "f16":
            out[name] = arr.astype(np.float16)
        else:
            out[name] = arr
    return out
