"""Oracle restatement of the CFM flow decoder (Euler solve with CFG).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/flow.py.
"""

from __future__ import annotations

import numpy as np

from . import ops
from .dit import DiT
from .torch_rng import randn

NOISE_SHAPE = (1, 80, 50 * 300)   # flow.py:16
NOISE_SEED = 0                     # flow.py:17


def cosine_t_span(steps: int) -> np.ndarray:
    """1 - cos(linspace(0,1,steps+1) pi/2) in float64, stored float32 (flow.py:68-69)."""
    return (1.0 - np.cos(np.linspace(0.0, 1.0, steps + 1, dtype=np.float64) * 0.5 * np.pi)).astype(np.float32)


class Flow:
    def __init__(self, weights, prefix: str = "flow."):
        self.w = weights
        self.p = prefix
        m = weights.meta.get("flow", {})
        self.token_mel_ratio = int(m.get("token_mel_ratio", 2))
        self.pre_lookahead_len = int(m.get("pre_lookahead_len", 3))
        self.output_size = int(m.get("output_size", 80))
        self.inference_cfg_rate = float(m.get("inference_cfg_rate", 0.7))
        self.n_timesteps = int(m.get("n_timesteps", 10))
        self.estimator = DiT(weights, prefix + "decoder.estimator.")
        self._noise = None

    def _t(self, name):
        return self.w.get(self.p + name)

    def rand_noise(self, n: int):
        """First n columns of a fixed torch.randn((1,80,15000)) seed 0 (flow.py:36-43)."""
        if self._noise is None:
            self._noise = randn(NOISE_SHAPE, NOISE_SEED)
        if n > self._noise.shape[2]:
            raise ValueError(f"utterance needs {n} mel frames but the fixed CFM noise only has "
                             f"{self._noise.shape[2]}; split the text into shorter segments")
        return self._noise[:, :, :n]

    def pre_lookahead(self, emb):
        """(T, 80) -> conv (right pad) -> leaky 0.01 -> causal conv -> + input (flow.py:46-56)."""
        x = np.ascontiguousarray(emb.T)
        h = ops.conv1d(x, self._t("pre_lookahead_layer.conv1.weight"),
                       self._t("pre_lookahead_layer.conv1.bias"), pad=(0, self.pre_lookahead_len))
        h = ops.leaky_relu(h, 0.01)
        w2 = self._t("pre_lookahead_layer.conv2.weight")
        k2 = (w2.orig_shape if hasattr(w2, "orig_shape") else w2.shape)[-1]
        h = ops.conv1d(h, w2, self._t("pre_lookahead_layer.conv2.bias"), pad=(k2 - 1, 0))
        return h.T + emb

    def solve_euler(self, mu, spks, cond, streaming=False, temperature=1.0, seq_chunk=512,
                    progress=None, x0=None):
        """Fixed-step Euler with classifier-free guidance (flow.py:58-93).

        The CFG batch holds the conditioned pair in slot 0 and zeros in slot 1;
        dphi = (1+w) d0 - w d1; x += dt dphi; t += dt; dt = t_span[s+1] - t.
        ``x0`` overrides the initial noise (tests only).
        """
        n = mu.shape[2]
        x = (self.rand_noise(n) if x0 is None else x0) * temperature
        t_span = cosine_t_span(self.n_timesteps)
        mu_in = np.zeros((2, 80, n), dtype=np.float32)
        mu_in[0] = mu[0]
        spk_in = np.zeros((2, spks.shape[1]), dtype=np.float32)
        spk_in[0] = spks[0]
        cond_in = np.zeros((2, 80, n), dtype=np.float32)
        cond_in[0] = cond[0]
        w = self.inference_cfg_rate
        t = t_span[0]
        dt = t_span[1] - t_span[0]
        for s in range(1, len(t_span)):
            d = self.estimator.forward(np.broadcast_to(x, (2, 80, n)), mu_in,
                                       np.array([t, t], dtype=np.float32), spk_in, cond_in,
                                       streaming=streaming, seq_chunk=seq_chunk)
            x = x + dt * ((1.0 + w) * d[0:1] - w * d[1:2])
            t = t + dt
            if s < len(t_span) - 1:
                dt = t_span[s + 1] - t
            if progress is not None:
                progress(s, len(t_span) - 1)
        return x.astype(np.float32)

    def inference(self, token, prompt_token, prompt_feat, embedding, streaming=False,
                  seq_chunk=512, progress=None):
        """Tokens (+ prompt) -> mel (80, T) with prompt frames stripped (flow.py:96-128)."""
        e = np.asarray(embedding, dtype=np.float32).reshape(1, -1)
        e = e / np.maximum(np.linalg.norm(e, axis=1, keepdims=True), 1e-12)
        e = ops.linear(e, self._t("spk_embed_affine_layer.weight"), self._t("spk_embed_affine_layer.bias"))
        ids = np.maximum(np.concatenate([np.asarray(prompt_token, dtype=np.int64),
                                         np.asarray(token, dtype=np.int64)]), 0)
        h = self.pre_lookahead(ops.embedding(self._t("input_embedding"), ids))
        h = np.repeat(h, self.token_mel_ratio, axis=0)
        pf = np.asarray(prompt_feat, dtype=np.float32)
        n_prompt = pf.shape[0]
        total = h.shape[0]
        if n_prompt > total:
            raise ValueError("prompt mel is longer than the token grid")
        cond = np.zeros((1, self.output_size, total), dtype=np.float32)
        cond[0, :, :n_prompt] = pf.T
        mu = np.ascontiguousarray(h.T)[None]
        feat = self.solve_euler(mu, e, cond, streaming=streaming, seq_chunk=seq_chunk, progress=progress)
        return feat[0, :, n_prompt:]
