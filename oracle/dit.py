"""Oracle restatement of the DiT flow-matching estimator call sequence.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/dit.py.  ``weights`` is any object with
``get(name) -> ndarray | QTensor`` and a ``meta`` dict (the reference's
WeightFile interface subset).
"""

from __future__ import annotations

import math

import numpy as np

from . import ops


def sinus_position_embedding(t, dim: int = 256, scale: float = 1000.0):
    """[sin(scale t f), cos(scale t f)], f = exp(-i log(1e4)/(dim/2-1)) in float32 (dit.py:13-18)."""
    half = dim // 2
    f = np.exp(np.arange(half, dtype=np.float32) * -(math.log(10000.0) / (half - 1)))
    arg = scale * np.asarray(t).reshape(-1, 1).astype(np.float32) * f[None, :]
    return np.concatenate([np.sin(arg), np.cos(arg)], axis=-1)


def rope_freqs(seq_len: int, dim_head: int, theta: float = 10000.0):
    """(T, dim_head) angles t*inv_freq, each frequency duplicated interleaved;
    computed in float64 and stored float32 (dit.py:21-29)."""
    inv = 1.0 / (theta ** (np.arange(0, dim_head, 2, dtype=np.float64) / dim_head))
    ang = np.arange(seq_len, dtype=np.float64)[:, None] * inv[None, :]
    return np.repeat(ang, 2, axis=-1).astype(np.float32)


def rotate_pairs(x):
    """GPT-J rotate_half: (a, b) pairs -> (-b, a) (dit.py:32-37)."""
    y = x.reshape(*x.shape[:-1], -1, 2)
    out = np.stack([-y[..., 1], y[..., 0]], axis=-1)
    return out.reshape(x.shape)


def apply_partial_rope(x, freqs):
    """Rotate the first freqs.shape[-1] channels of the full-width projection,
    i.e. before the head split (dit.py:40-54)."""
    r = freqs.shape[-1]
    c = np.cos(freqs)
    s = np.sin(freqs)
    head = x[..., :r]
    head = head * c + rotate_pairs(head) * s
    return np.concatenate([head, x[..., r:]], axis=-1)


class DiT:
    def __init__(self, weights, prefix: str = "flow.decoder.estimator."):
        self.w = weights
        self.p = prefix
        m = weights.meta.get("dit", {})
        self.dim = int(m.get("dim", 1024))
        self.depth = int(m.get("depth", 22))
        self.heads = int(m.get("heads", 16))
        self.dim_head = int(m.get("dim_head", 64))
        self.static_chunk_size = int(m.get("static_chunk_size", 50))
        self.num_decoding_left_chunks = int(m.get("num_decoding_left_chunks", -1))
        self.conv_pos_kernel = int(m.get("conv_pos_kernel", 31))
        self.conv_pos_groups = int(m.get("conv_pos_groups", 16))

    def _t(self, name):
        return self.w.get(self.p + name)

    def time_embed(self, t):
        """sinusoid(256) -> Linear -> SiLU -> Linear (dit.py:86-90)."""
        h = sinus_position_embedding(t, 256, 1000.0)
        h = ops.linear(h, self._t("time_embed.time_mlp.0.weight"), self._t("time_embed.time_mlp.0.bias"))
        return ops.linear(ops.silu(h), self._t("time_embed.time_mlp.2.weight"),
                          self._t("time_embed.time_mlp.2.bias"))

    def input_embed(self, x, cond, mu, spks):
        """concat[x, cond, mu, spk] -> Linear -> + Mish(conv(Mish(conv(.)))) per batch
        row, grouped causal convs (dit.py:92-112)."""
        b, t, _ = x.shape
        spk = np.broadcast_to(spks[:, None, :], (b, t, spks.shape[1]))
        h = ops.linear(np.concatenate([x, cond, mu, spk], axis=-1),
                       self._t("input_embed.proj.weight"), self._t("input_embed.proj.bias"))
        k = self.conv_pos_kernel
        pos = np.empty_like(h)
        for i in range(b):
            z = np.ascontiguousarray(h[i].T)
            for c in ("conv1", "conv2"):
                z = ops.conv1d(z, self._t(f"input_embed.conv_pos_embed.{c}.0.weight"),
                               self._t(f"input_embed.conv_pos_embed.{c}.0.bias"),
                               groups=self.conv_pos_groups, pad=(k - 1, 0))
                z = ops.mish(z)
            pos[i] = z.T
        return pos + h

    def attn(self, blk, x, freqs, mask_spec):
        """q/k/v linears, partial rope on q and k, per-batch head split, sdpa,
        out-projection (dit.py:114-129)."""
        b, t, _ = x.shape
        q = ops.linear(x, self._t(blk + "attn.to_q.weight"), self._t(blk + "attn.to_q.bias"))
        k = ops.linear(x, self._t(blk + "attn.to_k.weight"), self._t(blk + "attn.to_k.bias"))
        v = ops.linear(x, self._t(blk + "attn.to_v.weight"), self._t(blk + "attn.to_v.bias"))
        q = apply_partial_rope(q, freqs)
        k = apply_partial_rope(k, freqs)
        h, d = self.heads, self.dim_head
        out = np.empty((b, t, h * d), dtype=np.float32)
        for i in range(b):
            split = [np.ascontiguousarray(a[i].reshape(t, h, d).transpose(1, 0, 2)) for a in (q, k, v)]
            out[i] = ops.sdpa(*split, mask_spec).transpose(1, 0, 2).reshape(t, h * d)
        return ops.linear(out, self._t(blk + "attn.to_out.0.weight"), self._t(blk + "attn.to_out.0.bias"))

    def ff(self, blk, x, seq_chunk):
        """Linear -> GELU(tanh) -> Linear, chunked over time (dit.py:131-142)."""
        t = x.shape[1]
        out = np.empty_like(x)
        for t0 in range(0, t, seq_chunk):
            t1 = min(t, t0 + seq_chunk)
            hid = ops.gelu_tanh(ops.linear(x[:, t0:t1], self._t(blk + "ff.ff.0.0.weight"),
                                           self._t(blk + "ff.ff.0.0.bias")))
            out[:, t0:t1] = ops.linear(hid, self._t(blk + "ff.ff.2.weight"), self._t(blk + "ff.ff.2.bias"))
        return out

    def block(self, i, h, temb, freqs, mask_spec=None, seq_chunk=512):
        """One AdaLN transformer block (dit.py:163-173)."""
        blk = f"transformer_blocks.{i}."
        mod = ops.linear(ops.silu(temb), self._t(blk + "attn_norm.linear.weight"),
                         self._t(blk + "attn_norm.linear.bias"))
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = np.split(mod, 6, axis=1)
        n = ops.layer_norm(h, None, None, 1e-6) * (1.0 + sc_a[:, None]) + sh_a[:, None]
        h = h + g_a[:, None] * self.attn(blk, n, freqs, mask_spec)
        n = ops.layer_norm(h, None, None, 1e-6) * (1.0 + sc_m[:, None]) + sh_m[:, None]
        return h + g_m[:, None] * self.ff(blk, n, seq_chunk)

    def forward(self, x, mu, t, spks, cond, streaming=False, seq_chunk=512):
        """(B, 80, T) x/mu/cond, (B,) t, (B, 80) spks -> (B, 80, T) (dit.py:144-180)."""
        x, mu, cond = (np.ascontiguousarray(np.swapaxes(a, 1, 2)) for a in (x, mu, cond))
        n = x.shape[1]
        temb = self.time_embed(np.asarray(t, dtype=np.float32))
        h = self.input_embed(x, cond, mu, spks)
        freqs = rope_freqs(n, self.dim_head)
        mask = ("chunk", self.static_chunk_size, self.num_decoding_left_chunks) if streaming else None
        for i in range(self.depth):
            h = self.block(i, h, temb, freqs, mask, seq_chunk)
        mod = ops.linear(ops.silu(temb), self._t("norm_out.linear.weight"), self._t("norm_out.linear.bias"))
        scale, shift = np.split(mod, 2, axis=1)
        h = ops.layer_norm(h, None, None, 1e-6) * (1.0 + scale)[:, None] + shift[:, None]
        out = ops.linear(h, self._t("proj_out.weight"), self._t("proj_out.bias"))
        return np.ascontiguousarray(np.swapaxes(out, 1, 2))
