"""Oracle restatement of the Qwen2 decoder body with its KV cache.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/qwen2.py.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import ops


@dataclass
class Qwen2Config:
    """Model geometry (qwen2.py:14-32)."""

    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    vocab_size: int = 151936

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def from_meta(cls, meta):
        m = meta["qwen2"]
        return cls(**{k: m[k] for k in cls.__dataclass_fields__ if k in m})


def rope_tables(dim: int, theta: float, n: int):
    """HF half-split cos/sin tables: fp64 angles, fp64 cos/sin, stored float32 (qwen2.py:46-56)."""
    inv = 1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float64) / dim))
    ang = np.arange(n, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


class RopeCache:
    """Grows to max(n, 2*old, 256) positions (qwen2.py:35-61)."""

    def __init__(self, dim: int, theta: float, max_pos: int = 4096):
        self.dim, self.theta, self.n = dim, theta, 0
        self.cos = self.sin = None
        self.extend(max_pos)

    def extend(self, n: int):
        if n <= self.n:
            return
        n = max(n, self.n * 2, 256)
        self.cos, self.sin = rope_tables(self.dim, self.theta, n)
        self.n = n

    def get(self, pos):
        if pos.max() >= self.n:
            self.extend(int(pos.max()) + 1)
        return self.cos[pos], self.sin[pos]


def rotate_half(x):
    """concat(-x2, x1) (qwen2.py:64-66)."""
    d = x.shape[-1] // 2
    return np.concatenate([-x[..., d:], x[..., :d]], axis=-1)


def apply_rope(x, cos, sin):
    """x cos + rotate_half(x) sin over (H, T, D) (qwen2.py:69-71)."""
    return x * cos[None] + rotate_half(x) * sin[None]


class KVCache:
    """Per-layer (Hk, cap, D) K and V, grown geometrically; the length advances
    after the last layer appends (qwen2.py:74-121)."""

    def __init__(self, layers, heads, head_dim, dtype=np.float32):
        self.k = [None] * layers
        self.v = [None] * layers
        self.length = 0
        self.cap = 0
        self.heads, self.head_dim, self.dtype, self.layers = heads, head_dim, dtype, layers

    def __len__(self):
        return self.length

    def _reserve(self, need):
        if need <= self.cap:
            return
        cap = max(need, max(256, self.cap * 2))
        for store in (self.k, self.v):
            for i in range(self.layers):
                grown = np.zeros((self.heads, cap, self.head_dim), dtype=self.dtype)
                if store[i] is not None:
                    grown[:, :self.length] = store[i][:, :self.length]
                store[i] = grown
        self.cap = cap

    def append(self, layer, k, v):
        t = k.shape[1]
        if layer == 0:
            self._reserve(self.length + t)
        a = self.length
        self.k[layer][:, a:a + t] = k.astype(self.dtype)
        self.v[layer][:, a:a + t] = v.astype(self.dtype)
        if layer == self.layers - 1:
            self.length = a + t
        return self.k[layer][:, :a + t], self.v[layer][:, :a + t]


class Qwen2Model:
    def __init__(self, weights, cfg: Qwen2Config, prefix: str = "llm."):
        self.w = weights
        self.cfg = cfg
        self.prefix = prefix
        self.rope = RopeCache(cfg.head_dim, cfg.rope_theta)

    def _t(self, name):
        return self.w.get(self.prefix + name)

    def embed(self, ids):
        return ops.embedding(self._t("embed_tokens"), ids)

    def forward(self, x, cache=None, tile_bytes=ops.TILE_BYTES):
        """(T, hidden) embeddings -> final-normed hidden states (qwen2.py:139-179).

        Prefill (T > 1) is causal with offset = past; one decode step attends to
        the whole cache.  o_proj and the MLP have no bias; q/k/v do.
        """
        cfg = self.cfg
        t = x.shape[0]
        past = len(cache) if cache is not None else 0
        cos, sin = self.rope.get(np.arange(past, past + t))
        mask = ("causal", past) if t > 1 else None
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        h = x.astype(np.float32, copy=False)
        for i in range(cfg.num_hidden_layers):
            p = f"layers.{i}."
            n = ops.rms_norm(h, self._t(p + "input_layernorm"), cfg.rms_norm_eps)
            q = ops.linear(n, self._t(p + "self_attn.q_proj.weight"), self._t(p + "self_attn.q_proj.bias"))
            k = ops.linear(n, self._t(p + "self_attn.k_proj.weight"), self._t(p + "self_attn.k_proj.bias"))
            v = ops.linear(n, self._t(p + "self_attn.v_proj.weight"), self._t(p + "self_attn.v_proj.bias"))
            q = apply_rope(np.ascontiguousarray(q.reshape(t, nh, hd).transpose(1, 0, 2)), cos, sin)
            k = apply_rope(np.ascontiguousarray(k.reshape(t, nkv, hd).transpose(1, 0, 2)), cos, sin)
            v = np.ascontiguousarray(v.reshape(t, nkv, hd).transpose(1, 0, 2))
            if cache is not None:
                k, v = cache.append(i, k, v)
                k = k.astype(np.float32, copy=False)
                v = v.astype(np.float32, copy=False)
            a = ops.sdpa(q, k, v, mask, tile_bytes=tile_bytes).transpose(1, 0, 2).reshape(t, nh * hd)
            h = h + ops.linear(a, self._t(p + "self_attn.o_proj.weight"))
            n = ops.rms_norm(h, self._t(p + "post_attention_layernorm"), cfg.rms_norm_eps)
            g = ops.linear(n, self._t(p + "mlp.gate_proj.weight"))
            u = ops.linear(n, self._t(p + "mlp.up_proj.weight"))
            h = h + ops.linear(ops.silu(g) * u, self._t(p + "mlp.down_proj.weight"))
        return ops.rms_norm(h, self._t("norm"), cfg.rms_norm_eps)

    def new_cache(self):
        return KVCache(self.cfg.num_hidden_layers, self.cfg.num_key_value_heads, self.cfg.head_dim)
