"""Device-resident Qwen2 decode (the CosyVoice3 LM's token loop) on ``cv3_qwen2_decode_step``.

Restates the single-token path of cv3cpu/models/qwen2.py:139-179 and the head /
speech-embedding of cv3cpu/models/llm.py:68-77,121.  The reference samples
(llm.py:112-149); this path is greedy: argmax of the head logits with ties to
the lowest id, which is the first entry of the reference's stable
``np.argsort(-p)`` (llm.py:138).

Layout in HBM (L layers, D = hidden, dh = head_dim, I = intermediate):
  * per projection, one stacked int8 array for all layers: ``qkv`` [L*(H+2Hk)*dh, Kp]
    ([q; k; v] rows per layer), ``o`` [L*D, Kp], ``gate_up`` [L*2I, Kp]
    ([gate; up] rows per layer), ``down`` [L*D, Kp], each with its scales;
  * ``k_cache`` / ``v_cache`` [L, Hk, cap, dh] float32 (qwen2.py:74-121);
  * rotary tables cos / sin [cap, dh] built once on the host with the reference's
    float64 expressions (qwen2.py:46-56);
  * ``pos``, ``token``, ``history`` in device memory so that a captured graph of
    one step replays for every token.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional

import numpy as np

from . import _lib
from .device import DeviceArray, Graph, to_device

c_i64, c_vp = ctypes.c_int64, ctypes.c_void_p


class QWeight(ctypes.Structure):
    _fields_ = [("q", c_vp), ("scales", c_vp), ("rows", c_i64), ("k", c_i64), ("kp", c_i64), ("block", c_i64),
                ("scale_dtype", ctypes.c_int), ("kind", ctypes.c_int)]


class Model(ctypes.Structure):
    _fields_ = [("layers", c_i64), ("hidden", c_i64), ("heads", c_i64), ("kv_heads", c_i64), ("head_dim", c_i64),
                ("inter", c_i64), ("eps", ctypes.c_float),
                ("qkv", QWeight), ("o", QWeight), ("gate_up", QWeight), ("down", QWeight), ("head", QWeight),
                ("embedding", QWeight),
                ("qkv_bias", c_vp), ("ln1", c_vp), ("ln2", c_vp), ("norm", c_vp), ("head_bias", c_vp),
                ("rope_cos", c_vp), ("rope_sin", c_vp)]


class Persist(ctypes.Structure):
    _fields_ = [("words", c_vp), ("words_len", c_i64), ("err", c_vp), ("epoch_base", ctypes.c_uint32),
                ("workgroups", ctypes.c_int), ("cooperative", ctypes.c_int)]


class Sampler(ctypes.Structure):
    _fields_ = [("top_p", ctypes.c_double), ("rep_threshold", ctypes.c_double), ("top_k", c_i64),
                ("win_size", c_i64), ("speech_token_size", c_i64), ("min_len", c_i64),
                ("strict_min_len", ctypes.c_int), ("ctl", c_vp)]


_M64 = (1 << 64) - 1


class State(ctypes.Structure):
    _fields_ = [("k_cache", c_vp), ("v_cache", c_vp), ("cap", c_i64), ("pos", c_vp), ("token", c_vp),
                ("history", c_vp), ("x", c_vp), ("logits", c_vp), ("workspace", c_vp),
                ("workspace_floats", c_i64)]


def rope_tables(dim: int, theta: float, n: int):
    """HF half-split cos/sin: float64 angles and cos/sin, stored float32 (qwen2.py:46-56)."""
    inv = 1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float64) / dim))
    ang = np.arange(n, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _kind(w):
    return getattr(w, "kind", None)


def _host(a):
    return a.numpy() if isinstance(a, DeviceArray) else np.asarray(a)


def widen_q4_codes(packed: np.ndarray) -> np.ndarray:
    """q4 codes (quant.py:70-86: per 32-code block 16 bytes, byte j holding code j in its low
    nibble and code j + 16 in its high nibble, each + 8) as int8 codes n - 8, K in order."""
    b = np.ascontiguousarray(packed, dtype=np.uint8)
    rows, half = b.shape
    blocks = b.reshape(rows, half // 16, 16)
    codes = np.concatenate([blocks & 0x0F, blocks >> 4], axis=2).astype(np.int16) - 8
    return codes.reshape(rows, half * 2).astype(np.int8)


class _Stacked:
    """Rows of several q8 or q4 QTensors (per layer, in order) stacked into one device array.

    ``widen``: q4 rows are stored as int8 codes (n - 8) with their 32-code blocks and float16
    scales, i.e. the same weights, dequantised to the same floats, twice the bytes.  The decode
    step is latency-bound, and unpacking nibbles is VALU work on its critical path."""

    def __init__(self, per_layer: List[List[object]], widen: bool = False):
        qs, ss = [], []
        first = per_layer[0][0]
        self.k = int(first.shape[1])
        self.block = int(first.block)
        self.kind = _kind(first)
        sdt = np.dtype(_host(first.scales).dtype)
        for parts in per_layer:
            for w in parts:
                if _kind(w) not in ("q8", "q4"):
                    raise ValueError("the device decode takes q8 or q4 weights (the balanced and tiny profiles)")
                if (int(w.shape[1]) != self.k or int(w.block) != self.block or _host(w.scales).dtype != sdt
                        or _kind(w) != self.kind):
                    raise ValueError("stacked weights must share kind, K, block and scale dtype")
                qs.append(_host(w.q))
                ss.append(_host(w.scales))
        self.rows = sum(int(w.shape[0]) for w in per_layer[0])
        q = np.concatenate(qs, axis=0)
        s = np.concatenate(ss, axis=0)
        self.kp = int(s.shape[1]) * self.block  # q4 rows hold kp / 2 bytes
        self.source_nbytes = q.nbytes + s.nbytes   # the checkpoint's bytes (q4: packed nibbles)
        self.widened = bool(widen and self.kind == "q4")
        if self.widened:
            q = widen_q4_codes(q)
            self.kind = "q8"
        cpc = 32 if self.kind == "q4" else 16
        if self.kp % cpc or self.block % cpc:
            raise ValueError(f"padded K and block must be multiples of {cpc}")
        self.sf16 = sdt == np.dtype(np.float16)
        self.q = to_device(np.ascontiguousarray(q))
        self.scales = to_device(np.ascontiguousarray(s))

    def layer(self, layer: int, row0: int = 0, rows: Optional[int] = None):
        """linear_q arguments (kind, codes, scales, scale dtype, kp, block, n) of rows
        [row0, row0 + rows) of one layer."""
        rows = self.rows - row0 if rows is None else rows
        row_bytes = self.kp // 2 if self.kind == "q4" else self.kp
        nb = self.kp // self.block
        r = layer * self.rows + row0
        return (_lib.KIND_Q4 if self.kind == "q4" else _lib.KIND_Q8, self.q.ptr + r * row_bytes,
                self.scales.ptr + r * nb * (2 if self.sf16 else 4), _lib.F16 if self.sf16 else _lib.F32,
                self.kp, self.block, rows)

    def struct(self) -> QWeight:
        return QWeight(self.q.ptr, self.scales.ptr, self.rows, self.k, self.kp, self.block,
                       _lib.F16 if self.sf16 else _lib.F32, _lib.KIND_Q4 if self.kind == "q4" else _lib.KIND_Q8)

    @property
    def nbytes(self):
        """Bytes held in HBM (a widened q4 body: int8 codes)."""
        return self.q.nbytes + self.scales.nbytes


class DeviceQwen2:
    """Qwen2 body + CosyVoice3 LM head resident on the device, decoding greedily."""

    def __init__(self, weights, prefix: str = "llm.", cap: int = 1024, widen_q4: bool = False):
        """A q4 body (the tiny profile) is held in HBM as the checkpoint's packed nibbles; the
        one-launch step decodes it at the int8 body's rate.  ``widen_q4`` holds it as int8
        codes with the same blocks and scales instead (identical weights, twice the bytes),
        which the five-kernel step reads a little faster."""
        _lib.init()
        m = weights.meta["qwen2"]
        self.layers = int(m["num_hidden_layers"])
        self.hidden = int(m["hidden_size"])
        self.heads = int(m["num_attention_heads"])
        self.kv_heads = int(m["num_key_value_heads"])
        self.inter = int(m["intermediate_size"])
        self.eps = float(m.get("rms_norm_eps", 1e-6))
        self.theta = float(m.get("rope_theta", 1e6))
        self.head_dim = self.hidden // self.heads
        if cap % 64 or cap > 1024:
            raise ValueError("cache capacity must be a multiple of 64, at most 1024")
        self.cap = int(cap)
        body = prefix + "model."
        g = weights.get
        L = range(self.layers)
        lp = [f"{body}layers.{i}." for i in L]
        self.qkv = _Stacked([[g(p + f"self_attn.{x}_proj.weight") for x in "qkv"] for p in lp], widen_q4)
        self.o = _Stacked([[g(p + "self_attn.o_proj.weight")] for p in lp], widen_q4)
        self.gate_up = _Stacked([[g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")] for p in lp], widen_q4)
        self.down = _Stacked([[g(p + "mlp.down_proj.weight")] for p in lp], widen_q4)
        self.head = _Stacked([[g(prefix + "llm_decoder.weight")]])
        self.emb = _Stacked([[g(prefix + "speech_embedding")]])
        f32 = lambda a: np.asarray(_host(a), np.float32)  # noqa: E731
        self.qkv_bias = to_device(np.concatenate([f32(g(p + f"self_attn.{x}_proj.bias")) for p in lp for x in "qkv"]))
        self.ln1 = to_device(np.concatenate([f32(g(p + "input_layernorm")) for p in lp]))
        self.ln2 = to_device(np.concatenate([f32(g(p + "post_attention_layernorm")) for p in lp]))
        self.norm = to_device(f32(g(body + "norm")))
        hb = prefix + "llm_decoder.bias"
        self.head_bias = to_device(f32(g(hb))) if hb in weights else None
        c, s = rope_tables(self.head_dim, self.theta, self.cap)
        self.rope_cos, self.rope_sin = to_device(c), to_device(s)
        self.vocab = self.head.rows
        self.model = Model(self.layers, self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter,
                           self.eps, self.qkv.struct(), self.o.struct(), self.gate_up.struct(), self.down.struct(),
                           self.head.struct(), self.emb.struct(), self.qkv_bias.ptr, self.ln1.ptr, self.ln2.ptr,
                           self.norm.ptr, self.head_bias.ptr if self.head_bias is not None else None,
                           self.rope_cos.ptr, self.rope_sin.ptr)
        # state
        cache_shape = (self.layers, self.kv_heads, self.cap, self.head_dim)
        self.k_cache = DeviceArray(cache_shape).zero_()
        self.v_cache = DeviceArray(cache_shape).zero_()
        self.ints = DeviceArray((2 + self.cap,), np.int64).zero_()   # pos, token, history[cap]
        self.x = DeviceArray((self.hidden,))
        self.logits = DeviceArray((self.vocab,))
        nws = 1024 + self.heads * 16 * 64 + self.heads * 16 * 2 + self.inter + 64
        self.workspace = DeviceArray((nws,))
        p0 = self.ints.ptr
        self.state = State(self.k_cache.ptr, self.v_cache.ptr, self.cap, p0, p0 + 8, p0 + 16, self.x.ptr,
                           self.logits.ptr, self.workspace.ptr, nws)
        self._graph: Optional[Graph] = None
        self._pos_host = 0
        # sampler control block: [start, stop step + 1, PCG64 state hi, lo, inc hi, lo]
        self.ctl = DeviceArray((6,), np.int64).zero_()
        self._sampled_graphs = {}
        self._persist: Optional[Persist] = None   # exchange words of the one-launch step, made on first use
        # the one-launch step's launch: ordinary (the device runs nothing else meanwhile) or
        # hipLaunchCooperativeKernel, which guarantees co-residency at ~20 us more per token
        self.cooperative = False

    # -- weights streamed per token (the HBM roofline numerator) -----------
    def bytes_per_token(self, length: int) -> dict:
        """Algorithmic HBM bytes of one token at KV length ``length`` (keys read = length + 1): the
        checkpoint's weight bytes (a q4 body counts its packed nibbles even when held widened).
        ``body_held`` is what the kernels actually stream for the body: the widened int8 codes
        and their scales when a q4 body is held widened, else the same as ``body``."""
        body = self.qkv.source_nbytes + self.o.source_nbytes + self.gate_up.source_nbytes + self.down.source_nbytes
        held = self.qkv.nbytes + self.o.nbytes + self.gate_up.nbytes + self.down.nbytes
        kv = 2 * self.layers * self.kv_heads * (length + 1) * self.head_dim * 4
        small = 4 * (self.qkv_bias.size + self.ln1.size + self.ln2.size + self.norm.size)
        return {"body": body, "kv": kv, "norms_biases": small, "head": self.head.nbytes, "body_held": held}

    # -- state ------------------------------------------------------------
    def fill_cache(self, k: np.ndarray, v: np.ndarray):
        """Pre-fill positions [0, n) of every layer's cache from host (L, Hk, n, dh) arrays."""
        n = k.shape[2]
        if n >= self.cap:
            raise ValueError("prefill does not fit the cache")
        kc = np.zeros((self.layers, self.kv_heads, self.cap, self.head_dim), np.float32)
        vc = np.zeros_like(kc)
        kc[:, :, :n] = k
        vc[:, :, :n] = v
        self.k_cache.copy_from(kc)
        self.v_cache.copy_from(vc)

    def begin(self, token: int, pos: int):
        """Start decoding with input ``speech_embedding[token]`` at position ``pos``."""
        if not 0 <= pos < self.cap - 1:
            raise ValueError("position outside the cache")
        ints = np.zeros(2 + self.cap, np.int64)
        ints[0], ints[1] = pos, token
        self.ints.copy_from(ints)
        self._pos_host = pos
        _lib.call("qwen2_embed_token", ctypes.byref(self.model), ctypes.byref(self.state), None)

    def step(self, graph: bool = False):
        """Enqueue one greedy token (no host synchronisation)."""
        if self._pos_host + 1 >= self.cap:
            raise ValueError("the KV cache is full")
        if graph:
            if self._graph is None:
                g = Graph()
                with g:
                    _lib.call("qwen2_decode_step", ctypes.byref(self.model), ctypes.byref(self.state), None)
                self._graph = g
            self._graph.launch()
        else:
            _lib.call("qwen2_decode_step", ctypes.byref(self.model), ctypes.byref(self.state), None)
        self._pos_host += 1

    # -- prompt prefill (the body's multi-token forward) -----------------------
    def _linear(self, x: int, m: int, w: "_Stacked", layer: int, y: int, ldy: int, bias=None, row0: int = 0,
                rows: Optional[int] = None, epi=None):
        kind, q, sc, sdt, kp, block, n = w.layer(layer, row0, rows)
        _lib.call("linear_q", kind, x, m, w.k, w.k, q, sc, sdt, kp, block, n, bias, y, ldy,
                  ctypes.byref(epi) if epi is not None else None, None)

    def prefill(self, x, pos0: int = 0):
        """Qwen2Model.forward over T input embeddings at positions pos0 .. pos0 + T - 1
        (qwen2.py:139-179) on the device: RMSNorm, [q; k; v] projection with bias, half-split
        rotary, k and v appended to the cache, causal attention over the cache (mask
        ("causal", pos0) when T > 1), o_proj + residual, RMSNorm, SwiGLU, down + residual.
        Leaves the head logits of the last position in ``logits`` and ``pos`` at that
        position, so ``select`` / ``generate_*_after_prefill`` draw the next token."""
        xd = x if isinstance(x, DeviceArray) else to_device(np.ascontiguousarray(x, np.float32))
        if xd.ndim != 2 or xd.shape[1] != self.hidden or xd.shape[0] < 1:
            raise ValueError(f"prefill takes (T, {self.hidden}) embeddings, got {xd.shape}")
        t = xd.shape[0]
        if pos0 < 0 or pos0 + t >= self.cap:
            raise ValueError("the prompt does not fit the KV cache")
        D, H, Hk, dh, I, cap = self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter, self.cap
        R = self.qkv.rows
        h = DeviceArray((t, D))
        _lib.call("copy_d2d", h.ptr, xd.ptr, t * D * 4, None)
        n = DeviceArray((t, D))
        qkv = DeviceArray((t, R))
        att = DeviceArray((t, D))
        u = DeviceArray((t, I))
        a = DeviceArray((t, I))
        res = _lib.epilogue(residual=h.ptr, ld_res=D)
        swiglu = _lib.epilogue(act="silu", gate=u.ptr, gate_stride=I, rows_per_gate=1)
        c64 = ctypes.c_int64 * 3
        for l in range(self.layers):
            _lib.call("rms_norm", h.ptr, self.ln1.ptr + l * D * 4, n.ptr, t, D, self.eps, None)
            self._linear(n.ptr, t, self.qkv, l, qkv.ptr, R, bias=self.qkv_bias.ptr + l * R * 4)
            _lib.call("rope_half", qkv.ptr, t * H, H, R, dh, self.rope_cos.ptr, self.rope_sin.ptr, pos0, None)
            _lib.call("rope_half", qkv.ptr + H * dh * 4, t * Hk, Hk, R, dh, self.rope_cos.ptr, self.rope_sin.ptr,
                      pos0, None)
            for j, cache in enumerate((self.k_cache, self.v_cache)):   # rows pos0 .. of layer l
                _lib.call("copy_strided", qkv.ptr + (H + j * Hk) * dh * 4,
                          cache.ptr + ((l * Hk) * cap + pos0) * dh * 4, Hk, t, dh, c64(dh, R, 1),
                          c64(cap * dh, dh, 1), None)
            kv = l * Hk * cap * dh * 4
            _lib.call("attention", qkv.ptr, self.k_cache.ptr + kv, self.v_cache.ptr + kv, att.ptr, 1, H, Hk, t,
                      pos0 + t, dh, c64(0, dh, R), c64(0, cap * dh, dh), c64(0, cap * dh, dh), c64(0, dh, D),
                      1.0 / np.sqrt(dh), 1 if t > 1 else 0, pos0, 0, None)
            self._linear(att.ptr, t, self.o, l, h.ptr, D, epi=res)
            _lib.call("rms_norm", h.ptr, self.ln2.ptr + l * D * 4, n.ptr, t, D, self.eps, None)
            self._linear(n.ptr, t, self.gate_up, l, u.ptr, I, row0=I, rows=I)        # up
            self._linear(n.ptr, t, self.gate_up, l, a.ptr, I, row0=0, rows=I, epi=swiglu)  # u * silu(gate)
            self._linear(a.ptr, t, self.down, l, h.ptr, D, epi=res)
        _lib.call("rms_norm", h.ptr + (t - 1) * D * 4, self.norm.ptr, n.ptr, 1, D, self.eps, None)
        self._linear(n.ptr, 1, self.head, 0, self.logits.ptr, self.vocab,
                     bias=self.head_bias.ptr if self.head_bias is not None else None)
        p = np.array([pos0 + t - 1], np.int64)
        _lib.call("copy_h2d", self.ints.ptr, p.ctypes.data, 8, None)
        self._pos_host = pos0 + t - 1

    def select(self, smp: Optional["Sampler"] = None):
        """Draw the next token from the logits already in ``logits`` (greedy without a
        sampler), as a decode step's last kernel does."""
        _lib.call("qwen2_select", ctypes.byref(self.model), ctypes.byref(self.state),
                  ctypes.byref(smp) if smp is not None else None, None)
        self._pos_host += 1

    def step_sampled(self, smp: "Sampler", graph: bool = False, persistent: bool = False):
        """Enqueue one sampled token (no host synchronisation); ``persistent`` runs the
        body and head as one cooperative launch (cv3_qwen2_decode_step_persistent), then
        the draw (cv3_qwen2_select)."""
        if self._pos_host + 1 >= self.cap:
            raise ValueError("the KV cache is full")
        if persistent:
            self.step_persistent(select=False)
            _lib.call("qwen2_select", ctypes.byref(self.model), ctypes.byref(self.state), ctypes.byref(smp), None)
        elif graph:
            key = tuple(getattr(smp, f) for f, _ in Sampler._fields_)
            g = self._sampled_graphs.get(key)
            if g is None:
                g = Graph()
                with g:
                    _lib.call("qwen2_decode_step_sampled", ctypes.byref(self.model), ctypes.byref(self.state),
                              ctypes.byref(smp), None)
                self._sampled_graphs[key] = g
            g.launch()
        else:
            _lib.call("qwen2_decode_step_sampled", ctypes.byref(self.model), ctypes.byref(self.state),
                      ctypes.byref(smp), None)
        self._pos_host += 1

    def generate_sampled_after_prefill(self, max_len: int, min_len: int, sampling, speech_token_size: int,
                                       graph: bool = True, check_every: int = 16,
                                       persistent: bool = False) -> List[int]:
        """generate()'s loop after ``prefill``: the first token is drawn from the prompt's
        logits (llm.py:112-121 at i = 0), the rest by decode steps."""
        return self.generate_sampled(None, self._pos_host, max_len, min_len, sampling, speech_token_size, graph,
                                     check_every, persistent)

    def generate_sampled(self, first_token: Optional[int], pos: int, max_len: int, min_len: int, sampling,
                         speech_token_size: int, graph: bool = True, check_every: int = 16,
                         persistent: bool = False) -> List[int]:
        """The token loop of CosyVoice3LM.generate (llm.py:104-123) with its sampler
        (llm.py:125-149) on the device: up to max_len tokens from input
        speech_embedding[first_token] at position pos, ending before the first stop id.
        ``sampling`` has top_p, top_k, win_size, tau_r, strict_min_len and a NumPy
        PCG64 Generator ``rng``, whose state the device advances exactly as the
        reference's draws would and hands back.  The host looks for a stop every
        ``check_every`` tokens; steps after a stop change nothing.  ``first_token``
        None draws the first token from the logits already present (after ``prefill``,
        whose last position is ``pos``).  ``persistent`` decodes with the one-launch step
        (q8 weights) instead of the five-kernel step."""
        bg = sampling.rng.bit_generator
        st = bg.state
        if st.get("bit_generator") != "PCG64":
            raise ValueError("the device sampler draws from NumPy's PCG64 stream (np.random.default_rng)")
        if pos + max_len + 1 >= self.cap:
            raise ValueError("the generation does not fit the KV cache")
        if not sampling.top_p > 0 or int(sampling.top_k) < 1:
            raise ValueError("a draw needs top_p > 0 and top_k >= 1 (the nucleus would be empty)")
        s, inc = int(st["state"]["state"]), int(st["state"]["inc"])
        ctl = np.array([pos, 0, s >> 64, s & _M64, inc >> 64, inc & _M64], dtype=np.uint64).view(np.int64)
        self.ctl.copy_from(ctl)
        smp = Sampler(float(sampling.top_p), float(sampling.win_size * sampling.tau_r), int(sampling.top_k),
                      int(sampling.win_size), int(speech_token_size), int(min_len),
                      int(bool(getattr(sampling, "strict_min_len", False))), self.ctl.ptr)
        done = 0
        if first_token is None:
            self.select(smp)
            done = 1
        else:
            self.begin(first_token, pos)
        while done < max_len:
            n = min(check_every, max_len - done)
            for _ in range(n):
                self.step_sampled(smp, graph, persistent)
            done += n
            if int(self.ctl.numpy()[1]) != 0:
                break
        if persistent and self.persistent_error():
            raise RuntimeError("the one-launch decode step gave up waiting for an exchange")
        c = self.ctl.numpy().view(np.uint64)
        stop = int(c[1])
        count = stop - 1 if stop else max_len
        new = dict(st)
        new["state"] = {"state": (int(c[2]) << 64) | int(c[3]), "inc": (int(c[4]) << 64) | int(c[5])}
        bg.state = new
        ints = self.ints.numpy()
        self._pos_host = int(ints[0])
        return [int(t) for t in ints[2 + pos + 1: 2 + pos + 1 + count]]

    def generate_after_prefill(self, steps: int, graph: bool = True) -> List[int]:
        """Greedy tokens after ``prefill``: the argmax of the prompt's logits, then steps - 1
        decode steps."""
        pos = self._pos_host
        if pos + steps >= self.cap:
            raise ValueError("the generation does not fit the KV cache")
        self.select(None)
        for _ in range(steps - 1):
            self.step(graph)
        ints = self.ints.numpy()
        return [int(t) for t in ints[2 + pos + 1: 2 + pos + 1 + steps]]

    # -- the whole step as one cooperative launch --------------------------
    def step_persistent(self, select: bool = True):
        """Enqueue one token as a single launch of the whole step (cv3_qwen2_decode_step_persistent,
        cooperative if ``self.cooperative``): greedy selection inside (``select``), or logits only,
        for the sampler (``step_sampled(persistent=True)``)."""
        if self._pos_host + 1 >= self.cap:
            raise ValueError("the KV cache is full")
        need = ctypes.c_int64()
        _lib.call("qwen2_persist_words", ctypes.byref(self.model), 256, _lib.ptr(need))
        need = need.value
        if self._persist is None or self._persist.words_len < need:
            # fresh words are zero, the cleared state no epoch matches
            self._pwords = DeviceArray((need,), np.int64).zero_()
            self._perr = DeviceArray((1,), np.int64).zero_()
            base = self._persist.epoch_base if self._persist is not None else 0
            self._persist = Persist(self._pwords.ptr, need, self._perr.ptr, base, 0, 0)
        p = self._persist
        p.cooperative = 1 if self.cooperative else 0
        base = (p.epoch_base + 256) & 0xFFFFFFFF
        if base == 0:   # the launch counter wrapped: clear the words so no old epoch can match
            self._pwords.zero_()
            base = 256
        p.epoch_base = base
        _lib.call("qwen2_decode_step_persistent", ctypes.byref(self.model), ctypes.byref(self.state),
                  ctypes.byref(p), 1 if select else 0, None)
        self._pos_host += 1 if select else 0

    def persistent_error(self) -> bool:
        """True if a launch of the one-launch step gave up waiting (its results are invalid)."""
        return self._persist is not None and int(self._perr.numpy()[0]) != 0

    def generate_persistent(self, first_token: int, pos: int, steps: int) -> List[int]:
        """Greedy tokens with the one-launch step; raises if a launch gave up."""
        self.begin(first_token, pos)
        for _ in range(steps):
            self.step_persistent(True)
        if self.persistent_error():
            raise RuntimeError("the one-launch decode step gave up waiting for an exchange")
        ints = self.ints.numpy()
        return [int(t) for t in ints[2 + pos + 1: 2 + pos + 1 + steps]]

    def generate(self, first_token: int, pos: int, steps: int, graph: bool = True) -> List[int]:
        self.begin(first_token, pos)
        for _ in range(steps):
            self.step(graph)
        ints = self.ints.numpy()
        return [int(t) for t in ints[2 + pos + 1: 2 + pos + 1 + steps]]
