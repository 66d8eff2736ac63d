"""Device-resident DiT estimator and the Euler / classifier-free-guidance flow solve.

Restates the call sequences of cv3cpu/models/dit.py:86-180 (``DiT.forward``)
and cv3cpu/models/flow.py:58-93 (``Flow.solve_euler``) with every activation
resident in HBM and every step a kernel of ``libcv3hip.so``.  Only the
t-schedule and the sinusoidal time features (a few hundred floats, computed with
the reference's own float32 expressions) are prepared on the host.

Layout in HBM (B = 2 for the CFG pair, T mel frames, D = 1024):
  * ``h``   [B*T, D]     the residual stream, updated in place by the GEMM epilogues
  * ``qkv`` [B*T, 3D]    fused q|k|v projection (weights concatenated row-wise in
                         [q; k; v] order, biases likewise), the partial rotary of q
                         and k applied in the GEMM's epilogue
  * ``att`` [B*T, D]     attention output, heads interleaved as [T, H*dh]
  * ``ff``  [B*T, 2D]    GELU-tanh hidden
  * ``z1``  [B*T, D]     first conv_pos output (channels-last like everything else)
  * ``mod`` [S, L]       every AdaLN modulation row of the solve, one per Euler step:
                         the time embedding depends only on t, so the S = 10 rows of
                         ``Linear(silu(temb))`` for all 22 blocks and ``norm_out`` are
                         one GEMM over the concatenated weights (L = 22*6D + 2D).  Both
                         CFG rows share t (cv3cpu/models/flow.py:82-84), so one row
                         serves the pair.

Work per Euler step, in order (reference lines in brackets):
  pack x into the [x | cond | mu | spk] input  (dit.py:92-97, flow.py:72-84)
  input projection GEMM                        (dit.py:98)
  two grouped causal convs + Mish, residual    (dit.py:99-112)
  22 x [ LayerNorm+AdaLN -> QKV GEMM with partial rotary on q,k -> attention ->
         out GEMM with gate*y + h epilogue -> LayerNorm+AdaLN -> FF1 GEMM with
         GELU-tanh -> FF2 GEMM with gate*y + h ]  (dit.py:114-173)
  LayerNorm + (scale, shift) -> proj_out GEMM  (dit.py:175-180)
  CFG combine + Euler update                   (flow.py:86-90)
"""

from __future__ import annotations

import ctypes
import math
from typing import Dict, List, Optional

import numpy as np

from . import _lib
from .device import DeviceArray, Event, Graph, Stream, to_device, wait_event
from .quant import QTensor

ACT = _lib.ACT


def _is_q(w) -> bool:
    return hasattr(w, "kind") and hasattr(w, "scales")


def _host(a) -> np.ndarray:
    return a.numpy() if isinstance(a, DeviceArray) else np.asarray(a)


# True puts the per-channel q8 QKV and ff1 linears of the DiT on the int8 matrix cores as digit
# planes (cv3_linear_q8_digits; every product exact, 5x smaller error against float64 than the
# bfloat16 planes of cv3_linear_q8_x3_frag), their row exponents written by the layer norm that
# feeds them (cv3_layer_norm_rexp).  At the 30 s shapes (3000 rows) the digit-plane QKV ran
# 78.6-85.1 us against 85.6-86.3 us on the planes depending on the machine; with the CFG rows on
# two streams the 30 s solve ran level (86.3-87.0 against 86.9 ms).  out and ff2 (1024 outputs)
# were no faster on the digit planes and stay on the bfloat16 planes.
DIGITS = True
# From HALVES_MIN_T frames on, the two batch rows of the CFG pair (conditional, unconditional)
# go through the transformer blocks on two streams, so that one row's norms, attention and
# launch gaps overlap the other's GEMMs (bit-identical results).  30 s q8 solve: 90.4 -> 86.0 ms;
# at 10 s (500 frames) one row's GEMMs fill half the machine and the solve was 0.3 ms slower,
# so below the threshold both rows share each launch.  DeviceDiT.halves overrides it.
HALVES = True
HALVES_MIN_T = 1024


class DeviceLinear:
    """One resident linear weight: float32 ``[N, K]`` or q8 codes + scales.

    ``planes=True`` holds a float32 weight (K % 64 == 0) as its three bfloat16 planes
    instead (W = hi + mid + lo to all 24 bits), packed in the matrix cores' fragment order
    (``cv3_split_x3_frag``), and the product runs on the bfloat16 matrix cores as six plane
    products with float32 accumulation, each wave loading its weight fragments straight into
    registers (``cv3_linear_x3_frag``): the same float32 linear, with errors against float64
    no larger than the float32 matrix cores' own.  A q8 weight (blocks of a multiple of 64) then runs
    as the activation's three planes times its codes, exact in bfloat16, with the block
    scale on each block's sum (``cv3_linear_q8_x3``); with one scale per row (per-channel,
    K <= 2048) it runs on the int8 matrix cores instead, the activation's rows as four int8 digit
    planes (``cv3_linear_q8_digits``, exact products of the codes with each row rounded 30 bits
    below its largest element), given ``rexp``, an int32 workspace of at least m entries.
    """

    def __init__(self, weights: List[object], biases: List[Optional[np.ndarray]], planes: bool = False,
                 digits: bool = False):
        ws = list(weights)
        self.planes = None
        self.rexp: Optional[DeviceArray] = None
        if all(_is_q(w) for w in ws):
            kinds = {w.kind for w in ws}
            blocks = {int(w.block) for w in ws}
            sdt = {np.dtype(_host(w.scales).dtype) for w in ws}
            if kinds != {"q8"} or len(blocks) != 1 or len(sdt) != 1:
                raise ValueError("only q8 weights of one block size and scale dtype can be concatenated")
            self.q8 = True
            q = np.concatenate([_host(w.q) for w in ws], axis=0)
            s = np.concatenate([_host(w.scales) for w in ws], axis=0)
            self.k = int(ws[0].shape[1])
            if any(int(w.shape[1]) != self.k for w in ws):
                raise ValueError("concatenated weights disagree on K")
            self.n = int(q.shape[0])
            self.block = blocks.pop()
            self.kp = int(s.shape[1]) * self.block
            self.sf16 = sdt.pop() == np.dtype(np.float16)
            self.q = to_device(np.ascontiguousarray(q))
            self.scales = to_device(np.ascontiguousarray(s))
            # the activation's bfloat16 planes times the codes, held in the matrix cores' fragment
            # order (cv3_pack_q8_frag, cv3_linear_q8_x3_frag)
            self.q8_planes = bool(planes) and self.k % 64 == 0 and self.block % 64 == 0
            # per-channel codes on the int8 matrix cores (cv3_pack_q8_frag32, cv3_linear_q8_digits)
            self.q8_digits = (self.q8_planes and digits and DIGITS and self.kp == self.block
                              and self.k <= 2048)
            if self.q8_digits:
                npad = -(-self.n // 32) * 32
                qf = DeviceArray((npad * (self.k + 4),), np.int8)
                _lib.call("pack_q8_frag32", self.q.ptr, self.n, self.k, self.kp, qf.ptr, None)
                self.q = qf
                self.q8_planes = False
            elif self.q8_planes:
                qf = DeviceArray((-(-self.n // 32) * 32 * self.k,), np.int8)
                _lib.call("pack_q8_frag", self.q.ptr, self.n, self.k, self.kp, qf.ptr, None)
                self.q = qf
        elif not any(_is_q(w) for w in ws):
            self.q8 = self.q8_digits = False
            w = np.concatenate([np.asarray(_host(w), dtype=np.float32).reshape(np.shape(w)[0], -1) for w in ws],
                               axis=0)
            self.n, self.k = w.shape
            self.w = to_device(np.ascontiguousarray(w))
            if planes and self.k % 64 == 0:
                ne = ctypes.c_int64()
                _lib.call("x3_frag_elems", self.n, self.k, ctypes.byref(ne))
                self.planes = DeviceArray((ne.value,), np.uint16)
                _lib.call("split_x3_frag", self.w.ptr, self.n, self.k, self.k, self.planes.ptr, None)
                self.w = None
        else:
            raise ValueError("cannot concatenate quantised and float weights")
        if any(b is not None for b in biases):
            parts = []
            for w, b in zip(ws, biases):
                rows = int(w.shape[0])
                parts.append(np.zeros(rows, np.float32) if b is None else np.asarray(_host(b), np.float32))
            self.bias = to_device(np.concatenate(parts))
        else:
            self.bias = None

    @property
    def nbytes(self) -> int:
        if self.q8:
            return self.q.nbytes + self.scales.nbytes
        return self.planes.nbytes if self.planes is not None else self.w.nbytes

    def __call__(self, x: int, m: int, ldx: int, y: int, ldy: int, epi=None, rexp_given: bool = False,
                 st=None, rexp_row0: int = 0):
        """y[m, n] = epi(x[m, :k] . W^T + bias) on the calling thread's stream.  ``rexp_given``: the
        digit-plane path's row exponents of this x are already in ``rexp`` from row ``rexp_row0`` on
        (cv3_layer_norm_rexp); ``st``: a stream handle (None: the calling thread's)."""
        b = self.bias.ptr if self.bias is not None else None
        e = ctypes.byref(epi) if epi is not None else None
        if self.q8_digits:
            if self.rexp is None or self.rexp.size < rexp_row0 + m:
                raise ValueError("the digit-plane linear needs an int32 workspace of m entries (rexp)")
            _lib.call("linear_q8_digits", x, m, self.k, ldx, self.q.ptr, self.scales.ptr,
                      _lib.F16 if self.sf16 else _lib.F32, self.n, b, y, ldy, e, self.rexp.ptr + 4 * rexp_row0,
                      int(rexp_given), st)
        elif self.q8:
            fn = "linear_q8_x3_frag" if self.q8_planes else "linear_q"
            kind = () if self.q8_planes else (_lib.KIND_Q8,)
            _lib.call(fn, *kind, x, m, self.k, ldx, self.q.ptr, self.scales.ptr,
                      _lib.F16 if self.sf16 else _lib.F32, self.kp, self.block, self.n, b, y, ldy, e, st)
        elif self.planes is not None:
            _lib.call("linear_x3_frag", x, m, self.k, ldx, self.planes.ptr, self.n, b, y, ldy, e, st)
        else:
            _lib.call("linear_f32", x, m, self.k, ldx, self.w.ptr, self.k, self.n, b, y, ldy, e, st)


def sinus_features(t: np.ndarray, dim: int = 256, scale: float = 1000.0) -> np.ndarray:
    """[sin(scale t f), cos(scale t f)], f = exp(-i log(1e4)/(dim/2 - 1)), float32 (dit.py:13-18)."""
    half = dim // 2
    f = np.exp(np.arange(half, dtype=np.float32) * -(math.log(10000.0) / (half - 1)))
    arg = scale * np.asarray(t).reshape(-1, 1).astype(np.float32) * f[None, :]
    return np.concatenate([np.sin(arg), np.cos(arg)], axis=-1).astype(np.float32)


def cosine_t_span(steps: int) -> np.ndarray:
    """1 - cos(linspace(0, 1, steps+1) pi/2) in float64, stored float32 (flow.py:68-69)."""
    return (1.0 - np.cos(np.linspace(0.0, 1.0, steps + 1, dtype=np.float64) * 0.5 * np.pi)).astype(np.float32)


def euler_schedule(steps: int):
    """(t, dt) of each Euler step with the reference's float32 recurrence: t += dt, then
    dt = t_span[s+1] - t (flow.py:78-90), so t drifts from t_span by rounding exactly as there."""
    t_span = cosine_t_span(steps)
    t = t_span[0]
    dt = t_span[1] - t_span[0]
    ts, dts = [], []
    for s in range(1, len(t_span)):
        ts.append(t)
        dts.append(dt)
        t = t + dt
        if s < len(t_span) - 1:
            dt = t_span[s + 1] - t
    return np.array(ts, np.float32), np.array(dts, np.float32)


def dit_rope_tables(n: int, dim_head: int, theta: float = 10000.0):
    """cos/sin of the interleaved DiT rotary angles: fp64 angles stored float32, then
    float32 cos/sin (dit.py:21-29,51-52)."""
    inv = 1.0 / (theta ** (np.arange(0, dim_head, 2, dtype=np.float64) / dim_head))
    ang = np.repeat(np.arange(n, dtype=np.float64)[:, None] * inv[None, :], 2, axis=-1).astype(np.float32)
    return np.cos(ang), np.sin(ang)


class DeviceDiT:
    """The DiT estimator's weights resident in HBM, plus the solve driver.

    ``weights`` has the reference WeightFile read API (``get(name)`` returning a
    float array or a q8 QTensor, ``meta``).
    """

    def __init__(self, weights, prefix: str = "flow.decoder.estimator.", cfg_rate: float = 0.7,
                 steps: int = 10, planes: bool = True):
        _lib.init()
        m = weights.meta.get("dit", {})
        self.dim = int(m.get("dim", 1024))
        self.depth = int(m.get("depth", 22))
        self.heads = int(m.get("heads", 16))
        self.dim_head = int(m.get("dim_head", 64))
        self.conv_k = int(m.get("conv_pos_kernel", 31))
        self.conv_groups = int(m.get("conv_pos_groups", 16))
        self.cfg_rate = float(cfg_rate)
        self.steps = int(steps)
        g = lambda n: weights.get(prefix + n)  # noqa: E731
        D = self.dim
        self.time0 = DeviceLinear([g("time_embed.time_mlp.0.weight")], [g("time_embed.time_mlp.0.bias")])
        self.time2 = DeviceLinear([g("time_embed.time_mlp.2.weight")], [g("time_embed.time_mlp.2.bias")])
        # the linears over all B * T rows hold bfloat16 planes (DeviceLinear), and attention runs
        # on planes (cv3_attention_x3), unless planes=False
        self.planes = bool(planes)
        self.proj_in = DeviceLinear([g("input_embed.proj.weight")], [g("input_embed.proj.bias")], planes)
        self.mel = self.proj_in.k // 4
        self.conv_w, self.conv_b = [], []
        for c in ("conv1", "conv2"):
            w = g(f"input_embed.conv_pos_embed.{c}.0.weight")
            if _is_q(w):
                raise ValueError("conv_pos weights are float on this path")
            # (cout, cin/groups, k) -> (cout, k, cin/groups): K-contiguous rows for the implicit GEMM,
            # with planes held as bfloat16 planes in fragment order (cv3_conv1d_cl_x3f)
            wp = to_device(np.ascontiguousarray(np.asarray(w, np.float32).transpose(0, 2, 1)))
            cout, kk = wp.shape[0], wp.shape[1] * wp.shape[2]
            if self.planes and kk % 64 == 0:
                ne = ctypes.c_int64()
                _lib.call("x3_frag_elems", cout, kk, ctypes.byref(ne))
                fr = DeviceArray((ne.value,), np.uint16)
                _lib.call("split_x3_frag", wp.ptr, cout, kk, kk, fr.ptr, None)
                wp = fr
            self.conv_w.append(wp)
            self.conv_b.append(to_device(np.asarray(g(f"input_embed.conv_pos_embed.{c}.0.bias"), np.float32)))
        self.conv_planes = self.planes and self.conv_w[0].dtype == np.uint16
        mods = [g(f"transformer_blocks.{i}.attn_norm.linear.weight") for i in range(self.depth)]
        mods.append(g("norm_out.linear.weight"))
        mbias = [g(f"transformer_blocks.{i}.attn_norm.linear.bias") for i in range(self.depth)]
        mbias.append(g("norm_out.linear.bias"))
        self.mod = DeviceLinear(mods, mbias)
        self.ld_mod = self.mod.n
        self.qkv, self.out, self.ff1, self.ff2 = [], [], [], []
        for i in range(self.depth):
            b = f"transformer_blocks.{i}."
            self.qkv.append(DeviceLinear([g(b + f"attn.to_{p}.weight") for p in "qkv"],
                                         [g(b + f"attn.to_{p}.bias") for p in "qkv"], planes, digits=True))
            self.out.append(DeviceLinear([g(b + "attn.to_out.0.weight")], [g(b + "attn.to_out.0.bias")], planes))
            self.ff1.append(DeviceLinear([g(b + "ff.ff.0.0.weight")], [g(b + "ff.ff.0.0.bias")], planes,
                                         digits=True))
            self.ff2.append(DeviceLinear([g(b + "ff.ff.2.weight")], [g(b + "ff.ff.2.bias")], planes))
        self.ff_dim = self.ff1[0].n if self.depth else 2 * D
        self.proj_out = DeviceLinear([g("proj_out.weight")], [g("proj_out.bias")], planes)
        self._T = None
        self._graph = None
        self.halves = False                  # set by prepare() from HALVES and T
        self._side: Optional[Stream] = None
        self._ev = None

    # -- workspace ------------------------------------------------------------
    def prepare(self, mu: np.ndarray, spks: np.ndarray, cond: np.ndarray):
        """Upload the conditioning of one utterance and size the workspace.

        mu/cond (1, 80, T), spks (1, 80).  The CFG batch holds them in slot 0 and
        zeros in slot 1 (flow.py:72-77).
        """
        T = int(mu.shape[2])
        D, B, mel = self.dim, 2, self.mel
        inp = np.zeros((B, T, 4 * mel), np.float32)
        inp[0, :, mel:2 * mel] = np.asarray(cond[0], np.float32).T
        inp[0, :, 2 * mel:3 * mel] = np.asarray(mu[0], np.float32).T
        inp[0, :, 3 * mel:] = np.asarray(spks[0], np.float32)[None, :]
        self.inp = to_device(inp)
        self.halves = HALVES and T >= HALVES_MIN_T
        if self._T != T:
            self._T = T
            self.h = DeviceArray((B * T, D))
            self.n = DeviceArray((B * T, D))
            self.qkvb = DeviceArray((B * T, 3 * D))
            self.att = DeviceArray((B * T, D))
            self.ffb = DeviceArray((B * T, self.ff_dim))
            self.z1 = DeviceArray((B * T, D))
            self.outb = DeviceArray((B * T, mel))
            self.outT = DeviceArray((B, mel, T))
            self.x = DeviceArray((mel, T))
            c, s = dit_rope_tables(T, self.dim_head)
            self.cos, self.sin = to_device(c), to_device(s)
            # the row exponents of the digit-plane linears' input (the modulated norm), one at a time
            self.rexp = DeviceArray((B * T,), np.int32)
            for lin in (*self.qkv, *self.ff1):
                if lin.q8_digits:
                    lin.rexp = self.rexp
        self.ts, self.dts = euler_schedule(self.steps)
        S = self.steps
        self.sin_feat = to_device(sinus_features(self.ts))
        self.temb = DeviceArray((S, D))
        self.temb_h = DeviceArray((S, D))
        self.stemb = DeviceArray((S, D))
        self.mods = DeviceArray((S, self.ld_mod))
        self._graph = None

    # -- one estimator evaluation + Euler update ---------------------------
    def _time_and_mod(self):
        """temb = time_mlp(sinus(t_s)) for every step, then every AdaLN row (dit.py:86-90,164-167,175-177)."""
        S, D = self.steps, self.dim
        self.time0(self.sin_feat.ptr, S, 256, self.temb_h.ptr, D, _lib.epilogue("silu"))
        self.time2(self.temb_h.ptr, S, D, self.temb.ptr, D)
        _lib.call("act", ACT["silu"], 0.0, self.temb.ptr, self.stemb.ptr, S * D, None)
        self.mod(self.stemb.ptr, S, D, self.mods.ptr, self.ld_mod)

    def _norm(self, shift: int, scale: int, rexp: bool, r0: int, rows: int, st):
        """n = LN(h) (1 + scale) + shift over rows r0 .. r0 + rows (dit.py:168-169), with the rows'
        exponents into ``self.rexp`` when a digit-plane linear reads n next."""
        D = self.dim
        h, n = self.h.ptr + 4 * r0 * D, self.n.ptr + 4 * r0 * D
        if rexp:
            _lib.call("layer_norm_rexp", h, n, rows, D, 1e-6, None, None, shift, scale, 0, 0,
                      self.rexp.ptr + 4 * r0, st)
        else:
            _lib.call("layer_norm", h, n, rows, D, 1e-6, None, None, shift, scale, 0, 0, st)

    def _block(self, i: int, mrow: int, r0: int, nb: int, st):
        """Transformer block i (dit.py:114-141,160-171) over batch rows r0 / T .. + nb of the CFG
        pair, on stream handle ``st``."""
        T, D, H, dh, f4 = self._T, self.dim, self.heads, self.dim_head, 4
        S3 = ctypes.c_int64 * 3
        rows = nb * T
        h, n, att = (a.ptr + f4 * r0 * D for a in (self.h, self.n, self.att))
        qkvb, ffb = self.qkvb.ptr + f4 * r0 * 3 * D, self.ffb.ptr + f4 * r0 * self.ff_dim
        qs = S3(T * 3 * D, dh, 3 * D)
        os_ = S3(T * D, dh, D)
        scale = float(np.float32(1.0 / math.sqrt(dh)))
        base = mrow + i * 6 * D * f4
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = (base + j * D * f4 for j in range(6))
        self._norm(sh_a, sc_a, self.qkv[i].q8_digits, r0, rows, st)
        # partial rotary on q and k, channels 0..dh-1 (dit.py:119-120), in the GEMM epilogue
        rope_epi = _lib.epilogue(rope=(self.cos.ptr, self.sin.ptr, T, D, dh, 2 * D))
        self.qkv[i](n, rows, D, qkvb, 3 * D, rope_epi, rexp_given=True, st=st, rexp_row0=r0)
        _lib.call("attention_x3" if self.planes else "attention", qkvb, qkvb + D * f4, qkvb + 2 * D * f4, att,
                  nb, H, H, T, T, dh, qs, qs, qs, os_, scale, 0, 0, 0, st)
        self.out[i](att, rows, D, h, D,
                    _lib.epilogue(residual=h, ld_res=D, gate=g_a, gate_stride=0, rows_per_gate=1), st=st)
        self._norm(sh_m, sc_m, self.ff1[i].q8_digits, r0, rows, st)
        self.ff1[i](n, rows, D, ffb, self.ff_dim, _lib.epilogue("gelu_tanh"), rexp_given=True, st=st, rexp_row0=r0)
        self.ff2[i](ffb, rows, self.ff_dim, h, D,
                    _lib.epilogue(residual=h, ld_res=D, gate=g_m, gate_stride=0, rows_per_gate=1), st=st)

    def _step(self, s: int, dt: float, update: bool = True):
        T, D, B, mel, H, dh = self._T, self.dim, 2, self.mel, self.heads, self.dim_head
        BT = B * T
        f4 = 4
        S3 = ctypes.c_int64 * 3
        # x (80, T) -> columns 0..79 of both batch rows of the packed input (dit.py:151-153,96)
        _lib.call("copy_strided", self.x.ptr, self.inp.ptr, B, T, mel, S3(0, 1, T), S3(T * 4 * mel, 4 * mel, 1),
                  None)
        self.proj_in(self.inp.ptr, BT, 4 * mel, self.h.ptr, D)
        # conv_pos: two grouped causal convs with Mish on channels-last [B*T, D] activations,
        # the second adding the projection back in place (dit.py:99-112)
        k = self.conv_k
        conv = "conv1d_cl_x3f" if self.conv_planes else "conv1d_cl"
        _lib.call(conv, self.h.ptr, B, T, D, D, self.conv_w[0].ptr, D, k, self.conv_groups, k - 1,
                  self.conv_b[0].ptr, self.z1.ptr, D, ctypes.byref(_lib.epilogue("mish")), None)
        _lib.call(conv, self.z1.ptr, B, T, D, D, self.conv_w[1].ptr, D, k, self.conv_groups, k - 1,
                  self.conv_b[1].ptr, self.h.ptr, D,
                  ctypes.byref(_lib.epilogue("mish", residual=self.h.ptr, ld_res=D)), None)
        mrow = self.mods.ptr + s * self.ld_mod * f4
        if self.halves:
            # the CFG pair's two batch rows are independent through every block: the second on
            # a side stream, forked and joined around the blocks (graph edges under capture)
            if self._side is None:
                self._side, self._ev = Stream(), (Event(), Event())
            self._ev[0].record(None)
            self._side.wait(self._ev[0])
            for i in range(self.depth):
                self._block(i, mrow, 0, 1, None)
                self._block(i, mrow, T, 1, self._side.handle)
            self._ev[1].record(self._side)
            wait_event(self._ev[1])
        else:
            for i in range(self.depth):
                self._block(i, mrow, 0, B, None)
        base = mrow + self.depth * 6 * D * f4      # norm_out: (scale, shift) (dit.py:175-178)
        _lib.call("layer_norm", self.h.ptr, self.n.ptr, BT, D, 1e-6, None, None, base + D * f4, base, 0, 0, None)
        self.proj_out(self.n.ptr, BT, D, self.outb.ptr, mel)
        # (B, T, 80) -> (B, 80, T), then x += dt ((1 + w) d0 - w d1)  (dit.py:180, flow.py:86-87)
        _lib.call("copy_strided", self.outb.ptr, self.outT.ptr, B, T, mel, S3(T * mel, mel, 1),
                  S3(mel * T, 1, T), None)
        if not update:
            return
        _lib.call("cfg_euler", self.x.ptr, self.outT.ptr, self.outT.ptr + mel * T * f4, mel * T,
                  float(dt), float(self.cfg_rate), None)

    def _enqueue_solve(self):
        self._time_and_mod()
        for s in range(self.steps):
            self._step(s, float(self.dts[s]))

    def solve(self, x0: np.ndarray, graph: bool = False) -> DeviceArray:
        """Euler solve from x0 (1, 80, T) (already scaled by the temperature); returns the
        resident (80, T) result.  ``graph=True`` replays one captured HIP graph."""
        self.x.copy_from(np.asarray(x0, np.float32).reshape(self.mel, self._T))
        if not graph:
            self._enqueue_solve()
            return self.x
        if self._graph is None:
            g = Graph()
            with g:
                self._enqueue_solve()
            self._graph = g
        self._graph.launch()
        return self.x

    def estimate(self, x0: np.ndarray, s: int) -> np.ndarray:
        """One estimator evaluation at the s-th Euler time on the CFG pair built from x0 (1, 80, T);
        returns the (2, 80, T) velocity, i.e. ``DiT.forward`` (dit.py:144-180) without the update."""
        self.x.copy_from(np.asarray(x0, np.float32).reshape(self.mel, self._T))
        self._time_and_mod()
        self._step(s, 0.0, update=False)
        return self.outT.numpy()

    def flops_by_unit(self):
        """Flops of one solve by how they run: (float32 weights on bfloat16 planes, six
        products each; q8 weights on bfloat16 planes, three products each; the rest on the
        float32 matrix cores; per-channel q8 weights on the int8 matrix cores, four digit-plane
        products each)."""
        T, D, B = self._T, self.dim, 2
        M = B * T
        lins = [*self.qkv, *self.out, *self.ff1, *self.ff2, self.proj_in, self.proj_out]
        six = self.steps * sum(2.0 * M * l.n * l.k for l in lins if l.planes is not None)
        if self.planes and self.dim_head == 64:   # attention on planes too (cv3_attention_x3)
            six += self.steps * self.depth * 4.0 * B * self.heads * T * T * self.dim_head
        if self.conv_planes:                      # the conv_pos convs (cv3_conv1d_cl_x3f)
            six += self.steps * 2 * 2.0 * M * D * (D // self.conv_groups) * self.conv_k
        three = self.steps * sum(2.0 * M * l.n * l.k for l in lins if l.q8 and l.q8_planes)
        four = self.steps * sum(2.0 * M * l.n * l.k for l in lins if l.q8_digits)
        return six, three, self.flops_per_solve() - six - three - four, four

    def flops_per_solve(self) -> float:
        """Algorithmic flops of one solve (every contraction, 2 flops per MAC)."""
        T, D, B = self._T, self.dim, 2
        M = B * T
        per_block = 2 * M * D * (3 * D + D + 2 * self.ff_dim) + 4 * B * self.heads * T * T * self.dim_head
        conv = 2 * 2 * M * D * (D // self.conv_groups) * self.conv_k
        edges = 2 * M * (4 * self.mel) * D + 2 * M * D * self.mel
        mod = 2 * self.ld_mod * D * B
        return float(self.steps * (self.depth * per_block + conv + edges + mod))
