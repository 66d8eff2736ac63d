"""Device-resident causal HiFTNet: F0 -> NSF source -> source STFT -> conv stack -> iSTFT head.

Restates cv3cpu/models/hift.py:114-210 (``_resblock``, ``_spectral``,
``_spectral_chunked``, ``decode``) with every activation resident in HBM.  Inside the
stack activations are channels-last (time, channels): a stride-1 conv is then an
implicit GEMM whose A rows are shifted input rows, fed to LDS by DMA
(cv3_conv1d_cl_packed).  The mel and the source STFT come in the reference's
(channels, time) layout and are read through strides by the first convs; conv_post
writes (channels, time) for the iSTFT head.

``inference`` runs the whole vocoder on the device (hift.py:212-218): the F0
predictor's five causal convs + ELU (float32, like the reference's conv1d) and its
classifier summed in float64 (cv3_f0_classify), then the excitation
(cv3_nsf_source: float64 harmonic phase, dither, Linear(9 -> 1), tanh), then
``decode``.  The dither buffer is the seeded TorchMT19937 draw of hift.py:75-81,
made once on the host replica and kept in HBM.

Per upsampling stage i (reference lines in brackets):
  leaky(x, 0.1), nearest x r_i fused into the causal ``ups`` conv      (hift.py:137-142)
  last stage: reflect pad (1, 0) as a one-column copy                  (hift.py:143-144)
  source_downs conv on the source STFT (stride u_i) + source resblock  (hift.py:145-156)
  x + s, then the mean of three resblocks                              (hift.py:157-165)
A resblock's step is  snake(x, a1) -> dilated causal conv with snake(., a2) in its
epilogue -> causal conv with the residual x added in its epilogue  (hift.py:114-129).
"""

from __future__ import annotations

import ctypes
from typing import List, Optional

import numpy as np

from . import _lib
from .device import DeviceArray, Event, Graph, Stream, to_device, wait_event

ACT = _lib.ACT
F4 = 4
# The whole-input spectral stack's independent branches (each stage's source branch beside its
# upsampling conv, and its resblocks side by side) run on side streams forked off the thread's
# stream when the stack is recorded and captured; in the graph the forks and joins are edges.
# 10 s whole: 4.12 -> 3.37 ms.  The 1 s windows already run side by side on WINDOW_STREAMS
# streams, and their stacks with branches took 12.0 ms against 7.76, so they keep none.
BRANCHES = True
WINDOW_STREAMS = 16  # vocoder windows replayed side by side (one stream each, default priority); a
                     # 10 s decode in 1 s windows: 4 streams 10.1 ms, 10 or 16 streams 7.4 ms


def causal_pad(kernel_size: int, dilation: int = 1) -> int:
    """int((k d - d) / 2) * 2 + (k + 1) % 2 (hift.py:14-16)."""
    return int((kernel_size * dilation - dilation) / 2) * 2 + (kernel_size + 1) % 2


def receptive_frames(rates, up_k, rb_k, rb_d, src_k, src_d, src_kd, post_k) -> int:
    """Mel frames of history that the spectral stack's output at a frame depends on: the first
    output row of a frame far from the start is followed back through conv_post, the resblocks
    (each step reads (k - 1) d + (k - 1) rows back), the upsampling convs (nearest upsample,
    pad k - 1), the reflect-padded row of the last stage, and the strided source convs to the
    first mel frame and the first source-STFT frame it reads (hift.py:131-168).  conv_pre and
    the source STFT look only forward or at their own frame.  ``src_kd`` lists the source
    convs' kernel sizes; ``up_k`` the upsampling convs'."""
    up = int(np.prod(rates))
    m0 = 1 << 20                          # far from the start: no row is clamped at zero
    a = 1 + m0 * up - causal_pad(post_k)  # the frame's first output row, then conv_post's reach

    def resblock(k, dils, a):
        for d in reversed(dils):
            a -= causal_pad(k, d) + causal_pad(k, 1)
        return a

    downs = [1] + list(rates[::-1][:-1])
    down_cum = list(np.cumprod(downs))[::-1]
    first_src = a
    for i in reversed(range(len(rates))):
        a_xs = min(resblock(k, d, a) for k, d in zip(rb_k, rb_d))
        u = int(down_cum[i])
        a_si = resblock(src_k[i], src_d[i], a_xs)
        first_src = min(first_src, a_si * u - (causal_pad(src_kd[i]) if u == 1 else u - 1))
        a_c = a_xs - 1 if i == len(rates) - 1 else a_xs  # the last stage's rows sit one down
        a = (a_c - (up_k[i] - 1)) // rates[i]
    frames = max(m0 - a, m0 - first_src // up)
    return int(frames)


def split_k(t_out: int, cout: int, stages: int, even: bool = False) -> int:
    """K slices for the packed conv: grids under 160 tiles of 64 x 64 (a 1 s chunk's
    256-channel stage has 60) are split until they cover about two tiles per CU; the
    slices divide the k*cin/32 stages evenly (``even``: into an even count per slice, as the
    bfloat16-plane conv needs)."""
    tiles = -(-t_out // 64) * -(-cout // 64)
    if tiles >= 160:
        return 1
    step = 2 if even else 1
    for ks in (8, 6, 4, 3, 2):
        if tiles * ks <= 512 and stages % (ks * step) == 0:
            return ks
    return 1


def hann_window(n: int) -> np.ndarray:
    """Periodic Hann window, float64 -> float32 (ops.py:339-343)."""
    i = np.arange(n, dtype=np.float64)
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * i / n)).astype(np.float32)


class DeviceHiFT:
    """HiFTNet weights resident in HBM; ``weights`` has ``get(name)`` and ``meta``."""

    def __init__(self, weights, prefix: str = "hift.", planes: bool = True, trim_context: bool = True):
        """``planes``: the channels-last convs run on the bfloat16 matrix cores with their
        weights held as three bfloat16 planes in the matrix cores' fragment order
        (cv3_conv1d_cl_packed_x3f: the same float32 conv, errors against float64 below the
        float32 matrix cores'); False keeps them on the float32 matrix cores.
        ``trim_context``: a window of the windowed decode carries min(context, receptive field)
        frames of history rather than all ``context`` frames: the frames beyond the stack's
        receptive field cannot reach a kept sample, so the output is the same."""
        _lib.init()
        m = weights.meta.get("hift", {})
        self.rates = list(m.get("upsample_rates", [8, 5, 3]))
        self.rb_k = list(m.get("resblock_kernel_sizes", [3, 7, 11]))
        self.rb_d = [list(d) for d in m.get("resblock_dilation_sizes", [[1, 3, 5]] * 3)]
        self.src_k = list(m.get("source_resblock_kernel_sizes", [7, 7, 11]))
        self.src_d = [list(d) for d in m.get("source_resblock_dilation_sizes", [[1, 3, 5]] * 3)]
        self.n_fft = int(m.get("istft_n_fft", 16))
        self.hop = int(m.get("istft_hop_len", 4))
        self.slope = float(m.get("lrelu_slope", 0.1))
        self.limit = float(m.get("audio_limit", 0.99))
        self.sampling_rate = int(m.get("sampling_rate", 24000))
        self.harmonics = int(m.get("nb_harmonics", 8)) + 1
        self.nsf_alpha = float(m.get("nsf_alpha", 0.1))
        self.nsf_sigma = float(m.get("nsf_sigma", 0.003))
        self.nsf_threshold = float(m.get("nsf_voiced_threshold", 10.0))
        self.noise_seed = int(m.get("noise_seed", 0))
        self.nk = len(self.rb_k)
        self.up_total = int(np.prod(self.rates))
        self.trim_context = trim_context
        self.w = {}
        self.wp = {}   # conv weights repacked (out, k, in) for the channels-last implicit GEMM
        self.wpx = {}  # ... and as three bfloat16 planes in fragment order (planes=True)
        self.shape = {}
        for name in weights.keys():
            if not name.startswith(prefix) or "f0_predictor.classifier" in name or "m_source" in name:
                continue
            arr = np.asarray(weights.get(name), np.float32)
            key = name[len(prefix):]
            self.w[key] = to_device(np.ascontiguousarray(arr))
            self.shape[key] = arr.shape
            if arr.ndim == 3 and arr.shape[1] % 32 == 0:
                self.wp[key] = to_device(np.ascontiguousarray(arr.transpose(0, 2, 1)))
                cout, kin = arr.shape[0], arr.shape[1] * arr.shape[2]
                if planes and (kin // 32) % 2 == 0:
                    ne = ctypes.c_int64()
                    _lib.call("x3_frag_elems", cout, kin, ctypes.byref(ne))
                    pl = DeviceArray((ne.value,), np.uint16)
                    _lib.call("split_x3_frag", self.wp[key].ptr, cout, kin, kin, pl.ptr, None)
                    self.wpx[key] = pl
        self.receptive = receptive_frames(
            self.rates, [self.shape[f"ups.{i}.weight"][2] for i in range(len(self.rates))], self.rb_k, self.rb_d,
            self.src_k, self.src_d, [self.shape[f"source_downs.{i}.weight"][2] for i in range(len(self.rates))],
            self.shape["conv_post.weight"][2])
        # the F0 predictor's condnet convs sit with the stack's weights above; its
        # classifier and the source merge (hift.py:56-72,108-110) are float32 vectors
        self.f0_depth = 0
        while f"f0_predictor.condnet.{self.f0_depth}.weight" in self.shape:
            self.f0_depth += 1
        cls = f"{prefix}f0_predictor.classifier."
        self.f0_cls = None
        if cls + "weight" in weights:
            self.f0_cls = (to_device(np.asarray(weights.get(cls + "weight"), np.float32).reshape(-1)),
                           to_device(np.asarray(weights.get(cls + "bias"), np.float32).reshape(-1)))
        lin = f"{prefix}m_source.l_linear."
        self.l_linear = None
        if lin + "weight" in weights:
            lw = np.asarray(weights.get(lin + "weight"), np.float32).reshape(-1)
            if lw.size != self.harmonics:
                raise ValueError(f"m_source.l_linear has {lw.size} inputs, expected {self.harmonics} harmonics")
            self.l_linear = (to_device(lw), to_device(np.asarray(weights.get(lin + "bias"), np.float32).reshape(-1)))
        self._noise: Optional[DeviceArray] = None
        self.window = to_device(hann_window(self.n_fft))
        # captured spectral stacks, one per input length: (graph, mel in, source STFT in, out, arena)
        self._graphs = {}
        self._streams: List[Stream] = []
        self._recorded = set()   # (width, slot, stream) whose stack buffers are recorded on the stream
        self._side: List[Stream] = []   # branch streams of the spectral stack (BRANCHES)
        self._branch = False             # set while a whole-input stack is recorded and captured
        self._ev: List[Event] = []
        self._arena = None       # while recording or capturing: every intermediate of the stack
        self._arena_i = -1       # >= 0 while capturing: the next arena entry to hand out

    def _new(self, shape) -> DeviceArray:
        """A fresh intermediate.  While a stack is recorded, every intermediate is kept
        (the arena); while it is captured, the recorded arrays are handed out again in
        order, so the capture allocates and frees nothing and the graph owns its memory."""
        if self._arena is None:
            return DeviceArray(shape)
        if self._arena_i >= 0:
            a = self._arena[self._arena_i]
            self._arena_i += 1
            if a.shape != tuple(shape):
                raise RuntimeError(f"captured stack diverged from its recording: {a.shape} vs {tuple(shape)}")
            return a
        a = DeviceArray(shape)
        self._arena.append(a)
        return a

    # -- building blocks ------------------------------------------------------
    def _conv(self, x: DeviceArray, key: str, dilation: int = 1, pad=(0, 0), up: int = 1,
              act: str = "none", act_param: float = 0.0, snake: Optional[str] = None,
              residual: Optional[DeviceArray] = None, out: Optional[DeviceArray] = None, out_row0: int = 0,
              channels_first_out: bool = False, st: Optional[int] = None) -> DeviceArray:
        """Stride-1 conv1d (ops.py:165-219) on channels-last x (T_in, C_in) -> (T_out, C_out),
        or (C_out, T_out) with ``channels_first_out``; nearest upsample, activation / Snake
        and residual (channels-last) fused."""
        cout, cin, k = self.shape[key + ".weight"]
        t_in, c = x.shape
        if c != cin:
            raise ValueError(f"{key}: input has {c} channels, weight expects {cin}")
        n = max(0, t_in * up + pad[0] + pad[1] - dilation * (k - 1))
        if out is None:
            out = self._new((cout, n) if channels_first_out else (n, cout))
        y_ts, y_cs = (1, out.shape[1]) if channels_first_out else (out.shape[1], 1)
        alpha = self.w[snake].ptr if snake else None
        res = residual.ptr if residual is not None else None
        r_ts = residual.shape[1] if residual is not None else 0
        wkey = key + ".weight"
        if wkey in self.wpx:  # the bfloat16-plane implicit GEMM, weights in fragment order
            ks = split_k(n, cout, k * cin // 32, even=True)
            ws = self._new((ks * cout * n,)) if ks > 1 else None
            _lib.call("conv1d_cl_packed_x3f", x.ptr, t_in, cin, cin, self.wpx[wkey].ptr, cout, k,
                      self.w[key + ".bias"].ptr, dilation, pad[0], pad[1], up, out.ptr + out_row0 * y_ts * F4, y_ts,
                      y_cs, ACT[act], float(act_param), alpha, 1e-9, res, r_ts, 1, ks, ws.ptr if ws else None,
                      ws.size if ws else 0, st)
        elif wkey in self.wp:   # cin % 32 == 0: the DMA implicit GEMM
            ks = split_k(n, cout, k * cin // 32)
            ws = self._new((ks * cout * n,)) if ks > 1 else None
            _lib.call("conv1d_cl_packed", x.ptr, t_in, cin, cin, self.wp[wkey].ptr, cout, k,
                      self.w[key + ".bias"].ptr, dilation, pad[0], pad[1], up, out.ptr + out_row0 * y_ts * F4, y_ts,
                      y_cs, ACT[act], float(act_param), alpha, 1e-9, res, r_ts, 1, ks, ws.ptr if ws else None,
                      ws.size if ws else 0, st)
        else:                 # narrow stacks: the generic kernel, addressed channels-last
            _lib.call("conv1d", x.ptr, cin, t_in, 1, cin, self.w[wkey].ptr, cout, k, self.w[key + ".bias"].ptr, 1,
                      dilation, 1, pad[0], pad[1], up, out.ptr + out_row0 * y_ts * F4, y_cs, y_ts, None,
                      ACT[act], float(act_param), alpha, 1e-9, res, 1, r_ts, st)
        return out

    def _conv_in(self, x: DeviceArray, key: str, stride: int = 1, pad=(0, 0), act: str = "none",
                 act_param: float = 0.0, st: Optional[int] = None) -> DeviceArray:
        """conv1d (ops.py:165-219) from channels-first x (C_in, T_in) to channels-last output,
        for the convs on the stack's inputs (conv_pre on the mel, the strided source_downs on
        the source STFT), through the generic strided kernel."""
        cout, cin, k = self.shape[key + ".weight"]
        c, t_in = x.shape
        if c != cin:
            raise ValueError(f"{key}: input has {c} channels, weight expects {cin}")
        n = max(0, (t_in + pad[0] + pad[1] - k) // stride + 1)
        out = self._new((n, cout))
        _lib.call("conv1d", x.ptr, cin, t_in, t_in, 1, self.w[key + ".weight"].ptr, cout, k,
                  self.w[key + ".bias"].ptr, stride, 1, 1, pad[0], pad[1], 1, out.ptr, 1, cout, None,
                  ACT[act], float(act_param), None, 0.0, None, 0, 0, st)
        return out

    def _snake(self, x: DeviceArray, key: str, st: Optional[int] = None) -> DeviceArray:
        y = self._new(x.shape)
        _lib.call("snake_cl", x.ptr, self.w[key].ptr, y.ptr, x.shape[0], x.shape[1], 1e-9, st)
        return y

    def _act(self, x: DeviceArray, name: str, param: float) -> DeviceArray:
        y = self._new(x.shape)
        _lib.call("act", ACT[name], float(param), x.ptr, y.ptr, x.size, None)
        return y

    def _resblock(self, group: str, idx: int, x: DeviceArray, kernel: int, dilations,
                  st: Optional[int] = None) -> DeviceArray:
        """3 x [snake, dilated causal conv, snake, causal conv] + residual (hift.py:114-129),
        on stream handle ``st`` (None: the thread's).  ``x`` is left untouched; the result is a
        new buffer."""
        base = f"{group}.{idx}."
        cur = x
        for j, d in enumerate(dilations):
            y = self._snake(cur, base + f"activations1.{j}.alpha", st)
            y = self._conv(y, base + f"convs1.{j}", dilation=d, pad=(causal_pad(kernel, d), 0),
                           snake=base + f"activations2.{j}.alpha", st=st)
            out = self._new(x.shape) if cur is x else cur   # in place after the first step
            cur = self._conv(y, base + f"convs2.{j}", pad=(causal_pad(kernel, 1), 0), residual=cur, out=out, st=st)
        return cur

    def _branches(self, n: int):
        """n side streams and n + 1 events for forking independent branches off the thread's
        stream (inside a capture the forks and joins become graph edges)."""
        while len(self._side) < n:
            self._side.append(Stream())
        while len(self._ev) < n + 1:
            self._ev.append(Event())
        return self._side[:n], self._ev[:n + 1]

    # -- the spectral stack -------------------------------------------------
    def spectral(self, mel: DeviceArray, s_stft: DeviceArray) -> DeviceArray:
        """conv_pre .. conv_post: (80, T) -> (n_fft + 2, 120 T + 1) (hift.py:131-168)."""
        kpre = self.shape["conv_pre.weight"][2]
        x = self._conv_in(mel, "conv_pre", pad=(0, causal_pad(kpre)))
        downs = [1] + self.rates[::-1][:-1]
        down_cum = list(np.cumprod(downs))[::-1]
        # branches only while a stack is recorded or captured: its arena keeps every
        # intermediate alive, so no buffer a side stream uses is freed and reused meanwhile
        branch = self._branch and self._arena is not None
        for i, r in enumerate(self.rates):
            if branch:  # the source branch beside the leaky + upsampling conv
                side, ev = self._branches(max(1, self.nk - 1))
                sst = side[0].handle
                ev[0].record(None)
                side[0].wait(ev[0])
            else:
                sst = None
            xl = self._act(x, "leaky", self.slope)
            k = self.shape[f"ups.{i}.weight"][2]
            cout = self.shape[f"ups.{i}.weight"][0]
            t_up = x.shape[0] * r
            if i == len(self.rates) - 1:
                # reflect pad (1, 0): rows 1.. hold the conv, row 0 copies row 2 (hift.py:144)
                xu = self._new((t_up + 1, cout))
                self._conv(xl, f"ups.{i}", up=r, pad=(k - 1, 0), out=xu, out_row0=1)
                S3 = ctypes.c_int64 * 3
                _lib.call("copy_strided", xu.ptr + 2 * cout * F4, xu.ptr, 1, 1, cout, S3(0, 0, 1), S3(0, 0, 1),
                          None)
            else:
                xu = self._conv(xl, f"ups.{i}", up=r, pad=(k - 1, 0))
            u = int(down_cum[i])
            ks = self.shape[f"source_downs.{i}.weight"][2]
            if u == 1:
                si = self._conv_in(s_stft, f"source_downs.{i}", pad=(causal_pad(ks), 0), st=sst)
            else:
                si = self._conv_in(s_stft, f"source_downs.{i}", stride=u, pad=(u - 1, 0), st=sst)
            si = self._resblock("source_resblocks", i, si, self.src_k[i], self.src_d[i], st=sst)
            if branch:
                ev[1].record(side[0])
                wait_event(ev[1])
            if si.shape != xu.shape:
                raise ValueError(f"stage {i}: source branch {si.shape} vs upsampled {xu.shape}")
            xs = self._new(xu.shape)
            _lib.call("binary", 0, xu.ptr, si.ptr, xs.ptr, xs.size, 0.0, 0.0, None)
            # the resblocks read xs and write their own buffers: resblock j > 0 on side stream
            # j - 1, joined before the sum
            if branch:
                ev[0].record(None)
                for sd in side:
                    sd.wait(ev[0])
            rs = [self._resblock("resblocks", i * self.nk + j, xs, self.rb_k[j], self.rb_d[j],
                                 st=side[j - 1].handle if branch and j > 0 else None)
                  for j in range(self.nk)]
            if branch:
                for j, sd in enumerate(side):
                    ev[j + 1].record(sd)
                    wait_event(ev[j + 1])
            acc = rs[0]
            for j in range(1, self.nk):
                nxt = self._new(xs.shape)
                if j == self.nk - 1:   # ((r0 + r1) + r2) / 3 (hift.py:161-165)
                    _lib.call("binary", 4, acc.ptr, rs[j].ptr, nxt.ptr, nxt.size, float(self.nk), 0.0, None)
                else:
                    _lib.call("binary", 0, acc.ptr, rs[j].ptr, nxt.ptr, nxt.size, 0.0, 0.0, None)
                acc = nxt
            x = acc
        x = self._act(x, "leaky", 0.01)
        kpost = self.shape["conv_post.weight"][2]
        return self._conv(x, "conv_post", pad=(causal_pad(kpost), 0), channels_first_out=True)

    def _stack(self, w: int, slot: int = 0, branches: bool = False):
        """The spectral stack for a w-frame input, captured once per (w, slot): its staging
        inputs, its output and the graph (each slot owns its buffers, so windows on
        different streams run side by side).  Recorded eagerly first (on zeroed inputs),
        then captured with the recorded intermediates (see ``_new``)."""
        g = self._graphs.get((w, slot, branches))
        if g is None:
            mel_w = DeviceArray((self.shape["conv_pre.weight"][1], w))
            st_w = DeviceArray((self.n_fft + 2, w * self.up_total + 1))
            _lib.call("fill_zero", mel_w.ptr, mel_w.nbytes, None)
            _lib.call("fill_zero", st_w.ptr, st_w.nbytes, None)
            self._arena, self._arena_i = [], -1
            self._branch = branches and BRANCHES
            try:
                out = self.spectral(mel_w, st_w)
                self._arena_i = 0
                graph = Graph()
                with graph:
                    again = self.spectral(mel_w, st_w)
                if again is not out or self._arena_i != len(self._arena):
                    raise RuntimeError("captured stack diverged from its recording")
                g = (graph, mel_w, st_w, out, self._arena)
            finally:
                self._arena, self._arena_i = None, -1
                self._branch = False
            self._graphs[(w, slot, branches)] = g
        return g

    def spectral_graph(self, mel: DeviceArray, s_stft: DeviceArray, c0: int = 0, c1: Optional[int] = None,
                       slot: int = 0, stream: Optional[Stream] = None, branches: bool = False):
        """spectral() of mel[:, c0:c1] and its source STFT columns by graph replay on ``stream``
        (None: the calling thread's); returns the stack's own output buffer, valid until the
        next replay of the same (length, slot)."""
        t = mel.shape[1]
        c1 = t if c1 is None else c1
        w = c1 - c0
        graph, mel_w, st_w, out, arena = self._stack(w, slot, branches)
        S3 = ctypes.c_int64 * 3
        up = self.up_total
        sh = stream.handle if stream is not None else None
        if sh is not None and (w, slot, sh) not in self._recorded:
            # the stack's buffers are used on that stream: their blocks wait for it when freed
            for a in (mel_w, st_w, out, *arena):
                a.record_stream(stream)
            self._recorded.add((w, slot, sh))
        _lib.call("copy_strided", mel.ptr + c0 * F4, mel_w.ptr, 1, mel.shape[0], w, S3(0, t, 1), S3(0, w, 1), sh)
        fs = s_stft.shape[1]
        f0, f1 = c0 * up, min(fs, c1 * up + 1)
        if f1 - f0 != st_w.shape[1]:
            raise ValueError(f"source STFT has {fs} frames, expected {t * up + 1}")
        _lib.call("copy_strided", s_stft.ptr + f0 * F4, st_w.ptr, 1, s_stft.shape[0], f1 - f0, S3(0, fs, 1),
                  S3(0, f1 - f0, 1), sh)
        graph.launch(stream)
        return out

    def spectral_chunked(self, mel: DeviceArray, s_stft: DeviceArray, chunk: int, context: int,
                         graph: bool = True) -> DeviceArray:
        """Windows of ``chunk`` frames with ``context`` frames of history and conv_pre's
        lookahead, cut back to the window's own samples (hift.py:170-194).  With
        ``trim_context`` the history stops at the stack's receptive field (``receptive``
        frames), which reproduces the full-utterance result as the whole context does."""
        if self.trim_context:
            context = min(context, self.receptive)
        up = self.up_total
        t = mel.shape[1]
        look = causal_pad(self.shape["conv_pre.weight"][2])
        nout = self.n_fft + 2
        out = DeviceArray((nout, t * up + 1))
        S3 = ctypes.c_int64 * 3
        starts = list(range(0, t, chunk))
        # graph replay: the windows are independent, so they run side by side on up to
        # WINDOW_STREAMS streams (window i on stream i mod n), each with its own captured
        # stack; the thread's stream waits for all of them before anything reads `out`
        streams = self._window_streams(min(WINDOW_STREAMS, len(starts))) if graph else []
        if streams:
            for i, m0 in enumerate(starts):  # build (record + capture) every stack first, on this stream
                self._stack(min(t, m0 + chunk + look) - max(0, m0 - context), i % len(streams))
            ready = Event().record()
            for st in streams:
                st.wait(ready)
                out.record_stream(st)
        for i, m0 in enumerate(starts):
            m1 = min(t, m0 + chunk)
            c0 = max(0, m0 - context)
            c1 = min(t, m1 + look)
            lead = (m0 - c0) * up
            take = (m1 - m0) * up
            src0, dst0, n = (0, 0, 1 + take) if m0 == 0 else (1 + lead, 1 + m0 * up, take)
            if graph:
                slot = i % len(streams)
                st = streams[slot]
                sub = self.spectral_graph(mel, s_stft, c0, c1, slot=slot, stream=st)
                _lib.call("copy_strided", sub.ptr + src0 * F4, out.ptr + dst0 * F4, 1, nout, n,
                          S3(0, sub.shape[1], 1), S3(0, t * up + 1, 1), st.handle)
                continue
            sub_mel = DeviceArray((mel.shape[0], c1 - c0))
            _lib.call("copy_strided", mel.ptr + c0 * F4, sub_mel.ptr, 1, mel.shape[0], c1 - c0,
                      S3(0, t, 1), S3(0, c1 - c0, 1), None)
            fs = s_stft.shape[1]
            f0, f1 = c0 * up, min(fs, c1 * up + 1)
            sub_s = DeviceArray((s_stft.shape[0], f1 - f0))
            _lib.call("copy_strided", s_stft.ptr + f0 * F4, sub_s.ptr, 1, s_stft.shape[0], f1 - f0,
                      S3(0, fs, 1), S3(0, f1 - f0, 1), None)
            sub = self.spectral(sub_mel, sub_s)
            _lib.call("copy_strided", sub.ptr + src0 * F4, out.ptr + dst0 * F4, 1, nout, n,
                      S3(0, sub.shape[1], 1), S3(0, t * up + 1, 1), None)
        for st in streams:
            wait_event(Event().record(st))
        return out

    def _window_streams(self, n: int) -> List[Stream]:
        while len(self._streams) < n:
            self._streams.append(Stream())
        return self._streams[:n]

    def source_stft(self, source: DeviceArray) -> DeviceArray:
        """(n_fft + 2, frames) real / imaginary stack of the source STFT (hift.py:198-199)."""
        frames = ctypes.c_int64()
        _lib.call("stft", source.ptr, source.size, self.n_fft, self.hop, self.window.ptr, 1, None, None,
                  _lib.ptr(frames), None)
        half = self.n_fft // 2 + 1
        s = DeviceArray((2 * half, frames.value))
        _lib.call("stft", source.ptr, source.size, self.n_fft, self.hop, self.window.ptr, 1, s.ptr,
                  s.ptr + half * frames.value * F4, None, None)
        return s

    def istft_head(self, x: DeviceArray) -> DeviceArray:
        """clip(exp(min(x,80)),100) magnitude, sin(x) phase, iSTFT, clip +-limit (hift.py:204-210)."""
        half = self.n_fft // 2 + 1
        frames = x.shape[1]
        buf = DeviceArray((frames, self.n_fft))
        n = ctypes.c_int64()
        _lib.call("istft", 1, x.ptr, x.ptr + half * frames * F4, frames, self.n_fft, self.hop, self.window.ptr, 1,
                  -1, self.limit, buf.ptr, None, _lib.ptr(n), None)
        y = DeviceArray((n.value,))
        _lib.call("istft", 1, x.ptr, x.ptr + half * frames * F4, frames, self.n_fft, self.hop, self.window.ptr, 1,
                  -1, self.limit, buf.ptr, y.ptr, None, None)
        return y

    def decode(self, mel, source, chunk: Optional[int] = None, context: int = 64, graph: bool = True) -> DeviceArray:
        """(80, T) mel + (480 T,) source -> (480 T,) waveform (hift.py:196-210).  Host or
        device inputs; the result stays resident.  With ``graph`` the spectral stack of each
        input length is captured on first use and replayed (one launch per window)."""
        mel_d = mel if isinstance(mel, DeviceArray) else to_device(np.ascontiguousarray(mel, np.float32))
        src_d = source if isinstance(source, DeviceArray) else to_device(np.ascontiguousarray(source, np.float32))
        s_stft = self.source_stft(src_d)
        if chunk is None or mel_d.shape[1] <= chunk:
            x = self.spectral_graph(mel_d, s_stft, branches=True) if graph else self.spectral(mel_d, s_stft)
        else:
            x = self.spectral_chunked(mel_d, s_stft, chunk, context, graph=graph)
        return self.istft_head(x)

    # -- the source: F0 predictor + NSF excitation --------------------------------
    def f0_predict(self, mel) -> DeviceArray:
        """(80, T) mel -> (T,) F0 (hift.py:56-72), returned as the float32 values
        inference() feeds the excitation (hift.py:216)."""
        if not self.f0_depth or self.f0_cls is None:
            raise ValueError("the weights hold no f0_predictor")
        mel_d = mel if isinstance(mel, DeviceArray) else to_device(np.ascontiguousarray(mel, np.float32))
        t = mel_d.shape[1]
        # condnet: conv + ELU x depth, the first looking ahead (right pad), the rest causal;
        # channels-last after the first conv, so the wide ones run as split-K DMA GEMMs
        k0 = self.shape["f0_predictor.condnet.0.weight"][2]
        x = self._conv_in(mel_d, "f0_predictor.condnet.0", pad=(0, causal_pad(k0)), act="elu", act_param=1.0)
        for i in range(1, self.f0_depth):
            k = self.shape[f"f0_predictor.condnet.{i}.weight"][2]
            x = self._conv(x, f"f0_predictor.condnet.{i}", pad=(causal_pad(k), 0), act="elu", act_param=1.0)
        n, c = x.shape
        if n != t:
            raise ValueError(f"the F0 predictor gave {n} frames for {t}")
        f0 = DeviceArray((n,))
        _lib.call("f0_classify", x.ptr, c, n, 1, c, self.f0_cls[0].ptr, self.f0_cls[1].ptr, f0.ptr, None)
        return f0

    def source_noise(self, n: int) -> DeviceArray:
        """The first n rows of the [n, harmonics] dither buffer (hift.py:75-81), drawn once
        from TorchMT19937(noise_seed) on the host replica and kept resident; a longer
        request draws the buffer again at the new length, as the reference does."""
        if self._noise is None or self._noise.shape[0] < n:
            from .torch_rng import TorchMT19937
            need = max(n, 1)
            buf = TorchMT19937(self.noise_seed).random_float32(need * self.harmonics)
            self._noise = to_device(buf.reshape(need, self.harmonics))
        return self._noise

    def set_source_noise(self, buf) -> None:
        """Use a caller-supplied [n, harmonics] dither buffer (hift.py:83-88)."""
        buf = np.ascontiguousarray(buf, np.float32)
        if buf.ndim != 2 or buf.shape[1] != self.harmonics:
            raise ValueError(f"dither buffer of shape {buf.shape}, expected (n, {self.harmonics})")
        self._noise = to_device(buf)

    def excitation(self, f0) -> DeviceArray:
        """(T,) float32 F0 -> (480 T,) merged harmonic source (hift.py:90-111)."""
        if self.l_linear is None:
            raise ValueError("the weights hold no m_source.l_linear")
        f0_d = f0 if isinstance(f0, DeviceArray) else to_device(np.ascontiguousarray(f0, np.float32))
        t = f0_d.size
        up = self.up_total * self.hop
        noise = self.source_noise(up * t)
        phase = DeviceArray((max(t, 1), self.harmonics), np.float64)
        out = DeviceArray((up * t,))
        _lib.call("nsf_source", f0_d.ptr, t, up, self.harmonics, float(self.sampling_rate), self.nsf_alpha,
                  self.nsf_sigma, self.nsf_threshold, noise.ptr, self.l_linear[0].ptr, self.l_linear[1].ptr,
                  phase.ptr, out.ptr, None)
        return out

    def inference(self, mel, chunk: Optional[int] = 250, context: int = 64, graph: bool = True) -> DeviceArray:
        """(80, T) mel -> (480 T,) waveform, entirely on the device (hift.py:212-218)."""
        mel_d = mel if isinstance(mel, DeviceArray) else to_device(np.ascontiguousarray(mel, np.float32))
        source = self.excitation(self.f0_predict(mel_d))
        return self.decode(mel_d, source, chunk=chunk, context=context, graph=graph)

    def flops(self, t: int) -> float:
        """Algorithmic conv flops of a whole-utterance decode of t mel frames."""
        return sum(self.flops_by_unit(t))

    def flops_by_unit(self, t: int) -> tuple:
        """(flops on the bfloat16 planes, flops on the float32 units) of a whole-utterance
        decode of t mel frames: a conv runs on the planes when its weights were split."""
        on = [0.0, 0.0]

        def add(key, f):
            on[0 if key + ".weight" in self.wpx else 1] += f

        cur_t = t
        kpre = self.shape["conv_pre.weight"]
        add("conv_pre", 2.0 * kpre[0] * kpre[1] * kpre[2] * cur_t)
        for i, r in enumerate(self.rates):
            cur_t *= r
            co, ci, k = self.shape[f"ups.{i}.weight"]
            add(f"ups.{i}", 2.0 * co * ci * k * cur_t)
            co, ci, k = self.shape[f"source_downs.{i}.weight"]
            add(f"source_downs.{i}", 2.0 * co * ci * k * cur_t)
            for g, idx, kk in [("source_resblocks", i, self.src_k[i])] + \
                    [("resblocks", i * self.nk + j, self.rb_k[j]) for j in range(self.nk)]:
                c = self.shape[f"{g}.{idx}.convs1.0.weight"][0]
                add(f"{g}.{idx}.convs1.0", 2 * 3 * 2.0 * c * c * kk * cur_t)
        co, ci, k = self.shape["conv_post.weight"]
        add("conv_post", 2.0 * co * ci * k * cur_t)
        return tuple(on)
