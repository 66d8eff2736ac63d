"""Oracle restatement of the causal HiFTNet vocoder.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/hift.py.
"""

from __future__ import annotations

import numpy as np

from . import ops
from .torch_rng import TorchMT19937


def causal_pad(kernel_size: int, dilation: int = 1) -> int:
    """int((k d - d)/2)*2 + (k+1)%2 (hift.py:14-16)."""
    return int((kernel_size * dilation - dilation) / 2) * 2 + (kernel_size + 1) % 2


class HiFTGenerator:
    def __init__(self, weights, prefix: str = "hift."):
        self.w = weights
        self.p = prefix
        m = weights.meta.get("hift", {})
        self.upsample_rates = list(m.get("upsample_rates", [8, 5, 3]))
        self.resblock_kernel_sizes = list(m.get("resblock_kernel_sizes", [3, 7, 11]))
        self.resblock_dilation_sizes = [list(d) for d in m.get("resblock_dilation_sizes", [[1, 3, 5]] * 3)]
        self.source_resblock_kernel_sizes = list(m.get("source_resblock_kernel_sizes", [7, 7, 11]))
        self.source_resblock_dilation_sizes = [list(d) for d in
                                               m.get("source_resblock_dilation_sizes", [[1, 3, 5]] * 3)]
        self.n_fft = int(m.get("istft_n_fft", 16))
        self.hop_len = int(m.get("istft_hop_len", 4))
        self.lrelu_slope = float(m.get("lrelu_slope", 0.1))
        self.audio_limit = float(m.get("audio_limit", 0.99))
        self.sampling_rate = int(m.get("sampling_rate", 24000))
        self.nb_harmonics = int(m.get("nb_harmonics", 8))
        self.nsf_alpha = float(m.get("nsf_alpha", 0.1))
        self.nsf_sigma = float(m.get("nsf_sigma", 0.003))
        self.nsf_voiced_threshold = float(m.get("nsf_voiced_threshold", 10.0))
        self.num_kernels = len(self.resblock_kernel_sizes)
        self.num_upsamples = len(self.upsample_rates)
        self.upsample_scale = int(np.prod(self.upsample_rates)) * self.hop_len
        self.window = ops.hann_window(self.n_fft)
        self.noise_seed = int(m.get("noise_seed", 0))
        self._src_noise = None

    def _t(self, name):
        return self.w.get(self.p + name)

    def _k(self, name) -> int:
        return int(self.w.entry(self.p + name)["shape"][-1])

    def f0_predict(self, mel):
        """5x (conv + ELU) then the classifier in float64 (hift.py:56-72).  The convs
        themselves run in float32 because conv1d casts its operands."""
        x = np.asarray(mel, dtype=np.float64)
        for i in range(5):
            w = np.asarray(self.w.get_f32(self.p + f"f0_predictor.condnet.{i}.weight"), dtype=np.float64)
            b = np.asarray(self.w.get_f32(self.p + f"f0_predictor.condnet.{i}.bias"), dtype=np.float64)
            k = w.shape[-1]
            x = ops.elu(ops.conv1d(x, w, b, pad=(0, causal_pad(k)) if i == 0 else (causal_pad(k), 0)))
        cw = np.asarray(self.w.get_f32(self.p + "f0_predictor.classifier.weight"), dtype=np.float64)
        cb = np.asarray(self.w.get_f32(self.p + "f0_predictor.classifier.bias"), dtype=np.float64)
        return np.abs((x.T @ cw.T + cb)[:, 0])

    def source_noise(self, n: int, harmonics: int):
        """Lazily drawn TorchMT19937 uniform dither (hift.py:75-81)."""
        if self._src_noise is None or self._src_noise.shape[0] < n:
            g = TorchMT19937(self.noise_seed)
            need = max(n, 1)
            self._src_noise = g.random_float32(need * harmonics).reshape(need, harmonics)
        return self._src_noise[:n]

    def set_source_noise(self, buf):
        """hift.py:83-88"""
        self._src_noise = np.asarray(buf, dtype=np.float32)

    def excitation(self, f0):
        """Per-frame fp64 harmonic phase, held over ``upsample_scale`` samples, plus
        voiced/unvoiced dither, merged by Linear(9 -> 1) + tanh (hift.py:90-111)."""
        t = f0.shape[0]
        up = self.upsample_scale
        nh = self.nb_harmonics + 1
        rad = (f0[:, None] * np.arange(1, nh + 1)[None, :] / self.sampling_rate) % 1.0
        phase = np.cumsum(rad, axis=0) * (2.0 * np.pi) * up
        sines = np.sin(np.repeat(phase, up, axis=0)).astype(np.float32)
        sines *= self.nsf_alpha
        uv = (np.repeat(f0, up) > self.nsf_voiced_threshold).astype(np.float32)[:, None]
        amp = uv * self.nsf_sigma + (1.0 - uv) * (self.nsf_alpha / 3.0)
        src = sines * uv + amp * self.source_noise(up * t, nh)
        merged = ops.linear(src, self._t("m_source.l_linear.weight"), self._t("m_source.l_linear.bias"))
        return np.tanh(merged)[:, 0]

    def resblock(self, group, idx, x, kernel, dilations):
        """3x [Snake, dilated causal conv, Snake, causal conv] + residual (hift.py:114-129)."""
        base = f"{group}.{idx}."
        for j, d in enumerate(dilations):
            y = ops.snake(x, np.asarray(self._t(base + f"activations1.{j}.alpha"), dtype=np.float32))
            y = ops.conv1d(y, self._t(base + f"convs1.{j}.weight"), self._t(base + f"convs1.{j}.bias"),
                           dilation=d, pad=(causal_pad(kernel, d), 0))
            y = ops.snake(y, np.asarray(self._t(base + f"activations2.{j}.alpha"), dtype=np.float32))
            y = ops.conv1d(y, self._t(base + f"convs2.{j}.weight"), self._t(base + f"convs2.{j}.bias"),
                           dilation=1, pad=(causal_pad(kernel, 1), 0))
            x = y + x
        return x

    def spectral(self, mel, s_stft):
        """conv_pre .. conv_post: (80, T) -> (n_fft+2, 120 T + 1) (hift.py:131-168)."""
        x = ops.conv1d(mel, self._t("conv_pre.weight"), self._t("conv_pre.bias"),
                       pad=(0, causal_pad(self._k("conv_pre.weight"))))
        downs = [1] + self.upsample_rates[::-1][:-1]
        down_cum = list(np.cumprod(downs))[::-1]
        for i in range(self.num_upsamples):
            x = ops.interpolate_nearest(ops.leaky_relu(x, self.lrelu_slope), self.upsample_rates[i])
            k = self._k(f"ups.{i}.weight")
            x = ops.conv1d(x, self._t(f"ups.{i}.weight"), self._t(f"ups.{i}.bias"), pad=(k - 1, 0))
            if i == self.num_upsamples - 1:
                x = np.concatenate([x[:, 1:2], x], axis=1)
            u = int(down_cum[i])
            ks = self._k(f"source_downs.{i}.weight")
            if u == 1:
                si = ops.conv1d(s_stft, self._t(f"source_downs.{i}.weight"), self._t(f"source_downs.{i}.bias"),
                                pad=(causal_pad(ks), 0))
            else:
                si = ops.conv1d(s_stft, self._t(f"source_downs.{i}.weight"), self._t(f"source_downs.{i}.bias"),
                                stride=u, pad=(u - 1, 0))
            si = self.resblock("source_resblocks", i, si, self.source_resblock_kernel_sizes[i],
                               self.source_resblock_dilation_sizes[i])
            x = x + si
            acc = None
            for j in range(self.num_kernels):
                r = self.resblock("resblocks", i * self.num_kernels + j, x,
                                  self.resblock_kernel_sizes[j], self.resblock_dilation_sizes[j])
                acc = r if acc is None else acc + r
            x = acc / self.num_kernels
        x = ops.leaky_relu(x, 0.01)
        return ops.conv1d(x, self._t("conv_post.weight"), self._t("conv_post.bias"),
                          pad=(causal_pad(self._k("conv_post.weight")), 0))

    def spectral_chunked(self, mel, s_stft, chunk, context):
        """Windows of ``chunk`` mel frames with ``context`` frames of history and
        conv_pre's lookahead; reproduces :meth:`spectral` (hift.py:170-194)."""
        up = int(np.prod(self.upsample_rates))
        t = mel.shape[1]
        look = causal_pad(self._k("conv_pre.weight"))
        parts = []
        for m0 in range(0, t, chunk):
            m1 = min(t, m0 + chunk)
            c0 = max(0, m0 - context)
            c1 = min(t, m1 + look)
            sub = self.spectral(mel[:, c0:c1], s_stft[:, c0 * up:c1 * up + 1])
            lead = (m0 - c0) * up
            take = (m1 - m0) * up
            parts.append(sub[:, :1 + take] if m0 == 0 else sub[:, 1 + lead:1 + lead + take])
        return np.concatenate(parts, axis=1)

    def source_stft(self, source):
        """(18, frames) real/imag stack of the source STFT (hift.py:198-199)."""
        spec = ops.stft(source, self.n_fft, self.hop_len, self.window)
        return np.concatenate([spec.real, spec.imag], axis=0).astype(np.float32)

    def istft_head(self, x):
        """magnitude clip(exp(min(x,80)),100), phase sin(x), iSTFT, clip +-0.99 (hift.py:204-210)."""
        half = self.n_fft // 2 + 1
        mag = np.clip(np.exp(np.minimum(x[:half], 80.0)), None, 1e2)
        ph = np.sin(x[half:])
        y = ops.istft(mag * np.cos(ph) + 1j * mag * np.sin(ph), self.n_fft, self.hop_len, self.window)
        return np.clip(y, -self.audio_limit, self.audio_limit)

    def decode(self, mel, source, chunk=None, context=64):
        """hift.py:196-210"""
        s_stft = self.source_stft(source)
        if chunk is None or mel.shape[1] <= chunk:
            x = self.spectral(mel, s_stft)
        else:
            x = self.spectral_chunked(mel, s_stft, chunk, context)
        return self.istft_head(x)

    def inference(self, mel, chunk=250, context=64):
        """(80, T) mel -> (480 T,) waveform (hift.py:212-218)."""
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        f0 = self.f0_predict(mel)
        return self.decode(mel, self.excitation(f0.astype(np.float32)), chunk=chunk, context=context)
