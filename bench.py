#!/usr/bin/env python3
"""Benchmark of the MI355X tensor-kernel backend on its two headline workloads.

  * Qwen2-0.5B int8 greedy decode, batch 1 (the reported ``value``): 24 layers,
    hidden 896, 14/2 heads x 64, SwiGLU 4864, per-output-channel int8 weights with
    float32 scales, KV cache pre-filled to 512 positions of N(0, 1).  One step is one
    whole decode: 256 greedy tokens from speech_embedding[sos], KV 512 -> 768, each
    token one launch of the whole decode step (``--decode-step kernels``: five kernels
    per layer, whose rate is reported beside it in ``five_kernel_step``); the same
    decode with the reference's sampler on the device (``sampled_tok_s``); and with
    the tiny profile's q4 body layers (the ``decode_tiny`` object).
  * DiT flow decoder, 10 s of audio (the ``flow`` object): 22 blocks x [2, 500, 1024]
    fp32, 10 Euler steps with classifier-free guidance, noise from the host replica
    of torch.randn((1, 80, 15000), seed 0), checked against its pinned SHA-256; and
    the same solve over 30 s (T = 1500) with q8 linears, per-output-channel float32
    scales (``flow_q8_30s``) and block-64 float16 scales (``flow_q8_30s_block64``).
  * HiFTNet vocoder, 10 s of audio (the ``vocoder`` object), whole and in 1 s chunks.

Weights are synthetic (seeded N(0, 0.02), norms 1; cv3amd/synth.py); inputs are
resident in HBM before the timed regions start.  Each workload reports its
dominant kernel against the MI355X roofline (HBM 8 TB/s for the int8 GEMV; for the
DiT's float32 linears, held as three bfloat16 planes and run as six bfloat16 products
each, the dense bfloat16 matrix peak over six, 416.7 TFLOP/s of float32 products; fp32
matrix 157.3 TFLOP/s for what runs on the float32 matrix cores), timed live with HIP
events, next to the measured device copy rate and fp32 MFMA probe rate, and the
oracle's NumPy restatement timed on the host cores on a bounded sample.

Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "cosyvoice3-cpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "DiT flow RTF (10 s, CFG) + int8 LM decode tok/s, each as % of roofline"
HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
# HBM bytes per launch that rocprofv3 counted (FETCH_SIZE x2 + WRITE_SIZE x1, the factors a 256 MiB
# device copy needs; `bench.py --kernels --no-graph` under `rocprofv3 --pmc`, one counter per run):
# the one-launch decode step (24 layers, per-channel int8 with phase D on the int8 matrix cores,
# KV 512: 400.9 MB read + 9.2 MB written).  Counters cannot be read inside this process, so these
# are the measured figures for exactly these kernels and shapes.
TRAFFIC_DECODE_STEP = 410.1e6
# the same passes over the 10 s solve's fused QKV GEMM on bfloat16 planes in fragment order
# (k_gemm_x3f, [1000, 1024] x [3072, 1024]^T): 53.4 MB read + 12.3 MB written
TRAFFIC_QKV_GEMM_X3 = 65.7e6
FP32_MFMA_PEAK = 157.3e12  # flop/s, MI355X dense fp32 matrix
# float32 products on the bfloat16 matrix cores: six bfloat16 plane products each (cv3_linear_x3),
# so the dense bfloat16 peak (2.5 PFLOP/s) over six
SPLIT_BF16_PEAK = 2.5e15 / 6
# q8 weights on the same cores: three products per code (cv3_linear_q8_x3)
SPLIT_Q8_PEAK = 2.5e15 / 3
# per-channel q8 weights on the int8 matrix cores (5.0 POP/s dense): four digit-plane products
# per code (cv3_linear_q8_digits)
DIGITS_Q8_PEAK = 5.0e15 / 4


def matrix_floor_ms(by_unit) -> float:
    """The solve's matrix-core floor: each part of its flops at the peak of the unit it runs on."""
    six, three, f32 = by_unit[:3]
    four = by_unit[3] if len(by_unit) > 3 else 0.0
    return (six / SPLIT_BF16_PEAK + three / SPLIT_Q8_PEAK + four / DIGITS_Q8_PEAK + f32 / FP32_MFMA_PEAK) * 1e3
PREFILL = 512             # KV cache positions pre-filled before each decode
DECODE_TOKENS = 256       # tokens per decode: KV 512 -> 768
AUDIO_SECONDS = 10.0       # 500 mel frames at 50 Hz
# SHA-256 of torch.randn((1, 80, 15000)) under seed 0 as float32 bytes: the flow's initial noise
# (cv3cpu/models/flow.py:16,36-43).  tests/test_oracle_rng.py pins it to the oracle's replica.
NOISE_SHA256 = "ca8eb3b705dfa463ec872b622bd82459b5790c00f88f2529d993e40233bae482"


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_bandwidth(nbytes: int = 256 << 20, reps: int = 10) -> float:
    """Device-to-device copy rate (bytes/s) of one nbytes buffer: the achievable-HBM
    reference next to the 8 TB/s peak, and the known-size kernel that scales the
    FETCH_SIZE / WRITE_SIZE counters."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Timer, synchronize
    a = DeviceArray((nbytes // 4,)).zero_()
    b = DeviceArray((nbytes // 4,))
    _lib.call("copy_d2d", b.ptr, a.ptr, nbytes, None)
    synchronize()
    tm = Timer()
    tm.start()
    for _ in range(reps):
        _lib.call("copy_d2d", b.ptr, a.ptr, nbytes, None)
    ms = tm.stop() / reps
    return 2.0 * nbytes / (ms / 1e3)


def mfma_peak(cu_count: int, iters: int = 20000) -> float:
    """fp32 matrix-core rate (flop/s) the device sustains on register operands
    (cv3_mfma_peak_f32): the measured ceiling beside the published 157.3 TFLOP/s."""
    from cv3amd import _lib
    from cv3amd.device import DeviceArray, Timer, synchronize
    out = DeviceArray((cu_count * 512,))
    flops = ctypes.c_double()
    _lib.call("mfma_peak_f32", 1000, cu_count, out.ptr, ctypes.addressof(flops), None)   # clocks up
    synchronize()
    tm = Timer()
    tm.start()
    _lib.call("mfma_peak_f32", iters, cu_count, out.ptr, ctypes.addressof(flops), None)
    ms = tm.stop()
    return flops.value / (ms / 1e3)


def replayer(graph: bool, enqueue):
    """A callable that enqueues ``enqueue``'s launches: replayed from one captured HIP
    graph, or issued directly (the mode used under the kernel-trace profiler)."""
    if not graph:
        return enqueue
    from cv3amd.device import Graph
    g = Graph()
    with g:
        enqueue()
    return g.launch


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------

def build_lm(layers: int, profile: str):
    import cv3amd.quant as quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    t = synth.qwen2_tensors(layers=layers)
    t = synth.quantize_store(t, profile, quant.quantize_q8, quant.quantize_q4)   # device quantisers
    return t, synth.qwen2_meta(layers=layers)


def bench_decode(args, tensors, meta, label: str = "decode", decodes: int = None, warmup: int = None):
    """Greedy decodes of DECODE_TOKENS tokens from the KV cache pre-filled to PREFILL positions.
    One step = one whole decode: begin at position PREFILL with speech_embedding[sos], then
    DECODE_TOKENS tokens.  A decode only writes cache rows PREFILL and up, and each token reads
    the rows below its own position, so every decode sees the same pre-filled cache."""
    import cv3amd.quant as quant
    from cv3amd import _lib
    from cv3amd.device import Graph, Timer, synchronize
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore

    decodes = args.steps if decodes is None else decodes
    warmup = args.warmup if warmup is None else warmup
    store = WeightStore(tensors, meta, quant.QTensor)
    layers = meta["qwen2"]["num_hidden_layers"]
    lm = DeviceQwen2(store, cap=1024)
    rng = np.random.default_rng(0)
    shape = (layers, lm.kv_heads, PREFILL, lm.head_dim)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    lm.fill_cache(k, v)
    sos = int(meta["speech_token_size"])
    persistent = args.decode_step == "persistent"
    lm.cooperative = args.cooperative
    tm = Timer()

    def one_decode(one_launch: bool):
        lm.begin(sos, PREFILL)
        for _ in range(DECODE_TOKENS):
            lm.step_persistent() if one_launch else lm.step(graph=args.graph)

    def timed_decodes(one_launch: bool, n: int, w: int):
        """w untimed decodes, then n timed ones; returns (ms per decode, tokens of the last)."""
        what = "one-launch step" if one_launch else "five-kernel step"
        log(f"{label}: {what}: {w} warmup + {n} timed decodes of {DECODE_TOKENS} tokens from KV {PREFILL}")
        for _ in range(w):
            one_decode(one_launch)
        synchronize()
        tm.start()
        for _ in range(n):
            one_decode(one_launch)
        ms_ = tm.stop() / n
        synchronize()
        if one_launch and lm.persistent_error():
            raise RuntimeError("the one-launch decode step gave up waiting for an exchange")
        toks = [int(t) for t in lm.ints.numpy()[2 + PREFILL + 1: 2 + PREFILL + 1 + DECODE_TOKENS]]
        log(f"{label}: {what}: {ms_:.2f} ms per decode = {DECODE_TOKENS / (ms_ / 1e3):.1f} tok/s")
        return ms_, toks

    side = max(1, min(decodes, 3))     # the step not reported as the value: a shorter sample
    if persistent:
        ms, tokens = timed_decodes(True, decodes, warmup)
        ms_k, tokens_k = timed_decodes(False, side, 1)
    else:
        ms_k, tokens_k = timed_decodes(False, decodes, warmup)
        ms, tokens = ms_k, tokens_k
    if tokens != tokens_k:
        raise RuntimeError("the one-launch and five-kernel steps chose different tokens")
    tok_s = DECODE_TOKENS / (ms / 1e3)
    # algorithmic bytes averaged over the decode's tokens: token s reads PREFILL + s + 1 cache rows
    parts = [lm.bytes_per_token(PREFILL + s) for s in range(DECODE_TOKENS)]
    b = {key: sum(p[key] for p in parts) / DECODE_TOKENS for key in parts[0]}
    per_token = b["body"] + b["kv"] + b["norms_biases"] + b["head"]
    held = per_token - b["body"] + b["body_held"]   # what the kernels stream (a q4 body held widened: int8 codes)
    if held != per_token:
        log(f"{label}: {tok_s:.1f} tok/s; checkpoint bytes {per_token / 1e6:.1f} MB/token -> "
            f"{per_token * tok_s / 1e9:.0f} GB/s algorithmic; held in HBM {held / 1e6:.1f} MB/token -> "
            f"{held * tok_s / 1e9:.0f} GB/s streamed")
    else:
        log(f"{label}: {tok_s:.1f} tok/s; {per_token / 1e6:.1f} MB/token -> {per_token * tok_s / 1e9:.0f} GB/s")

    # Dominant kernel: the gate/up GEMV (RMSNorm prologue + SwiGLU), one layer's
    # [gate; up] = 2 x 4864 x 896 int8 + scales per launch.  Timed back-to-back
    # over the 24 layers (so the weights stream from HBM, as in the decode),
    # replayed from a captured graph.
    gu = lm.gate_up.struct()
    gu_bytes = lm.gate_up.nbytes // layers + lm.hidden * 4 * 2 + lm.inter * 4
    out = lm.workspace
    def gate_up_sweep():
        for layer in range(layers):
            _lib.call("gemv_q8", ctypes.byref(gu), layer, lm.x.ptr, lm.ln2.ptr + layer * lm.hidden * 4, lm.eps,
                      None, out.ptr, 2, None)
    run = replayer(args.graph, gate_up_sweep)
    run()
    synchronize()
    reps = 20
    tm.start()
    for _ in range(reps):
        run()
    kms = tm.stop() / (reps * layers)
    achieved = gu_bytes / (kms / 1e3)
    log(f"{label}: gate/up GEMV {kms * 1e3:.2f} us/launch, {achieved / 1e9:.0f} GB/s")
    # the reference's sampler (SamplingConfig defaults) on the device, stop ids held back
    # for the whole run (strict min_len = all steps) so every timed token is decoded
    class _Sampling:
        top_p, top_k, win_size, tau_r, strict_min_len = 0.8, 25, 10, 0.1, True
        rng = np.random.default_rng(0)
    lm.generate_sampled(sos, PREFILL, 8, 8, _Sampling, sos, graph=args.graph, persistent=persistent)
    synchronize()
    tm.start()
    sampled = lm.generate_sampled(sos, PREFILL, DECODE_TOKENS, DECODE_TOKENS, _Sampling, sos, graph=args.graph,
                                  persistent=persistent)
    sms = tm.stop()
    sampled_tok_s = len(sampled) / (sms / 1e3)
    log(f"{label}: sampled (top_p 0.8, top_k 25, repetition window 10) {sms:.2f} ms for {len(sampled)} tokens "
        f"= {sampled_tok_s:.1f} tok/s")
    sf16 = lm.gate_up.sf16
    gs = lm.gate_up.struct()
    mx = lm.gate_up.kind != "q4" and gs.kp <= gs.block   # phase D on the int8 matrix cores
    return {
        "sampled_tok_s": sampled_tok_s, "persistent": persistent,
        "tok_s": tok_s, "ms": ms, "tokens": tokens, "bytes_per_token": per_token, "bytes_parts": b,
        "bytes_per_token_held": held,
        "five_kernel_tok_s": DECODE_TOKENS / (ms_k / 1e3), "decodes": decodes,
        # the one-launch step is a single kernel per token: its bytes are the token's
        "step_kernel": {"name": f"k_dec_persist<{'true' if sf16 else 'false'}, "
                                f"{'true' if lm.gate_up.kind == 'q4' else 'false'}, {'true' if mx else 'false'}> "
                                "(the whole decode step)",
                        "bytes_per_launch": per_token, "us_per_launch": ms / DECODE_TOKENS * 1e3,
                        "achieved_Bps": per_token / (ms / DECODE_TOKENS / 1e3)},
        "kernel": {"name": "k_dec_gemv<8,4,2,q4> (RMSNorm + [gate;up] q4 GEMV + SwiGLU)" if lm.gate_up.kind == "q4"
                   else "k_dec_gemv<16,4,2> (RMSNorm + [gate;up] int8 GEMV + SwiGLU)",
                   "bytes_per_launch": gu_bytes, "us_per_launch": kms * 1e3, "achieved_Bps": achieved},
    }


def cpu_decode(tensors, meta, n_tokens: int):
    """The oracle's NumPy restatement of the same decode on the host cores."""
    import oracle.quant
    from oracle.llm import CosyVoice3LM
    from cv3amd.weights import WeightStore
    store = WeightStore(tensors, meta, oracle.quant.QTensor)
    lm = CosyVoice3LM(store, "llm.")
    layers = lm.cfg.num_hidden_layers
    rng = np.random.default_rng(0)
    shape = (layers, lm.cfg.num_key_value_heads, PREFILL, lm.cfg.head_dim)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    cache = lm.body.new_cache()
    cache._reserve(PREFILL + n_tokens + 2)
    for i in range(layers):
        cache.k[i][:, :PREFILL] = k[i]
        cache.v[i][:, :PREFILL] = v[i]
    cache.length = PREFILL
    x = lm.speech_emb([lm.sos])
    logits0 = lm.head(lm.body.forward(x, cache)[-1:])[0]   # warm-up token
    x = lm.speech_emb([int(np.argmax(logits0))])
    t0 = time.perf_counter()
    toks = []
    for _ in range(n_tokens):
        logits = lm.head(lm.body.forward(x, cache)[-1:])[0]
        top = int(np.argmax(logits))
        toks.append(top)
        x = lm.speech_emb([top])
    dt = time.perf_counter() - t0
    return n_tokens / dt, dt, [int(np.argmax(logits0))] + toks


# ---------------------------------------------------------------------------
# flow
# ---------------------------------------------------------------------------

def flow_inputs(T: int):
    import hashlib
    from cv3amd.torch_rng import randn
    rng = np.random.default_rng(0)
    mu = rng.standard_normal((1, 80, T), dtype=np.float32)
    cond = rng.standard_normal((1, 80, T), dtype=np.float32)
    spks = rng.standard_normal((1, 80), dtype=np.float32)
    noise = randn((1, 80, 15000), 0)                      # flow.py:16-17,36-43
    digest = hashlib.sha256(np.ascontiguousarray(noise, np.float32).tobytes()).hexdigest()
    if digest != NOISE_SHA256:
        raise RuntimeError(f"the host torch.randn replica drew different ODE noise on this host (sha256 {digest})")
    return mu, cond, spks, np.ascontiguousarray(noise[:, :, :T])


def bench_flow(args, tensors, meta):
    import cv3amd.quant as quant
    from cv3amd import _lib
    from cv3amd.device import Graph, Timer, synchronize
    from cv3amd.dit import DeviceDiT
    from cv3amd.weights import WeightStore
    T = 500
    store = WeightStore(tensors, meta, quant.QTensor)
    d = DeviceDiT(store)
    mu, cond, spks, x0 = flow_inputs(T)
    d.prepare(mu, spks, cond)
    log("flow: warmup solve (captures the solve graph)")
    d.solve(x0, graph=args.graph)
    synchronize()
    tm = Timer()
    n = args.flow_solves
    log(f"flow: timing {n} solves")
    tm.start()
    for _ in range(n):
        d.solve(x0, graph=args.graph)
    ms = tm.stop() / n
    flops = d.flops_per_solve()
    by_unit = d.flops_by_unit()
    log(f"flow: {ms:.2f} ms/solve, RTF {ms / 1e3 / AUDIO_SECONDS:.2e}, {flops / (ms / 1e3) / 1e12:.1f} TFLOP/s")

    # Dominant kernel: the fused QKV projection GEMM, [1000, 1024] x [3072, 1024]^T, timed
    # over the 22 blocks' weights back-to-back from a captured graph.
    M, K, N = 2 * T, d.dim, 3 * d.dim
    def qkv_sweep():
        for i in range(d.depth):
            d.qkv[i](d.n.ptr, M, K, d.qkvb.ptr, N)
    run = replayer(args.graph, qkv_sweep)
    run()
    synchronize()
    reps = 10
    tm.start()
    for _ in range(reps):
        run()
    kms = tm.stop() / (reps * d.depth)
    kflops = 2.0 * M * N * K
    log(f"flow: QKV GEMM {kms * 1e3:.1f} us/launch, {kflops / (kms / 1e3) / 1e12:.1f} TFLOP/s")
    planes = d.qkv[0].planes is not None if d.depth else False
    name = ("k_gemm_x3f (float32 GEMM as six bfloat16 plane products, weight fragments straight to registers, "
            "fused QKV 1000x3072x1024)" if planes
            else "k_gemm<0> (fp32 MFMA GEMM, fused QKV 1000x3072x1024)")
    return {"ms": ms, "flops": flops, "by_unit": by_unit, "T": T, "depth": d.depth,
            "kernel": {"name": name, "flops_per_launch": kflops, "peak": SPLIT_BF16_PEAK if planes else FP32_MFMA_PEAK,
                       "traffic": TRAFFIC_QKV_GEMM_X3 if planes else None,
                       "us_per_launch": kms * 1e3, "achieved_flops": kflops / (kms / 1e3)}}


def bench_flow_q8(args, tensors, meta, profile: str):
    """The 30 s solve (T = 1500) with the DiT linears stored q8, dequantised inside the GEMM's
    B load: ``per_channel`` (one float32 scale per output row) or ``balanced`` (block 64,
    float16 scales; the reference converter's default profile)."""
    import cv3amd.quant as quant
    from cv3amd import synth
    from cv3amd.device import Timer, synchronize
    from cv3amd.dit import DeviceDiT
    from cv3amd.weights import WeightStore
    T = 1500
    qt = synth.quantize_store(tensors, profile, quant.quantize_q8)   # device quantiser
    d = DeviceDiT(WeightStore(qt, meta, quant.QTensor))
    mu, cond, spks, x0 = flow_inputs(T)
    d.prepare(mu, spks, cond)
    log(f"flow q8 ({profile}) 30 s: warmup solve (captures the solve graph)")
    d.solve(x0, graph=args.graph)
    synchronize()
    n = max(1, args.flow_solves - 1)
    log(f"flow q8 ({profile}) 30 s: timing {n} solves")
    tm = Timer()
    tm.start()
    for _ in range(n):
        d.solve(x0, graph=args.graph)
    ms = tm.stop() / n
    flops = d.flops_per_solve()
    log(f"flow q8 ({profile}) 30 s: {ms:.2f} ms/solve, RTF {ms / 1e3 / 30.0:.2e}, "
        f"{flops / (ms / 1e3) / 1e12:.1f} TFLOP/s")
    return {"ms": ms, "flops": flops, "by_unit": d.flops_by_unit(), "T": T, "halves": d.halves,
            "digits": d.qkv[0].q8_digits if d.depth else False}


def bench_kernels(args):
    """The roofline kernels one by one, for per-kernel tables and rocprofv3 counter passes:
    16 tokens of the one-launch decode step (24 layers, per-channel int8, KV 512), each launch of
    one DiT block at the 10 s solve's shapes (T = 500, CFG batch 2) timed alone (`reps`
    back-to-back launches of the same kernel, replayed from a captured graph unless --no-graph,
    on the buffers a real estimator evaluation left behind), the 30 s q8 GEMMs (block-64 / f16
    weights), one whole-utterance vocoder inference (10 s), then optionally the whole 10 s
    solve.  The five-kernel decode step is left out (its kernels have their own bench lines)."""
    import ctypes
    import math
    import cv3amd.quant as quant
    from cv3amd import _lib, synth
    from cv3amd.device import Timer, synchronize, to_device, DeviceArray
    from cv3amd.dit import DeviceDiT
    from cv3amd.weights import WeightStore
    T, B = 500, 2
    info = _lib.device_info()
    copy_bps = copy_bandwidth()   # also the known-size kernel the traffic counters are scaled by
    log(f"kernels: device copy {copy_bps / 1e9:.0f} GB/s (read + write of 256 MiB)")
    peak = mfma_peak(info["cu_count"])
    log(f"kernels: fp32 MFMA probe {peak / 1e12:.1f} TFLOP/s (k_mfma_peak, the matrix-core busy reference)")
    out = {"mfma_probe_tflops": round(peak / 1e12, 2)}
    # the one-launch decode step
    from cv3amd.qwen2 import DeviceQwen2
    lm_t, lm_meta = build_lm(args.layers, args.profile)
    lm = DeviceQwen2(WeightStore(lm_t, lm_meta, quant.QTensor), cap=1024)
    rng = np.random.default_rng(0)
    kv_shape = (args.layers, lm.kv_heads, PREFILL, lm.head_dim)
    lm.fill_cache(rng.standard_normal(kv_shape, dtype=np.float32), rng.standard_normal(kv_shape, dtype=np.float32))
    lm.begin(int(lm_meta["speech_token_size"]), PREFILL)
    for _ in range(4):
        lm.step_persistent()
    synchronize()
    tm = Timer()
    tm.start()
    for _ in range(16):
        lm.step_persistent()
    us = tm.stop() / 16 * 1e3
    if lm.persistent_error():
        raise RuntimeError("the one-launch decode step gave up waiting")
    nbytes = sum(lm.bytes_per_token(PREFILL + 12).values())   # the timed tokens' midpoint (KV 524)
    log(f"kernels: one-launch decode step {us:.1f} us per token ({nbytes / (us * 1e-6) / 1e9:.0f} GB/s)")
    out["decode_step_us"] = round(us, 2)
    del lm, lm_t
    tensors, meta = synth.dit_tensors(depth=2), synth.dit_meta(depth=2)
    d = DeviceDiT(WeightStore(tensors, meta, quant.QTensor))
    mu, cond, spks, x0 = flow_inputs(T)
    d.prepare(mu, spks, cond)
    d.solve(x0, graph=False)
    synchronize()
    D, H, dh, F = d.dim, d.heads, d.dim_head, d.ff_dim
    BT = B * T
    f4 = 4
    S3 = ctypes.c_int64 * 3
    qs = S3(T * 3 * D, dh, 3 * D)
    os_ = S3(T * D, dh, D)
    scale = float(np.float32(1.0 / math.sqrt(dh)))
    rope_epi = _lib.epilogue(rope=(d.cos.ptr, d.sin.ptr, T, D, dh, 2 * D))
    g = d.mods.ptr   # any AdaLN row: the timing does not depend on its values
    res_epi = _lib.epilogue(residual=d.h.ptr, ld_res=D, gate=g, gate_stride=0, rows_per_gate=1)
    k = d.conv_k
    mish = _lib.epilogue("mish")
    # the block linears on bfloat16 planes (six products per float32 product) or fp32 MFMA
    lin_peak, lin_unit = ((SPLIT_BF16_PEAK, "split-bf16") if d.qkv[0].planes is not None
                          else (FP32_MFMA_PEAK, "fp32 MFMA"))
    f32 = (FP32_MFMA_PEAK, "fp32 MFMA")
    launches = {
        "layer_norm + AdaLN [1000, 1024]": (
            lambda: _lib.call("layer_norm", d.h.ptr, d.n.ptr, BT, D, 1e-6, None, None, g, g + D * f4, 0, 0, None),
            None, None),
        f"QKV GEMM [{BT}, {D}] x [{3 * D}, {D}]^T + rotary": (
            lambda: d.qkv[0](d.n.ptr, BT, D, d.qkvb.ptr, 3 * D, rope_epi), 2.0 * BT * 3 * D * D, (lin_peak, lin_unit)),
        f"QKV GEMM [{BT}, {D}] x [{3 * D}, {D}]^T, bias only": (
            lambda: d.qkv[0](d.n.ptr, BT, D, d.qkvb.ptr, 3 * D), 2.0 * BT * 3 * D * D, (lin_peak, lin_unit)),
        f"flash attention B={B} H={H} T={T} d={dh}": (
            lambda: _lib.call("attention_x3" if d.planes else "attention", d.qkvb.ptr, d.qkvb.ptr + D * f4,
                              d.qkvb.ptr + 2 * D * f4, d.att.ptr, B, H, H, T, T, dh, qs, qs, qs, os_, scale, 0, 0, 0,
                              None), 4.0 * B * H * T * T * dh, (lin_peak, lin_unit)),
        f"out GEMM [{BT}, {D}] x [{D}, {D}]^T + gated residual": (
            lambda: d.out[0](d.att.ptr, BT, D, d.z1.ptr, D, res_epi), 2.0 * BT * D * D, (lin_peak, lin_unit)),
        f"ff1 GEMM [{BT}, {D}] x [{F}, {D}]^T + GELU": (
            lambda: d.ff1[0](d.n.ptr, BT, D, d.ffb.ptr, F, _lib.epilogue("gelu_tanh")), 2.0 * BT * F * D,
            (lin_peak, lin_unit)),
        f"ff2 GEMM [{BT}, {F}] x [{D}, {F}]^T + gated residual": (
            lambda: d.ff2[0](d.ffb.ptr, BT, F, d.z1.ptr, D, res_epi), 2.0 * BT * D * F, (lin_peak, lin_unit)),
        f"grouped causal conv k={k} groups={d.conv_groups} [{B}, {T}, {D}] + Mish": (
            lambda: _lib.call("conv1d_cl_x3f" if d.conv_planes else "conv1d_cl", d.h.ptr, B, T, D, D,
                              d.conv_w[0].ptr, D, k, d.conv_groups, k - 1, d.conv_b[0].ptr, d.z1.ptr, D,
                              ctypes.byref(mish), None),
            2.0 * BT * D * (D // d.conv_groups) * k, (lin_peak, lin_unit) if d.conv_planes else f32),
    }
    reps = args.kernel_reps
    for name, (fn, flops, pk) in launches.items():
        run = replayer(args.graph, lambda: [fn() for _ in range(reps)])
        run()
        synchronize()
        tm.start()
        for _ in range(5):
            run()
        us = tm.stop() / (5 * reps) * 1e3
        rate = flops / (us * 1e-6) / 1e12 if flops else None
        log(f"kernels: {name}: {us:.1f} us" + (f", {rate:.1f} TFLOP/s ({rate / (pk[0] / 1e12):.1%} of the "
                                                   f"{pk[1]} peak)" if rate else ""))
        out[name] = {"us": round(us, 2), "tflops": round(rate, 2) if rate else None}
    # the 30 s solve's q8 GEMMs (the activation's bfloat16 planes times the codes, held in the matrix
    # cores' fragment order as the solve holds them): per-output-channel f32 scales and block-64 / f16
    T3 = 1500
    BT3 = B * T3
    rng = np.random.default_rng(0)
    a = rng.standard_normal((BT3, F), dtype=np.float32)
    a_d = to_device(a)
    for (n, kk, label) in ((3 * D, D, "QKV"), (F, D, "ff1"), (D, D, "out"), (D, F, "ff2")):
        w = to_device(rng.standard_normal((n, kk), dtype=np.float32) * np.float32(0.02))
        for block, sdt, what in ((kk, np.float32, "per-channel f32 scales"), (64, np.float16, "block 64, f16 scales")):
            qd, sd, kp = quant.quantize_q8(w, block, sdt)   # device quantiser
            qf = DeviceArray((-(-n // 32) * 32 * kp,), np.int8)
            _lib.call("pack_q8_frag", qd.ptr, n, kp, kp, qf.ptr, None)
            y = DeviceArray((BT3, n), np.float32)
            sdt_c = _lib.F16 if sdt == np.float16 else _lib.F32
            fn = lambda: _lib.call("linear_q8_x3_frag", a_d.ptr, BT3, kk, F, qf.ptr, sd.ptr, sdt_c, kp, block, n,
                                   None, y.ptr, n, None, None)
            run = replayer(args.graph, lambda: [fn() for _ in range(reps)])
            run()
            synchronize()
            tm.start()
            for _ in range(5):
                run()
            us = tm.stop() / (5 * reps) * 1e3
            rate = 2.0 * BT3 * n * kk / (us * 1e-6) / 1e12
            name = f"q8 {label} GEMM [{BT3}, {kk}] x [{n}, {kk}]^T ({what})"
            log(f"kernels: {name}: {us:.1f} us, {rate:.1f} TFLOP/s ({rate / (SPLIT_Q8_PEAK / 1e12):.1%} of the "
                f"split q8 peak)")
            out[name] = {"us": round(us, 2), "tflops": round(rate, 2)}
            if block != kk:
                continue
            # the same per-channel weight on the int8 matrix cores as the solve runs it (digit planes)
            qf32 = DeviceArray((-(-n // 32) * 32 * (kp + 4),), np.int8)
            _lib.call("pack_q8_frag32", qd.ptr, n, kp, kp, qf32.ptr, None)
            rexp = DeviceArray((BT3,), np.int32)
            fn = lambda: _lib.call("linear_q8_digits", a_d.ptr, BT3, kk, F, qf32.ptr, sd.ptr, sdt_c, n, None, y.ptr,
                                   n, None, rexp.ptr, 0, None)
            run = replayer(args.graph, lambda: [fn() for _ in range(reps)])
            run()
            synchronize()
            tm.start()
            for _ in range(5):
                run()
            us = tm.stop() / (5 * reps) * 1e3
            rate = 2.0 * BT3 * n * kk / (us * 1e-6) / 1e12
            name = f"q8 {label} GEMM [{BT3}, {kk}] x [{n}, {kk}]^T (per-channel, int8 digit planes)"
            log(f"kernels: {name}: {us:.1f} us, {rate:.1f} TFLOP/s ({rate / (DIGITS_Q8_PEAK / 1e12):.1%} of the "
                f"digit-plane q8 peak)")
            out[name] = {"us": round(us, 2), "tflops": round(rate, 2)}
    # the 30 s solve's attention: 1500 x 1500 per head, the CFG pair x 16 heads, on bfloat16 planes
    qkv3 = to_device(rng.standard_normal((BT3, 3 * D), dtype=np.float32))
    att3 = DeviceArray((BT3, D), np.float32)
    qs3, os3 = S3(T3 * 3 * D, dh, 3 * D), S3(T3 * D, dh, D)
    fn = lambda: _lib.call("attention_x3" if d.planes else "attention", qkv3.ptr, qkv3.ptr + D * f4,
                           qkv3.ptr + 2 * D * f4, att3.ptr, B, H, H, T3, T3, dh, qs3, qs3, qs3, os3, scale, 0, 0, 0,
                           None)
    run = replayer(args.graph, lambda: [fn() for _ in range(reps)])
    run()
    synchronize()
    tm.start()
    for _ in range(5):
        run()
    us = tm.stop() / (5 * reps) * 1e3
    rate = 4.0 * B * H * T3 * T3 * dh / (us * 1e-6) / 1e12
    name = f"flash attention B={B} H={H} T={T3} d={dh}"
    log(f"kernels: {name}: {us:.1f} us, {rate:.1f} TFLOP/s ({rate / (lin_peak / 1e12):.1%} of the {lin_unit} peak)")
    out[name] = {"us": round(us, 2), "tflops": round(rate, 2)}
    del qkv3, att3
    # one whole-utterance vocoder inference (F0 net, excitation, decode; its convs are k_conv_cl_dma)
    from cv3amd.hift import DeviceHiFT
    h = DeviceHiFT(WeightStore(synth.hift_tensors(base=512), synth.hift_meta()))
    mel_d = to_device(hift_inputs(500)[0])
    h.inference(mel_d, graph=args.graph)
    synchronize()
    tm.start()
    h.inference(mel_d, graph=args.graph)
    ms = tm.stop()
    log(f"kernels: vocoder inference, 10 s whole: {ms:.2f} ms")
    out["vocoder_inference_ms"] = round(ms, 3)
    del h
    if args.kernel_solve:
        # the whole 10 s solve (22 blocks, 10 steps, CFG) for the end-to-end figure
        del d
        t22, m22 = synth.dit_tensors(depth=22), synth.dit_meta(depth=22)
        d = DeviceDiT(WeightStore(t22, m22, quant.QTensor))
        d.prepare(mu, spks, cond)
        d.solve(x0, graph=args.graph)
        synchronize()
        tm.start()
        for _ in range(3):
            d.solve(x0, graph=args.graph)
        ms = tm.stop() / 3
        log(f"kernels: 10 s solve {ms:.2f} ms ({d.flops_per_solve() / (ms / 1e3) / 1e12:.1f} TFLOP/s)")
        out["solve_10s_ms"] = round(ms, 3)
    return out


def cpu_flow(tensors, meta):
    """One estimator evaluation (22 blocks, the 10-step solve's unit) of the oracle."""
    import oracle.quant
    from oracle.dit import DiT
    from cv3amd.weights import WeightStore
    store = WeightStore(tensors, meta, oracle.quant.QTensor)
    mu, cond, spks, x0 = flow_inputs(500)
    T = 500
    mu_in = np.zeros((2, 80, T), np.float32)
    mu_in[0] = mu[0]
    cond_in = np.zeros((2, 80, T), np.float32)
    cond_in[0] = cond[0]
    spk_in = np.zeros((2, 80), np.float32)
    spk_in[0] = spks[0]
    dit = DiT(store, "flow.decoder.estimator.")
    t0 = time.perf_counter()
    dit.forward(np.broadcast_to(x0, (2, 80, T)), mu_in, np.array([0.0, 0.0], np.float32), spk_in, cond_in)
    return time.perf_counter() - t0


# ---------------------------------------------------------------------------
# vocoder
# ---------------------------------------------------------------------------

def hift_inputs(T: int):
    rng = np.random.default_rng(0)
    mel = (rng.standard_normal((80, T), dtype=np.float32) * np.float32(2.0) - np.float32(5.0)).astype(np.float32)
    # the NSF excitation's range: tanh of a small harmonic + noise mix (hift.py:90-111)
    source = np.tanh(rng.standard_normal(480 * T, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    return mel, source


def bench_hift(args, tensors, meta):
    from cv3amd.device import Timer, synchronize, to_device
    from cv3amd.hift import DeviceHiFT
    from cv3amd.weights import WeightStore
    T = 500
    d = DeviceHiFT(WeightStore(tensors, meta))
    mel, source = hift_inputs(T)
    mel_d, src_d = to_device(mel), to_device(source)
    out = {}
    for label, chunk, trim in (("whole", None, True), ("chunked_1s", 50, True), ("chunked_1s_context64", 50, False)):
        d.trim_context = trim   # False: every window carries all 64 frames of history
        d.decode(mel_d, src_d, chunk=chunk, graph=args.graph)
        synchronize()
        tm = Timer()
        tm.start()
        for _ in range(args.hift_runs):
            d.decode(mel_d, src_d, chunk=chunk, graph=args.graph)
        ms = tm.stop() / args.hift_runs
        out[label] = ms
        log(f"vocoder ({label}): {ms:.2f} ms per 10 s of audio, RTF {ms / 1e3 / AUDIO_SECONDS:.2e}")
    d.trim_context = True
    out["window_history"] = d.receptive
    # mel -> waveform with the F0 predictor and the excitation on the device as well
    for label, chunk in (("inference_whole", None), ("inference_chunked_1s", 50)):
        d.inference(mel_d, chunk=chunk, graph=args.graph)
        synchronize()
        tm = Timer()
        tm.start()
        for _ in range(args.hift_runs):
            d.inference(mel_d, chunk=chunk, graph=args.graph)
        ms = tm.stop() / args.hift_runs
        out[label] = ms
        log(f"vocoder ({label}): {ms:.2f} ms per 10 s of audio, RTF {ms / 1e3 / AUDIO_SECONDS:.2e}")
    out["flops_whole"] = d.flops(T)
    planes, f32 = d.flops_by_unit(T)
    out["by_unit_whole"] = (planes, 0.0, f32)
    return out


def cpu_hift(tensors, meta):
    """The oracle's whole-utterance inference (F0, excitation, decode) of the same mel
    on the host cores."""
    import oracle.quant
    from oracle.hift import HiFTGenerator
    from cv3amd.weights import WeightStore
    h = HiFTGenerator(WeightStore(tensors, meta, oracle.quant.QTensor), "hift.")
    mel, _ = hift_inputs(500)
    t0 = time.perf_counter()
    h.decode(mel, h.excitation(h.f0_predict(mel).astype(np.float32)))
    return time.perf_counter() - t0


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10,
                    help=f"timed steps; one step is one greedy decode of {DECODE_TOKENS} tokens from KV {PREFILL}")
    ap.add_argument("--warmup", type=int, default=2, help="untimed decodes first")
    ap.add_argument("--flow-solves", type=int, default=3)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--profile", default="per_channel", choices=["per_channel", "balanced"],
                    help="int8 scale layout of the LM weights")
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-core baseline")
    ap.add_argument("--no-tiny", action="store_true", help="skip the q4-body (tiny profile) decode")
    ap.add_argument("--no-flow", action="store_true")
    ap.add_argument("--no-flow-q8", action="store_true", help="skip the 30 s q8-weight solve")
    ap.add_argument("--no-hift", action="store_true")
    ap.add_argument("--hift-runs", type=int, default=3)
    ap.add_argument("--cpu-tokens", type=int, default=128)
    ap.add_argument("--decode-step", choices=("persistent", "kernels"), default="persistent",
                    help="the decode step the reported value times: one cooperative launch per token, or "
                         "five kernels per layer (replayed from a graph unless --no-graph)")
    ap.add_argument("--cooperative", action="store_true",
                    help="launch the one-launch step with hipLaunchCooperativeKernel (guaranteed co-residency, "
                         "about 20 us more per token) instead of an ordinary launch")
    ap.add_argument("--kernels", action="store_true",
                    help="time the roofline kernels one by one (one-launch decode tokens, each DiT block launch at "
                         "the 10 s shapes, the 30 s q8 GEMMs, a vocoder inference), print them as one JSON line "
                         "and exit: for per-kernel rooflines and rocprofv3 counter passes")
    ap.add_argument("--kernel-reps", type=int, default=20, help="launches per replay in --kernels")
    ap.add_argument("--no-kernel-solve", dest="kernel_solve", action="store_false",
                    help="--kernels without the closing 22-block 10 s solve")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="issue every launch directly instead of replaying captured HIP graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU layout is "
              "described in DESIGN.md and is not measured", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be at least 1 and --warmup at least 0")

    from cv3amd import _lib
    _lib.lib()
    _lib.init(0)
    info = _lib.device_info()
    log(f"device {info['arch']} with {info['cu_count']} CUs")
    if args.kernels:
        print(json.dumps({"kernels": bench_kernels(args)}), flush=True)
        return

    copy_bps = copy_bandwidth()
    log(f"device copy: {copy_bps / 1e9:.0f} GB/s (read + write of 256 MiB)")
    mfma_fps = mfma_peak(info["cu_count"])
    log(f"fp32 MFMA probe: {mfma_fps / 1e12:.1f} TFLOP/s (v_mfma_f32_32x32x2f32 on registers, "
        f"{info['cu_count']} workgroups x 8 waves)")
    t0 = time.time()
    lm_t, lm_meta = build_lm(args.layers, args.profile)
    log(f"LM weights ready ({time.time() - t0:.1f} s)")
    dec = bench_decode(args, lm_t, lm_meta)
    tiny = None
    if not args.no_tiny:
        t0 = time.time()
        tiny_t, tiny_meta = build_lm(args.layers, "tiny")
        log(f"LM weights, tiny profile (q4 body), ready ({time.time() - t0:.1f} s)")
        tiny = bench_decode(args, tiny_t, tiny_meta, label="decode tiny", decodes=max(1, min(args.steps, 3)),
                            warmup=1)
        del tiny_t

    flow = flow_q8 = None
    dit_t = dit_meta = None
    if not args.no_flow:
        from cv3amd import synth
        dit_t = synth.dit_tensors(depth=22)
        dit_meta = synth.dit_meta(depth=22)
        flow = bench_flow(args, dit_t, dit_meta)
        if not args.no_flow_q8:
            flow_q8 = {p: bench_flow_q8(args, dit_t, dit_meta, p) for p in ("per_channel", "balanced")}

    voc = None
    hift_t = hift_meta = None
    if not args.no_hift:
        from cv3amd import synth
        hift_t = synth.hift_tensors(base=512)
        hift_meta = synth.hift_meta()
        voc = bench_hift(args, hift_t, hift_meta)

    cores = cpu_cores()
    cpu = None
    cpu_flow_s = None
    cpu_hift_s = None
    if not args.no_cpu:
        log(f"cpu baseline: oracle decode of {args.cpu_tokens} tokens on {cores} host cores")
        cpu_tok_s, cpu_dt, cpu_toks = cpu_decode(lm_t, lm_meta, args.cpu_tokens)
        log(f"cpu baseline: {cpu_tok_s:.2f} tok/s ({cpu_dt:.1f} s)")
        if cpu_toks != dec["tokens"][:len(cpu_toks)]:
            raise RuntimeError("the oracle's greedy tokens differ from the device decode's")
        cpu = {"value": round(cpu_tok_s, 3), "unit": "tok/s", "cores": cores, "kind": "port",
               "sample": f"tokens 2..{args.cpu_tokens + 1} of the same 24-layer per-channel int8 greedy decode "
                         f"(KV {PREFILL + 1}->{PREFILL + 1 + args.cpu_tokens}, after one untimed token) by the "
                         f"oracle's NumPy restatement, its tokens identical to the device's; "
                         f"OpenBLAS threads = {cores}, host '{cpu_model()}'"}
        if flow is not None:
            log("cpu baseline: one 22-block estimator evaluation of the oracle")
            cpu_flow_s = cpu_flow(dit_t, dit_meta)
            log(f"cpu baseline: {cpu_flow_s:.2f} s per evaluation")
        if voc is not None:
            log("cpu baseline: one whole-utterance vocoder inference (F0 net, excitation, decode) of the oracle")
            cpu_hift_s = cpu_hift(hift_t, hift_meta)
            log(f"cpu baseline: {cpu_hift_s:.2f} s per 10 s of audio")

    kern = dec["kernel"]
    step_k = dec["step_kernel"] if dec["persistent"] else kern
    line = {
        "metric": METRIC,
        "decode_step": (("one cooperative launch" if args.cooperative else "one kernel launch") + " per token")
        if dec["persistent"] else "five kernels per layer",
        "launch_mode": "direct launches" if dec["persistent"] or not args.graph else "hip-graph replay",
        "value": round(dec["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 4),
        "ms_per_token": round(dec["ms"] / DECODE_TOKENS, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (int8 weights, per-channel f32 scales)" if args.profile == "per_channel"
        else "f32 (int8 weights, block-64 f16 scales)",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) KV prefill)",
        "config": {"workload": f"Qwen2-0.5B greedy decode, batch 1, {args.layers} layers, hidden 896, 14/2 heads x 64, "
                               f"SwiGLU 4864, int8 {args.profile}; one step = one decode of {DECODE_TOKENS} "
                               f"tokens, KV {PREFILL}->{PREFILL + DECODE_TOKENS}",
                   "decode_tokens": DECODE_TOKENS, "kv_prefill": PREFILL},
        "hbm_roofline_frac": round(dec["bytes_per_token"] * dec["tok_s"] / HBM_PEAK, 4),
        "bytes_per_token": dec["bytes_per_token"],
        "roofline": {"bound": "hbm", "achieved": round(step_k["achieved_Bps"] / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(step_k["achieved_Bps"] / HBM_PEAK, 4),
                     "traffic": TRAFFIC_DECODE_STEP if (dec["persistent"] and args.profile == "per_channel"
                                                         and args.layers == 24 and not args.cooperative) else None,
                     "kernel": step_k["name"], "bytes_per_launch": step_k["bytes_per_launch"],
                     "us_per_launch": round(step_k["us_per_launch"], 3)},
        "five_kernel_step": {
            "tok_s": round(dec["five_kernel_tok_s"], 2),
            "launch_mode": "hip-graph replay" if args.graph else "direct launches",
            "roofline": {"bound": "hbm", "achieved": round(kern["achieved_Bps"] / 1e9, 1), "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": round(kern["achieved_Bps"] / HBM_PEAK, 4), "traffic": None,
                         "kernel": kern["name"], "bytes_per_launch": kern["bytes_per_launch"],
                         "us_per_launch": round(kern["us_per_launch"], 3)}},
        "cpu_baseline": cpu,
        "copy_GBps": round(copy_bps / 1e9, 1),
        "mfma_f32_probe_TFLOPs": round(mfma_fps / 1e12, 2),
        "tokens_head": dec["tokens"][:8],
        "sampled_tok_s": round(dec["sampled_tok_s"], 2),
    }
    if tiny is not None:
        tk = tiny["kernel"]
        tsk = tiny["step_kernel"] if tiny["persistent"] else tk
        line["decode_tiny"] = {
            "workload": f"the same decode with the tiny profile: Qwen2 body layers q4 (block 32, f16 scales; held "
                        f"in HBM as the checkpoint's packed nibbles), head and speech embedding q8, "
                        f"KV {PREFILL}->{PREFILL + DECODE_TOKENS}",
            "decodes_timed": tiny["decodes"],
            "decode_step": "one kernel launch per token" if tiny["persistent"] else "five kernels per layer",
            "tok_s": round(tiny["tok_s"], 2), "ms_per_token": round(tiny["ms"] / DECODE_TOKENS, 5),
            "five_kernel_tok_s": round(tiny["five_kernel_tok_s"], 2),
            "bytes_per_token": tiny["bytes_per_token"],
            "hbm_roofline_frac": round(tiny["bytes_per_token"] * tiny["tok_s"] / HBM_PEAK, 4),
            # what the kernels stream per token as the body is held (equal to bytes_per_token
            # for packed nibbles; int8 codes with DeviceQwen2(widen_q4=True))
            "bytes_per_token_held": tiny["bytes_per_token_held"],
            "held_GBps": round(tiny["bytes_per_token_held"] * tiny["tok_s"] / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(tsk["achieved_Bps"] / 1e9, 1), "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": round(tsk["achieved_Bps"] / HBM_PEAK, 4), "kernel": tsk["name"],
                         "bytes_per_launch": tsk["bytes_per_launch"], "us_per_launch": round(tsk["us_per_launch"], 3)},
            "five_kernel_roofline": {"bound": "hbm", "achieved": round(tk["achieved_Bps"] / 1e9, 1),
                                     "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                                     "frac": round(tk["achieved_Bps"] / HBM_PEAK, 4), "kernel": tk["name"],
                                     "bytes_per_launch": tk["bytes_per_launch"],
                                     "us_per_launch": round(tk["us_per_launch"], 3)},
            "tokens_head": tiny["tokens"][:8],
        }
    if flow is not None:
        fk = flow["kernel"]
        rtf = flow["ms"] / 1e3 / AUDIO_SECONDS
        # the solve's matrix-core floor: its linears' flops at the split-bfloat16 peak, attention,
        # conv_pos and the AdaLN rows at the fp32 matrix peak
        floor_ms = matrix_floor_ms(flow["by_unit"])
        line["flow"] = {
            "workload": "DiT flow decoder, 10 s audio (500 frames), 22 blocks, 10 Euler steps, CFG, fp32 "
                        "(linears as six bfloat16 plane products, float32 accumulate)",
            "ms_per_solve": round(flow["ms"], 3), "rtf": round(rtf, 6),
            "tflops": round(flow["flops"] / (flow["ms"] / 1e3) / 1e12, 2),
            "roofline_ms": round(floor_ms, 3),
            "mfma_roofline_frac": round(floor_ms / flow["ms"], 4),
            # against the floor of running every flop on the fp32 matrix cores (26.9 ms)
            "fp32_mfma_frac": round(flow["flops"] / (flow["ms"] / 1e3) / FP32_MFMA_PEAK, 4),
            "flops_per_solve": flow["flops"], "flops_on_bf16_planes": flow["by_unit"][0],
            "roofline": {"bound": "mfma", "achieved": round(fk["achieved_flops"] / 1e12, 2),
                         "peak": round(fk["peak"] / 1e12, 1), "unit": "TFLOP/s",
                         "frac": round(fk["achieved_flops"] / fk["peak"], 4), "traffic": fk["traffic"],
                         "kernel": fk["name"], "us_per_launch": round(fk["us_per_launch"], 2)},
            "cpu_baseline": None if cpu_flow_s is None else {
                "value": round(cpu_flow_s * 10 / AUDIO_SECONDS, 3), "unit": "RTF", "cores": cores, "kind": "port",
                "sample": "one 22-block estimator evaluation (of the solve's 10) by the oracle, x10 extrapolated"},
        }
    if flow_q8 is not None:
        scales = {"per_channel": "per-output-channel int8 + float32 scales",
                  "balanced": "block-64 int8 + float16 scales (the converter's balanced profile)"}
        planes = ("the activation's three bfloat16 planes times the codes (exact in bfloat16), the {} scale on "
                  "each {} sum, fp32 accumulate")
        how = {"per_channel": planes.format("output channel's", "row"),
               "balanced": planes.format("block", "block")}
        if flow_q8.get("per_channel", {}).get("digits"):
            how["per_channel"] = ("QKV and ff1 with each activation row rounded 30 bits below its largest element "
                                  "and split into four int8 digit planes, each times the codes an exact int32 sum "
                                  "on the int8 matrix cores, combined in float64 and scaled per output channel; "
                                  "out and ff2 " + how["per_channel"])
        halves = ("; the CFG pair's two rows through the blocks on two streams"
                  if any(fq.get("halves") for fq in flow_q8.values()) else "")
        for prof, fq in flow_q8.items():
            line["flow_q8_30s" if prof == "per_channel" else "flow_q8_30s_block64"] = {
                "workload": f"DiT flow decoder, 30 s audio (1500 frames), 22 blocks, 10 Euler steps, CFG, q8 linears "
                            f"({scales[prof]}): {how[prof]}{halves}",
                "ms_per_solve": round(fq["ms"], 3), "rtf": round(fq["ms"] / 1e3 / 30.0, 6),
                "tflops": round(fq["flops"] / (fq["ms"] / 1e3) / 1e12, 2),
                "roofline_ms": round(matrix_floor_ms(fq["by_unit"]), 3),
                "mfma_roofline_frac": round(matrix_floor_ms(fq["by_unit"]) / fq["ms"], 4),
                "fp32_mfma_frac": round(fq["flops"] / (fq["ms"] / 1e3) / FP32_MFMA_PEAK, 4),
                "flops_per_solve": fq["flops"],
            }
    if voc is not None:
        line["vocoder"] = {
            "workload": "causal HiFTNet, mel [1, 80, 500] (10 s), base 512, ups x8/x5/x3, iSTFT 16/4, fp32; "
                        "ms_whole / ms_chunked_1s decode a precomputed source, ms_inference_* run mel -> waveform "
                        "(F0 net, NSF excitation and decode) on the device; 1 s windows with 64 frames of context, "
                        "each window computed from window_history_frames of it (the stack's receptive field: "
                        "the same samples), ms_chunked_1s_context64 from all 64",
            "ms_whole": round(voc["whole"], 3), "rtf_whole": round(voc["whole"] / 1e3 / AUDIO_SECONDS, 6),
            "ms_chunked_1s": round(voc["chunked_1s"], 3),
            "rtf_chunked_1s": round(voc["chunked_1s"] / 1e3 / AUDIO_SECONDS, 6),
            "window_history_frames": voc["window_history"],
            "ms_chunked_1s_context64": round(voc["chunked_1s_context64"], 3),
            "ms_inference_whole": round(voc["inference_whole"], 3),
            "rtf_inference_whole": round(voc["inference_whole"] / 1e3 / AUDIO_SECONDS, 6),
            "ms_inference_chunked_1s": round(voc["inference_chunked_1s"], 3),
            "conv_tflops_whole": round(voc["flops_whole"] / (voc["whole"] / 1e3) / 1e12, 2),
            "roofline_ms_whole": round(matrix_floor_ms(voc["by_unit_whole"]), 3),
            "flops_on_bf16_planes_whole": round(voc["by_unit_whole"][0] / voc["flops_whole"], 4),
            "mfma_roofline_frac_whole": round(matrix_floor_ms(voc["by_unit_whole"]) / voc["whole"], 4),
            "fp32_mfma_frac_whole": round(voc["flops_whole"] / (voc["whole"] / 1e3) / FP32_MFMA_PEAK, 4),
            "cpu_baseline": None if cpu_hift_s is None else {
                "value": round(cpu_hift_s / AUDIO_SECONDS, 3), "unit": "RTF", "cores": cores, "kind": "port",
                "sample": "one whole-utterance inference (F0 net, excitation, decode) of the same mel by the "
                          "oracle; compare with rtf_inference_whole"},
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
