"""Device-resident DiT estimator and Euler/CFG solve against the oracle.

The oracle (oracle/dit.py, oracle/flow.py) restates cv3cpu/models/dit.py and
cv3cpu/models/flow.py on NumPy and is itself pinned to the reference's frozen
upstream flow output (tests/test_oracle_models.py).  Here both run the same
seeded synthetic weights (cv3amd/synth.py) at the full block geometry:
* one estimator evaluation (config 0's block, whole-forward form) <= 1e-5;
* a 10-step CFG solve at reduced depth <= 1e-4 (the flow parity bar);
* the balanced-profile q8 DiT at T = 1500 (in-GEMM dequantisation) <= 1e-4.
"""

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _stores(depth, profile="f32", T=None):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.weights import WeightStore
    t = synth.dit_tensors(depth=depth)
    if profile != "f32":
        t = synth.quantize_store(t, profile, oracle.quant.quantize_q8)
    meta = synth.dit_meta(depth=depth)
    return WeightStore(t, meta, oracle.quant.QTensor), WeightStore(t, meta, cv3amd.quant.QTensor)


def _inputs(T, seed=1):
    rng = np.random.default_rng(seed)
    mu = rng.standard_normal((1, 80, T), dtype=np.float32)
    cond = rng.standard_normal((1, 80, T), dtype=np.float32)
    spks = rng.standard_normal((1, 80), dtype=np.float32)
    x0 = rng.standard_normal((1, 80, T), dtype=np.float32)
    return mu, cond, spks, x0


def _oracle_forward(store, x0, mu, cond, spks, t):
    from oracle.dit import DiT
    T = mu.shape[2]
    mu_in = np.zeros((2, 80, T), np.float32)
    mu_in[0] = mu[0]
    cond_in = np.zeros((2, 80, T), np.float32)
    cond_in[0] = cond[0]
    spk_in = np.zeros((2, 80), np.float32)
    spk_in[0] = spks[0]
    return DiT(store, "flow.decoder.estimator.").forward(np.broadcast_to(x0, (2, 80, T)), mu_in,
                                                         np.array([t, t], np.float32), spk_in, cond_in)


@pytest.mark.parametrize("step,planes", [(0, True), (7, True), (0, False)])
def test_estimator_one_block_full_width(gpu, step, planes):
    """x [2, 500, 1024] through one AdaLN block plus the DiT's edges, with the linears on
    bfloat16 planes (the default) and on the float32 matrix cores."""
    from cv3amd.dit import DeviceDiT, euler_schedule
    cpu, dev = _stores(1)
    T = 500
    mu, cond, spks, x0 = _inputs(T)
    print(f"[flow] one-block estimator T={T} step={step} planes={planes}", flush=True)
    d = DeviceDiT(dev, planes=planes)
    d.prepare(mu, spks, cond)
    got = d.estimate(x0, step)
    ts, _ = euler_schedule(10)
    want = _oracle_forward(cpu, x0, mu, cond, spks, ts[step])
    e = rel_err(got, want)
    print(f"[flow] rel err {e:.2e}", flush=True)
    assert e < 1e-5


def test_solve_ten_steps_two_blocks(gpu):
    from oracle.flow import Flow
    from cv3amd.dit import DeviceDiT
    cpu, dev = _stores(2)
    T = 500
    mu, cond, spks, x0 = _inputs(T, seed=2)
    print(f"[flow] 10-step CFG solve depth=2 T={T}", flush=True)
    want = Flow(cpu, "flow.").solve_euler(mu, spks, cond, x0=x0)
    d = DeviceDiT(dev)
    d.prepare(mu, spks, cond)
    got = d.solve(x0).numpy()
    e = rel_err(got, want[0])
    print(f"[flow] eager rel err {e:.2e}", flush=True)
    assert e < 1e-4
    # the same solve replayed from a captured HIP graph, twice
    for rep in range(2):
        g = d.solve(x0, graph=True).numpy()
        print(f"[flow] graph replay {rep} rel err {rel_err(g, want[0]):.2e}", flush=True)
        assert rel_err(g, got) < 1e-6


def test_q8_dit_long_utterance(gpu):
    """Balanced profile (q8 block-64, f16 scales; time_embed/proj_out f16) at T = 1500."""
    from oracle.flow import Flow
    from cv3amd.dit import DeviceDiT
    cpu, dev = _stores(1, "balanced")
    T = 1500
    mu, cond, spks, x0 = _inputs(T, seed=3)
    print(f"[flow] q8 DiT depth=1 T={T}, 2 steps", flush=True)
    f = Flow(cpu, "flow.")
    f.n_timesteps = 2
    want = f.solve_euler(mu, spks, cond, x0=x0)
    d = DeviceDiT(dev, steps=2)
    d.prepare(mu, spks, cond)
    got = d.solve(x0).numpy()
    e = rel_err(got, want[0])
    print(f"[flow] rel err {e:.2e}", flush=True)
    assert e < 1e-4


@pytest.mark.parametrize("profile", ["f32", "per_channel"])
def test_cfg_halves_on_two_streams_change_nothing(gpu, profile):
    """From 1024 frames the CFG pair's two batch rows run through the blocks on two streams
    (forked and joined around them): the solve, eager and replayed from its graph three times,
    is bit-identical to the one with both rows in every launch."""
    import cv3amd.dit as dit
    _, dev = _stores(2, profile)
    T = 1100
    mu, cond, spks, x0 = _inputs(T, seed=7)
    d = dit.DeviceDiT(dev, steps=2)
    d.prepare(mu, spks, cond)
    assert d.halves == dit.HALVES and T >= dit.HALVES_MIN_T
    print(f"[flow] halves {profile} depth=2 T={T}", flush=True)
    d.halves = False
    want = d.solve(x0).numpy().copy()
    d.halves, d._graph = True, None
    np.testing.assert_array_equal(d.solve(x0).numpy(), want)
    for _ in range(3):
        np.testing.assert_array_equal(d.solve(x0, graph=True).numpy(), want)
    d.prepare(mu[:, :, :500], spks, cond[:, :, :500])
    assert not d.halves
