"""Layout of the streamed one-launch decode step's weights (cv3_qwen2_stream_pack).

The plan must cover every row of every matrix exactly once per layer (q, k, v rows
in rotary pairs, o_proj rows, [gate; up] pairs, down rows in four K quarters, head
rows), and each packed 1 KB tile must hold, at lane l's 16 bytes, codes
16 (l // 16) .. +16 of the 64-code block of the row its column l % 16 names: the
B-operand order of v_mfma_i32_16x16x64_i8.  Checked against a NumPy gather of the
same stacked weights, with the scales beside them.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# plan fields (the table's int64 words per workgroup)
P_A, P_C, P_ND, P_D0, P_D1, P_NE, P_E0, P_E1, P_NH, P_H0, P_H1 = range(11)
P_SB, P_SBH, P_NL, P_NHT, P_OFF, P_STRIDE, P_HOFF, P_SPAD, P_SPADH = range(11, 20)
QUARTERS = 4


def _rows(unit_type, u, j, kt, D, I, dh, V, KB, KBQ):
    """(matrix, row, k-block) of column j of tile kt of a unit, as the pack lays it out."""
    if unit_type == "A":
        upk = dh // 16
        hd, sub = divmod(u, upk)
        return "qkv", hd * dh + sub * 8 + (j & 7) + (dh // 2 if j >= 8 else 0), kt
    if unit_type == "C":
        return "o", u * 16 + j, kt
    if unit_type == "D":
        return "gate_up", (0 if kt < KB else I) + u * 16 + j, kt % KB
    if unit_type == "E":
        return "down", (u // QUARTERS) * 16 + j, (u % QUARTERS) * KBQ + kt
    return "head", min(u * 16 + j, V - 1), kt


def _units(P, head):
    if head:
        return [("H", int(P[P_H0 + i])) for i in range(int(P[P_NH]))]
    out = []
    if P[P_A] >= 0:
        out.append(("A", int(P[P_A])))
    if P[P_C] >= 0:
        out.append(("C", int(P[P_C])))
    out += [("D", int(P[P_D0 + i])) for i in range(int(P[P_ND]))]
    out += [("E", int(P[P_E0 + i])) for i in range(int(P[P_NE]))]
    return out


@pytest.mark.parametrize("profile", ["per_channel", "balanced"])
def test_stream_plan_and_packed_tiles(gpu, profile):
    import oracle.quant
    import cv3amd.quant
    from cv3amd import synth
    from cv3amd.qwen2 import DeviceQwen2
    from cv3amd.weights import WeightStore
    L = 2
    t = synth.quantize_store(synth.qwen2_tensors(layers=L), profile, oracle.quant.quantize_q8)
    d = DeviceQwen2(WeightStore(t, synth.qwen2_meta(layers=L), cv3amd.quant.QTensor), cap=1024)
    plan = d.stream_plan()
    data = d._sdata.numpy()
    G = plan.shape[0]
    D, I, dh, H = d.hidden, d.inter, d.head_dim, d.heads
    V = d.head.rows
    KB, KBQ = D // 64, I // 64 // QUARTERS
    mats = {"qkv": d.qkv, "o": d.o, "gate_up": d.gate_up, "down": d.down, "head": d.head}
    host = {k: (m.q.numpy(), m.scales.numpy()) for k, m in mats.items()}
    print(f"[stream] {G} workgroups, {profile}, {data.nbytes / 1e6:.1f} MB packed", flush=True)
    # coverage: every (matrix, row, k-block) of a layer exactly once (head rows past V are clamped copies)
    cover = {k: np.zeros((m.rows, m.k // 64), np.int64) for k, m in mats.items()}   # rows per layer
    per_wg_tiles = []
    for w in range(G):
        P = plan[w]
        n_tiles = 0
        for head in (False, True):
            for ut, u in _units(P, head):
                nt = 2 * KB if ut == "D" else KBQ if ut == "E" else KB
                n_tiles += nt if not head else 0
                for kt in range(nt):
                    for j in range(16):
                        mat, row, kb = _rows(ut, u, j, kt, D, I, dh, V, KB, KBQ)
                        if ut != "H" or u * 16 + j < V:
                            cover[mat][row, kb] += 1
        per_wg_tiles.append(n_tiles)
        assert n_tiles == P[P_NL]
    for mat, c in cover.items():
        assert c.min() == 1 and c.max() == 1, f"{mat}: rows covered {c.min()}..{c.max()} times"
    assert plan[:, P_ND].min() >= 1                           # every workgroup owns [gate; up] rows
    # attention items live on the last H * 8 workgroups, which own no qkv or o_proj unit
    assert (plan[G - 8 * H:, P_A] < 0).all() and (plan[G - 8 * H:, P_C] < 0).all()
    print(f"[stream] tiles per workgroup and layer: {min(per_wg_tiles)}..{max(per_wg_tiles)}", flush=True)
    # bytes: every tile of a sample of workgroups, both layers and the head region
    rng = np.random.default_rng(0)
    lanes = np.arange(64)
    for w in sorted(set(rng.integers(0, G, 12).tolist()) | {0, G - 1}):
        P = plan[w]
        for l in range(L + 1):
            head = l == L
            region = int(P[P_OFF]) + (int(P[P_HOFF]) if head else l * int(P[P_STRIDE]))
            tiles0 = region + int(P[P_SPADH] if head else P[P_SPAD])
            ti, soff = 0, region
            for ut, u in _units(P, head):
                nt = 2 * KB if ut == "D" else KBQ if ut == "E" else KB
                lay = 0 if head else l
                for kt in range(nt):
                    got = data[tiles0 + (ti + kt) * 1024: tiles0 + (ti + kt + 1) * 1024].reshape(64, 16)
                    for lane in lanes:
                        mat, row, kb = _rows(ut, u, lane % 16, kt, D, I, dh, V, KB, KBQ)
                        q, _ = host[mat]
                        rows_per_layer = mats[mat].rows
                        want = q[lay * rows_per_layer + row, kb * 64 + (lane // 16) * 16: kb * 64 + (lane // 16) * 16 + 16]
                        assert np.array_equal(got[lane].view(np.int8), want), (w, l, ut, u, kt, lane)
                # scales
                if profile == "balanced":
                    sc = data[soff: soff + nt * 32].view(np.float16).reshape(nt, 16)
                    for kt in range(nt):
                        for j in range(16):
                            mat, row, kb = _rows(ut, u, j, kt, D, I, dh, V, KB, KBQ)
                            s = host[mat][1]
                            rows_per_layer = mats[mat].rows
                            assert sc[kt, j] == s[lay * rows_per_layer + row, kb]
                    soff += nt * 32
                else:
                    sets = 2 if ut == "D" else 1
                    sc = data[soff: soff + sets * 64].view(np.float32).reshape(sets, 16)
                    for st in range(sets):
                        for j in range(16):
                            mat, row, _ = _rows(ut, u, j, st * KB, D, I, dh, V, KB, KBQ)
                            s = host[mat][1]
                            rows_per_layer = mats[mat].rows
                            assert sc[st, j] == s[lay * rows_per_layer + row, 0]
                    soff += sets * 64
                ti += nt
