"""The reference's weight file (cv3cpu/io/weights.py, io/safetensors_io.py) read by
cv3amd.weightfile.DeviceWeightFile.

Pinned against the official ``safetensors`` library (files it writes are read here,
files written here are read by it) and against the reference's own weight tests
(tests/test_weights.py:170-300): round trip with a folded conv, alignment of
tensors after an odd-length one, foreign files, page eviction, BF16 widening.
"""

import json
import struct

import numpy as np
import pytest

import oracle.quant as oq
from cv3amd.weightfile import DeviceWeightFile, write_weight_file


def _q8(w, orig_shape=None):
    q, s, _ = oq.quantize_q8(w)
    return {"kind": "q8", "q": q, "scales": s, "shape": w.shape, "block": oq.Q8_BLOCK, "orig_shape": orig_shape}


def _q4(w, orig_shape=None):
    q, s, _ = oq.quantize_q4(w)
    return {"kind": "q4", "q": q, "scales": s, "shape": w.shape, "block": oq.Q4_BLOCK, "orig_shape": orig_shape}


def _open(path):
    return DeviceWeightFile(str(path), oq.QTensor)


def test_roundtrip_folded_conv_and_half(tmp_path):
    """tests/test_weights.py:170-192 with this package's reader."""
    rng = np.random.default_rng(2)
    w = rng.normal(size=(200, 301)).astype(np.float32)
    b = rng.normal(size=200).astype(np.float32)
    conv = rng.normal(size=(64, 32, 5)).astype(np.float32)
    p = tmp_path / "t.safetensors"
    write_weight_file(str(p), {"lin.weight": _q8(w), "lin.bias": b,
                               "conv.weight": _q8(conv.reshape(64, -1), conv.shape),
                               "half": w.astype(np.float16)}, meta={"hello": "world"})
    with _open(p) as f:
        assert f.meta["hello"] == "world"
        assert np.array_equal(f.get("lin.bias"), b)
        assert f.get("conv.weight").kernel_size == 5
        assert f.entry("conv.weight")["shape"] == [64, 32, 5]
        assert f.entry("conv.weight")["mshape"] == [64, 160]
        assert f.entry("half") == {"kind": "f16", "shape": [200, 301], "nbytes": 200 * 301 * 2}
        assert np.abs(f.get_f32("half") - w).max() < 1e-2
        x = rng.normal(size=(3, 301)).astype(np.float32)
        ref = x @ w.T + b
        got = oq.qmatmul(x, f.get("lin.weight"), f.get("lin.bias"))
        assert np.abs(got - ref).mean() / np.abs(ref).mean() < 0.02
        assert set(f.subset("lin.")) == {"weight", "bias"}
        assert sorted(f.keys()) == ["conv.weight", "half", "lin.bias", "lin.weight"]
        assert "lin.weight.__scales__" not in f
        assert f.get("lin.weight") is f.get("lin.weight")


@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_quantised_entries_are_the_stored_codes(tmp_path, kind):
    """Payload and scales come back bit for bit, ragged K included."""
    rng = np.random.default_rng(5)
    w = rng.normal(size=(9, 100)).astype(np.float32)
    rec = _q8(w) if kind == "q8" else _q4(w)
    p = tmp_path / "q.safetensors"
    write_weight_file(str(p), {"w": rec})
    with _open(p) as f:
        t = f.get("w")
        assert t.kind == kind and t.shape == (9, 100) and t.block == rec["block"]
        assert t.q.dtype == (np.int8 if kind == "q8" else np.uint8)
        assert t.scales.dtype == np.float16
        assert np.array_equal(t.q, rec["q"]) and np.array_equal(t.scales, rec["scales"])
        want = oq.QTensor(kind, rec["q"], rec["scales"], (9, 100), rec["block"]).dequant()
        assert np.array_equal(f.get_f32("w"), want)


def test_files_are_readable_by_the_official_library(tmp_path):
    """tests/test_weights.py:223-256: the layout is plain safetensors."""
    stnp = pytest.importorskip("safetensors.numpy")
    from safetensors import safe_open
    rng = np.random.default_rng(0)
    w = rng.normal(size=(64, 96)).astype(np.float32)
    conv = rng.normal(size=(8, 4, 5)).astype(np.float32)
    p = str(tmp_path / "m.safetensors")
    write_weight_file(p, {"llm.w": _q8(w), "hift.conv.weight": _q4(conv.reshape(8, -1), conv.shape),
                          "hift.bias": np.arange(8, dtype=np.float32)}, meta={"sample_rate": 24000})
    loaded = stnp.load_file(p)
    assert loaded["llm.w"].dtype == np.int8
    assert loaded["llm.w.__scales__"].dtype == np.float16
    assert loaded["hift.conv.weight"].dtype == np.uint8
    with safe_open(p, framework="numpy") as fh:
        blob = json.loads(fh.metadata()["cv3cpu"])
    assert blob["version"] == 1
    assert blob["meta"]["sample_rate"] == 24000
    assert blob["quant"]["hift.conv.weight"] == {"kind": "q4", "block": 32, "shape": [8, 4, 5], "mshape": [8, 20]}
    with _open(p) as ours:
        assert np.array_equal(ours.get("llm.w").q, loaded["llm.w"])
        assert np.array_equal(ours.get("llm.w").scales, loaded["llm.w.__scales__"])
        assert np.array_equal(ours.get("hift.bias"), loaded["hift.bias"])


def test_reads_what_the_official_library_writes(tmp_path):
    """A file in the reference layout written by the official library, quant blob by hand."""
    stnp = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(1)
    w = rng.normal(size=(16, 128)).astype(np.float32)
    q, s, _ = oq.quantize_q8(w)
    blob = {"version": 1, "meta": {"llm": {"hidden_size": 16}},
            "quant": {"m.w": {"kind": "q8", "block": 64, "shape": [16, 128], "mshape": [16, 128]}}}
    p = str(tmp_path / "official.safetensors")
    stnp.save_file({"m.w": q, "m.w.__scales__": s, "a": np.arange(6, dtype=np.float32).reshape(2, 3),
                    "i": np.arange(5, dtype=np.int64)}, p, metadata={"cv3cpu": json.dumps(blob)})
    with _open(p) as f:
        assert f.meta == {"llm": {"hidden_size": 16}}
        assert np.array_equal(f.get("a"), np.arange(6, dtype=np.float32).reshape(2, 3))
        assert f.entry("i") == {"kind": "i64", "shape": [5], "nbytes": 40}
        t = f.get("m.w")
        assert np.array_equal(t.q, q) and np.array_equal(t.scales, s)
        assert np.array_equal(t.dequant(), oq.QTensor("q8", q, s, (16, 128), 64).dequant())
    p2 = str(tmp_path / "plain.safetensors")
    stnp.save_file({"a": np.ones(3, np.float32)}, p2, metadata={"note": "hi"})
    with _open(p2) as f:
        assert f.meta == {}  # no cv3cpu blob in a foreign file


def test_misaligned_tensors_are_still_read_correctly(tmp_path):
    """tests/test_weights.py:273-300: an odd-length int8 tensor shifts the rest."""
    rng = np.random.default_rng(9)
    w = rng.normal(size=(16, 64)).astype(np.float32)
    p = tmp_path / "odd.safetensors"
    write_weight_file(str(p), {"odd_bytes": np.arange(7, dtype=np.uint8), "w": _q8(w), "f": w})
    with _open(p) as f:
        assert f.get("w").scales.ctypes.data % 2 == 0
        assert f.get("f").ctypes.data % 4 == 0
        assert not f.get("f").flags.writeable
        assert np.abs(f.get_f32("f") - w).max() == 0.0


def test_bf16_is_widened(tmp_path):
    vals = np.array([1.0, -2.5, 3.140625, 0.0], np.float32)
    raw = (vals.view(np.uint32) >> 16).astype("<u2").tobytes()
    head = json.dumps({"b": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, len(raw)]}}).encode()
    p = tmp_path / "bf.safetensors"
    p.write_bytes(struct.pack("<Q", len(head)) + head + raw)
    with _open(p) as f:
        got = f.get("b")
        assert got.dtype == np.float32 and np.array_equal(got.ravel(), vals)


def test_rejects_foreign_and_truncated_files(tmp_path):
    p = tmp_path / "nope.safetensors"
    p.write_bytes(b"XXXX" + b"\0" * 128)
    with pytest.raises(Exception):
        DeviceWeightFile(str(p))
    head = json.dumps({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    p2 = tmp_path / "short.safetensors"
    p2.write_bytes(struct.pack("<Q", len(head)) + head + b"\0" * 8)
    with pytest.raises(ValueError, match="outside the file"):
        DeviceWeightFile(str(p2))


def test_evict_releases_pages_and_rereads(tmp_path):
    """tests/test_weights.py:207-219."""
    rng = np.random.default_rng(3)
    p = tmp_path / "big.safetensors"
    write_weight_file(str(p), {"stage1.w": _q8(rng.normal(size=(4000, 4000)).astype(np.float32)),
                               "stage2.w": _q8(rng.normal(size=(1000, 1000)).astype(np.float32))})
    with _open(p) as f:
        x = np.ones((1, 4000), np.float32)
        first = f.get("stage1.w")
        before = oq.qmatmul(x, first)
        assert f.stage_bytes("stage1.") == 4000 * 4032 + 4000 * 63 * 2  # K padded to 63 blocks of 64
        assert f.evict("stage1.") > 8 << 20
        again = f.get("stage1.w")
        assert again is not first  # the cached object went with the pages
        assert np.array_equal(oq.qmatmul(x, again), before)
        assert f.evict("nothing.") == 0


def test_evict_spares_other_stages_between(tmp_path):
    """A stage's tensors stored around another stage's: eviction advises only the stage's
    own byte runs (each run's whole pages), never the pages of the tensor in between."""
    import mmap
    rng = np.random.default_rng(4)
    p = tmp_path / "interleaved.safetensors"
    big = lambda: rng.normal(size=(512, 2048)).astype(np.float32)   # 4 MiB each
    write_weight_file(str(p), {"a.first": big(), "b.middle": big(), "a.last": big()})
    with _open(p) as f:
        middle = np.array(f.get("b.middle"))
        freed = f.evict("a.")
        page = mmap.PAGESIZE
        # two runs of 4 MiB each: at most their sizes, at least their whole interior pages
        assert 2 * (4 << 20) - 2 * 2 * page <= freed <= 2 * (4 << 20)
        assert f.evict("b.") <= 4 << 20
        assert np.array_equal(np.asarray(f.get("b.middle")), middle)
        assert f.stage_bytes("a.") == 2 * (4 << 20) and f.total_bytes() == 3 * (4 << 20)
