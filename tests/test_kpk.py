"""KPK1 model files (host only): the product's reader against a file built
byte by byte in the layout tools/pack_model.py:11-19 writes, the loader
checks of runtime/kpk_model.gd:67-139, a round trip of every dtype through
the writer, and -- where the reference's packed model is present (this
container, not the GPU box) -- the reference loader test's own checks
(tests/test_load_model.gd:32-86) plus equality with the packaged structure."""
import importlib
import json
import os
import struct

import numpy as np
import pytest

KPK_REF = "/root/reference/addons/best-tts/assets/model.kpk"


def kpk():
    return importlib.import_module("best-tts-godot_amd.kpk")


def graph_mod():
    return importlib.import_module("best-tts-godot_amd.graph")


def hand_built():
    """A two-node graph, written field by field: magic, <III header, JSON
    padded with NULs to 4 bytes, then the blob with 4-byte-aligned tensors."""
    emb = np.arange(-6, 6, dtype=np.int8).reshape(3, 4)
    bias = np.array([0.5, -1.25, 3.0], np.float32)
    shape = np.array([1, 3], np.int64)
    blob = emb.tobytes()                       # offset 0, 12 bytes
    blob += b"\0" * (-len(blob) % 4)
    o_bias = len(blob)
    blob += bias.tobytes()                     # offset 12
    o_shape = len(blob)
    blob += shape.tobytes()                    # offset 24
    desc = {
        "version": 1, "ops": ["Gather", "Add"],
        "tensors": ["emb", "bias", "shape", "ids", "style", "speed", "h", "waveform"],
        "weights": {"0": {"o": 0, "n": 12, "d": 1, "s": [3, 4]},
                    "1": {"o": o_bias, "n": 12, "d": 0, "s": [3]},
                    "2": {"o": o_shape, "n": 16, "d": 4, "s": [2]}},
        "nodes": [[0, [0, 3], [6], {"axis": 0}, 1], [1, [6, 1], [7], None, 1]],
        "inputs": {"input_ids": 3, "style": 4, "speed": 5}, "output": 7,
        "sample_rate": 24000, "samples_per_frame": 300,
    }
    payload = json.dumps(desc).encode()
    payload += b"\0" * (-len(payload) % 4)
    raw = b"KPK1" + struct.pack("<III", 1, len(payload), len(blob)) + payload + blob
    return raw, desc, {0: emb, 1: bias, 2: shape}


def test_reads_a_hand_built_file():
    raw, desc, want = hand_built()
    got_desc, got = kpk().parse_kpk(raw)
    for key in ("ops", "tensors", "nodes", "inputs", "output", "sample_rate"):
        assert got_desc[key] == desc[key]
    assert sorted(got) == [0, 1, 2]
    for tid, arr in want.items():
        assert got[tid].dtype == arr.dtype and got[tid].shape == arr.shape
        np.testing.assert_array_equal(got[tid], arr)
        assert not got[tid].flags.writeable  # views of the file's bytes


def test_loader_checks():
    K = kpk()
    raw, _desc, _w = hand_built()
    cases = {
        "not a .kpk file": b"KPK2" + raw[4:],
        "unsupported version": raw[:4] + struct.pack("<I", 2) + raw[8:],
        "truncated weight blob": raw[:-3],
        "malformed graph description": raw[:16] + b"[" + raw[17:],
    }
    for msg, bad in cases.items():
        with pytest.raises(K.KpkError, match=msg):
            K.parse_kpk(bad)
    # a weight that runs past the blob
    _v, jl, bl = struct.unpack_from("<III", raw, 4)
    desc = json.loads(raw[16:16 + jl].rstrip(b"\0"))
    desc["weights"]["2"]["o"] = bl - 8
    payload = json.dumps(desc).encode()
    payload += b"\0" * (-len(payload) % 4)
    bad = raw[:4] + struct.pack("<III", 1, len(payload), bl) + payload + raw[16 + jl:]
    with pytest.raises(K.KpkError, match="runs past the blob"):
        K.parse_kpk(bad)
    # byte count that does not match the shape
    desc["weights"]["2"]["o"] = 24
    desc["weights"]["2"]["n"] = 12
    payload = json.dumps(desc).encode()
    payload += b"\0" * (-len(payload) % 4)
    bad = raw[:4] + struct.pack("<III", 1, len(payload), bl) + payload + raw[16 + jl:]
    with pytest.raises(K.KpkError, match="bytes for shape"):
        K.parse_kpk(bad)


def test_round_trip_every_dtype(tmp_path):
    K = kpk()
    r = np.random.default_rng(0)
    weights = {5: r.normal(size=(2, 3)).astype(np.float32), 9: r.integers(-128, 128, 7).astype(np.int8),
               1: r.integers(0, 256, (3, 1, 5)).astype(np.uint8), 4: np.array([1, -2], np.int32),
               2: np.array([[7]], np.int64), 3: np.array([True, False, True]),
               8: r.normal(size=5).astype(np.float16), 6: np.zeros((0, 4), np.float32),
               7: np.array(2.5, np.float32), 11: np.asfortranarray(r.normal(size=(3, 4)).astype(np.float32))}
    desc = {"ops": ["Identity"], "tensors": [f"t{i}" for i in range(14)],
            "nodes": [[0, [5], [10], None, 1]], "inputs": {"input_ids": 0, "style": 12, "speed": 13},
            "output": 10, "sample_rate": 24000, "samples_per_frame": 300}
    path = os.path.join(tmp_path, "m.kpk")
    K.write_kpk(path, desc, weights)
    got_desc, got = K.read_kpk(path)
    assert got_desc["nodes"] == desc["nodes"] and got_desc["version"] == 1
    for tid, arr in weights.items():
        assert got[tid].dtype == arr.dtype and got[tid].shape == arr.shape
        np.testing.assert_array_equal(got[tid], arr)
        assert got_desc["weights"][str(tid)]["o"] % 4 == 0
    raw = open(path, "rb").read()
    _v, jl, bl = struct.unpack_from("<III", raw, 4)
    assert jl % 4 == 0 and 16 + jl + bl == len(raw)


def test_synthetic_model_round_trips(tmp_path):
    """The synthetic Kokoro model packed to KPK1 and read back holds the same
    description and the same weight bits."""
    G, K = graph_mod(), kpk()
    desc, weights = G.synth_model(seed=0)
    path = os.path.join(tmp_path, "synth.kpk")
    K.write_kpk(path, desc, weights)
    got_desc, got = K.read_kpk(path)
    for key in ("ops", "tensors", "nodes", "inputs", "output"):
        assert got_desc[key] == desc[key]
    assert sorted(got) == sorted(weights)
    for tid, arr in weights.items():
        assert got[tid].dtype == arr.dtype and got[tid].shape == arr.shape
        assert got[tid].tobytes() == arr.tobytes()


@pytest.mark.skipif(not os.path.exists(KPK_REF), reason="the reference's model.kpk is not here")
def test_reference_model_file():
    """The reference's packed model through the product's reader: the checks
    of tests/test_load_model.gd:32-86, and the packaged structure equals it
    (constants exactly, learned tensors by their statistics)."""
    G, K = graph_mod(), kpk()
    desc, w = K.read_kpk(KPK_REF)
    assert len(desc["nodes"]) == 3945 and len(w) == 781 and len(desc["ops"]) > 40
    assert desc["sample_rate"] == 24000 and desc["samples_per_frame"] == 300
    assert desc["tensors"][desc["output"]] == "waveform"
    assert sum(1 for n in desc["nodes"] if n[4] == 0) == 409
    emb = [a for a in w.values() if a.shape == (178, 128)]
    assert emb and emb[0].dtype == np.int8 and emb[0].nbytes == 178 * 128
    produced = set(w) | {desc["inputs"][k] for k in ("input_ids", "style", "speed")}
    for _op, ins, outs, _at, _pl in desc["nodes"]:
        assert all(t < 0 or t in produced for t in ins)
        produced |= {t for t in outs if t >= 0}
    assert desc["output"] in produced
    st = G.load_graph()
    for key in ("ops", "tensors", "nodes", "inputs", "output"):
        assert st[key] == desc[key]
    assert sorted(int(k) for k in st["weights"]) == sorted(w)
    for tid, arr in w.items():
        rec = st["weights"][str(tid)]
        assert list(arr.shape) == rec["s"] and K.NP_TO_CODE[arr.dtype] == rec["d"]
        if "v" in rec:
            np.testing.assert_array_equal(arr.reshape(-1).astype(np.float64 if arr.dtype.kind == "f" else np.int64),
                                          np.asarray(rec["v"]))
        else:
            f = arr.astype(np.float64)
            np.testing.assert_allclose([f.mean(), f.std(), f.min(), f.max()], rec["stat"], rtol=1e-9, atol=1e-12)
