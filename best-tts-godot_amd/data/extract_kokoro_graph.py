"""Extracts the Kokoro-82M graph *structure* from the reference's packed model
into kokoro_graph.json.gz -- data only, no weights.

Source: addons/best-tts/assets/model.kpk (KPK1: 16-byte header, JSON graph,
weight blob; layout per tools/pack_model.py:11-19, read here with struct/json
/numpy.frombuffer, which execute nothing from the file).

The fixture keeps
  * ops, nodes (op id, input ids, output ids, attributes, placement), the
    graph inputs/output, sample rate and samples per frame;
  * for every weight tensor: dtype code and shape;
  * the exact values of structural constants: every int64/int32/bool tensor
    and every tensor of at most 16 elements (shape vectors, axes, epsilons,
    zero points, SineGen constants, Resize scales ...);
  * for every other (learned) tensor: mean, std, min and max, so a seeded
    generator can draw random weights of the same dtype, shape and scale.
The learned values themselves are not stored.
"""
import gzip
import json
import os
import struct
import sys

import numpy as np

KPK = "/root/reference/addons/best-tts/assets/model.kpk"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kokoro_graph.json.gz")
CODE_TO_NP = {0: np.float32, 1: np.int8, 2: np.uint8, 3: np.int32, 4: np.int64, 5: np.bool_,
              6: np.float16}
SMALL = 16


def main(path=KPK, out=OUT):
    raw = open(path, "rb").read()
    if raw[:4] != b"KPK1":
        raise ValueError("not a KPK1 file")
    _ver, jl, bl = struct.unpack_from("<III", raw, 4)
    g = json.loads(raw[16:16 + jl].rstrip(b"\0"))
    blob = raw[16 + jl:16 + jl + bl]
    weights = {}
    n_const = n_learned = 0
    for tid, w in g["weights"].items():
        dt = CODE_TO_NP[w["d"]]
        a = np.frombuffer(blob, dtype=dt, count=w["n"] // np.dtype(dt).itemsize,
                          offset=w["o"]).reshape(w["s"])
        rec = {"d": w["d"], "s": w["s"]}
        if w["d"] in (3, 4, 5) or a.size <= SMALL:
            rec["v"] = a.reshape(-1).astype(np.float64 if w["d"] in (0, 6) else np.int64).tolist()
            n_const += 1
        else:
            f = a.astype(np.float64)
            rec["stat"] = [float(f.mean()), float(f.std()), float(f.min()), float(f.max())]
            n_learned += 1
        weights[tid] = rec
    fixture = {
        "source": "addons/best-tts/assets/model.kpk (structure and constants only)",
        "ops": g["ops"], "nodes": g["nodes"], "inputs": g["inputs"], "output": g["output"],
        "tensors": g["tensors"], "sample_rate": g.get("sample_rate"),
        "samples_per_frame": g.get("samples_per_frame"), "weights": weights,
    }
    with gzip.open(out, "wt") as f:
        json.dump(fixture, f, separators=(",", ":"))
    print(f"wrote {out}: {len(g['nodes'])} nodes, {n_const} constants, {n_learned} learned "
          f"tensors, {os.path.getsize(out)} bytes")


if __name__ == "__main__":
    main(*sys.argv[1:])
