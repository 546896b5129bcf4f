"""Packed-graph runner: the Kokoro graph walked node by node through the
drop-in dispatch on the GPU.

The walk restates PackedModel.run (tools/kpk_runtime.py:52-81) with the GPU
executor's memory discipline (executor.gd:190-195, 270-280): every
intermediate tensor is dropped from `env` after its last use, which returns
its buffer to libkk's pool.

`load_graph` reads the structure fixture extracted from the reference's
model.kpk (nodes, ops, shapes, structural constants, per-tensor statistics of
the learned weights); `synth_weights` draws seeded random learned weights of
the same dtype, shape and scale, which together give the full
Kokoro-82M-architecture graph with random-init weights (int8/uint8 for the
quantized contractions, fp16 elsewhere).
"""
import gzip
import json
import os

import numpy as np

from .dispatch import dispatch, to_device, to_host
from .fuse import fuse as fuse_chains
from .tensor import DeviceTensor

CODE_TO_NP = {0: np.float32, 1: np.int8, 2: np.uint8, 3: np.int32, 4: np.int64, 5: np.bool_,
              6: np.float16}


def load_graph(path):
    with gzip.open(path, "rt") as f:
        return json.load(f)


def synth_weights(graph, seed=0):
    """{tensor id: ndarray}: structural constants exact, learned tensors drawn
    from N(mean, std) of the original tensor, clipped to its [min, max] (and
    rounded for the integer types), one RNG stream per tensor id."""
    out = {}
    for tid, w in graph["weights"].items():
        dt = CODE_TO_NP[w["d"]]
        shape = tuple(w["s"])
        if "v" in w:
            out[int(tid)] = np.array(w["v"], dtype=dt).reshape(shape)
            continue
        mean, std, lo, hi = w["stat"]
        r = np.random.default_rng([int(seed), int(tid)])
        v = r.normal(mean, std, shape)
        if np.dtype(dt).kind in "iu":
            info = np.iinfo(dt)
            v = np.clip(np.rint(v), max(lo, info.min), min(hi, info.max))
        else:
            v = np.clip(v, lo, hi)
        out[int(tid)] = v.astype(dt)
    return out


def synth_inputs(n_ids=128, seed=0):
    """128 phoneme ids U{1..177} padded with 0 at both ends; a voice pack
    [510, 1, 256] ~ N(0, 0.1) indexed by length (row len(ids) - 3, as
    tools/voice_util.py:49-57 does for the padded ids); speed 1.0."""
    r = np.random.default_rng(seed)
    ids = np.concatenate([[0], r.integers(1, 178, n_ids), [0]]).astype(np.int64)
    pack = r.normal(0, 0.1, (510, 1, 256)).astype(np.float32)
    style = pack[min(max(len(ids) - 3, 0), 509)].reshape(1, 256)
    return ids, style, 1.0


def _decode_attrs(at):
    attrs = {}
    for k, v in (at or {}).items():
        if isinstance(v, dict) and "__t" in v:
            v = np.array(v["v"], dtype=CODE_TO_NP[v["__t"]]).reshape(v["s"])
        attrs[k] = v
    return attrs


class PackedGraph:
    """A packed graph with its weights resident on the device.

    With `fuse` (the default) the quantised-conv tails, InstanceNorm chains
    and snake chains run as single kernels; `groups[k]` lists the original
    node indices that node k stands for.  Tensors in `protect` stay
    readable after a run (they are never fused away)."""

    def __init__(self, graph, weights, fuse=True, protect=()):
        self.graph = graph
        self.ops = graph["ops"]
        nodes = [(self.ops[op], ["" if t < 0 else str(t) for t in ins],
                  ["" if t < 0 else str(t) for t in outs], _decode_attrs(at))
                 for op, ins, outs, at, _pl in graph["nodes"]]
        self.inputs = {k: str(v) for k, v in graph["inputs"].items()}
        self.output = str(graph["output"])
        # Weights: float data on the device once (fp16 widened to fp32 there,
        # except the fp16 weights that only Conv/ConvTranspose read, which
        # keep fp16 for the fp16 matrix-core convolutions), integer data
        # as-is; integer constants also stay on the host, where the
        # shape-domain nodes read them.
        conv_w, other = set(), set()
        for op, ins, _outs, _at in nodes:
            for k, name in enumerate(ins):
                (conv_w if op in ("Conv", "ConvTranspose") and k == 1 else other).add(name)
        conv_w -= other
        self.weights = {}
        for tid, arr in weights.items():
            arr = np.asarray(arr)
            if arr.dtype.kind in "iub" and arr.dtype.itemsize >= 4 or arr.dtype == np.bool_:
                self.weights[str(tid)] = arr
                continue
            if arr.dtype == np.float16 and str(tid) in conv_w:
                self.weights[str(tid)] = to_device(arr)
                continue
            if arr.dtype == np.float16:
                t = to_device(arr).astype(np.float32)
                host = arr.astype(np.float32)
            else:
                t = to_device(arr)
                host = arr
            if arr.size <= 16:
                t.host = host  # small constants are also read on the host
            self.weights[str(tid)] = t
        if fuse:
            keep = {self.output} | {str(p) for p in protect}
            self.nodes, self.groups = fuse_chains(nodes, self.weights, keep)
        else:
            self.nodes, self.groups = nodes, [[i] for i in range(len(nodes))]
        # Last use of every non-weight tensor (executor.gd:190-195).
        self.last_use = {}
        for i, (_op, ins, _outs, _at) in enumerate(self.nodes):
            for name in ins:
                if name and name not in self.weights:
                    self.last_use[name] = i
        self.last_use.pop(self.output, None)
        self.frees = [[] for _ in self.nodes]  # names whose last use is node i
        for name, i in self.last_use.items():
            self.frees[i].append(name)

    def run(self, input_ids, style, speed=1.0, keep=()):
        """Returns the waveform on the host (a numpy array)."""
        env = dict(self.weights)
        env[self.inputs["input_ids"]] = np.asarray(input_ids, np.int64).reshape(1, -1)
        env[self.inputs["style"]] = to_device(np.asarray(style, np.float32).reshape(1, 256))
        env[self.inputs["speed"]] = to_device(np.asarray([speed], np.float32))
        keep = {str(k) for k in keep}
        frees = self.frees
        for i, (op, ins, outs, at) in enumerate(self.nodes):
            try:
                dispatch(op, ins, outs, at, env)
            except Exception as exc:
                raise RuntimeError(f"node {i} {op}: {exc}") from exc
            for name in frees[i]:
                if name not in keep:
                    env.pop(name, None)
        out = env[self.output]
        self.last_env = {k: env[k] for k in keep if k in env}
        return to_host(out)


def default_graph_path():
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    return os.path.join(here, "tests", "golden", "kokoro_graph.json.gz")


__all__ = ["load_graph", "synth_weights", "synth_inputs", "PackedGraph", "DeviceTensor",
           "default_graph_path"]
