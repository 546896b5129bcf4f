"""CPU oracle for whole-graph runs: walks a packed Kokoro graph node by node
through oracle.ref_ops.dispatch.

TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline, never the
product).  Restates PackedModel.run (tools/kpk_runtime.py:52-81): tensor ids
become string names ("" for -1), tensor-valued attributes {"__t","v","s"}
are decoded to numpy arrays, and every node goes through the same dispatch
the per-op oracle uses.
"""
import numpy as np

from . import ref_ops

CODE_TO_NP = {0: np.float32, 1: np.int8, 2: np.uint8, 3: np.int32, 4: np.int64, 5: np.bool_,
              6: np.float16}


def decode_attrs(at):
    attrs = {}
    for k, v in (at or {}).items():
        if isinstance(v, dict) and "__t" in v:
            v = np.array(v["v"], dtype=CODE_TO_NP[v["__t"]]).reshape(v["s"])
        attrs[k] = v
    return attrs


def run(graph, weights, input_ids, style, speed=1.0, max_nodes=None, capture=None):
    """graph: the fixture dict (ops, nodes, inputs, output); weights:
    {tensor id: ndarray}.  Returns the output waveform (and, with `capture`,
    a dict of the named intermediate tensor ids)."""
    env = {str(k): v for k, v in weights.items()}
    env[str(graph["inputs"]["input_ids"])] = np.asarray(input_ids, np.int64).reshape(1, -1)
    env[str(graph["inputs"]["style"])] = np.asarray(style, np.float32).reshape(1, 256)
    env[str(graph["inputs"]["speed"])] = np.asarray([speed], np.float32)
    ops = graph["ops"]
    # Intermediates are dropped after their last reader (the captured ones,
    # the weights and the output are kept), so that long utterances fit in
    # host memory; the values computed are the same.
    keep = {str(k) for k in weights} | {str(graph["output"])}
    keep |= {str(t) for t in (capture or ())}
    last = {}
    for i, (_op, ins, _outs, _at, _pl) in enumerate(graph["nodes"]):
        for t in ins:
            if t >= 0:
                last[str(t)] = i
    for i, (op_id, ins, outs, at, _place) in enumerate(graph["nodes"]):
        if max_nodes is not None and i >= max_nodes:
            break
        try:
            ref_ops.dispatch(ops[op_id], ["" if t < 0 else str(t) for t in ins],
                             ["" if t < 0 else str(t) for t in outs], decode_attrs(at), env)
        except Exception as exc:
            raise RuntimeError(f"node {i} {ops[op_id]}: {exc}") from exc
        if max_nodes is None:
            for t in ins:
                name = str(t)
                if t >= 0 and last.get(name) == i and name not in keep:
                    env.pop(name, None)
    out = env.get(str(graph["output"]))
    if capture is not None:
        return out, {t: env.get(str(t)) for t in capture}
    return out
