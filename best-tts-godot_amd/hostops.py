"""Host shape-domain ops: integer/bool tensors of shapes, axes and indices.

These are the nodes the reference's GPU executor also keeps on the CPU
(executor.gd:483-518 -> runtime/cpu_ops.gd:66-140): a handful of int64
elements each.  Only integer/bool data reaches this module (dispatch routes
it here when every input is a host integer array); float tensors never do.
Semantics follow the matching branches of tools/ref_runtime.py:446-586.
"""
import numpy as np

ONNX_DTYPE = {
    1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16, 5: np.int16,
    6: np.int32, 7: np.int64, 9: np.bool_, 10: np.float16, 11: np.float64,
    12: np.uint32, 13: np.uint64,
}


def slice_clamp(dim, s, e, st):
    """Clamp one axis's start/end like op_slice (ref_runtime.py:307-325):
    into [0, dim] for a positive step, into [-1, dim - 1] for a negative one,
    where a python slice then reads -1 as the last element."""
    if st > 0:
        s = min(max(s if s >= 0 else s + dim, 0), dim)
        e = min(max(e if e >= 0 else e + dim, 0), dim)
    else:
        s = min(max(s if s >= 0 else s + dim, -1), dim - 1)
        e = min(max(e if e >= 0 else e + dim, -1), dim - 1)
    return s, e


def _slice(data, starts, ends, axes, steps):
    r = data.ndim
    axes = list(range(len(starts))) if axes is None else axes
    steps = [1] * len(starts) if steps is None else steps
    sl = [slice(None)] * r
    for s, e, a, st in zip(starts, ends, axes, steps):
        a = int(a) % r
        st = int(st)
        s, e = slice_clamp(data.shape[a], int(s), int(e), st)
        sl[a] = slice(s, e, st)
    return data[tuple(sl)]


def run(op, node_input, node_output, at, env):
    def inp(i):
        if i >= len(node_input) or not node_input[i]:
            return None
        return np.asarray(env[node_input[i]])

    x, y = inp(0), inp(1)
    if op == "Add":
        out = x + y
    elif op == "Sub":
        out = x - y
    elif op == "Mul":
        out = x * y
    elif op == "Div":
        out = x // y
    elif op == "Equal":
        out = np.equal(x, y)
    elif op == "Greater":
        out = np.greater(x, y)
    elif op == "Less":
        out = np.less(x, y)
    elif op == "GreaterOrEqual":
        out = np.greater_equal(x, y)
    elif op == "And":
        out = np.logical_and(x, y)
    elif op == "Where":
        out = np.where(x, y, inp(2))
    elif op == "Reshape":
        shape = [int(v) for v in y.reshape(-1)]
        if not at.get("allowzero", 0):
            shape = [x.shape[i] if v == 0 else v for i, v in enumerate(shape)]
        out = x.reshape(shape)
    elif op == "Transpose":
        out = np.transpose(x, at.get("perm"))
    elif op in ("Unsqueeze", "Squeeze"):
        axes = y if len(node_input) > 1 else at.get("axes")
        if op == "Unsqueeze":
            for a in sorted(int(v) for v in np.asarray(axes).reshape(-1)):
                x = np.expand_dims(x, a)
            out = x
        else:
            out = np.squeeze(x) if axes is None else \
                np.squeeze(x, tuple(int(v) for v in np.asarray(axes).reshape(-1)))
    elif op == "Concat":
        out = np.concatenate([np.asarray(env[i]) for i in node_input if i], axis=at["axis"])
    elif op == "Split":
        axis = at.get("axis", 0)
        if y is None:
            parts = np.array_split(x, len(node_output), axis=axis)
        else:
            parts = np.split(x, np.cumsum([int(v) for v in y])[:-1], axis=axis)
        for name, p in zip(node_output, parts):
            if name:
                env[name] = p
        return
    elif op == "Slice":
        out = _slice(x, y, inp(2), inp(3), inp(4))
    elif op == "Gather":
        out = np.take(x, y.astype(np.int64), axis=at.get("axis", 0))
    elif op == "Expand":
        out = np.broadcast_to(x, np.broadcast_shapes(x.shape, tuple(int(v) for v in y))).copy()
    elif op == "ConstantOfShape":
        v = np.asarray(at.get("value", np.array([0], dtype=np.float32)))
        dt = np.float32 if v.dtype == np.float16 else v.dtype
        out = np.full([int(s) for s in x], v.reshape(-1)[0], dtype=dt)
    elif op == "Range":
        out = np.arange(x.item(), y.item(), inp(2).item(), dtype=x.dtype)
    elif op == "NonZero":
        out = np.array(np.nonzero(x), dtype=np.int64)
    elif op == "CumSum":
        out = np.cumsum(x, axis=int(y.item()))
    elif op == "Cast":
        to = ONNX_DTYPE[at["to"]]
        out = x.astype(np.float32 if to == np.float16 else to)
    else:
        raise NotImplementedError(f"{op} (host)")
    env[node_output[0]] = out
