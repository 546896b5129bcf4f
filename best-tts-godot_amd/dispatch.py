"""Drop-in op dispatch: ``dispatch(op, node_input, node_output, attrs, env)``.

Same signature, op names, attribute names and defaults as the reference's
``RefRuntime.dispatch`` (tools/ref_runtime.py:428-668): `env` maps tensor
names to values, inputs are read by name (``""`` = absent), outputs are
written by name.  Values are :class:`DeviceTensor` for tensor data on the
GPU; numpy arrays are host values.

Placement follows the reference's GPU executor: float tensors are computed
on the device by libkk's HIP kernels; small integer/bool "shape-domain"
tensors (shapes, axes, indices, sizes) live on the host and the ops that
only touch them run there, as executor.gd places its 409 CPU shape nodes
(executor.gd:483-518 -> cpu_ops.gd:66-140).  A float op given host data
uploads it first; nothing float is ever computed on the host.

fp16 is storage only (tools/NOTES.md:44-59): fp16 data is widened to fp32 on
the device when it enters a device op, every float result is fp32, and
Cast(to=float16) yields fp32.
"""
import numpy as np

from . import ops
from .hostops import slice_clamp
from .tensor import DeviceTensor

# ONNX TensorProto element types -> numpy (ref_runtime.py:24-28)
ONNX_DTYPE = {
    1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16, 5: np.int16,
    6: np.int32, 7: np.int64, 9: np.bool_, 10: np.float16, 11: np.float64,
    12: np.uint32, 13: np.uint64,
}

# Shape-domain nodes stay on the host when all their inputs are host values
# (cpu_ops.gd:66-140 lists the same family): pure data movement for any
# dtype, arithmetic and comparisons only on integer/bool data.
_HOST_MOVE_OPS = {
    "Shape", "Reshape", "Unsqueeze", "Squeeze", "Concat", "Slice", "Gather",
    "Cast", "Transpose", "Expand", "Split",
}
# The shortest conv output whose InstanceNorm takes the block-wise
# statistics (rows of nine 8192-blocks or more; shorter rows are held on
# chip, read once): only there do leaf sums save a pass.
_LEAF_MIN_STEPS = 9 * 8192

_HOST_INT_OPS = {
    "Equal", "Where", "Greater", "Less", "GreaterOrEqual", "And", "Add", "Sub", "Mul",
    "Div", "CumSum",
}


def _is_dev(v):
    return isinstance(v, DeviceTensor)


def to_device(v):
    """Device copy of a host value; fp16 data is widened to fp32 on the GPU."""
    if v is None or _is_dev(v):
        return v
    arr = np.asarray(v)
    if arr.dtype == np.float64:
        raise TypeError("float64 host data has no device type (fp32 compute only)")
    t = DeviceTensor.from_numpy(arr)
    return t


def _f32(t):
    """_f32 of the reference (ref_runtime.py:49-51): widen fp16 storage."""
    if t is not None and t.dtype == np.float16:
        return t.astype(np.float32)
    return t


def to_host(v):
    """Host array of a value.  A device value is downloaded (a sync point)
    unless it is a constant whose host copy was kept at upload."""
    if _is_dev(v):
        return v.host if v.host is not None else v.numpy()
    return v


def _host_int(v):
    return v is not None and not _is_dev(v) and np.asarray(v).dtype.kind in "iub"


def _slice_params(dim, s, e, st):
    """Clamp like op_slice (ref_runtime.py:307-325) and resolve the python
    slice to (start, stop, step) of the selected range."""
    s, e = slice_clamp(dim, s, e, st)
    r = range(dim)[slice(s, e, st)]
    return r.start, r.stop, r.step, len(r)


def _per_channel(t, x):
    """True when t is absent or holds x's C values broadcasting along T
    (shape [..., C, 1]; any shape of one value when C is 1), the operand form
    the fused instance-norm kernels apply per channel."""
    if t is None:
        return True
    C = x.shape[-2] if len(x.shape) >= 2 else 0
    sh = tuple(t.shape)
    if int(np.prod(sh, dtype=np.int64)) != C or len(sh) > len(x.shape):
        return False
    return C == 1 or (len(sh) >= 2 and sh[-1] == 1 and sh[-2] == C)


def _norm_chain(xd, sc, sh, eps, leaky_alpha):
    """The fused InstanceNorm chain's float result: one launch when scale and
    shift are per channel, else the statistics' launch and then the chain's
    Mul, Add and LeakyRelu nodes, broadcasting as numpy does."""
    if _per_channel(sc, xd) and _per_channel(sh, xd):
        return ops.instance_norm_scale_shift(xd, sc, sh, eps, leaky_alpha)
    y = ops.instance_norm_scale_shift(xd, None, None, eps, None)
    if sc is not None:
        y = ops.binary("Mul", y, sc)
    if sh is not None:
        y = ops.binary("Add", y, sh)
    if leaky_alpha is not None:
        y = ops.unary("LeakyRelu", y, np.float32(leaky_alpha))
    return y


def _qconv_resid(at, inp, x, w):
    """A quantised conv that took in the residual Add after it (attribute
    "resid", the residual's input index): the residual when the epilogue can
    add it -- an fp32 device tensor of the conv output's shape (the Add's
    x + y in fp32, ref_runtime.py:446-447, commutes) -- else None (and the
    Add runs after the conv, with its broadcasting)."""
    k = at.get("resid")
    if k is None:
        return None
    r = inp(k)
    pads = at.get("pads", [0, 0])
    s, d = at.get("strides", [1])[0], at.get("dilations", [1])[0]
    n, _, L = x.shape
    cout, _, kw = w.shape
    lout = (L + pads[0] + pads[1] - d * (kw - 1) - 1) // s + 1
    if isinstance(r, DeviceTensor) and r.dtype == np.float32 and tuple(r.shape) == (n, cout, lout):
        return r
    return None


def dispatch(op, node_input, node_output, at, env):
    """Execute one node.  Mirrors tools/ref_runtime.py:428-668."""

    def inp(i, default=None):
        if i >= len(node_input) or not node_input[i]:
            return default
        return env[node_input[i]]

    x = inp(0)
    y = inp(1)

    # ---------------------------------------------------- host shape domain
    if op in ("Range", "NonZero"):
        # Shape-domain results the host needs (frame counts, alignment
        # indices): device inputs are downloaded here -- the data-dependent
        # sync points of the GPU executor (executor.gd:474-491, 543-563).
        from . import hostops
        local = {n: to_host(env[n]) for n in node_input if n}
        hostops.run(op, node_input, node_output, at, local)
        env[node_output[0]] = local[node_output[0]]
        return
    if (op in _HOST_MOVE_OPS or op in _HOST_INT_OPS) and not (_is_dev(x) or _is_dev(y)):
        present = [inp(i) for i in range(len(node_input)) if inp(i) is not None]
        host = bool(present) and all(not _is_dev(v) for v in present)
        if host and op in _HOST_INT_OPS:
            host = all(_host_int(v) for v in present)
        if host and op != "Shape":
            from . import hostops
            hostops.run(op, node_input, node_output, at, env)
            return

    out = None
    # ------------------------------------------------ elementwise / math
    if op in ("Add", "Sub", "Mul", "Div", "Pow"):
        out = ops.binary(op, to_device(x), to_device(y))
    elif op in ("Sqrt", "Exp", "Sin", "Cos", "Atan", "Tanh", "Sigmoid", "Floor", "Round", "Erf"):
        out = ops.unary(op, _f32(to_device(x)))
    elif op == "LeakyRelu":
        out = ops.unary(op, to_device(x), np.float32(at.get("alpha", 0.01)))
    elif op == "Clip":
        lo, hi = inp(1), inp(2)
        out = ops.clip(to_device(x), to_device(lo), to_device(hi))

    # --------------------------------------------- comparison / logic
    elif op in ("Equal", "Greater", "Less", "GreaterOrEqual", "And"):
        out = ops.binary(op, to_device(x), to_device(y))
    elif op == "Where":
        out = ops.where(to_device(x), to_device(y), to_device(inp(2)))

    # --------------------------------------------------- shape / layout
    elif op == "Shape":
        s = np.array(x.shape, dtype=np.int64)
        out = s[at.get("start", 0):at.get("end", len(s))]
    elif op == "Reshape":
        shape = [int(v) for v in np.asarray(to_host(y)).reshape(-1)]
        if not at.get("allowzero", 0):
            shape = [x.shape[i] if v == 0 else v for i, v in enumerate(shape)]
        out = x.reshape(shape)
    elif op == "Transpose":
        out = x.transpose(at.get("perm"))
    elif op == "Unsqueeze":
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        for a in sorted(int(v) for v in np.asarray(to_host(axes)).reshape(-1)):
            x = x.expand_dims(a)
        out = x
    elif op == "Squeeze":
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        out = x.squeeze(None if axes is None else
                        [int(v) for v in np.asarray(to_host(axes)).reshape(-1)])
    elif op == "Concat":
        vals = [to_device(env[i]) for i in node_input if i]
        if any(v.dtype == np.float16 for v in vals):
            vals = [_f32(v) for v in vals]
        axis = int(at["axis"]) % vals[0].ndim
        dt = np.result_type(*[v.dtype for v in vals])
        shape = list(vals[0].shape)
        shape[axis] = sum(v.shape[axis] for v in vals)
        out = DeviceTensor.empty(shape, dt)
        pos = 0
        for v in vals:
            n = v.shape[axis]
            if n:
                ops.copy_into(out.slice_axis(axis, pos, pos + n), v)
            pos += n
    elif op == "Split":
        axis = int(at.get("axis", 0)) % x.ndim
        split = inp(1)
        dim = x.shape[axis]
        if split is None:
            n = len(node_output)
            q, r = divmod(dim, n)
            sizes = [q + 1] * r + [q] * (n - r)
        else:
            sizes = [int(v) for v in np.asarray(to_host(split)).reshape(-1)]
        # np.split at the running sums: the last part runs to the end.
        pos = 0
        for k, (name, sz) in enumerate(zip(node_output, sizes)):
            lo = min(pos, dim)
            hi = dim if k == len(sizes) - 1 else min(max(pos + sz, lo), dim)
            if name:
                env[name] = x.slice_axis(axis, lo, hi)
            pos += sz
        return
    elif op == "Slice":
        starts = np.asarray(to_host(inp(1))).reshape(-1)
        ends = np.asarray(to_host(inp(2))).reshape(-1)
        axes = inp(3)
        steps = inp(4)
        axes = list(range(len(starts))) if axes is None else np.asarray(to_host(axes)).reshape(-1)
        steps = [1] * len(starts) if steps is None else np.asarray(to_host(steps)).reshape(-1)
        out = x
        for s, e, a, st in zip(starts, ends, axes, steps):
            a = int(a) % x.ndim
            start, _, step, n = _slice_params(x.shape[a], int(s), int(e), int(st))
            out = out.slice_axis(a, start, start + n * step, step) if n else \
                out.slice_axis(a, 0, 0)
    elif op == "Gather":
        axis = int(at.get("axis", 0))
        idx = y
        if not _is_dev(idx):
            idx = np.asarray(idx).astype(np.int64)
            dim = x.shape[axis]
            if idx.size and (idx.min() < -dim or idx.max() >= dim):
                raise IndexError(f"index out of bounds for axis {axis} with size {dim}")
        out = ops.gather(to_device(x), to_device(idx), axis)
    elif op == "Expand":
        shape = np.broadcast_shapes(x.shape, tuple(int(v) for v in to_host(y)))
        out = to_device(x).broadcast_to(shape).contiguous()
    elif op == "ConstantOfShape":
        v = at.get("value", np.array([0], dtype=np.float32))
        v = np.asarray(v)
        dt = np.float32 if v.dtype == np.float16 else v.dtype
        shape = [int(s) for s in np.asarray(to_host(x)).reshape(-1)]
        if np.dtype(dt).kind == "f":
            out = ops.fill(shape, v.reshape(-1)[0], dt)
        else:  # integer fills are shape-domain data: host
            out = np.full(shape, v.reshape(-1)[0], dtype=dt)
    elif op == "Cast":
        to = ONNX_DTYPE[at["to"]]
        dt = np.float32 if to == np.float16 else to
        if _is_dev(x) and x.dtype == dt:
            out = x
        else:
            out = to_device(x).astype(dt)

    # --------------------------------------------- reductions / norms
    elif op in ("ReduceMean", "ReduceSum"):
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        keep = bool(at.get("keepdims", 1))
        v = _f32(to_device(x))
        if axes is None:
            if at.get("noop_with_empty_axes", 0):
                out = v
            else:
                out = ops.reduce(op, v, range(v.ndim), keep)
        else:
            axes_t = [int(a) for a in np.asarray(to_host(axes)).reshape(-1)]
            out = v if not axes_t else ops.reduce(op, v, axes_t, keep)
    elif op == "Softmax":
        out = ops.softmax(_f32(to_device(x)), at.get("axis", -1))
    elif op == "LayerNormalization":
        out = ops.layernorm(_f32(to_device(x)), _f32(to_device(y)),
                            _f32(to_device(inp(2))), at.get("axis", -1),
                            at.get("epsilon", 1e-5))
    elif op == "SkipLayerNormalization":
        out = ops.layernorm(_f32(to_device(x)), _f32(to_device(inp(2))),
                            _f32(to_device(inp(3))), -1, at.get("epsilon", 1e-12),
                            skip=_f32(to_device(y)), skip_bias=_f32(to_device(inp(4))))
    elif op == "FastGelu":
        out = ops.fast_gelu(to_device(x), to_device(y))

    # --------------------------------------------------- matmul / conv
    elif op == "MatMul":
        out = ops.matmul(to_device(x), to_device(y))
    elif op == "FusedMatMul":
        a, b = to_device(x), to_device(y)
        if at.get("transA", 0):
            a = a.transpose(list(range(a.ndim - 2)) + [a.ndim - 1, a.ndim - 2])
        if at.get("transB", 0):
            b = b.transpose(list(range(b.ndim - 2)) + [b.ndim - 1, b.ndim - 2])
        out = ops.matmul(a, b, alpha=np.float32(at.get("alpha", 1.0)))
    elif op == "DequantizeLinear":
        out = ops.dequantize(to_device(x), to_device(y), to_device(inp(2)))
    elif op == "Conv":
        # attribute "packed" (set by a graph at load): the name of this
        # constant weight's kk_conv_pack layout in env
        out = ops.conv1d(_f32(to_device(x)), to_device(y), _f32(to_device(inp(2))),
                         at.get("pads", [0, 0]), at.get("strides", [1])[0],
                         at.get("dilations", [1])[0], at.get("group", 1),
                         packed=env.get(at.get("packed")))
    elif op == "ConvTranspose":
        out = ops.conv_transpose1d(_f32(to_device(x)), to_device(y), _f32(to_device(inp(2))),
                                   at.get("pads", [0, 0]), at.get("strides", [1])[0],
                                   at.get("dilations", [1])[0], at.get("group", 1),
                                   at.get("output_padding", [0])[0],
                                   packed=env.get(at.get("packed")))

    elif op == "CumSum":
        out = ops.cumsum(_f32(to_device(x)), int(np.asarray(to_host(y)).item()))
    elif op == "Pad":
        pads = np.asarray(to_host(inp(1))).reshape(-1)
        value = 0.0 if inp(2) is None else float(np.asarray(to_host(inp(2))).item())
        out = ops.pad(_f32(to_device(x)), pads, at.get("mode", "constant"), value)
    elif op == "Resize":
        scales = inp(2) if inp(2) is not None else inp(3)
        mode = at.get("mode", "nearest")
        ctm = at.get("coordinate_transformation_mode", "half_pixel")
        nearest = at.get("nearest_mode", "round_prefer_floor")
        if mode == "nearest" and (ctm != "asymmetric" or nearest != "floor"):
            raise NotImplementedError(f"resize nearest {ctm}/{nearest}")
        if mode == "linear" and ctm != "half_pixel":
            raise NotImplementedError(f"resize linear {ctm}")
        if mode not in ("nearest", "linear"):
            raise NotImplementedError(f"resize mode {mode}")
        scale = float(np.asarray(to_host(scales)).reshape(-1)[-1])
        out = ops.resize(_f32(to_device(x)), scale, mode)
    elif op == "ScatterND":
        out = ops.scatter_nd(_f32(to_device(x)), to_host(y), _f32(to_device(inp(2))))
    elif op == "STFT":
        out = ops.stft(_f32(to_device(x)), _f32(to_device(inp(2))),
                       int(np.asarray(to_host(y)).item()),
                       int(np.asarray(to_host(inp(3))).item()), at.get("onesided", 1))
    elif op == "DynamicQuantizeLinear":
        for name, v in zip(node_output, ops.dynamic_quantize_linear(_f32(to_device(x)))):
            if name:
                env[name] = v
        return
    elif op == "MatMulInteger":
        out = ops.matmul_integer(to_device(x), to_device(y), to_device(inp(2)),
                                 to_device(inp(3)))
    elif op == "ConvInteger":
        out = ops.conv_integer(to_device(x), to_device(y), to_device(inp(2)), to_device(inp(3)),
                               at.get("pads", [0, 0]), at.get("strides", [1])[0],
                               at.get("dilations", [1])[0], at.get("group", 1))
    elif op == "DynamicQuantizeLSTM":
        res = ops.lstm(_f32(to_device(x)), to_device(y), to_device(inp(2)),
                       _f32(to_device(inp(3))), _f32(to_device(inp(5))),
                       _f32(to_device(inp(6))), _f32(to_device(inp(8))), to_device(inp(9)),
                       _f32(to_device(inp(10))), to_device(inp(11)), int(at["hidden_size"]),
                       at.get("direction") == "bidirectional")
        for name, v in zip(node_output, res):
            if name:
                env[name] = v
        return

    # -------------------------------------- fused composites (libkk only)
    elif op == "Snake":
        # x + recip * sin(alpha * x)^2: the Mul/Sin/Pow/Mul/Add chain fused.
        out = ops.snake(to_device(x), to_device(y), to_device(inp(2)))
    elif op == "QConvScaled" and at.get("bias_quant"):
        # the same with the bias quantisation ahead of it folded in: inputs
        # x, w, x_zp, w_zp, "", "", scale_a, scale_w, bias (fp32); scale =
        # scale_a * scale_w, int32 bias = Cast(Floor(Div(bias, scale))).
        x, y = to_device(x), to_device(y)
        resid = _qconv_resid(at, inp, x, y)
        packed = env.get(at.get("packed"))
        # a second output: the leaf sums of the result for the InstanceNorm
        # that reads it, where its rows take the block-wise statistics
        # (at least nine 8192-blocks; none otherwise)
        pads, st, dil = at.get("pads", [0, 0]), at.get("strides", [1])[0], at.get("dilations", [1])[0]
        lout = (x.shape[2] + pads[0] + pads[1] - dil * (y.shape[2] - 1) - 1) // st + 1
        leafy = (len(node_output) > 1 and node_output[1] and packed is not None and
                 ("resid" not in at or resid is not None) and lout >= _LEAF_MIN_STEPS)
        out = ops.conv_integer_scaled_qbias(x, y, to_device(inp(2)),
                                            to_device(inp(3)), _f32(to_device(inp(8))),
                                            _f32(to_device(inp(6))), _f32(to_device(inp(7))),
                                            pads, st, dil, at.get("group", 1), resid=resid,
                                            packed=packed, leaves=leafy)
        if leafy:
            out, env[node_output[1]] = out
        elif len(node_output) > 1 and node_output[1]:
            env[node_output[1]] = None
        if "resid" in at and resid is None:  # the Add it took in, after it
            out = ops.binary("Add", out, to_device(inp(at["resid"])))
    elif op == "QConvScaled":
        # ConvInteger -> Add(int32 bias) -> Cast(float) -> Mul(scale), fused;
        # inputs x, w, x_zp, w_zp, bias ("" if absent), scale.
        x, y = to_device(x), to_device(y)
        resid = _qconv_resid(at, inp, x, y)
        out = ops.conv_integer_scaled(x, y, to_device(inp(2)),
                                      to_device(inp(3)), to_device(inp(4)),
                                      _f32(to_device(inp(5))), at.get("pads", [0, 0]),
                                      at.get("strides", [1])[0], at.get("dilations", [1])[0],
                                      at.get("group", 1), resid=resid)
        if "resid" in at and resid is None:
            out = ops.binary("Add", out, to_device(inp(at["resid"])))
    elif op == "QMatMulScaled":
        # MatMulInteger -> Cast(float) -> Mul(scale) (-> Add(bias)), fused;
        # inputs a, b, a_zp, b_zp, scale, bias ("" if absent), and with
        # scale_product the scale's two factors (the Mul that formed it) as
        # inputs 6 and 7.  A scale or bias that is not one value or one per
        # output column (it would broadcast the product to another shape)
        # runs the chain node by node.
        a, b = to_device(x), to_device(y)
        a_zp, b_zp = to_device(inp(2)), to_device(inp(3))
        bias = _f32(to_device(inp(5)))
        n, rank = b.shape[-1], max(a.ndim, b.ndim)

        def per_col(t):
            return t is None or (t.ndim <= rank and t.size in (1, n) and
                                 (t.size == 1 or t.shape[-1] == n))
        scale2 = None
        if at.get("scale_product"):
            scale, scale2 = _f32(to_device(inp(6))), _f32(to_device(inp(7)))
            if not (per_col(scale) and per_col(scale2)):
                scale, scale2 = ops.binary("Mul", scale, scale2), None
        else:
            scale = _f32(to_device(inp(4)))
        # attribute "packed" (set by a graph at load): the name of this
        # constant B's kk_matmul_integer_pack layout in env
        packed = env.get(at.get("packed"))
        if a.shape[-1] and per_col(scale) and per_col(bias):
            out = ops.matmul_integer_scaled(a, b, a_zp, b_zp, scale, bias, scale2, packed=packed)
        else:
            if scale2 is not None:
                scale = ops.binary("Mul", scale, scale2)
            out = ops.binary("Mul", ops.matmul_integer(a, b, a_zp, b_zp, packed=packed)
                             .astype(np.float32), scale)
            if bias is not None:
                out = ops.binary("Add", out, bias)
    elif op == "InstanceNormScaleShift":
        # ReduceMean/Sub/Mul/ReduceMean/Add/Sqrt/Div [-> Mul -> Add -> LeakyRelu], fused;
        # inputs x, scale ("" if absent), shift ("" if absent).
        # Operands that are not per channel run past the statistics node by node.
        out = _norm_chain(_f32(to_device(x)), _f32(to_device(y)), _f32(to_device(inp(2))),
                          at["epsilon"], at.get("leaky_alpha"))
    elif op == "InstanceNormSnake":
        # the InstanceNorm chain (+ Mul scale, Add shift), then the snake chain on its
        # output; inputs x, scale, shift ("" if absent), alpha, recip (C values each).
        xd, a, rc = _f32(to_device(x)), _f32(to_device(inp(3))), _f32(to_device(inp(4)))
        sc, sh = _f32(to_device(y)), _f32(to_device(inp(2)))
        if all(_per_channel(t, xd) for t in (sc, sh, a, rc)):
            out = ops.instance_norm_scale_shift_snake(xd, sc, sh, a, rc, at["epsilon"])
        else:  # an operand not per channel: the two chains one after the other
            out = ops.snake(_norm_chain(xd, sc, sh, at["epsilon"], None), a, rc)
    elif op == "InstanceNormQuant":
        # the InstanceNorm chain (+ Mul scale, Add shift, then LeakyRelu or the snake
        # chain) -> Cast(float) -> DynamicQuantizeLinear, fused; inputs x, scale,
        # shift, alpha, recip ("" if absent); the outputs are the quantiser's.
        xd = _f32(to_device(x))
        sc, sh = _f32(to_device(y)), _f32(to_device(inp(2)))
        a, rc = inp(3), inp(4)
        a = _f32(to_device(a)) if a is not None else None
        rc = _f32(to_device(rc)) if rc is not None else None
        if all(_per_channel(t, xd) for t in (sc, sh, a, rc)):
            # input 5: x's leaf sums from the conv that produced it, or None
            res = ops.instance_norm_quant(xd, sc, sh, a, rc, at["epsilon"], at.get("leaky_alpha"),
                                          leaves=env.get(node_input[5]) if len(node_input) > 5
                                          and node_input[5] and xd is x else None)
        else:  # an operand not per channel: the chains one after the other
            yv = _norm_chain(xd, sc, sh, at["epsilon"], None if a is not None else
                             at.get("leaky_alpha"))
            res = ops.dynamic_quantize_linear(ops.snake(yv, a, rc) if a is not None else yv)
        for name, v in zip(node_output, res):
            if name:
                env[name] = v
        return
    elif op == "AdaIN":
        # inputs: x, style, W, bias; attribute epsilon.
        out = ops.adain(to_device(x), to_device(y), to_device(inp(2)),
                        to_device(inp(3)), at.get("epsilon", 1e-5))
    else:
        raise NotImplementedError(f"{op}")

    env[node_output[0]] = out
