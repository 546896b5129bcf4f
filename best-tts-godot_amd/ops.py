"""Device ops: allocate the output from the pool and call libkk.

Each function takes DeviceTensors (or None for optional operands) and
returns a new DeviceTensor.  Shapes are computed here with numpy's rules;
the kernels re-validate them before launching.
"""
import numpy as np

from . import _lib
from .tensor import DeviceTensor


def _d(t):
    return None if t is None else t.desc()


def _float_out(*ts):
    return np.float32


def broadcast_shape(*shapes):
    return tuple(np.broadcast_shapes(*[tuple(s) for s in shapes]))


# ------------------------------------------------------------ elementwise
def binary(op, a, b, out_dtype=None):
    shape = broadcast_shape(a.shape, b.shape)
    if out_dtype is None:
        fa, fb = a.dtype.kind == "f", b.dtype.kind == "f"
        if op in ("Equal", "Greater", "Less", "GreaterOrEqual", "And"):
            out_dtype = np.bool_
        elif fa and fb:
            out_dtype = np.float32
        elif not fa and not fb:
            out_dtype = np.result_type(a.dtype, b.dtype)
        else:
            raise NotImplementedError(f"{op}: mixed float/integer operands {a.dtype}, {b.dtype}")
    out = DeviceTensor.empty(shape, out_dtype)
    _lib.call("kk_binary", _lib.OP[op], out.desc(), a.desc(), b.desc())
    return out


def unary(op, x, alpha=0.0):
    out = DeviceTensor.empty(x.shape, np.float32 if x.dtype.kind == "f" or op not in
                             ("Neg", "Abs", "Identity") else x.dtype)
    _lib.call("kk_unary", _lib.OP[op], out.desc(), x.desc(), float(alpha))
    return out


def where(cond, x, y):
    shape = broadcast_shape(cond.shape, x.shape, y.shape)
    if x.dtype.kind == "f" or y.dtype.kind == "f":
        dt = np.float32
    else:
        dt = np.result_type(x.dtype, y.dtype)
    out = DeviceTensor.empty(shape, dt)
    _lib.call("kk_where", out.desc(), cond.desc(), x.desc(), y.desc())
    return out


def clip(x, lo=None, hi=None):
    shape = broadcast_shape(x.shape, *[t.shape for t in (lo, hi) if t is not None])
    out = DeviceTensor.empty(shape, np.float32)
    _lib.call("kk_clip", out.desc(), x.desc(), _d(lo), _d(hi))
    return out


def snake(x, alpha, recip=None):
    """y = x + r*sin(alpha*x)^2 with r = recip, or 1/alpha when recip is None."""
    shapes = [x.shape, alpha.shape] + ([recip.shape] if recip is not None else [])
    out = DeviceTensor.empty(broadcast_shape(*shapes), np.float32)
    _lib.call("kk_snake", out.desc(), x.desc(), alpha.desc(), _d(recip))
    return out


def fast_gelu(x, bias=None):
    shape = broadcast_shape(x.shape, bias.shape) if bias is not None else x.shape
    out = DeviceTensor.empty(shape, np.float32)
    _lib.call("kk_fast_gelu", out.desc(), x.desc(), _d(bias))
    return out


def dequantize(q, scale, zp=None):
    shapes = [q.shape, scale.shape] + ([zp.shape] if zp is not None else [])
    out = DeviceTensor.empty(broadcast_shape(*shapes), np.float32)
    _lib.call("kk_dequantize", out.desc(), q.desc(), scale.desc(), _d(zp))
    return out


def cast(x, dtype):
    return x.astype(dtype)


def fill(shape, value, dtype=np.float32):
    out = DeviceTensor.empty(shape, dtype)
    _lib.call("kk_fill", out.desc(), float(value))
    return out


def copy_into(dst_view, src):
    _lib.call("kk_copy", dst_view.desc(), src.desc())


def gather(data, indices, axis=0):
    axis = int(axis) % data.ndim
    data = data.contiguous()
    indices = indices.contiguous()
    shape = data.shape[:axis] + indices.shape + data.shape[axis + 1:]
    out = DeviceTensor.empty(shape, data.dtype)
    _lib.call("kk_gather", out.desc(), data.desc(), indices.desc(), axis)
    return out


# ------------------------------------------------------------- reductions
def reduce(op, x, axes, keepdims=True):
    code = {"ReduceSum": _lib.REDUCE_SUM, "ReduceMean": _lib.REDUCE_MEAN,
            "ReduceMax": _lib.REDUCE_MAX}[op]
    axes = sorted({int(a) % x.ndim for a in axes}) if x.ndim else []
    mask = 0
    for a in axes:
        mask |= 1 << a
    kept = [d for i, d in enumerate(x.shape) if i not in axes]
    out = DeviceTensor.empty(kept, np.float32)
    _lib.call("kk_reduce", code, out.desc(), x.desc(), mask)
    if keepdims:
        return out.reshape([1 if i in axes else d for i, d in enumerate(x.shape)])
    return out


def instance_norm(x, gamma_beta=None, eps=1e-5):
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_instance_norm_affine", out.desc(), x.desc(), _d(gamma_beta), float(eps))
    return out


def adain(x, style, w, bias=None, eps=1e-5, w_scale=None, w_zp=None):
    """InstanceNorm over T of x [1, C, T] with (1+gamma, beta) = style.W + b."""
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_adain", out.desc(), x.desc(), style.contiguous().desc(), w.desc(),
              _d(w_scale), _d(w_zp), _d(bias), float(eps))
    return out


def layernorm(x, scale, bias=None, axis=-1, eps=1e-5, skip=None, skip_bias=None):
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_layernorm", out.desc(), x.desc(),
              _d(skip.contiguous() if skip is not None else None),
              _d(skip_bias.contiguous() if skip_bias is not None else None),
              scale.contiguous().desc(),
              _d(bias.contiguous() if bias is not None else None), int(axis), float(eps))
    return out


def softmax(x, axis=-1):
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_softmax", out.desc(), x.desc(), int(axis))
    return out


# ----------------------------------------------------------- contractions
def matmul(a, w, w_scale=None, w_zp=None, alpha=1.0):
    """numpy matmul (1-D operands promoted and the added axis dropped)."""
    squeeze = []
    if a.ndim == 1:
        a = a.expand_dims(0)
        squeeze.append(-2)
    if w.ndim == 1:
        w = w.expand_dims(1)
        squeeze.append(-1)
    batch = broadcast_shape(a.shape[:-2], w.shape[:-2])
    out = DeviceTensor.empty(batch + (a.shape[-2], w.shape[-1]), np.float32)
    _lib.call("kk_gemm", out.desc(), a.desc(), w.desc(), _d(w_scale), _d(w_zp), float(alpha))
    if squeeze:
        out = out.squeeze([out.ndim + s for s in squeeze])
    return out


def conv1d(x, w, bias=None, pads=(0, 0), stride=1, dilation=1, group=1,
           w_scale=None, w_zp=None):
    x = x.contiguous()
    n, _, L = x.shape
    cout, _, k = w.shape
    lout = (L + pads[0] + pads[1] - dilation * (k - 1) - 1) // stride + 1
    out = DeviceTensor.empty((n, cout, max(lout, 0)), np.float32)
    _lib.call("kk_conv1d", out.desc(), x.desc(), w.contiguous().desc(), _d(w_scale), _d(w_zp),
              _d(bias), int(stride), int(dilation), int(pads[0]), int(pads[1]), int(group))
    return out


def conv_transpose1d(x, w, bias=None, pads=(0, 0), stride=1, dilation=1, group=1,
                     output_padding=0, w_scale=None, w_zp=None):
    x = x.contiguous()
    n, _, L = x.shape
    _, cout_g, k = w.shape
    lfull = (L - 1) * stride + dilation * (k - 1) + 1 + output_padding
    out = DeviceTensor.empty((n, cout_g * group, lfull - pads[0] - pads[1]), np.float32)
    _lib.call("kk_conv_transpose1d", out.desc(), x.desc(), w.contiguous().desc(), _d(w_scale),
              _d(w_zp), _d(bias), int(stride), int(dilation), int(pads[0]), int(pads[1]),
              int(group), int(output_padding))
    return out
