"""Device ops: allocate the output from the pool and call libkk.

Each function takes DeviceTensors (or None for optional operands) and
returns a new DeviceTensor.  Shapes are computed here with numpy's rules;
the kernels re-validate them before launching.
"""
import ctypes

import numpy as np

from . import _lib
from .tensor import NP_TO_CODE, DeviceTensor


def _d(t):
    return None if t is None else t.desc()


def broadcast_shape(*shapes):
    """numpy's broadcast rule (right-aligned; 1 stretches; else must match)."""
    if len(shapes) == 2 and tuple(shapes[0]) == tuple(shapes[1]):
        return tuple(shapes[0])
    rank = max(len(s) for s in shapes)
    out = [1] * rank
    for s in shapes:
        off = rank - len(s)
        for i, d in enumerate(s):
            d = int(d)
            o = out[off + i]
            if o == 1:
                out[off + i] = d
            elif d != 1 and d != o:
                raise ValueError(f"shapes {shapes} do not broadcast")
    return tuple(out)


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
def matmul(a, w, w_scale=None, w_zp=None, alpha=1.0, packed=None):
    """numpy matmul (1-D operands promoted and the added axis dropped); with
    `packed` (gemm_pack(w, w_zp) of this very 2-D w) the weights are not
    converted for the call."""
    squeeze = []
    if a.ndim == 1:
        a = a.expand_dims(0)
        squeeze.append(-2)
    if w.ndim == 1:
        w = w.expand_dims(1)
        squeeze.append(-1)
    batch = broadcast_shape(a.shape[:-2], w.shape[:-2])
    out = DeviceTensor.empty(batch + (a.shape[-2], w.shape[-1]), np.float32)
    if packed is not None:
        _lib.call("kk_gemm_packed", out.desc(), a.desc(), w.desc(), packed.desc(), _d(w_scale),
                  _d(w_zp), float(alpha))
    else:
        _lib.call("kk_gemm", out.desc(), a.desc(), w.desc(), _d(w_scale), _d(w_zp), float(alpha))
    if squeeze:
        out = out.squeeze([out.ndim + s for s in squeeze])
    return out


def conv1d(x, w, bias=None, pads=(0, 0), stride=1, dilation=1, group=1,
           w_scale=None, w_zp=None, packed=None):
    """Conv1d; with `packed` (conv_pack(w, w_zp) of this very w) the
    weights are not laid out for the call."""
    x = x.contiguous()
    w = w.contiguous()
    n, _, L = x.shape
    cout, _, k = w.shape
    lout = (L + pads[0] + pads[1] - dilation * (k - 1) - 1) // stride + 1
    out = DeviceTensor.empty((n, cout, max(lout, 0)), np.float32)
    if packed is not None:
        if group != 1:
            raise ValueError("conv1d: packed weights need group 1")
        _lib.call("kk_conv1d_packed", out.desc(), x.desc(), w.desc(), packed.desc(), _d(w_scale),
                  _d(w_zp), _d(bias), int(stride), int(dilation), int(pads[0]), int(pads[1]))
        return out
    _lib.call("kk_conv1d", out.desc(), x.desc(), w.desc(), _d(w_scale), _d(w_zp),
              _d(bias), int(stride), int(dilation), int(pads[0]), int(pads[1]), int(group))
    return out


def conv_transpose1d(x, w, bias=None, pads=(0, 0), stride=1, dilation=1, group=1,
                     output_padding=0, w_scale=None, w_zp=None, packed=None):
    """ConvTranspose1d; with `packed` (conv_pack(w, w_zp, True, stride) of
    this very w) the weights are not laid out for the call."""
    x = x.contiguous()
    w = w.contiguous()
    n, _, L = x.shape
    _, cout_g, k = w.shape
    lfull = (L - 1) * stride + dilation * (k - 1) + 1 + output_padding
    out = DeviceTensor.empty((n, cout_g * group, lfull - pads[0] - pads[1]), np.float32)
    if packed is not None:
        if group != 1 or dilation != 1:
            raise ValueError("conv_transpose1d: packed weights need group 1 and dilation 1")
        _lib.call("kk_conv_transpose1d_packed", out.desc(), x.desc(), w.desc(), packed.desc(),
                  _d(w_scale), _d(w_zp), _d(bias), int(stride), int(pads[0]), int(pads[1]),
                  int(output_padding))
        return out
    _lib.call("kk_conv_transpose1d", out.desc(), x.desc(), w.desc(), _d(w_scale),
              _d(w_zp), _d(bias), int(stride), int(dilation), int(pads[0]), int(pads[1]),
              int(group), int(output_padding))
    return out


def gemm_pack(w, w_zp=None):
    """The packed form of a constant [K, N] MatMul weight (fp16, or int8/uint8
    with its zero point of the same type) as the bf16 matrix cores' operands
    (uint8 bytes on the device), for matmul(packed=...)."""
    nbytes = ctypes.c_int64(0)
    _lib.call("kk_gemm_packed_bytes", int(w.shape[0]), int(w.shape[1]), int(NP_TO_CODE[w.dtype]),
              ctypes.byref(nbytes))
    packed = DeviceTensor.empty((nbytes.value,), np.uint8)
    _lib.call("kk_gemm_pack", packed.desc(), w.desc(), _d(w_zp))
    return packed


def conv_pack(w, w_zp=None, transposed=False, stride=1):
    """The packed form of a constant Conv (transposed=False, any stride) or
    ConvTranspose (transposed=True, this stride) weight: fp16, or int8/uint8
    with its int8/uint8 zero point, laid out once for the fp16 matrix cores
    (uint8 bytes on the device), for conv1d / conv_transpose1d(packed=...)."""
    w = w.contiguous()
    cin, cout = (w.shape[0], w.shape[1]) if transposed else (w.shape[1], w.shape[0])
    nbytes = ctypes.c_int64(0)
    _lib.call("kk_conv_packed_bytes", int(bool(transposed)), int(cin), int(cout), int(w.shape[2]),
              int(stride), ctypes.byref(nbytes))
    packed = DeviceTensor.empty((nbytes.value,), np.uint8)
    _lib.call("kk_conv_pack", packed.desc(), w.desc(), _d(w_zp), int(bool(transposed)), int(stride))
    return packed


# ------------------------------------------------- quantized integer path
def dynamic_quantize_linear(x):
    """(y uint8, scale fp32 scalar, zero point uint8 scalar), all on device."""
    x = x.contiguous()
    y = DeviceTensor.empty(x.shape, np.uint8)
    scale = DeviceTensor.empty((), np.float32)
    zp = DeviceTensor.empty((), np.uint8)
    _lib.call("kk_dynamic_quantize_linear", y.desc(), scale.desc(), zp.desc(), x.desc())
    return y, scale, zp


def matmul_integer_pack(b):
    """The packed form of a constant [K, N] int8/uint8 MatMulInteger B for
    the int8 matrix cores (uint8 bytes on the device), for
    matmul_integer(packed=...) and matmul_integer_scaled(packed=...)."""
    nbytes = ctypes.c_size_t(0)
    _lib.call("kk_matmul_integer_pack_bytes", b.desc(), ctypes.byref(nbytes))
    packed = DeviceTensor.empty((nbytes.value,), np.uint8)
    _lib.call("kk_matmul_integer_pack", packed.desc(), b.desc())
    return packed


def matmul_integer(a, b, a_zp=None, b_zp=None, packed=None):
    batch = broadcast_shape(a.shape[:-2], b.shape[:-2])
    out = DeviceTensor.empty(batch + (a.shape[-2], b.shape[-1]), np.int32)
    if packed is None:
        _lib.call("kk_matmul_integer", out.desc(), a.desc(), b.desc(), _d(a_zp), _d(b_zp))
    else:
        _lib.call("kk_matmul_integer_packed", out.desc(), a.desc(), b.desc(), packed.desc(),
                  _d(a_zp), _d(b_zp))
    return out


def matmul_integer_scaled(a, b, a_zp, b_zp, scale, bias=None, scale2=None, packed=None):
    """MatMulInteger -> Cast(float) -> Mul(scale) (-> Add(bias)) in one
    launch, the scale optionally the product scale * scale2 (rounded once,
    as a Mul node forms it); each holds 1 or N (the output's columns)
    values.  `packed`: b's matmul_integer_pack."""
    batch = broadcast_shape(a.shape[:-2], b.shape[:-2])
    out = DeviceTensor.empty(batch + (a.shape[-2], b.shape[-1]), np.float32)
    sc = scale.contiguous().desc()
    s2 = _d(None if scale2 is None else scale2.contiguous())
    bi = _d(None if bias is None else bias.contiguous())
    if packed is None:
        _lib.call("kk_matmul_integer_scaled", out.desc(), a.desc(), b.desc(), _d(a_zp), _d(b_zp),
                  sc, s2, bi)
    else:
        _lib.call("kk_matmul_integer_scaled_packed", out.desc(), a.desc(), b.desc(), packed.desc(),
                  _d(a_zp), _d(b_zp), sc, s2, bi)
    return out


def conv_integer(x, w, x_zp=None, w_zp=None, pads=(0, 0), stride=1, dilation=1, group=1):
    x = x.contiguous()
    w = w.contiguous()
    n, _, L = x.shape
    cout, _, k = w.shape
    lout = (L + pads[0] + pads[1] - dilation * (k - 1) - 1) // stride + 1
    out = DeviceTensor.empty((n, cout, max(lout, 0)), np.int32)
    _lib.call("kk_conv_integer", out.desc(), x.desc(), w.desc(), _d(x_zp), _d(w_zp),
              int(stride), int(dilation), int(pads[0]), int(pads[1]), int(group))
    return out


def conv_integer_scaled(x, w, x_zp, w_zp, bias, scale, pads=(0, 0), stride=1, dilation=1,
                        group=1, resid=None):
    """float(ConvInteger(x, w) + bias[co]) * scale, fp32 out (bias int32 [Cout] or None);
    with `resid` (fp32, the output's shape) that added too: the residual Add fused."""
    x = x.contiguous()
    w = w.contiguous()
    n, _, L = x.shape
    cout, _, k = w.shape
    lout = (L + pads[0] + pads[1] - dilation * (k - 1) - 1) // stride + 1
    out = DeviceTensor.empty((n, cout, max(lout, 0)), np.float32)
    b = _d(bias.contiguous() if bias is not None else None)
    tail = (int(stride), int(dilation), int(pads[0]), int(pads[1]), int(group))
    if resid is None:
        _lib.call("kk_conv_integer_scaled", out.desc(), x.desc(), w.desc(), _d(x_zp), _d(w_zp),
                  b, scale.contiguous().desc(), *tail)
    else:
        _lib.call("kk_conv_integer_scaled_add", out.desc(), x.desc(), w.desc(), _d(x_zp),
                  _d(w_zp), b, scale.contiguous().desc(), resid.contiguous().desc(), *tail)
    return out


def conv_integer_pack(w, w_zp=None):
    """The packed form of a ConvInteger weight (uint8/int8 [Cout, Cin, K])
    and its zero point, for conv_integer_scaled_qbias(packed=...): the
    per-call weight re-layout done once (uint8 bytes on the device)."""
    w = w.contiguous()
    nbytes = ctypes.c_int64(0)
    _lib.call("kk_conv_integer_packed_bytes", *[int(v) for v in w.shape], ctypes.byref(nbytes))
    packed = DeviceTensor.empty((nbytes.value,), np.uint8)
    _lib.call("kk_conv_integer_pack", packed.desc(), w.desc(), _d(w_zp))
    return packed


def conv_integer_scaled_qbias(x, w, x_zp, w_zp, bias, scale_a, scale_w, pads=(0, 0), stride=1,
                              dilation=1, group=1, noalloc=False, resid=None, packed=None,
                              leaves=False):
    """conv_integer_scaled with its int32 bias and scale formed in the same
    launch sequence: scale = scale_a * scale_w, bias_int32 =
    int32(floor(bias / scale)) (bias fp32 [Cout], the scales one value each).
    With `noalloc` the library allocates nothing for the call (its workspace
    is a fixed device array); the output is still allocated here.  With
    `resid` (fp32, the output's shape) that is added too: the residual Add
    fused (not with `noalloc`).  With `packed` (conv_integer_pack of this w
    and w_zp) the weights are not re-laid for the call; with `leaves` too
    (and an output of at least 8192 steps) the result is (out, leaf sums of
    out for instance_norm_quant(leaves=...))."""
    x = x.contiguous()
    w = w.contiguous()
    n, _, L = x.shape
    cout, _, k = w.shape
    lout = (L + pads[0] + pads[1] - dilation * (k - 1) - 1) // stride + 1
    out = DeviceTensor.empty((n, cout, max(lout, 0)), np.float32)
    args = [out.desc(), x.desc(), w.desc(), _d(x_zp), _d(w_zp), bias.contiguous().desc(),
            scale_a.contiguous().desc(), scale_w.contiguous().desc()]
    tail = (int(stride), int(dilation), int(pads[0]), int(pads[1]), int(group))
    if packed is not None:
        if noalloc:
            raise ValueError("conv_integer_scaled_qbias: packed with noalloc is not supported")
        args.insert(3, packed.desc())
        rd = None if resid is None else resid.contiguous().desc()
        if leaves:
            lv = DeviceTensor.empty((n * cout, (lout // 8192) * 64), np.float32)
            _lib.call("kk_conv_integer_scaled_qbias_packed_leaves", *args, rd, lv.desc(), *tail)
            return out, lv
        _lib.call("kk_conv_integer_scaled_qbias_packed", *args, rd, *tail)
    elif resid is not None:
        if noalloc:
            raise ValueError("conv_integer_scaled_qbias: resid with noalloc is not supported")
        _lib.call("kk_conv_integer_scaled_qbias_add", *args, resid.contiguous().desc(), *tail)
    else:
        entry = "kk_conv_integer_scaled_qbias_noalloc" if noalloc else "kk_conv_integer_scaled_qbias"
        _lib.call(entry, *args, *tail)
    return out


def instance_norm_scale_shift(x, scale=None, shift=None, eps=1e-5, leaky_alpha=None):
    """(x - mean_T) / sqrt(var_T + eps) * scale[c] + shift[c] over the last
    axis, then LeakyRelu(leaky_alpha) when given."""
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_instance_norm_scale_shift", out.desc(), x.desc(),
              _d(scale.contiguous() if scale is not None else None),
              _d(shift.contiguous() if shift is not None else None), float(eps),
              0 if leaky_alpha is None else 1, 0.0 if leaky_alpha is None else float(leaky_alpha))
    return out


def instance_norm_scale_shift_snake(x, scale, shift, alpha, recip, eps=1e-5):
    """instance_norm_scale_shift, then the snake y + recip[c]*sin(alpha[c]*y)^2,
    in one pass; alpha and recip hold C values."""
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_instance_norm_scale_shift_snake", out.desc(), x.desc(),
              _d(scale.contiguous() if scale is not None else None),
              _d(shift.contiguous() if shift is not None else None), alpha.contiguous().desc(),
              recip.contiguous().desc(), float(eps))
    return out


def instance_norm_quant(x, scale=None, shift=None, alpha=None, recip=None, eps=1e-5,
                        leaky_alpha=None, leaves=None):
    """The instance norm chain (affine, then LeakyRelu or snake) and the
    DynamicQuantizeLinear of its result: (y uint8, scale fp32 [], zero point
    uint8 []), the float result never stored.  `leaves`: x's leaf sums from
    the convolution that produced it (conv_integer_scaled_qbias(leaves=True))."""
    x = x.contiguous()
    y = DeviceTensor.empty(x.shape, np.uint8)
    ys = DeviceTensor.empty((), np.float32)
    yz = DeviceTensor.empty((), np.uint8)
    args = [y.desc(), ys.desc(), yz.desc(), x.desc(),
            _d(scale.contiguous() if scale is not None else None),
            _d(shift.contiguous() if shift is not None else None),
            _d(alpha.contiguous() if alpha is not None else None),
            _d(recip.contiguous() if recip is not None else None), float(eps),
            0 if leaky_alpha is None else 1, 0.0 if leaky_alpha is None else float(leaky_alpha)]
    if leaves is None:
        _lib.call("kk_instance_norm_quant", *args)
    else:
        _lib.call("kk_instance_norm_quant_leaves", *args, leaves.desc())
    return y, ys, yz


# ------------------------------------------------ recurrent / vocoder
def lstm(x, w, r, b, init_h, init_c, w_scale, w_zp, r_scale, r_zp, hidden_size, bidirectional):
    x = x.contiguous()
    seq, batch, _ = x.shape
    ndir = 2 if bidirectional else 1
    ys = DeviceTensor.empty((seq, ndir, batch, hidden_size), np.float32)
    yh = DeviceTensor.empty((ndir, batch, hidden_size), np.float32)
    yc = DeviceTensor.empty((ndir, batch, hidden_size), np.float32)
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    _lib.call("kk_lstm", ys.desc(), yh.desc(), yc.desc(), x.desc(), c(w).desc(), c(r).desc(),
              _d(c(b)), _d(c(init_h)), _d(c(init_c)), c(w_scale).desc(), _d(c(w_zp)),
              c(r_scale).desc(), _d(c(r_zp)), int(hidden_size), 1 if bidirectional else 0)
    return ys, yh, yc


def stft(signal, window, frame_step, frame_length, onesided=1):
    signal = signal.contiguous()
    batch = signal.shape[0]
    slen = signal.size // max(batch, 1)
    n, step = int(frame_length), int(frame_step)
    nframes = (slen - n) // step + 1 if slen >= n else 0
    nfreq = n // 2 + 1 if onesided else n
    out = DeviceTensor.empty((batch, nframes, nfreq, 2), np.float32)
    _lib.call("kk_stft", out.desc(), signal.desc(), window.contiguous().desc(), step, n,
              1 if onesided else 0)
    return out


def resize(x, scale, mode):
    """mode 'nearest' (asymmetric/floor) or 'linear' (half_pixel), last axis."""
    x = x.contiguous()
    lout = int(np.floor(x.shape[-1] * scale))
    out = DeviceTensor.empty(x.shape[:-1] + (lout,), np.float32)
    _lib.call("kk_resize", out.desc(), x.desc(), 0 if mode == "nearest" else 1, float(scale))
    return out


def pad(x, pads, mode="constant", value=0.0):
    r = x.ndim
    pads = np.ascontiguousarray(np.asarray(pads, dtype=np.int64).reshape(-1))
    shape = [x.shape[i] + int(pads[i]) + int(pads[i + r]) for i in range(r)]
    out = DeviceTensor.empty(shape, np.float32)
    m = {"constant": 0, "reflect": 1, "edge": 2}[mode]
    _lib.call("kk_pad", out.desc(), x.desc(), pads.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), m, float(value))
    return out


def cumsum(x, axis):
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, x.dtype)
    _lib.call("kk_cumsum", out.desc(), x.desc(), int(axis))
    return out


def scatter_nd(data, indices, updates):
    """indices: host int64 [..., k]; later duplicates win (the host keeps the
    last occurrence of each index, so the device writes never collide)."""
    out = data.astype(data.dtype)  # a fresh copy, as numpy's data.copy()
    idx = np.asarray(indices).astype(np.int64)
    k = idx.shape[-1]
    flat = idx.reshape(-1, k)
    inner = int(np.prod(out.shape[k:], dtype=np.int64)) if k < out.ndim else 1
    for a in range(k):
        dim = out.shape[a]
        if flat.size and (flat[:, a].min() < -dim or flat[:, a].max() >= dim):
            raise IndexError(f"ScatterND index out of bounds for axis {a} with size {dim}")
    flat = np.where(flat < 0, flat + np.array(out.shape[:k]), flat)
    strides = np.array([int(np.prod(out.shape[a + 1:], dtype=np.int64)) for a in range(k)],
                       dtype=np.int64)
    offsets = flat @ strides if flat.size else np.zeros(0, np.int64)
    upd = updates.contiguous()
    if upd.size != len(offsets) * inner:
        raise ValueError("ScatterND: updates do not match indices")
    # keep the last occurrence of each offset
    _, last = np.unique(offsets[::-1], return_index=True)
    keep = np.sort(len(offsets) - 1 - last)
    if len(keep) != len(offsets):
        upd = upd.reshape((len(offsets), inner))
        sel = DeviceTensor.empty((len(keep), inner), upd.dtype)
        for j, i in enumerate(keep):
            copy_into(sel.slice_axis(0, j, j + 1), upd.slice_axis(0, int(i), int(i) + 1))
        upd, offsets = sel, offsets[keep]
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    _lib.call("kk_scatter_nd", out.desc(), upd.desc(),
              offsets.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
              int(len(offsets)), int(inner))
    return out


# ------------------------------------------------------ audio output stage
def fir(x, taps, center=-1):
    """The notch FIR over the flattened waveform (kernels/fir.glsl:35-47);
    center < 0: (len(taps) - 1) / 2."""
    x = x.contiguous()
    out = DeviceTensor.empty(x.shape, np.float32)
    _lib.call("kk_fir", out.desc(), x.desc(), taps.contiguous().desc(), int(center))
    return out


def pcm16(x, gain=1.0):
    """16-bit PCM bytes of the waveform (kernels/pcm16.glsl:28-46): uint8
    [2 * numel], the little-endian int16 stream."""
    x = x.contiguous()
    out = DeviceTensor.empty((2 * x.size,), np.uint8)
    _lib.call("kk_pcm16", out.desc(), x.desc(), float(gain))
    return out


def fir_pcm16(x, taps, center=-1, gain=1.0):
    """fir then pcm16 in one pass."""
    x = x.contiguous()
    out = DeviceTensor.empty((2 * x.size,), np.uint8)
    _lib.call("kk_fir_pcm16", out.desc(), x.desc(), taps.contiguous().desc(), int(center),
              float(gain))
    return out
