"""CPU oracle: a numpy restatement of the reference op layer's semantics.

TEST INFRASTRUCTURE ONLY.  This module is the checker for libkk's HIP
kernels and the CPU baseline timed by bench.py.  Only tests/, the smoke
check in __graft_entry__.py and bench.py's cpu_baseline leg may import it;
the product (best-tts-godot_amd/) never does.

It restates, in its own code, what ``RefRuntime.dispatch``
(tools/ref_runtime.py:428-668) computes for the ops on the hot path; each
function cites the reference lines it follows.  fp16 is storage only and
every float computation is float32 (tools/NOTES.md:44-59).

Pinning (how each function is checked independently of its own formula,
see tests/test_oracle.py):
  f32, binary, broadcast  -- reference KATs (tests/test_gpu_elementwise.gd
                             :31-40, :165-181) and a brute-force coordinate
                             walk; IEEE correct rounding makes them exact.
  unary                   -- float64 closed forms within an ulp bound; the
                             LeakyRelu KAT.
  snake                   -- float64 closed form x + sin^2(a x)/a.
  reduce, adain,          -- float64 closed forms, torch.nn.functional
  layernorm, softmax         instance_norm/layer_norm/softmax on the CPU,
                             invariants (zero mean, unit variance, rows
                             summing to 1), a large-offset case that fails a
                             one-pass variance.
  matmul, dequantize      -- float64 matmul; exact int8 dequant.
  conv1d, conv_transpose  -- direct loops on tiny shapes, torch conv1d /
                             conv_transpose1d, the adjoint identity
                             <conv(x), y> = <x, convT(y)>, delta kernels.
  fast_gelu               -- float64 closed form.
  bucket                  -- closed-form properties (multiple of 256, at most
                             4 significant bits, monotone, <= 12.5% slack).
  (tests/test_oracle_graphops.py:)
  dynamic_quantize_linear -- the ONNX specification's example; zero exact,
                             reconstruction within half a quantum, the
                             float32 division of x by the double scale.
  matmul_integer,         -- integer brute force (int64 loops), padding
  conv_integer               contributing zero after the zero-point shift.
  lstm                    -- torch.nn.LSTM (float64, bidirectional) on the
                             dequantised weights, gates reordered.
  stft                    -- numpy.fft.rfft of the windowed frames (float64).
  resize                  -- np.repeat (nearest x300), torch interpolate
                             (linear, half_pixel).
  pad                     -- torch.nn.functional.pad (reflect/replicate/
                             constant).
  scatter_nd, CumSum      -- loops; integer prefix sums in closed form.
  (tests/test_oracle_audio.py:)
  notch_taps              -- scipy.signal.firwin's Blackman band-pass designs
                             (an impulse minus one per tone), symmetry, the
                             frequency response (>= 40 dB nulls at 4800 and
                             9600 Hz, < 0.1 dB elsewhere); planted mistakes
                             (Hamming window, a missing tone, half the
                             bandwidth) fail the comparison.
  fir                     -- np.correlate of the edge-clamped signal, brute
                             force on tiny inputs, impulse response = taps,
                             DC gain = sum of the taps.
  pcm16                   -- known answers (clamp, rounding, byte order);
                             .5 ties round away from zero, which GLSL leaves
                             open: ties are parity unpinned.
"""
import numpy as np

F32 = np.float32


# --------------------------------------------------------------- dtypes
def f32(x):
    """fp16 -> fp32 widening at every use (ref_runtime.py:49-51)."""
    x = np.asarray(x)
    return x.astype(F32) if x.dtype == np.float16 else x


# ---------------------------------------------------------- elementwise
def binary(op, x, y):
    """Add/Sub/Mul/Div/Pow with numpy broadcasting (ref_runtime.py:446-457).
    Div of two integer arrays is floor division (:453-455)."""
    a, b = f32(x), f32(y)
    if op == "Add":
        return a + b
    if op == "Sub":
        return a - b
    if op == "Mul":
        return a * b
    if op == "Div":
        if np.issubdtype(a.dtype, np.integer) and np.issubdtype(b.dtype, np.integer):
            return a // b
        return a / b
    if op == "Pow":
        return np.power(a, b)
    raise NotImplementedError(op)


def unary(op, x, alpha=0.01):
    """ref_runtime.py:458-479: Sqrt/Exp/Sin/Cos/Atan/Tanh/Sigmoid/Floor/
    Round/LeakyRelu.  Sigmoid is 1/(1+exp(-x)); LeakyRelu uses a float32
    alpha (default 0.01)."""
    v = f32(x)
    if op == "Sqrt":
        return np.sqrt(v)
    if op == "Exp":
        return np.exp(v)
    if op == "Sin":
        return np.sin(v)
    if op == "Cos":
        return np.cos(v)
    if op == "Atan":
        return np.arctan(v)
    if op == "Tanh":
        return np.tanh(v)
    if op == "Sigmoid":
        return 1.0 / (1.0 + np.exp(-v))
    if op == "Floor":
        return np.floor(v)
    if op == "Round":
        return np.rint(v)
    if op == "LeakyRelu":
        a = F32(alpha)
        return np.where(v < 0, v * a, v)
    raise NotImplementedError(op)


def where(c, x, y):
    """ref_runtime.py:502-503."""
    return np.where(c, x, y)


def snake(x, alpha, recip=None):
    """The graph's snake chain (kpk #2853-2857): Mul(alpha, x) -> Sin ->
    Pow(., 2) -> Mul(recip, .) -> Add(x, .), each node as its dispatch
    branch computes it (ref_runtime.py:446-463).  With no folded `recip`
    constant, recip = 1/alpha in float32."""
    x = f32(x)
    alpha = f32(alpha)
    r = (F32(1.0) / alpha).astype(F32) if recip is None else f32(recip)
    t = binary("Mul", alpha, x)
    s = unary("Sin", t)
    p = binary("Pow", s, np.asarray(2.0, dtype=F32))
    q = binary("Mul", r, p)
    return binary("Add", x, q)


def fast_gelu(x, bias=None):
    """op_fast_gelu (ref_runtime.py:288-293)."""
    x = f32(x).astype(F32)
    if bias is not None:
        x = x + f32(bias).astype(F32)
    c = F32(0.7978845608028654)
    return 0.5 * x * (1.0 + np.tanh(c * (x + 0.044715 * x * x * x)))


def dequantize(q, scale, zp=None):
    """DequantizeLinear (ref_runtime.py:631-636): (q - zp) * scale in fp32."""
    v = np.asarray(q).astype(F32)
    if zp is not None:
        v = v - np.asarray(zp).astype(F32)
    return v * f32(scale).astype(F32)


# ------------------------------------------------------------ reductions
def reduce(op, x, axes=None, keepdims=True):
    """ReduceMean/ReduceSum (ref_runtime.py:589-598)."""
    v = f32(x)
    fn = np.mean if op == "ReduceMean" else np.sum
    ax = None if axes is None else tuple(int(a) for a in np.asarray(axes).reshape(-1))
    if ax == ():
        return v
    return fn(v, axis=ax, keepdims=keepdims)


def softmax(x, axis=-1):
    """op_softmax (ref_runtime.py:269-273)."""
    x = f32(x).astype(F32)
    m = x.max(axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def layernorm(x, scale, bias=None, axis=-1, eps=1e-5):
    """op_layernorm (ref_runtime.py:276-285): two-pass variance over the
    trailing axes from `axis`, a true division by sqrt(var + eps)."""
    x = f32(x).astype(F32)
    axes = tuple(range(axis if axis >= 0 else x.ndim + axis, x.ndim))
    mu = x.mean(axis=axes, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=axes, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    y = y * f32(scale).astype(F32)
    if bias is not None:
        y = y + f32(bias).astype(F32)
    return y


def skip_layernorm(x, skip, scale, bias=None, skip_bias=None, eps=1e-12):
    """SkipLayerNormalization (ref_runtime.py:604-609)."""
    s = f32(x) + f32(skip)
    if skip_bias is not None:
        s = s + f32(skip_bias)
    return layernorm(s, scale, bias, -1, eps)


def linear(style, w, b=None):
    """The AdaIN fc: style [1,S] @ W [S,2C] (+ b) in fp32 (MatMul branch,
    ref_runtime.py:614-615, then Add :446-447)."""
    h = f32(style).astype(F32) @ f32(w).astype(F32)
    if b is not None:
        h = h + f32(b).astype(F32)
    return h


def instance_norm_affine(x, gamma, beta, eps):
    """The AdaIN norm chain of the graph (kpk #2844-2852), node by node:
    ReduceMean(ax 2) -> Sub -> Mul(d, d) -> ReduceMean(ax 2) -> Add(eps)
    -> Sqrt -> Div -> Mul(1 + gamma) -> Add(beta); gamma/beta [1, C, 1]."""
    x = f32(x).astype(F32)
    mu = reduce("ReduceMean", x, [x.ndim - 1])
    d = binary("Sub", x, mu)
    var = reduce("ReduceMean", binary("Mul", d, d), [x.ndim - 1])
    den = unary("Sqrt", binary("Add", var, np.asarray(eps, dtype=F32)))
    q = binary("Div", d, den)
    g1 = binary("Add", gamma, np.asarray(1.0, dtype=F32))
    return binary("Add", binary("Mul", q, g1), beta)


def adain(x, style, w, b=None, eps=1e-5):
    """AdaIN: h = style . W + b, gamma = h[:, :C], beta = h[:, C:] (Split of
    kpk #80 -> #138, Unsqueeze to [1, C, 1]), then instance_norm_affine."""
    c = x.shape[-2]
    h = linear(np.asarray(style).reshape(1, -1), w, b)
    gamma = h[:, :c].reshape(1, c, 1)
    beta = h[:, c:].reshape(1, c, 1)
    return instance_norm_affine(x, gamma, beta, eps)


# ---------------------------------------------------------- contractions
def matmul(a, b):
    """MatMul (ref_runtime.py:614-615)."""
    return f32(a) @ f32(b)


def fused_matmul(a, b, trans_a=0, trans_b=0, alpha=1.0):
    """FusedMatMul (ref_runtime.py:616-622)."""
    a, b = f32(a), f32(b)
    if trans_a:
        a = np.swapaxes(a, -1, -2)
    if trans_b:
        b = np.swapaxes(b, -1, -2)
    return (a @ b) * F32(alpha)


def conv1d(x, w, b=None, pads=(0, 0), stride=1, dilation=1, group=1):
    """op_conv1d forward (ref_runtime.py:58-82, 101-103): zero pad, im2col
    per group, contraction over (cin, k), bias."""
    x = f32(x).astype(F32)
    w = f32(w).astype(F32)
    p0, p1 = int(pads[0]), int(pads[1])
    n, cin, _ = x.shape
    cout, cing, k = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (p0, p1)))
    lout = (xp.shape[2] - dilation * (k - 1) - 1) // stride + 1
    out = np.empty((n, cout, lout), dtype=F32)
    coutg = cout // group
    for g in range(group):
        xs = xp[:, g * cing:(g + 1) * cing, :]
        cols = np.empty((n, cing * k, lout), dtype=F32)
        for j in range(k):
            cols[:, j::k, :] = xs[:, :, j * dilation: j * dilation + lout * stride: stride]
        wg = w[g * coutg:(g + 1) * coutg].reshape(coutg, cing * k)
        out[:, g * coutg:(g + 1) * coutg, :] = np.einsum("oc,ncl->nol", wg, cols)
    if b is not None:
        out = out + f32(b).astype(F32).reshape(1, -1, 1)
    return out


def conv_transpose1d(x, w, b=None, pads=(0, 0), stride=1, dilation=1, group=1,
                     output_padding=0):
    """op_conv1d transposed (ref_runtime.py:83-99): per-tap contributions
    scattered with stride into the uncropped length
    (L-1)*s + d*(K-1) + 1 + output_padding, then cropped [p0 : end - p1]."""
    x = f32(x).astype(F32)
    w = f32(w).astype(F32)
    p0, p1 = int(pads[0]), int(pads[1])
    n, cin, lin = x.shape
    _, coutg, k = w.shape
    cout = coutg * group
    cing = cin // group
    lfull = (lin - 1) * stride + dilation * (k - 1) + 1 + output_padding
    acc = np.zeros((n, cout, lfull), dtype=F32)
    for g in range(group):
        xs = x[:, g * cing:(g + 1) * cing, :]
        wg = w[g * cing:(g + 1) * cing]
        contrib = np.einsum("nil,iok->nokl", xs, wg)
        for j in range(k):
            st = j * dilation
            acc[:, g * coutg:(g + 1) * coutg, st:st + (lin - 1) * stride + 1:stride] += \
                contrib[:, :, j, :]
    out = acc[:, :, p0:lfull - p1] if (p0 or p1) else acc
    if b is not None:
        out = out + f32(b).astype(F32).reshape(1, -1, 1)
    return out


# ------------------------------------------------- quantized integer path
def dynamic_quantize_linear(x):
    """DynamicQuantizeLinear (ref_runtime.py:106-116): uint8 asymmetric
    quantisation with the range widened to include 0; scale and zero point
    in float64, x / scale in float32 (a Python float is a weak scalar), the
    float64 zero point added after rounding."""
    x = f32(x).astype(F32)
    lo = min(0.0, float(x.min())) if x.size else 0.0
    hi = max(0.0, float(x.max())) if x.size else 0.0
    scale = (hi - lo) / 255.0
    if scale == 0:
        scale = 1.0
    zp = np.clip(np.rint(0.0 - lo / scale), 0.0, 255.0)
    y = np.clip(np.rint(x / scale) + zp, 0.0, 255.0).astype(np.uint8)
    return y, F32(scale), np.uint8(zp)


def matmul_integer(a, b, a_zp=None, b_zp=None):
    """MatMulInteger (ref_runtime.py:119-127): exact int32 (a - a_zp) @ (b - b_zp)
    with a per-tensor a_zp and a per-tensor or per-column b_zp."""
    ai = np.asarray(a).astype(np.int64)
    bi = np.asarray(b).astype(np.int64)
    if a_zp is not None:
        ai = ai - np.asarray(a_zp).astype(np.int64)
    if b_zp is not None:
        z = np.asarray(b_zp).astype(np.int64)
        bi = bi - (z if z.ndim == 0 else z.reshape(1, -1))
    return (ai @ bi).astype(np.int32)


def conv_integer(x, w, x_zp=None, w_zp=None, pads=(0, 0), stride=1, dilation=1, group=1):
    """ConvInteger (ref_runtime.py:130-134): the zero-point-shifted integers
    convolved in float32 by op_conv1d, then rounded to int32 (exact while
    partial sums stay below 2**24)."""
    xi = np.asarray(x).astype(np.int32) - (0 if x_zp is None else np.int32(x_zp))
    wi = np.asarray(w).astype(np.int32) - (0 if w_zp is None else np.int32(w_zp))
    out = conv1d(xi.astype(F32), wi.astype(F32), None, pads, stride, dilation, group)
    return out.round().astype(np.int32)


# ------------------------------------------------------------------- LSTM
def lstm(x, w, r, b, init_h, init_c, w_scale, w_zp, r_scale, r_zp, hidden_size,
         bidirectional):
    """DynamicQuantizeLSTM as the shipped runtime computes it (op_lstm with
    quantize_activations=False, ref_runtime.py:137-210): int8 W [dir, in, 4H]
    and R [dir, H, 4H] dequantised to fp32, the input projection x @ W for all
    steps, then per step g = xw[t] + h @ R with ONNX gate order i, o, f, c;
    the reverse direction walks time backwards."""
    x = f32(x).astype(F32)
    seq, batch, _ = x.shape
    ndir = 2 if bidirectional else 1
    hs = int(hidden_size)

    def deq(q, scale, zp):
        q = np.asarray(q).astype(F32)
        if zp is not None:
            q = q - np.asarray(zp).astype(F32)
        return q * np.asarray(scale, dtype=F32)

    ys = np.zeros((seq, ndir, batch, hs), F32)
    y_h = np.zeros((ndir, batch, hs), F32)
    y_c = np.zeros((ndir, batch, hs), F32)
    ws = np.asarray(w_scale).reshape(-1)
    rs = np.asarray(r_scale).reshape(-1)
    for d in range(ndir):
        wz = None if w_zp is None else np.asarray(w_zp).reshape(-1)[d]
        rz = None if r_zp is None else np.asarray(r_zp).reshape(-1)[d]
        wd = deq(w[d], ws[d] if ws.size == ndir else ws, wz)
        rd = deq(r[d], rs[d] if rs.size == ndir else rs, rz)
        bd = np.zeros(8 * hs, F32) if b is None else f32(b)[d].astype(F32)
        h = np.zeros((batch, hs), F32) if init_h is None else f32(init_h)[d].astype(F32).copy()
        c = np.zeros((batch, hs), F32) if init_c is None else f32(init_c)[d].astype(F32).copy()
        xw = (x.reshape(seq * batch, -1) @ wd).reshape(seq, batch, 4 * hs) + (bd[:4 * hs] + bd[4 * hs:])
        for t in (range(seq) if d == 0 else range(seq - 1, -1, -1)):
            g = xw[t] + h @ rd
            i = 1.0 / (1.0 + np.exp(-g[:, 0:hs]))
            o = 1.0 / (1.0 + np.exp(-g[:, hs:2 * hs]))
            fg = 1.0 / (1.0 + np.exp(-g[:, 2 * hs:3 * hs]))
            cc = np.tanh(g[:, 3 * hs:4 * hs])
            c = fg * c + i * cc
            h = o * np.tanh(c)
            ys[t, d] = h
        y_h[d], y_c[d] = h, c
    return ys, y_h, y_c


# --------------------------------------------------- vocoder tail / misc
def stft(signal, frame_step, window, frame_length, onesided=1):
    """op_stft (ref_runtime.py:213-233): direct DFT of windowed frames with a
    float64 cos/sin basis; the products are float64 and stored as float32."""
    sig = f32(signal).astype(F32)
    if sig.ndim == 3 and sig.shape[-1] == 1:
        sig = sig[:, :, 0]
    win = f32(window).astype(F32)
    n, step = int(frame_length), int(frame_step)
    batch, slen = sig.shape
    nframes = (slen - n) // step + 1
    nfreq = n // 2 + 1 if onesided else n
    ang = -2.0 * np.pi * np.arange(nfreq)[:, None] * np.arange(n)[None, :] / n
    cos_b, sin_b = np.cos(ang), np.sin(ang)
    out = np.empty((batch, nframes, nfreq, 2), F32)
    idx = np.arange(nframes)[:, None] * step + np.arange(n)[None, :]
    for bi in range(batch):
        frames = sig[bi][idx] * win
        out[bi, :, :, 0] = frames @ cos_b.T
        out[bi, :, :, 1] = frames @ sin_b.T
    return out


def resize(x, scales, mode, ctm, nearest_mode):
    """op_resize (ref_runtime.py:236-256): 1-D resize of the last axis,
    nearest (asymmetric, floor) or linear (half_pixel) with float64 source
    positions and a float32 blend."""
    x = f32(x).astype(F32)
    scale = float(np.asarray(scales).reshape(-1)[-1])
    lin = x.shape[-1]
    lout = int(np.floor(lin * scale))
    if mode == "nearest":
        if ctm != "asymmetric" or nearest_mode != "floor":
            raise NotImplementedError(f"resize nearest {ctm}/{nearest_mode}")
        src = np.floor(np.arange(lout) / scale).astype(np.int64)
        return x[..., np.clip(src, 0, lin - 1)]
    if mode == "linear":
        if ctm != "half_pixel":
            raise NotImplementedError(f"resize linear {ctm}")
        pos = np.clip((np.arange(lout) + 0.5) / scale - 0.5, 0, lin - 1)
        i0 = np.floor(pos).astype(np.int64)
        i1 = np.clip(i0 + 1, 0, lin - 1)
        frac = (pos - i0).astype(F32)
        return x[..., i0] * (1.0 - frac) + x[..., i1] * frac
    raise NotImplementedError(f"resize mode {mode}")


def pad(x, pads, mode="constant", value=0.0):
    """op_pad (ref_runtime.py:259-266): numpy pad, ONNX pads layout
    [begin_0 .. begin_r-1, end_0 .. end_r-1]."""
    r = x.ndim
    widths = [(int(pads[i]), int(pads[i + r])) for i in range(r)]
    if mode == "reflect":
        return np.pad(x, widths, mode="reflect")
    if mode == "edge":
        return np.pad(x, widths, mode="edge")
    return np.pad(x, widths, mode="constant", constant_values=value)


def scatter_nd(data, indices, updates):
    """op_scatternd (ref_runtime.py:296-304): later duplicates win."""
    out = np.array(data, copy=True)
    idx = np.asarray(indices).astype(np.int64)
    k = idx.shape[-1]
    flat = idx.reshape(-1, k)
    upd = np.asarray(updates).reshape((flat.shape[0],) + out.shape[k:])
    for i in range(flat.shape[0]):
        out[tuple(flat[i])] = upd[i]
    return out


# ------------------------------------------------- audio output stage
def notch_taps(sample_rate=24000, tones=(4800.0, 9600.0), bw=80.0, n=1023):
    """KokoroAudio.notch_taps (runtime/audio.gd:30-45): an impulse at the
    centre tap c = (n - 1) // 2 minus one Blackman-windowed sinc band-pass
    [f0 - bw, f0 + bw] per tone.  GDScript computes in double and stores in a
    PackedFloat32Array, so each tone's subtraction is rounded to float32."""
    k = np.arange(n, dtype=np.float64)
    c = (n - 1) // 2
    m = k - c
    taps = np.zeros(n, F32)
    taps[c] = 1.0
    two_pi = 2.0 * np.pi

    def sinc(x):
        out = np.ones_like(x)
        big = np.abs(x) >= 1e-9
        out[big] = np.sin(np.pi * x[big]) / (np.pi * x[big])
        return out

    w = 0.42 - 0.5 * np.cos(two_pi * k / (n - 1)) + 0.08 * np.cos(2.0 * two_pi * k / (n - 1))
    for f0 in tones:
        f1 = (f0 - bw) / sample_rate
        f2 = (f0 + bw) / sample_rate
        band = (2.0 * f2 * sinc(2.0 * f2 * m) - 2.0 * f1 * sinc(2.0 * f1 * m)) * w
        taps = (taps.astype(np.float64) - band).astype(F32)
    return taps


def fir(x, h, center=None):
    """The notch FIR of kernels/fir.glsl:35-47 over one waveform:
    y[i] = sum_k h[k] * x[clamp(i - center + k, 0, n - 1)], the taps summed
    in order in float32 (edges clamp to the first and last sample; center
    defaults to (taps - 1) / 2, as audio.gd:72-76 passes it)."""
    x = np.asarray(x, F32).reshape(-1)
    h = np.asarray(h, F32).reshape(-1)
    n, t = x.size, h.size
    c = (t - 1) // 2 if center is None else int(center)
    if n == 0:
        return x.copy()
    xp = x[np.clip(np.arange(-c, n - c + t - 1), 0, n - 1)]
    acc = np.zeros(n, F32)
    for k in range(t):
        acc = acc + h[k] * xp[k:k + n]
    return acc


def pcm16(x, gain=1.0):
    """16-bit PCM of a waveform (kernels/pcm16.glsl:28-46 as audio.gd:59-106
    drives it): round(clamp(x * gain, -1, 1) * 32767) as int16, the
    little-endian pairs of the GLSL being the int16 stream itself.  GLSL's
    round() leaves the direction of a .5 tie to the implementation; here a
    tie rounds away from zero (so ties are parity unpinned)."""
    v = np.asarray(x, F32) * F32(gain)
    c = np.minimum(np.maximum(v, F32(-1.0)), F32(1.0))
    s = (c * F32(32767.0)).astype(np.float64)
    return (np.sign(s) * np.floor(np.abs(s) + 0.5)).astype(np.int16)


# ------------------------------------------------------------------ pool
def bucket(nbytes):
    """Pool bucket size: 256-byte floor, four significant bits above 4 KiB
    (executor.gd:206-216)."""
    size = max(256, (int(nbytes) + 255) & ~255)
    if size <= 4096:
        return size
    shift, v = 0, size
    while v > 15:
        v >>= 1
        shift += 1
    gran = 1 << shift
    return (size + gran - 1) & ~(gran - 1)


# ----------------------------------------------------------- dispatch
def dispatch(op, node_input, node_output, at, env):
    """The reference dispatch for the hot-path ops, same signature and
    conventions (ref_runtime.py:428-668) over numpy values in `env`."""

    def inp(i, default=None):
        if i >= len(node_input) or not node_input[i]:
            return default
        return env[node_input[i]]

    x, y = inp(0), inp(1)
    if op in ("Add", "Sub", "Mul", "Div", "Pow"):
        out = binary(op, x, y)
    elif op == "LeakyRelu":
        out = unary(op, x, at.get("alpha", 0.01))
    elif op in ("Sqrt", "Exp", "Sin", "Cos", "Atan", "Tanh", "Sigmoid", "Floor", "Round"):
        out = unary(op, x)
    elif op == "Clip":
        out = f32(x)
        if inp(1) is not None:
            out = np.maximum(out, f32(inp(1)))
        if inp(2) is not None:
            out = np.minimum(out, f32(inp(2)))
    elif op == "Equal":
        out = np.equal(x, y)
    elif op == "Greater":
        out = np.greater(f32(x), f32(y))
    elif op == "Less":
        out = np.less(f32(x), f32(y))
    elif op == "GreaterOrEqual":
        out = np.greater_equal(f32(x), f32(y))
    elif op == "And":
        out = np.logical_and(x, y)
    elif op == "Where":
        out = where(x, y, inp(2))
    elif op == "Reshape":
        shape = [int(v) for v in np.asarray(y).reshape(-1)]
        if not at.get("allowzero", 0):
            shape = [x.shape[i] if v == 0 else v for i, v in enumerate(shape)]
        out = x.reshape(shape)
    elif op == "Transpose":
        out = np.transpose(x, at.get("perm"))
    elif op == "Unsqueeze":
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        for a in sorted(int(v) for v in np.asarray(axes).reshape(-1)):
            x = np.expand_dims(x, a)
        out = x
    elif op == "Squeeze":
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        out = np.squeeze(x) if axes is None else \
            np.squeeze(x, tuple(int(v) for v in np.asarray(axes).reshape(-1)))
    elif op == "Concat":
        vals = [env[i] for i in node_input if i]
        if any(v.dtype == np.float16 for v in vals):
            vals = [f32(v) for v in vals]
        out = np.concatenate(vals, axis=at["axis"])
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
        out = slice_op(x, inp(1), inp(2), inp(3), inp(4))
    elif op == "Gather":
        out = np.take(x, np.asarray(y).astype(np.int64), axis=at.get("axis", 0))
    elif op == "Expand":
        out = np.broadcast_to(x, np.broadcast_shapes(x.shape, tuple(int(v) for v in y))).copy()
    elif op == "ConstantOfShape":
        v = np.asarray(at.get("value", np.array([0], dtype=F32)))
        dt = F32 if v.dtype == np.float16 else v.dtype
        out = np.full([int(s) for s in x], v.reshape(-1)[0], dtype=dt)
    elif op == "Cast":
        to = {1: F32, 2: np.uint8, 3: np.int8, 6: np.int32, 7: np.int64, 9: np.bool_,
              10: np.float16}[at["to"]]
        out = f32(x).astype(F32 if to == np.float16 else to)
    elif op in ("ReduceMean", "ReduceSum"):
        axes = inp(1) if len(node_input) > 1 else at.get("axes")
        keep = bool(at.get("keepdims", 1))
        if axes is None:
            out = f32(x) if at.get("noop_with_empty_axes", 0) else \
                reduce(op, x, None, keep)
        else:
            out = reduce(op, x, axes, keep)
    elif op == "Softmax":
        out = softmax(x, at.get("axis", -1))
    elif op == "LayerNormalization":
        out = layernorm(x, y, inp(2), at.get("axis", -1), at.get("epsilon", 1e-5))
    elif op == "SkipLayerNormalization":
        out = skip_layernorm(x, y, inp(2), inp(3), inp(4), at.get("epsilon", 1e-12))
    elif op == "FastGelu":
        out = fast_gelu(x, y)
    elif op == "MatMul":
        out = matmul(x, y)
    elif op == "FusedMatMul":
        out = fused_matmul(x, y, at.get("transA", 0), at.get("transB", 0), at.get("alpha", 1.0))
    elif op == "DequantizeLinear":
        out = dequantize(x, y, inp(2))
    elif op == "Conv":
        out = conv1d(x, y, inp(2), at.get("pads", [0, 0]), at.get("strides", [1])[0],
                     at.get("dilations", [1])[0], at.get("group", 1))
    elif op == "ConvTranspose":
        out = conv_transpose1d(x, y, inp(2), at.get("pads", [0, 0]), at.get("strides", [1])[0],
                               at.get("dilations", [1])[0], at.get("group", 1),
                               at.get("output_padding", [0])[0])
    elif op == "Snake":
        out = snake(x, y, inp(2))
    elif op == "AdaIN":
        out = adain(x, y, inp(2), inp(3), at.get("epsilon", 1e-5))
    # ---- the rest of the graph's branches (ref_runtime.py:446-664)
    elif op == "Erf":
        from scipy.special import erf
        out = erf(f32(x))
    elif op == "Shape":
        s = np.array(x.shape, dtype=np.int64)
        out = s[at.get("start", 0):at.get("end", len(s))]
    elif op == "Range":
        out = np.arange(x.item(), y.item(), inp(2).item(), dtype=x.dtype)
    elif op == "NonZero":
        out = np.array(np.nonzero(x), dtype=np.int64)
    elif op == "CumSum":
        out = np.cumsum(f32(x), axis=int(np.asarray(y).item()))
    elif op == "Pad":
        out = pad(f32(x), np.asarray(inp(1)).reshape(-1), at.get("mode", "constant"),
                  0.0 if inp(2) is None else float(inp(2)))
    elif op == "ScatterND":
        out = scatter_nd(f32(x), y, f32(inp(2)))
    elif op == "Resize":
        out = resize(x, inp(2) if inp(2) is not None else inp(3), at.get("mode", "nearest"),
                     at.get("coordinate_transformation_mode", "half_pixel"),
                     at.get("nearest_mode", "round_prefer_floor"))
    elif op == "STFT":
        out = stft(x, np.asarray(y).item(), inp(2), np.asarray(inp(3)).item(),
                   at.get("onesided", 1))
    elif op == "DynamicQuantizeLinear":
        for name, v in zip(node_output, dynamic_quantize_linear(x)):
            if name:
                env[name] = v
        return
    elif op == "MatMulInteger":
        out = matmul_integer(x, y, inp(2), inp(3))
    elif op == "ConvInteger":
        out = conv_integer(x, y, inp(2), inp(3), at.get("pads", [0, 0]),
                           at.get("strides", [1])[0], at.get("dilations", [1])[0],
                           at.get("group", 1))
    elif op == "DynamicQuantizeLSTM":
        res = lstm(x, y, inp(2), inp(3), inp(5), inp(6), inp(8), inp(9), inp(10), inp(11),
                   at["hidden_size"], at.get("direction") == "bidirectional")
        for name, v in zip(node_output, res):
            if name:
                env[name] = v
        return
    else:
        raise NotImplementedError(op)
    env[node_output[0]] = out


def slice_op(data, starts, ends, axes, steps):
    """op_slice (ref_runtime.py:307-325): ONNX clamping, then a numpy
    slice (whose own negative-index rule applies to the clamped ends)."""
    r = data.ndim
    starts = np.asarray(starts).reshape(-1)
    ends = np.asarray(ends).reshape(-1)
    axes = list(range(len(starts))) if axes is None else np.asarray(axes).reshape(-1)
    steps = [1] * len(starts) if steps is None else np.asarray(steps).reshape(-1)
    sl = [slice(None)] * r
    for s, e, a, st in zip(starts, ends, axes, steps):
        a = int(a) % r
        s, e, st = int(s), int(e), int(st)
        dim = data.shape[a]
        if st > 0:
            s = min(max(s if s >= 0 else s + dim, 0), dim)
            e = min(max(e if e >= 0 else e + dim, 0), dim)
        else:
            s = min(max(s if s >= 0 else s + dim, -1), dim - 1)
            e = min(max(e if e >= 0 else e + dim, -1), dim - 1)
        sl[a] = slice(s, e, st)
    return data[tuple(sl)]
