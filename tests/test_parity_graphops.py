"""Parity of the rest of the graph's device ops with the oracle:
DynamicQuantizeLinear, MatMulInteger, ConvInteger, DynamicQuantizeLSTM, STFT,
Resize, Pad, CumSum, ScatterND, and the host-side Range/NonZero fed from the
device.

Bars: bit-exact for the integer/quantised outputs, indexing and sequential
sums; rel 1e-4 (+1e-5*max|ref|) for the LSTM and STFT, whose sums run in a
different order than numpy's."""
import numpy as np
import pytest

from conftest import assert_bitexact, assert_close, rng

pytestmark = pytest.mark.gpu


def node(kk, op, inputs, attrs=None, nout=1):
    env, names = {}, []
    for i, v in enumerate(inputs):
        if v is None:
            names.append("")
            continue
        if isinstance(v, tuple) and v[0] == "host":
            env[f"i{i}"] = v[1]
        else:
            env[f"i{i}"] = kk.to_device(np.asarray(v))
        names.append(f"i{i}")
    outs = [f"o{k}" for k in range(nout)]
    kk.dispatch(op, names, outs, attrs or {}, env)
    res = [kk.to_host(env[o]) for o in outs]
    return res[0] if nout == 1 else res


def onode(oracle, op, inputs, attrs=None, nout=1):
    env, names = {}, []
    for i, v in enumerate(inputs):
        if v is None:
            names.append("")
            continue
        env[f"i{i}"] = v[1] if isinstance(v, tuple) else np.asarray(v)
        names.append(f"i{i}")
    outs = [f"o{k}" for k in range(nout)]
    oracle.dispatch(op, names, outs, attrs or {}, env)
    res = [env[o] for o in outs]
    return res[0] if nout == 1 else res


@pytest.mark.parametrize("case", ["normal", "positive", "negative", "zeros", "big", "odd_small",
                                  "just_over", "one_block_max", "two_launch_min", "ragged"])
def test_dynamic_quantize_linear(gpu, oracle, case):
    """Inputs up to 16384 elements take the one-block kernel, larger ones
    the two launches (many blocks' (min, max), the last block folding them;
    then the bytes); both against the oracle, bit for bit, the two-launch
    cases one after another (each leaves its arrival count at zero for the
    next)."""
    r = rng(1)
    x = {"normal": r.normal(0, 1, (1, 130, 768)),
         "positive": r.uniform(0.5, 3, (4, 1000)),
         "negative": -r.uniform(0.5, 3, (4, 1000)),
         "zeros": np.zeros((3, 7)),
         "big": r.normal(0, 50, (1, 512, 2400)),
         "odd_small": r.normal(0.3, 2, (1, 3, 43689)),
         "just_over": r.normal(-0.2, 1, (2, 65537)),
         "one_block_max": r.normal(0, 1, (4, 4096)),
         "two_launch_min": r.normal(0, 1, (1, 16385)),
         "ragged": r.normal(1, 3, (7, 3001))}[case].astype(np.float32)
    y, s, z = node(gpu, "DynamicQuantizeLinear", [x], nout=3)
    yo, so, zo = onode(oracle, "DynamicQuantizeLinear", [x], nout=3)
    assert_bitexact(np.asarray(s, np.float32).reshape(()), np.asarray(so, np.float32), "scale")
    assert_bitexact(np.asarray(z, np.uint8).reshape(()), np.asarray(zo, np.uint8), "zero point")
    assert_bitexact(y, yo, f"quantised {case}")


def test_matmul_integer(gpu, oracle):
    r = rng(2)
    a = r.integers(0, 256, (1, 130, 768)).astype(np.uint8)
    b = r.integers(-127, 128, (768, 2048)).astype(np.int8)
    azp = np.uint8(117)
    bzp = r.integers(-4, 5, 2048).astype(np.int8)
    got = node(gpu, "MatMulInteger", [a, b, azp, bzp])
    assert_bitexact(got, onode(oracle, "MatMulInteger", [a, b, azp, bzp]), "MatMulInteger")
    got = node(gpu, "MatMulInteger", [a[0, :7, :33], b[:33, :50], None, None])
    assert_bitexact(got, oracle.matmul_integer(a[0, :7, :33], b[:33, :50]), "no zero points")
    # the duration projection's shape: K a multiple of 4, N = 50 is not
    ins = [a[:, :10, :512], np.ascontiguousarray(b[:512, :50]), azp, bzp[:50]]
    assert_bitexact(node(gpu, "MatMulInteger", ins), onode(oracle, "MatMulInteger", ins),
                    "MatMulInteger N=50")
    # the FFN's down projection: K = 2048
    a2 = r.integers(0, 256, (1, 130, 2048)).astype(np.uint8)
    b2 = r.integers(-127, 128, (2048, 768)).astype(np.int8)
    ins = [a2, b2, azp, bzp[:768]]
    assert_bitexact(node(gpu, "MatMulInteger", ins), onode(oracle, "MatMulInteger", ins),
                    "MatMulInteger K=2048")


def brute_matmul_integer(a, b, azp, bzp):
    """int64 sums, one output at a time, wrapped to int32 as numpy's int32
    matmul wraps (ref_runtime.py:119-127)."""
    a = np.asarray(a, np.int64) - (0 if azp is None else int(azp))
    b = np.asarray(b, np.int64) - (0 if bzp is None else np.asarray(bzp, np.int64).reshape(1, -1))
    out = np.einsum("mk,kn->mn", a, b)
    return ((out + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)


def test_matmul_integer_sums_beyond_fp32(gpu, oracle):
    """Partial sums far above 2^24, where fp32 accumulation would round: K =
    2048, all-255 activations (zero point 0), weights +-127 against the
    opposite extreme of an int8 per-column zero point, so every product is
    255 * 255 (|sum| = 1.33e8).  Bit-exact against int64 brute force and the
    oracle."""
    K, M, N = 2048, 70, 192
    a = np.full((1, M, K), 255, np.uint8)
    r = rng(21)
    sign = r.choice([-1, 1], N)
    b = np.tile((127 * sign).astype(np.int8), (K, 1))
    bzp = np.where(sign > 0, -128, 127).astype(np.int8)
    bzp[:8] = r.integers(-128, 128, 8)  # a few ordinary columns
    want = brute_matmul_integer(a[0], b, 0, bzp)[None]
    assert int(np.abs(want.astype(np.int64)).max()) > 2 ** 26
    assert_bitexact(want, onode(oracle, "MatMulInteger", [a, b, np.uint8(0), bzp]), "oracle")
    got = node(gpu, "MatMulInteger", [a, b, np.uint8(0), bzp])
    assert_bitexact(got, want, "MatMulInteger |sum| 1.3e8")
    # and a random case at the same size, with an extreme activation zero point
    a = r.integers(0, 256, (1, M, K)).astype(np.uint8)
    b = r.integers(-128, 128, (K, N)).astype(np.int8)
    for azp in (np.uint8(0), np.uint8(255)):
        want = brute_matmul_integer(a[0], b, azp, bzp)[None]
        assert_bitexact(node(gpu, "MatMulInteger", [a, b, azp, bzp]), want, f"random, a_zp {azp}")


@pytest.mark.parametrize("case", ["u8_u8", "i8_i8", "batch_broadcast", "gather_paths", "strided",
                                  "wraps_mod_2_32"])
def test_matmul_integer_variants(gpu, oracle, case):
    """Both byte types on both sides, numpy batch broadcasting, the byte-gather
    loaders (K not a multiple of 16, N not of 4, strided views) and results
    beyond int32, which wrap modulo 2^32 as numpy's int32 matmul does."""
    r = rng(22)
    if case == "u8_u8":
        a = r.integers(0, 256, (1, 77, 300)).astype(np.uint8)
        b = r.integers(0, 256, (300, 130)).astype(np.uint8)
        azp, bzp = np.uint8(200), np.uint8(3)
    elif case == "i8_i8":
        a = r.integers(-128, 128, (65, 512)).astype(np.int8)
        b = r.integers(-128, 128, (512, 68)).astype(np.int8)
        azp, bzp = np.int8(-100), r.integers(-128, 128, 68).astype(np.int8)
    elif case == "batch_broadcast":
        a = r.integers(0, 256, (2, 3, 40, 96)).astype(np.uint8)
        b = r.integers(-128, 128, (2, 1, 96, 72)).astype(np.int8)
        azp, bzp = np.uint8(9), r.integers(-5, 6, 72).astype(np.int8)
    elif case == "gather_paths":
        a = r.integers(0, 256, (1, 33, 37)).astype(np.uint8)
        b = r.integers(-128, 128, (37, 50)).astype(np.int8)
        azp, bzp = np.uint8(128), r.integers(-128, 128, 50).astype(np.int8)
    elif case == "strided":
        # device views: every other column of A (a_sj = 2), and B the
        # transpose of an [N, K] buffer (b_si = 1, b_sj = K)
        a_full = r.integers(0, 256, (64, 200)).astype(np.uint8)
        bt = r.integers(-128, 128, (96, 100)).astype(np.int8)
        a, b, azp = a_full[:, ::2], bt.T, np.uint8(1)
        want = brute_matmul_integer(a, b, azp, None)
        assert_bitexact(onode(oracle, "MatMulInteger", [a, b, azp, None]), want, "oracle")
        da = gpu.to_device(a_full).slice_axis(1, 0, 200, 2)
        db = gpu.to_device(bt).transpose((1, 0))
        got = gpu.to_host(gpu.ops.matmul_integer(da, db, gpu.to_device(np.asarray(azp)), None))
        assert_bitexact(got, want, "MatMulInteger on strided views")
        return
    else:
        a = np.full((1, 4, 40000), 255, np.uint8)
        b = np.full((40000, 8), 127, np.int8)
        azp, bzp = np.uint8(0), np.full(8, -128, np.int8)
    ins = [a, b, azp, bzp]
    want = onode(oracle, "MatMulInteger", ins)
    if a.ndim == 2 and b.ndim == 2:
        assert_bitexact(want, brute_matmul_integer(a, b, azp, bzp), "oracle vs brute force")
    got = node(gpu, "MatMulInteger", ins)
    assert_bitexact(got, want, f"MatMulInteger {case}")


PACKED_CASES = {
    # (M, K, N, a dtype, b dtype, zero points): the text encoder's ALBERT
    # shapes, the predictors' style Linear (M = 1), the duration projection
    # (N = 50), partial tiles, both byte types
    "albert_qkv": (130, 768, 768, np.uint8, np.int8, "col"),
    "ffn_up": (130, 768, 2048, np.uint8, np.int8, "col"),
    "ffn_down": (130, 2048, 768, np.uint8, np.int8, "col"),
    "gemv": (1, 128, 1024, np.uint8, np.int8, "tensor"),
    "n50": (10, 512, 50, np.uint8, np.int8, "col"),
    "tails": (33, 48, 33, np.uint8, np.uint8, "tensor"),
    "i8_i8": (65, 512, 68, np.int8, np.int8, "col"),
    "no_zp": (7, 32, 50, np.uint8, np.int8, None),
    "k_odd": (9, 37, 40, np.uint8, np.int8, "col"),  # K % 16: the unpacked kernel on b
}


@pytest.mark.parametrize("case", list(PACKED_CASES) + ["batch", "strided_a", "wraps_mod_2_32"])
def test_matmul_integer_packed(gpu, case):
    """kk_matmul_integer_pack'ed B: kk_matmul_integer_packed and
    kk_matmul_integer_scaled_packed give the unpacked kernels' bits (and
    int64 brute force's, wrapped to int32), one launch of the packed kernel
    where A and out are contiguous and K % 16 == 0, the unpacked kernel on b
    otherwise (a strided A, K = 37)."""
    r = rng(27)
    ops, D = gpu.ops, gpu.to_device
    if case in PACKED_CASES:
        m, k, n, adt, bdt, zps = PACKED_CASES[case]
        lo = -128 if adt == np.int8 else 0
        a = r.integers(lo, lo + 256, (1, m, k)).astype(adt)
        lo = -128 if bdt == np.int8 else 0
        b = r.integers(lo, lo + 256, (k, n)).astype(bdt)
        azp = None if zps is None else np.asarray(r.integers(0, 256) if adt == np.uint8
                                                  else r.integers(-128, 128), adt)
        bzp = (None if zps is None else
               np.asarray(r.integers(-4, 5, n if zps == "col" else ()), bdt) if bdt == np.int8
               else np.asarray(r.integers(120, 136, n if zps == "col" else ()), bdt))
        da = D(a)
    elif case == "batch":
        a = r.integers(0, 256, (2, 3, 40, 96)).astype(np.uint8)
        b = r.integers(-128, 128, (96, 72)).astype(np.int8)
        azp, bzp = np.uint8(9), r.integers(-5, 6, 72).astype(np.int8)
        da = D(a)
    elif case == "strided_a":
        a_full = r.integers(0, 256, (64, 256)).astype(np.uint8)
        a = a_full[:, ::2]
        b = r.integers(-128, 128, (128, 100)).astype(np.int8)
        azp, bzp = np.uint8(1), None
        da = D(a_full).slice_axis(1, 0, 256, 2)
    else:
        a = np.full((1, 4, 40000), 255, np.uint8)
        b = np.full((40000, 8), 127, np.int8)
        azp, bzp = np.uint8(0), np.full(8, -128, np.int8)
        da = D(a)
    db = D(np.ascontiguousarray(b))
    dazp = None if azp is None else D(np.asarray(azp))
    dbzp = None if bzp is None else D(np.asarray(bzp))
    packed = ops.matmul_integer_pack(db)
    want = gpu.to_host(ops.matmul_integer(da, db, dazp, dbzp))
    got = gpu.to_host(ops.matmul_integer(da, db, dazp, dbzp, packed=packed))
    assert_bitexact(got, want, f"packed MatMulInteger {case}")
    if a.ndim == 2 or a.shape[0] == 1 and a.ndim == 3:
        brute = brute_matmul_integer(a.reshape(a.shape[-2:]), b, azp, bzp)
        assert_bitexact(np.asarray(want).reshape(brute.shape), brute, f"unpacked vs brute {case}")
    n = b.shape[1]
    scale = D(r.uniform(1e-4, 1e-3, (n,)).astype(np.float32))
    scale2 = D(np.asarray([0.02], np.float32))
    bias = D(r.normal(0, 1, (n,)).astype(np.float32))
    want = gpu.to_host(ops.matmul_integer_scaled(da, db, dazp, dbzp, scale, bias, scale2))
    got = gpu.to_host(ops.matmul_integer_scaled(da, db, dazp, dbzp, scale, bias, scale2,
                                                packed=packed))
    assert_bitexact(got, want, f"packed scaled MatMulInteger {case}")


def test_matmul_integer_packed_refuses_mismatch(gpu):
    r = rng(28)
    ops, D = gpu.ops, gpu.to_device
    b1 = D(r.integers(-128, 128, (64, 32)).astype(np.int8))
    b2 = D(r.integers(-128, 128, (64, 32)).astype(np.int8))
    a = D(r.integers(0, 256, (1, 5, 64)).astype(np.uint8))
    packed = ops.matmul_integer_pack(b1)
    with pytest.raises(Exception, match="another B"):
        ops.matmul_integer(a, b2, None, None, packed=packed)


@pytest.mark.parametrize("cin,cout,k,L,pad,dil", [(512, 512, 3, 240, 1, 1), (1090, 1024, 3, 40, 1, 1),
                                                  (256, 256, 7, 300, 9, 3), (1, 1, 3, 50, 1, 1),
                                                  (22, 128, 1, 480, 0, 1)])
def test_conv_integer(gpu, oracle, cin, cout, k, L, pad, dil):
    r = rng(3)
    x = r.integers(0, 256, (1, cin, L)).astype(np.uint8)
    w = r.integers(0, 256, (cout, cin, k)).astype(np.uint8)
    xzp, wzp = np.uint8(121), np.uint8(63)
    at = {"pads": [pad, pad], "dilations": [dil], "strides": [1], "group": 1}
    got = node(gpu, "ConvInteger", [x, w, xzp, wzp], at)
    assert_bitexact(got, onode(oracle, "ConvInteger", [x, w, xzp, wzp], at),
                    f"ConvInteger {cin}->{cout} k{k}")


def brute_conv_integer(x, w, xzp, wzp, pad, dil):
    """int64 ConvInteger, group 1, stride 1: sum over (ci, k) of
    (x - xzp)[ci, l + k*dil - pad] * (w - wzp)[co, ci, k], padding 0 after
    the shift."""
    xi = np.asarray(x, np.int64)[0] - int(xzp)
    wi = np.asarray(w, np.int64) - int(wzp)
    cout, cin, k = wi.shape
    L = xi.shape[1]
    xp = np.zeros((cin, L + 2 * pad), np.int64)
    xp[:, pad:pad + L] = xi
    lout = L + 2 * pad - dil * (k - 1)
    out = np.zeros((cout, lout), np.int64)
    for t in range(k):
        out += wi[:, :, t] @ xp[:, t * dil:t * dil + lout]
    return out[None]


def test_conv_integer_exact_beyond_2_24(gpu, oracle):
    """Sums above 2^24: the device is exact int32 (int8 matrix cores), while
    the reference convolves the shifted integers in float32 and rounds
    (ref_runtime.py:130-134), which can miss by a few units there.  The
    device matches int64 brute force bit for bit; the oracle, which restates
    the reference, stays within float32 rounding of it."""
    r = rng(23)
    x = np.full((1, 512, 64), 255, np.uint8)
    x[0, :, ::7] = r.integers(0, 256, (512, 10))
    w = r.integers(0, 256, (96, 512, 3)).astype(np.uint8)
    xzp, wzp = np.uint8(0), np.uint8(255)
    at = {"pads": [1, 1], "dilations": [1], "strides": [1], "group": 1}
    exact = brute_conv_integer(x, w, xzp, wzp, 1, 1)
    assert np.abs(exact).max() > 2 ** 25
    got = node(gpu, "ConvInteger", [x, w, xzp, wzp], at)
    assert_bitexact(got, exact.astype(np.int32), "ConvInteger |sum| > 2^25")
    ref = onode(oracle, "ConvInteger", [x, w, xzp, wzp], at).astype(np.int64)
    assert np.abs(ref - exact).max() <= 2.0 ** -23 * 1536 * np.abs(exact).max()


@pytest.mark.parametrize("case", ["no_zero_points", "int8_weights", "stride2_batch2", "one_output",
                                  "zp_extremes", "stride6_k12"])
def test_conv_integer_variants(gpu, oracle, case):
    r = rng(13)
    n, cin, cout, k, L, pad, stride = 1, 96, 40, 5, 333, 2, 1
    wdt, xzp, wzp = np.uint8, np.uint8(77), np.uint8(140)
    if case == "no_zero_points":
        xzp = wzp = None
    elif case == "int8_weights":
        wdt, wzp = np.int8, np.int8(-5)
    elif case == "stride2_batch2":
        n, stride = 2, 2
    elif case == "one_output":
        L, pad = 5, 0
    elif case == "zp_extremes":
        xzp, wzp = np.uint8(255), np.uint8(0)
    elif case == "stride6_k12":  # the graph's noise conv: a 64-step time tile
        cin, cout, k, L, pad, stride = 22, 256, 12, 6000, 3, 6
    x = r.integers(0, 256, (n, cin, L)).astype(np.uint8)
    lo, hi = (-128, 128) if wdt == np.int8 else (0, 256)
    w = r.integers(lo, hi, (cout, cin, k)).astype(wdt)
    at = {"pads": [pad, pad], "dilations": [1], "strides": [stride], "group": 1}
    ins = [x, w, xzp, wzp]
    want = onode(oracle, "ConvInteger", ins, at)
    assert_bitexact(node(gpu, "ConvInteger", ins, at), want, f"ConvInteger {case}")


@pytest.mark.parametrize("seq,inp,init", [(40, 640, "zero"), (7, 512, "zero"), (1, 64, "zero"),
                                          (9, 128, "large")])
def test_lstm(gpu, oracle, seq, inp, init):
    """Bidirectional int8 LSTM; "large" starts from initial states of
    |h0| up to ~6 (the first step's scale comes from max|h0|)."""
    r = rng(4)
    H = 256
    x = r.normal(0, 1, (seq, 1, inp)).astype(np.float32)
    w = r.integers(-127, 128, (2, inp, 4 * H)).astype(np.int8)
    rr = r.integers(-127, 128, (2, H, 4 * H)).astype(np.int8)
    b = r.normal(0, 0.05, (2, 8 * H)).astype(np.float32)
    h0 = (np.zeros((2, 1, H)) if init == "zero" else r.normal(0, 2, (2, 1, H))).astype(np.float32)
    ws = r.uniform(0.002, 0.006, 2).astype(np.float32)
    rs = r.uniform(0.002, 0.006, 2).astype(np.float32)
    wz = np.array([0, 1], np.int8)
    rz = np.array([-1, 0], np.int8)
    c0 = (np.zeros((2, 1, H)) if init == "zero" else r.normal(0, 1, (2, 1, H))).astype(np.float32)
    ins = [x, w, rr, b, None, h0, c0, None, ws, wz, rs, rz]
    at = {"hidden_size": H, "direction": "bidirectional"}
    got = node(gpu, "DynamicQuantizeLSTM", ins, at, nout=3)
    want = onode(oracle, "DynamicQuantizeLSTM", ins, at, nout=3)
    for g, wv, name in zip(got, want, ("Y", "Y_h", "Y_c")):
        assert_close(g, wv, 1e-4, floor_rel=1e-5, what=f"LSTM {name} seq={seq}")


@pytest.mark.parametrize("batch,slen,n,step,onesided", [(1, 3005, 20, 5, 1), (2, 999, 16, 3, 0),
                                                         (1, 1400003, 20, 5, 1)])
def test_stft(gpu, oracle, batch, slen, n, step, onesided):
    """Frames of n samples every `step` (the graph's n_fft 20, hop 5), the
    one-sided and full spectra, two signals, and more frames than the grid
    has threads (1400003 samples: 280,000 frames)."""
    r = rng(5)
    sig = r.normal(0, 1, (batch, slen)).astype(np.float32)
    win = np.hanning(n).astype(np.float16)
    ins = [sig, ("host", np.array(step)), win, ("host", np.array(n))]
    got = node(gpu, "STFT", ins, {"onesided": onesided})
    assert_close(got, onode(oracle, "STFT", ins, {"onesided": onesided}), 1e-6, floor_rel=1e-7,
                 what=f"STFT batch={batch} n={n} step={step}")


@pytest.mark.parametrize("mode,ctm,nm,scale,L", [("nearest", "asymmetric", "floor", 300.0, 37),
                                                 ("linear", "half_pixel", "", 2.0, 101),
                                                 ("nearest", "asymmetric", "floor", 2.0, 64)])
def test_resize(gpu, oracle, mode, ctm, nm, scale, L):
    x = rng(6).normal(0, 1, (1, 3, L)).astype(np.float32)
    scales = np.array([1.0, 1.0, scale], np.float32)
    at = {"mode": mode, "coordinate_transformation_mode": ctm, "nearest_mode": nm}
    ins = [x, None, scales]
    got = node(gpu, "Resize", ins, at)
    want = onode(oracle, "Resize", ins, at)
    assert_bitexact(got, want.astype(np.float32), f"Resize {mode} x{scale}")


@pytest.mark.parametrize("mode", ["reflect", "edge", "constant"])
@pytest.mark.parametrize("shape,pads", [((1, 4, 30), [0, 0, 5, 0, 0, 3]),
                                        ((1, 5, 2000), [0, 2, 7, 0, 1, 9]),
                                        ((2, 3, 4097), [0, 0, 0, 0, 0, 1])])
def test_pad(gpu, oracle, mode, shape, pads):
    """Short rows (element-wise kernel) and rows of >= 1024 outputs (a block
    row per output row), padding the middle axis and the last."""
    x = rng(7).normal(0, 1, shape).astype(np.float32)
    pads = np.array(pads, np.int64)
    got = node(gpu, "Pad", [x, ("host", pads)], {"mode": mode})
    assert_bitexact(got, onode(oracle, "Pad", [x, ("host", pads)], {"mode": mode}),
                    f"Pad {mode} {shape}")


def test_cumsum_scatter_range_nonzero(gpu, oracle):
    r = rng(8)
    x = r.normal(0, 1, (1, 2, 5000)).astype(np.float32)
    got = node(gpu, "CumSum", [x, ("host", np.array(2, np.int32))])
    assert_bitexact(got, onode(oracle, "CumSum", [x, ("host", np.array(2, np.int32))]), "CumSum f32")
    # the harmonic source's phase sum: 9 strided lines of 7180; and a line
    # longer than the LDS stage (the thread-per-line kernel)
    for shape, axis in (((1, 7180, 9), 1), ((2, 20000), 1)):
        x = r.uniform(0, 0.1, shape).astype(np.float32)
        ax = ("host", np.array(axis, np.int32))
        assert_bitexact(node(gpu, "CumSum", [x, ax]), onode(oracle, "CumSum", [x, ax]),
                        f"CumSum f32 {shape}")
    d = r.integers(1, 40, (1, 6)).astype(np.int64)
    got = node(gpu, "CumSum", [d, ("host", np.array(1, np.int32))])
    assert_bitexact(got, np.cumsum(d, axis=1), "CumSum int64")
    data = r.normal(0, 1, (6, 10, 4)).astype(np.float32)
    idx = np.array([[1], [3], [1], [5]], np.int64)
    upd = r.normal(0, 1, (4, 10, 4)).astype(np.float32)
    got = node(gpu, "ScatterND", [data, ("host", idx), upd])
    assert_bitexact(got, onode(oracle, "ScatterND", [data, ("host", idx), upd]), "ScatterND")
    # Range / NonZero with device inputs: the host computes them after a download
    env = {"s": gpu.to_device(np.array(0, np.int64)), "e": gpu.to_device(np.array(11, np.int64)),
           "d": np.array(3, np.int64)}
    gpu.dispatch("Range", ["s", "e", "d"], ["o"], {}, env)
    assert np.array_equal(env["o"], np.arange(0, 11, 3))
    env["b"] = gpu.to_device(np.array([[True, False, True], [False, False, True]]))
    gpu.dispatch("NonZero", ["b"], ["nz"], {}, env)
    assert np.array_equal(env["nz"], np.array(np.nonzero([[1, 0, 1], [0, 0, 1]]), np.int64))
