"""Parity of the contractions -- weight-dequant MatMul, Conv1d and
ConvTranspose1d -- with the oracle, on the GPU through the C ABI.

Bar: |got - ref| <= 1e-4*|ref| + 1e-5*max|ref|.  Both sides accumulate in
fp32 but in different orders (numpy: OpenBLAS / einsum loops; libkk: MFMA
tiles), so the absolute floor scales with the size of the terms: for K in
the thousands an element whose exact value is near zero still carries
~sqrt(K)*eps*|partial sums| of rounding on either side.  Each test also
checks that the worst relative error over elements with |ref| >= 1% of
max|ref| stays below 1e-4."""
import numpy as np
import pytest

from conftest import assert_bitexact, assert_close, rng

pytestmark = pytest.mark.gpu
RTOL, FLOOR = 1e-4, 1e-5


def check(got, want, what):
    assert_close(got, want, RTOL, floor_rel=FLOOR, what=what)
    w = np.abs(np.asarray(want, np.float64))
    big = w >= 0.01 * w.max()
    rel = np.abs(np.asarray(got, np.float64) - want)[big] / w[big]
    assert rel.max() < 1e-4, f"{what}: worst relative error {rel.max():.2e} on large elements"


def int8_weight(r, shape):
    q = r.integers(-127, 128, shape).astype(np.int8)
    s = np.float32(r.uniform(1e-3, 1e-2))
    return q, s


# -------------------------------------------------- dequant GEMM workloads
@pytest.mark.parametrize("m,k,n", [(256, 768, 2048), (256, 2048, 768)])
def test_int8_matmul_config(gpu, oracle, m, k, n):
    """A ~ N(0,1); W ~ U{-127..127} int8, per-tensor scale ~ U(1e-3,1e-2),
    zero point 0: DequantizeLinear then MatMul."""
    r = rng(0)
    a = r.normal(0, 1, (m, k)).astype(np.float32)
    q, s = int8_weight(r, (k, n))
    zp = np.int8(0)
    got = gpu.ops.matmul(gpu.to_device(a), gpu.to_device(q), gpu.to_device(np.array(s)),
                         gpu.to_device(np.array(zp))).numpy()
    want = oracle.matmul(a, oracle.dequantize(q, s, zp))
    check(got, want, f"int8 matmul {m}x{k}x{n}")


def test_fp16_matmul_config(gpu, oracle):
    r = rng(0)
    a = r.normal(0, 1, (256, 768)).astype(np.float32)
    w = r.normal(0, 0.02, (768, 768)).astype(np.float16)
    env = {"a": gpu.to_device(a), "w": gpu.to_device(w)}
    gpu.dispatch("MatMul", ["a", "w"], ["y"], {}, env)
    check(env["y"].numpy(), oracle.matmul(a, w), "fp16 matmul")


def test_per_column_dequant_u8_and_i8(gpu, oracle):
    r = rng(1)
    a = r.normal(0, 1, (130, 128)).astype(np.float32)
    q = r.integers(-127, 128, (128, 1028)).astype(np.int8)
    sc = r.uniform(1e-3, 1e-2, 1028).astype(np.float32)
    zp = r.integers(-3, 4, 1028).astype(np.int8)
    got = gpu.ops.matmul(gpu.to_device(a), gpu.to_device(q), gpu.to_device(sc),
                         gpu.to_device(zp)).numpy()
    check(got, oracle.matmul(a, oracle.dequantize(q, sc, zp)), "int8 per-column")
    u = r.integers(0, 256, (128, 96)).astype(np.uint8)
    got = gpu.ops.matmul(gpu.to_device(a), gpu.to_device(u), gpu.to_device(np.float32(0.01)),
                         gpu.to_device(np.uint8(128))).numpy()
    check(got, oracle.matmul(a, oracle.dequantize(u, np.float32(0.01), np.uint8(128))), "uint8")


@pytest.mark.parametrize("m,k,n,wdt", [(1024, 256, 1024, "i8"),   # 32x64 tiles, eight waves
                                       (256, 768, 2048, "i8"),    # 32x64, eight waves
                                       (256, 512, 1024, "u8"),    # 32x32, four waves
                                       (256, 768, 768, "u8"),     # 32x32, eight waves
                                       (256, 768, 768, "f16"),    # the same, two weight planes
                                       (1024, 256, 1024, "f16"),  # 32x64, four waves, two planes
                                       (45, 200, 80, "i8"),       # ragged M, K (a partial
                                       (45, 200, 88, "f16"),      #   K-step) and N
                                       (5, 12, 16, "u8"),         # K under one K-step
                                       (1, 36, 48, "f16"),        # waves with no K-steps
                                       (300, 2052, 64, "i8"),     # runs of 8 and 9 K-steps
                                       (300, 2052, 64, "f16"),
                                       # weight rows not 16-byte aligned: fp32 matrix cores
                                       (1, 100, 36, "i8"), (33, 36, 100, "f16"),
                                       (70, 4, 8, "u8"), (300, 2052, 68, "i8")])
def test_dequant_matmul_bf16_split_accuracy(gpu, oracle, m, k, n, wdt):
    """The 8-bit- and fp16-weight MatMul on the bf16 matrix cores
    (activations split into three bf16 parts, fp16 weights into two, every
    product exact): the oracle's bar, and no less accurate than numpy's own
    fp32 result against a float64 product (M, K and N off the tile sizes,
    M = 1, per-column and per-tensor zero points of both byte types; weights
    whose rows are not 16-byte aligned take the fp32 matrix cores)."""
    r = rng(12)
    a = r.normal(0, 1, (m, k)).astype(np.float32)
    if wdt == "f16":
        w = r.normal(0, 0.05, (k, n)).astype(np.float16)
        sc = zp = None
        wdeq = w.astype(np.float32)
    elif wdt == "i8":
        w = r.integers(-128, 128, (k, n)).astype(np.int8)
        sc = r.uniform(1e-3, 1e-2, n).astype(np.float32)
        zp = r.integers(-127, 128, n).astype(np.int8)  # |q - zp| up to 255
        wdeq = oracle.dequantize(w, sc, zp)
    else:
        w = r.integers(0, 256, (k, n)).astype(np.uint8)
        sc = np.float32(0.004)
        zp = np.uint8(255)
        wdeq = oracle.dequantize(w, sc, zp)
    dv = gpu.to_device
    got = gpu.ops.matmul(dv(a), dv(w), dv(np.asarray(sc)) if sc is not None else None,
                         dv(np.asarray(zp)) if zp is not None else None).numpy()
    want = oracle.matmul(a, wdeq)
    check(got, want, f"{wdt} {m}x{k}x{n}")
    exact = a.astype(np.float64) @ wdeq.astype(np.float64)
    terms = np.abs(a.astype(np.float64)) @ np.abs(wdeq.astype(np.float64))
    e_dev = (np.abs(got - exact) / np.maximum(terms, 1e-300)).max()
    e_np = (np.abs(want - exact) / np.maximum(terms, 1e-300)).max()
    assert e_dev <= 4 * e_np + 2 ** -22, (e_dev, e_np)


@pytest.mark.parametrize("mag", [1e-30, 1e-7, 1e20])
def test_dequant_matmul_activation_range(gpu, oracle, mag):
    """Activations of any magnitude keep fp32 accuracy (on the bf16 matrix
    cores the split needs no scaling); inf and NaN activations reach the
    same outputs as numpy's."""
    r = rng(13)
    a = (r.normal(0, 1, (40, 256)) * mag).astype(np.float32)
    for wdt in ("i8", "f16"):
        if wdt == "i8":
            w = r.integers(-127, 128, (256, 96)).astype(np.int8)
            sc, wdeq = np.float32(0.01), None
            wdeq = oracle.dequantize(w, sc, np.int8(0))
        else:
            w = r.normal(0, 0.05, (256, 96)).astype(np.float16)
            sc, wdeq = None, w.astype(np.float32)
        dv = gpu.to_device
        got = gpu.ops.matmul(dv(a), dv(w), dv(np.asarray(sc)) if sc is not None else None).numpy()
        check(got, oracle.matmul(a, wdeq), f"{wdt} activations ~{mag:g}")
    a2 = r.normal(0, 1, (40, 256)).astype(np.float32)
    a2[3, 17], a2[9, 200] = np.inf, np.nan
    w = r.integers(-127, 128, (256, 96)).astype(np.int8)
    w[17, :] = np.where(w[17, :] == 0, 1, w[17, :])  # inf meets no zero weight
    got = gpu.ops.matmul(gpu.to_device(a2), gpu.to_device(w),
                         gpu.to_device(np.float32(0.01))).numpy()
    want = oracle.matmul(a2, oracle.dequantize(w, np.float32(0.01), np.int8(0)))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.sign(got[np.isinf(want)]), np.sign(want[np.isinf(want)]))
    check(np.where(fin, got, 0), np.where(fin, want, 0), "finite rows beside inf/NaN")


def test_fp16_matmul_nonfinite_and_extreme_weights(gpu, oracle):
    """fp16 weights on the bf16 matrix cores: subnormal, largest and
    zero weights at fp32 accuracy; an infinite or NaN weight or activation
    gives numpy's inf / NaN pattern (those calls take the exact scalar
    tiles), and the next finite call is back on the matrix cores."""
    r = rng(14)
    m, k, n = 64, 320, 96
    a = r.normal(0, 1, (m, k)).astype(np.float32)
    w = r.normal(0, 0.05, (k, n)).astype(np.float16)
    w[:40, 3] = np.float16(6.0e-8)      # fp16 subnormals (2^-24 steps)
    w[40:80, 3] = np.float16(3.0e-6)
    w[5, 7] = np.float16(65504.0)       # the largest fp16
    w[:, 9] = 0
    w[::7, 11] = np.float16(1.0)        # 8 significant bits or fewer: second plane 0
    dv = gpu.to_device

    def run(a_, w_):
        return gpu.ops.matmul(dv(a_), dv(w_)).numpy()

    def same_nonfinite(got, want, what):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want), err_msg=what)
        np.testing.assert_array_equal(np.isinf(got), np.isinf(want), err_msg=what)
        inf = np.isinf(want)
        assert np.array_equal(np.sign(got[inf]), np.sign(want[inf])), what
        fin = np.isfinite(want)
        check(np.where(fin, got, 0), np.where(fin, want, 0), what)

    check(run(a, w), oracle.matmul(a, w.astype(np.float32)), "fp16 extremes")
    w2 = w.copy()
    w2[17, 20], w2[30, 21], w2[31, 21] = np.inf, -np.inf, np.inf   # column 21: inf - inf
    w2[50, 22] = np.nan
    a2 = a.copy()
    a2[4, 17] = 0.0                     # 0 * inf in row 4, column 20
    with np.errstate(invalid="ignore", over="ignore"):
        same_nonfinite(run(a2, w2), oracle.matmul(a2, w2.astype(np.float32)), "inf/NaN weights")
    w[100, 30] = np.float16(0.5)        # second plane 0: inf * (b0 + 0) must stay inf
    a3 = a.copy()
    a3[6, 100], a3[8, 5] = np.inf, np.nan
    with np.errstate(invalid="ignore", over="ignore"):
        same_nonfinite(run(a3, w), oracle.matmul(a3, w.astype(np.float32)), "inf/NaN activations")
    check(run(a, w), oracle.matmul(a, w.astype(np.float32)), "finite call after a stamped one")


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (33, 65, 97), (130, 512, 50),
                                   (64, 64, 64)])
def test_matmul_odd_shapes(gpu, oracle, m, k, n):
    r = rng(2)
    a = r.normal(0, 1, (m, k)).astype(np.float32)
    w = r.normal(0, 0.1, (k, n)).astype(np.float32)
    check(gpu.ops.matmul(gpu.to_device(a), gpu.to_device(w)).numpy(), oracle.matmul(a, w),
          f"matmul {m}x{k}x{n}")


@pytest.mark.parametrize("wdt", ["f16", "i8c", "u8c"])
def test_matmul_weights_batched(gpu, oracle, wdt):
    """fp16 / 8-bit weights (per-column scale and zero point) shared by a
    batch of fp32 rows; FusedMatMul's alpha; a large activation.  [2,300,512]
    x [512,640] leaves CUs idle at one K range per tile, so K is split and
    the partials summed in split order."""
    r = rng(11)
    a = r.normal(0, 1, (2, 300, 512)).astype(np.float32)
    n = 640
    if wdt == "f16":
        w = r.normal(0, 0.05, (512, n)).astype(np.float16)
        sc = zp = None
        wdeq = w.astype(np.float32)
    else:
        dt = np.int8 if wdt == "i8c" else np.uint8
        lo, hi = (-127, 128) if wdt == "i8c" else (0, 256)
        w = r.integers(lo, hi, (512, n)).astype(dt)
        sc = r.uniform(1e-3, 1e-2, n).astype(np.float32)
        zp = r.integers(-3, 4, n).astype(dt) if wdt == "i8c" else r.integers(120, 136, n).astype(dt)
        wdeq = oracle.dequantize(w, sc, zp)
    dv = gpu.to_device
    got = gpu.ops.matmul(dv(a), dv(w), dv(sc) if sc is not None else None,
                         dv(zp) if zp is not None else None).numpy()
    check(got, oracle.matmul(a, wdeq), f"matmul {wdt} batched")
    if wdt == "f16":
        env = {"a": dv(a), "w": dv(w)}
        gpu.dispatch("FusedMatMul", ["a", "w"], ["y"], {"alpha": 0.125}, env)
        check(env["y"].numpy(), oracle.fused_matmul(a, wdeq, 0, 0, 0.125), "FusedMatMul alpha")
        a2 = a.copy()
        a2[1, 7, 100] = 7.0e4
        got = gpu.ops.matmul(dv(a2), dv(w)).numpy()
        check(got, oracle.matmul(a2, wdeq), "matmul with a 7e4 activation")


@pytest.mark.parametrize("shape_a,shape_w", [((1, 50000, 9), (9, 1)), ((3, 2000, 7), (7, 3)),
                                             ((4100, 32), (32, 4))])
def test_matmul_skinny(gpu, oracle, shape_a, shape_w):
    """Tall, skinny products (N <= 4, K <= 32: a thread per row), as the
    harmonic source's Linear(9 -> 1) over every sample."""
    r = rng(4)
    a = r.normal(0, 1, shape_a).astype(np.float32)
    w = r.normal(0, 0.3, shape_w).astype(np.float32)
    check(gpu.ops.matmul(gpu.to_device(a), gpu.to_device(w)).numpy(), oracle.matmul(a, w),
          f"matmul {shape_a} x {shape_w}")


def test_attention_batched_and_fused(gpu, oracle):
    """[1,12,T,64] x [1,12,64,T] with the right operand a transposed view,
    FusedMatMul with transB and alpha, and vector operands."""
    r = rng(3)
    t = 130
    q = r.normal(0, 1, (1, 12, t, 64)).astype(np.float32)
    kx = r.normal(0, 1, (1, 12, t, 64)).astype(np.float32)
    env = {"q": gpu.to_device(q), "k": gpu.to_device(kx)}
    gpu.dispatch("Transpose", ["k"], ["kt"], {"perm": [0, 1, 3, 2]}, env)
    gpu.dispatch("MatMul", ["q", "kt"], ["s"], {}, env)
    check(env["s"].numpy(), oracle.matmul(q, np.transpose(kx, (0, 1, 3, 2))), "QK^T")
    gpu.dispatch("FusedMatMul", ["q", "k"], ["f"], {"transB": 1, "alpha": 0.125}, env)
    check(env["f"].numpy(), oracle.fused_matmul(q, kx, 0, 1, 0.125), "FusedMatMul")
    gpu.dispatch("FusedMatMul", ["k", "q"], ["g"], {"transA": 1}, env)
    check(env["g"].numpy(), oracle.fused_matmul(kx, q, 1, 0, 1.0), "FusedMatMul transA")
    v = r.normal(0, 1, 64).astype(np.float32)
    env["v"] = gpu.to_device(v)
    gpu.dispatch("MatMul", ["q", "v"], ["qv"], {}, env)
    check(env["qv"].numpy(), oracle.matmul(q, v), "matrix @ vector")
    w = r.normal(0, 1, (64, 40)).astype(np.float32)
    env["w"] = gpu.to_device(w)
    gpu.dispatch("MatMul", ["q", "w"], ["qw"], {}, env)
    check(env["qw"].numpy(), oracle.matmul(q, w), "batched @ broadcast weight")


# --------------------------------------------------------------- conv1d
def test_int8_conv1d_config(gpu, oracle):
    """x ~ N(0,1) [1,512,2400]; W int8 [512,512,3], per-tensor scale; pad 1."""
    r = rng(0)
    x = r.normal(0, 1, (1, 512, 2400)).astype(np.float32)
    q, s = int8_weight(r, (512, 512, 3))
    got = gpu.ops.conv1d(gpu.to_device(x), gpu.to_device(q), None, (1, 1),
                         w_scale=gpu.to_device(np.array(s))).numpy()
    want = oracle.conv1d(x, oracle.dequantize(q, s), None, (1, 1))
    check(got, want, "int8 conv1d 512->512 k3")


CONV = [  # (n, cin, cout, k, L, p0, p1, s, d, g, wdt)
    (1, 256, 256, 3, 2400, 1, 1, 1, 1, 1, "i8"),
    (1, 256, 256, 3, 2400, 3, 3, 1, 3, 1, "i8"),
    (1, 256, 256, 3, 2400, 5, 5, 1, 5, 1, "f32"),
    (2, 22, 256, 12, 600, 3, 3, 6, 1, 1, "f16"),
    (1, 128, 22, 7, 480, 3, 3, 1, 1, 1, "f16"),
    (1, 512, 512, 5, 130, 2, 2, 1, 1, 1, "u8"),
    (1, 64, 64, 3, 101, 1, 0, 2, 1, 64, "f16"),
    (1, 1090, 1090, 3, 50, 1, 1, 1, 1, 1090, "f32"),
    (1, 12, 6, 4, 33, 0, 2, 3, 2, 3, "f32"),
    (1, 1, 1, 3, 40, 1, 1, 2, 1, 1, "f32"),
]


@pytest.mark.parametrize("case", CONV)
def test_conv1d_cases(gpu, oracle, case):
    n, cin, cout, k, L, p0, p1, s, d, g, wdt = case
    r = rng(4)
    x = r.normal(0, 1, (n, cin, L)).astype(np.float32)
    b = r.normal(0, 0.1, cout).astype(np.float32)
    shape = (cout, cin // g, k)
    ws = wz = None
    if wdt == "i8":
        w, sc = int8_weight(r, shape)
        ws = np.array(sc)
        wdeq = oracle.dequantize(w, sc)
    elif wdt == "u8":
        w = r.integers(0, 256, shape).astype(np.uint8)
        ws, wz = np.array(np.float32(0.004)), np.array(np.uint8(114))
        wdeq = oracle.dequantize(w, ws, wz)
    else:
        w = (r.normal(0, 0.05, shape)).astype(np.float16 if wdt == "f16" else np.float32)
        wdeq = w
    got = gpu.ops.conv1d(gpu.to_device(x), gpu.to_device(w), gpu.to_device(b), (p0, p1), s, d, g,
                         w_scale=gpu.to_device(ws) if ws is not None else None,
                         w_zp=gpu.to_device(wz) if wz is not None else None).numpy()
    check(got, oracle.conv1d(x, wdeq, b, (p0, p1), s, d, g), f"conv1d {case}")


def test_conv_dispatch_f16(gpu, oracle):
    r = rng(5)
    x = r.normal(0, 1, (1, 128, 240)).astype(np.float32)
    w = r.normal(0, 0.05, (22, 128, 7)).astype(np.float16)
    b = r.normal(0, 0.1, 22).astype(np.float16)
    env = {"x": gpu.to_device(x), "w": gpu.to_device(w), "b": gpu.to_device(b)}
    at = {"pads": [3, 3], "strides": [1], "dilations": [1], "group": 1}
    gpu.dispatch("Conv", ["x", "w", "b"], ["y"], at, env)
    oenv = {"x": x, "w": w, "b": b}
    oracle.dispatch("Conv", ["x", "w", "b"], ["y"], at, oenv)
    check(env["y"].numpy(), oenv["y"], "Conv dispatch")


# ------------------------------------------------------ conv transpose
def test_int8_conv_transpose_config(gpu, oracle):
    """x ~ N(0,1) [1,512,240]; W int8 [512,256,20]; stride 10, pad 5."""
    r = rng(0)
    x = r.normal(0, 1, (1, 512, 240)).astype(np.float32)
    q, s = int8_weight(r, (512, 256, 20))
    got = gpu.ops.conv_transpose1d(gpu.to_device(x), gpu.to_device(q), None, (5, 5), 10,
                                   w_scale=gpu.to_device(np.array(s))).numpy()
    assert got.shape == (1, 256, 2400)
    want = oracle.conv_transpose1d(x, oracle.dequantize(q, s), None, (5, 5), 10)
    check(got, want, "int8 convT 512->256 k20 s10 p5")


CONVT = [  # (n, cin, cout_g, k, L, p0, p1, s, d, g, op, wdt)
    (1, 256, 128, 12, 300, 3, 3, 6, 1, 1, 0, "f16"),
    (1, 22, 1, 20, 101, 0, 0, 5, 1, 1, 0, "f32"),
    (1, 512, 1, 3, 40, 1, 1, 2, 1, 512, 1, "f16"),
    (2, 8, 3, 5, 17, 2, 1, 3, 1, 1, 2, "f32"),
    (1, 6, 4, 3, 9, 1, 1, 2, 2, 1, 0, "f32"),
    (1, 4, 4, 4, 10, 0, 0, 1, 1, 1, 0, "i8"),
    (1, 3, 2, 2, 8, 0, 0, 4, 1, 1, 3, "f32"),
]


@pytest.mark.parametrize("case", CONVT)
def test_conv_transpose_cases(gpu, oracle, case):
    n, cin, cout_g, k, L, p0, p1, s, d, g, op, wdt = case
    r = rng(6)
    x = r.normal(0, 1, (n, cin, L)).astype(np.float32)
    b = r.normal(0, 0.1, cout_g * g).astype(np.float32)
    shape = (cin, cout_g, k)
    ws = None
    if wdt == "i8":
        w, sc = int8_weight(r, shape)
        ws = np.array(sc)
        wdeq = oracle.dequantize(w, sc)
    else:
        w = r.normal(0, 0.1, shape).astype(np.float16 if wdt == "f16" else np.float32)
        wdeq = w
    got = gpu.ops.conv_transpose1d(gpu.to_device(x), gpu.to_device(w), gpu.to_device(b), (p0, p1),
                                   s, d, g, op,
                                   w_scale=gpu.to_device(ws) if ws is not None else None).numpy()
    check(got, oracle.conv_transpose1d(x, wdeq, b, (p0, p1), s, d, g, op), f"convT {case}")


# ---------------------------------------------------- decoder stage chain
# fp16 or 8-bit weights, channels in multiples of 32, enough work: the fp16
# matrix cores with each activation split into two fp16 halves (fp32
# accuracy); 8-bit weights less their zero point, the scale on the sums
F16MC = [  # (kind, n, cin, cout, k, L, p0, p1, s, d, op, wdt)
    ("convT", 1, 256, 128, 12, 2000, 3, 3, 6, 1, 0, "f16"),     # generator ups.1
    ("convT", 1, 512, 256, 20, 700, 5, 5, 10, 1, 0, "f16"),     # generator ups.0
    ("convT", 2, 256, 64, 7, 1500, 2, 1, 3, 1, 1, "f16"),       # two items, K not a multiple of s
    ("conv", 1, 128, 22, 7, 20000, 3, 3, 1, 1, 0, "f16"),       # conv_post
    ("conv", 1, 128, 40, 5, 30000, 4, 2, 2, 3, 0, "f16"),       # stride 2, dilation 3
    ("conv", 2, 64, 160, 3, 8000, 1, 1, 1, 1, 0, "f16"),        # two items, 160 channels
    ("convT", 1, 512, 256, 20, 240, 5, 5, 10, 1, 0, "i8"),      # the upsample config, int8
    ("convT", 1, 256, 128, 12, 1000, 3, 3, 6, 1, 0, "u8c"),     # uint8, per-channel scale + zp
    ("conv", 1, 256, 96, 3, 6000, 1, 1, 1, 2, 0, "i8"),         # int8 per tensor, dilation 2
    ("conv", 1, 128, 64, 5, 8000, 2, 2, 1, 1, 0, "u8c"),        # uint8, per-channel scale + zp
    # input channels a multiple of the 32-wide K step but not of 64
    ("conv", 1, 96, 64, 3, 12000, 1, 1, 1, 1, 0, "i8"),
    ("convT", 1, 160, 64, 12, 1200, 3, 3, 6, 1, 0, "f16"),
]


@pytest.mark.parametrize("case", F16MC)
def test_fp16_weight_conv_matrix_cores(gpu, oracle, case):
    kind, n, cin, cout, k, L, p0, p1, s, d, op, wdt = case
    r = rng(9)
    x = r.normal(0, 1, (n, cin, L)).astype(np.float32)
    x[0, 0, :50] *= 1e-6  # tiny activations (their low halves are fp16 subnormals)
    b = r.normal(0, 0.1, cout).astype(np.float32)
    shape = (cin, cout, k) if kind == "convT" else (cout, cin, k)
    bshape = (1, cout, 1) if kind == "convT" else (cout, 1, 1)  # per output channel
    sc = zp = None
    if wdt == "f16":
        w = r.normal(0, 0.05, shape).astype(np.float16)
        wdeq = w
    elif wdt == "i8":
        w, sc = int8_weight(r, shape)
        wdeq = oracle.dequantize(w, sc)
    else:
        w = r.integers(0, 256, shape).astype(np.uint8)
        sc = r.uniform(1e-4, 1e-3, cout).astype(np.float32)
        zp = r.integers(100, 156, cout).astype(np.uint8)
        wdeq = oracle.dequantize(w, sc.reshape(bshape), zp.reshape(bshape))
    dv = gpu.to_device
    kw = dict(w_scale=dv(np.asarray(sc)) if sc is not None else None,
              w_zp=dv(zp) if zp is not None else None)
    if kind == "convT":
        got = gpu.ops.conv_transpose1d(dv(x), dv(w), dv(b), (p0, p1), s, d, 1, op, **kw).numpy()
        want = oracle.conv_transpose1d(x, wdeq, b, (p0, p1), s, d, 1, op)
    else:
        got = gpu.ops.conv1d(dv(x), dv(w), dv(b), (p0, p1), s, d, **kw).numpy()
        want = oracle.conv1d(x, wdeq, b, (p0, p1), s, d)
    check(got, want, f"{wdt}-weight {case}")


def test_fp16_weight_conv_large_activations(gpu, oracle):
    """Activations far beyond fp16's range: the input is scaled by a power of
    two before the split, so the matrix-core pass stays exact in range."""
    r = rng(10)
    x = r.normal(0, 1, (1, 256, 2000)).astype(np.float32)
    x[0, 5, 123] = 1.0e5
    w = r.normal(0, 0.05, (256, 128, 12)).astype(np.float16)
    b = r.normal(0, 0.1, 128).astype(np.float32)
    got = gpu.ops.conv_transpose1d(gpu.to_device(x), gpu.to_device(w), gpu.to_device(b), (3, 3),
                                   6).numpy()
    check(got, oracle.conv_transpose1d(x, w, b, (3, 3), 6), "convT with a 1e5 activation")
    x2 = r.normal(0, 3e8, (1, 128, 20000)).astype(np.float32)
    x2[0, 100, 7] = -np.float32(4.0e12)
    w2 = r.normal(0, 0.05, (22, 128, 7)).astype(np.float16)
    got = gpu.ops.conv1d(gpu.to_device(x2), gpu.to_device(w2), None, (3, 3)).numpy()
    check(got, oracle.conv1d(x2, w2, None, (3, 3)), "conv with activations ~3e8 and -4e12")


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_fp16_weight_conv_nonfinite_falls_back(gpu, oracle, bad):
    """A non-finite activation sends each block whose input window holds it
    to scalar fp32 products and sums (inside the same launch), which
    propagate it as numpy does; the other blocks, and the next call, run on
    the matrix cores."""
    r = rng(11)
    x = r.normal(0, 1, (1, 256, 2000)).astype(np.float32)
    x[0, 5, 123] = bad
    w = r.normal(0, 0.05, (256, 128, 12)).astype(np.float16)
    b = r.normal(0, 0.1, 128).astype(np.float32)
    got = gpu.ops.conv_transpose1d(gpu.to_device(x), gpu.to_device(w), gpu.to_device(b), (3, 3),
                                   6).numpy()
    with np.errstate(invalid="ignore"):
        want = oracle.conv_transpose1d(x, w, b, (3, 3), 6)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    check(np.where(fin, got, 0), np.where(fin, want, 0), f"convT with a {bad} activation")
    x[0, 5, 123] = 0.5
    got = gpu.ops.conv_transpose1d(gpu.to_device(x), gpu.to_device(w), gpu.to_device(b), (3, 3),
                                   6).numpy()
    check(got, oracle.conv_transpose1d(x, w, b, (3, 3), 6), "convT after the fallback")


@pytest.mark.parametrize("sigma", [1e-4, 1e-5, 1e-7])
@pytest.mark.parametrize("kind", ["conv_i8", "convT_i8", "conv_f16", "convT_f16"])
def test_fp16_weight_conv_small_activations(gpu, oracle, sigma, kind):
    """Whole inputs of magnitude 1e-4 .. 1e-7 (a quiet stretch of the vocoder),
    where an unscaled split's low halves would be fp16 subnormals: held to the
    same bar as unit-scale inputs.  K = 1536 reductions, as in the 512-channel
    convolutions."""
    r = rng(12)
    if kind.startswith("conv_"):
        x = r.normal(0, sigma, (1, 512, 600)).astype(np.float32)
        shape = (256, 512, 3)
    else:
        x = r.normal(0, sigma, (1, 512, 120)).astype(np.float32)
        shape = (512, 256, 20)
    if kind.endswith("i8"):
        w, sc = int8_weight(r, shape)
        wdeq, kw = oracle.dequantize(w, sc), dict(w_scale=gpu.to_device(np.array(sc)))
    else:
        w = r.normal(0, 0.05, shape).astype(np.float16)
        wdeq, kw = w, {}
    dv = gpu.to_device
    if kind.startswith("conv_"):
        got = gpu.ops.conv1d(dv(x), dv(w), None, (1, 1), **kw).numpy()
        want = oracle.conv1d(x, wdeq, None, (1, 1))
    else:
        got = gpu.ops.conv_transpose1d(dv(x), dv(w), None, (5, 5), 10, **kw).numpy()
        want = oracle.conv_transpose1d(x, wdeq, None, (5, 5), 10)
    check(got, want, f"{kind} sigma {sigma}")


def decoder_stage(r):
    """The decoder upsample stage's operands (the fixed draws of the stage
    tests and of the bench): int8 ConvTranspose1d(512->256, k20, s10, p5)
    on [1,512,240], snake, AdaIN with style [1,128], then two residual blocks
    AdaIN -> snake -> conv(d) -> AdaIN -> snake -> conv(d1) -> + x with
    dilations 1 and 3 (int8 weights, per-tensor scales)."""
    return dict(
        x=r.normal(0, 1, (1, 512, 240)).astype(np.float32),
        style=r.normal(0, 0.1, (1, 128)).astype(np.float32),
        convt=int8_weight(r, (512, 256, 20)),
        alphas=[r.uniform(0.5, 2, (1, 256, 1)).astype(np.float32) for _ in range(5)],
        fcs=[r.normal(0, 0.05, (128, 512)).astype(np.float32) for _ in range(5)],
        convs=[int8_weight(r, (256, 256, 3)) for _ in range(4)])


def decoder_stage_ops(P):
    """The stage as a list of (name, bar, run(lib_or_None, inputs...)) steps,
    each taking the previous step's output (and, for the residual Add, the
    stage input of its block); lib None runs the oracle."""
    qt, st = P["convt"]

    def convt(L, O, h):
        if L is None:
            return O.conv_transpose1d(h, O.dequantize(qt, st), None, (5, 5), 10)
        return L.ops.conv_transpose1d(L.to_device(h), L.to_device(qt), None, (5, 5), 10,
                                      w_scale=L.to_device(np.array(st))).numpy()

    def snake(i):
        def f(L, O, h):
            a = P["alphas"][i]
            return O.snake(h, a) if L is None else \
                L.ops.snake(L.to_device(h), L.to_device(a)).numpy()
        return f

    def adain(i):
        def f(L, O, h):
            if L is None:
                return O.adain(h, P["style"], P["fcs"][i], None, 1e-5)
            return L.ops.adain(L.to_device(h), L.to_device(P["style"]), L.to_device(P["fcs"][i]),
                               None, 1e-5).numpy()
        return f

    def conv(i, dil):
        def f(L, O, h):
            q, s = P["convs"][i]
            if L is None:
                return O.conv1d(h, O.dequantize(q, s), None, (dil, dil), 1, dil)
            return L.ops.conv1d(L.to_device(h), L.to_device(q), None, (dil, dil), 1, dil,
                                w_scale=L.to_device(np.array(s))).numpy()
        return f

    ew, red, mm = (1e-5, 1e-6), (1e-4, 1e-5), (1e-4, 1e-5)
    steps = [("convT", mm, convt), ("snake0", ew, snake(0)), ("adain0", red, adain(0))]
    for blk, dil in enumerate((1, 3)):
        steps += [(f"res{blk}.adain1", red, adain(1 + 2 * blk)),
                  (f"res{blk}.snake1", ew, snake(1 + 2 * blk)),
                  (f"res{blk}.conv_d{dil}", mm, conv(2 * blk, dil)),
                  (f"res{blk}.adain2", red, adain(2 + 2 * blk)),
                  (f"res{blk}.snake2", ew, snake(2 + 2 * blk)),
                  (f"res{blk}.conv1", mm, conv(2 * blk + 1, 1)),
                  (f"res{blk}.add", (0.0, 0.0), "add")]
    return steps


def test_decoder_upsample_stage_teacher_forced(gpu, oracle):
    """Every step of the decoder upsample stage against the oracle, each fed
    the oracle's output of the step before: contractions and the AdaINs at
    rel 1e-4 + 1e-5 max, the snakes at rel 1e-5 + 1e-6 max, the residual Add
    bit for bit."""
    P = decoder_stage(rng(0))
    h = P["x"]
    block_in = None
    for name, (rtol, floor), fn in decoder_stage_ops(P):
        if name.endswith("adain1"):
            block_in = h
        if fn == "add":
            want = oracle.binary("Add", block_in, h)
            got = gpu.ops.binary("Add", gpu.to_device(block_in), gpu.to_device(h)).numpy()
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
        else:
            want = fn(None, oracle, h)
            got = fn(gpu, oracle, h)
            if rtol == RTOL:
                check(got, want, f"decoder stage {name}")
            else:
                assert_close(got, want, rtol, floor_rel=floor, what=f"decoder stage {name}")
        h = want


def test_decoder_upsample_stage_free_running(gpu, oracle):
    """The whole stage run through on each side: five normalisations in
    series amplify the per-step rounding, so the end result is held to 10x
    the single-step bar (each step is held to its own bar above)."""
    P = decoder_stage(rng(0))

    def run(L):
        h = P["x"]
        block_in = None
        for name, _bar, fn in decoder_stage_ops(P):
            if name.endswith("adain1"):
                block_in = h
            if fn == "add":
                h = oracle.binary("Add", block_in, h) if L is None else \
                    L.ops.binary("Add", L.to_device(block_in), L.to_device(h)).numpy()
            else:
                h = fn(L, oracle, h)
        return h

    assert_close(run(gpu), run(None), 1e-3, floor_rel=1e-4, what="decoder stage")


@pytest.mark.parametrize("cin,cout,k,L,pad,dil,stride,wdt,wzp,resid", [
    (128, 128, 11, 3001, 5, 1, 1, np.uint8, 129, False),
    (100, 200, 3, 777, 3, 3, 1, np.int8, None, True),
    (512, 256, 7, 1203, 9, 3, 1, np.uint8, 66, True),
    (64, 40, 5, 500, 2, 1, 2, np.uint8, 0, False)])
def test_conv_packed_weights(gpu, cin, cout, k, L, pad, dil, stride, wdt, wzp, resid):
    """kk_conv_integer_scaled_qbias_packed: the weights packed once by
    kk_conv_integer_pack, the bias quantisation formed in the conv's
    prologue -- bit-identical to the per-call path (with and without the
    residual Add), on two calls in a row with different activations."""
    r = rng(41)
    lo, hi = (0, 256) if wdt == np.uint8 else (-128, 128)
    w = gpu.to_device(r.integers(lo, hi, (cout, cin, k)).astype(wdt))
    wz = None if wzp is None else gpu.to_device(np.array(wzp, wdt))
    bias = gpu.to_device(r.normal(0, 0.5, (cout,)).astype(np.float32))
    sw = gpu.to_device(np.array(0.0037, np.float32))
    packed = gpu.ops.conv_integer_pack(w, wz)
    lout = (L + 2 * pad - dil * (k - 1) - 1) // stride + 1
    for call in range(2):
        x = gpu.to_device(r.integers(0, 256, (1, cin, L)).astype(np.uint8))
        xz = gpu.to_device(np.array(100 + call, np.uint8))
        sa = gpu.to_device(np.array(r.uniform(1e-3, 1e-2), np.float32))
        res = gpu.to_device(r.normal(0, 1, (1, cout, lout)).astype(np.float32)) if resid else None
        kw = dict(pads=(pad, pad), stride=stride, dilation=dil, resid=res)
        want = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, **kw).numpy()
        got = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, packed=packed,
                                                **kw).numpy()
        assert_bitexact(got, want, f"packed conv {cin}->{cout} k{k} call {call}")


@pytest.mark.parametrize("cin,cout,k,L,pad,dil,resid", [
    (64, 64, 3, 20000, 1, 1, False),      # two whole 8192-blocks and a tail
    (128, 130, 7, 17000, 9, 3, True),     # a second, partial channel block; the residual
    (96, 128, 11, 16400, 25, 5, False)])
def test_conv_leaf_sums(gpu, cin, cout, k, L, pad, dil, resid):
    """kk_conv_integer_scaled_qbias_packed_leaves: the output bit-identical to
    the packed conv's, and leaf t of each row -- the sum of its elements
    128 t .. 128 t + 127 -- equal to numpy's np.add.reduce of that slice
    (eight accumulators of sixteen terms, then their tree) for every leaf of
    the rows' whole 8192-blocks."""
    r = rng(45)
    w = gpu.to_device(r.integers(0, 256, (cout, cin, k)).astype(np.uint8))
    wz = gpu.to_device(np.array(128, np.uint8))
    bias = gpu.to_device(r.normal(0, 0.5, (cout,)).astype(np.float32))
    sw = gpu.to_device(np.array(0.0037, np.float32))
    sa = gpu.to_device(np.array(0.0051, np.float32))
    packed = gpu.ops.conv_integer_pack(w, wz)
    x = gpu.to_device(r.integers(0, 256, (1, cin, L)).astype(np.uint8))
    xz = gpu.to_device(np.array(117, np.uint8))
    lout = L + 2 * pad - dil * (k - 1)
    res = gpu.to_device(r.normal(0, 1, (1, cout, lout)).astype(np.float32)) if resid else None
    kw = dict(pads=(pad, pad), dilation=dil, resid=res, packed=packed)
    want = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, **kw).numpy()
    out, leaves = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, leaves=True, **kw)
    got = out.numpy()
    assert_bitexact(got, want, f"conv with leaf sums {cin}->{cout} k{k}")
    lv = leaves.numpy()
    nleaf = (lout // 8192) * 64
    assert lv.shape == (cout, nleaf)
    ref = np.add.reduce(got[0, :, :nleaf * 128].reshape(cout, nleaf, 128), axis=2)
    # (np.add.reduce over the last axis of a [.., 128] view sums each row of
    # 128 contiguous values with numpy's pairwise loop, as the oracle's
    # ReduceMean does)
    for t in (0, 1, nleaf - 1):
        assert_bitexact(np.float32(np.add.reduce(got[0, 0, 128 * t:128 * t + 128])), ref[0, t],
                        "numpy leaf order")
    assert_bitexact(lv, ref.astype(np.float32), f"leaf sums {cin}->{cout} k{k}")


@pytest.mark.parametrize("kind", ["leaky", "snake", "affine"])
def test_instance_norm_quant_with_leaf_sums(gpu, kind):
    """kk_instance_norm_quant_leaves on a conv's output with that conv's leaf
    sums: the same bytes, scale and zero point as without them, on rows
    long enough for the block-wise statistics (100,000 steps: twelve whole
    8192-blocks and a tail).  Leaf sums formed from another tensor are
    refused."""
    r = rng(46)
    cin, cout, L = 32, 48, 100000
    w = gpu.to_device(r.integers(0, 256, (cout, cin, 3)).astype(np.uint8))
    wz = gpu.to_device(np.array(128, np.uint8))
    bias = gpu.to_device(r.normal(0, 0.5, (cout,)).astype(np.float32))
    sw = gpu.to_device(np.array(0.004, np.float32))
    sa = gpu.to_device(np.array(0.006, np.float32))
    packed = gpu.ops.conv_integer_pack(w, wz)
    x = gpu.to_device(r.integers(0, 256, (1, cin, L)).astype(np.uint8))
    xz = gpu.to_device(np.array(100, np.uint8))
    y, leaves = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, pads=(1, 1),
                                                  packed=packed, leaves=True)
    D = gpu.to_device
    g = D((1 + 0.1 * r.normal(0, 1, (1, cout, 1))).astype(np.float32))
    b = D((0.1 * r.normal(0, 1, (1, cout, 1))).astype(np.float32))
    a = D(r.uniform(0.5, 2, (1, cout, 1)).astype(np.float32))
    rc = D((1.0 / r.uniform(0.5, 2, (1, cout, 1))).astype(np.float32))
    args = {"leaky": dict(leaky_alpha=0.2), "snake": dict(alpha=a, recip=rc),
            "affine": {}}[kind]
    want = gpu.ops.instance_norm_quant(y, g, b, eps=1e-5, **args)
    got = gpu.ops.instance_norm_quant(y, g, b, eps=1e-5, leaves=leaves, **args)
    for gt, wt, what in zip(got, want, ("bytes", "scale", "zero point")):
        assert_bitexact(gpu.to_host(gt), gpu.to_host(wt), f"{kind} {what}")
    other = y.astype(np.float32)  # same values, another buffer
    with pytest.raises(gpu._lib.KKError, match="not formed from x"):
        gpu.ops.instance_norm_quant(other, g, b, eps=1e-5, leaves=leaves, **args)
    # freeing x forgets its leaf sums: a tensor that the pool hands the same
    # address next is refused with them
    addr = y.ptr
    del y, got, want
    gpu.sync()
    again = [gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, pads=(1, 1),
                                               packed=packed) for _ in range(4)]
    reused = [t for t in again if t.ptr == addr]
    assert reused, "the pool did not hand out the freed address again"
    for t in reused:
        with pytest.raises(gpu._lib.KKError, match="not formed from x"):
            gpu.ops.instance_norm_quant(t, g, b, eps=1e-5, leaves=leaves, **args)


def test_conv_packed_refuses_another_weight(gpu):
    """A packed buffer is used only with the weight and zero-point tensors it
    was packed from: another weight of the same shape, or another zero point,
    is refused with an error before any launch."""
    r = rng(43)
    w = gpu.to_device(r.integers(0, 256, (64, 64, 3)).astype(np.uint8))
    w2 = gpu.to_device(r.integers(0, 256, (64, 64, 3)).astype(np.uint8))
    wz = gpu.to_device(np.array(120, np.uint8))
    wz2 = gpu.to_device(np.array(121, np.uint8))
    packed = gpu.ops.conv_integer_pack(w, wz)
    x = gpu.to_device(r.integers(0, 256, (1, 64, 300)).astype(np.uint8))
    xz = gpu.to_device(np.array(100, np.uint8))
    bias = gpu.to_device(r.normal(0, 0.5, (64,)).astype(np.float32))
    sa = gpu.to_device(np.array(0.004, np.float32))
    sw = gpu.to_device(np.array(0.003, np.float32))
    kw = dict(pads=(1, 1), packed=packed)
    ok = gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, **kw).numpy()
    assert ok.shape == (1, 64, 300)
    with pytest.raises(gpu._lib.KKError, match="another weight tensor"):
        gpu.ops.conv_integer_scaled_qbias(x, w2, xz, wz, bias, sa, sw, **kw)
    with pytest.raises(gpu._lib.KKError, match="another weight zero point"):
        gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz2, bias, sa, sw, **kw)
    with pytest.raises(gpu._lib.KKError, match="not made by kk_conv_integer_pack"):
        other = gpu.DeviceTensor.empty(packed.shape, np.uint8)
        gpu.ops.conv_integer_scaled_qbias(x, w, xz, wz, bias, sa, sw, pads=(1, 1), packed=other)


@pytest.mark.parametrize("case", F16MC)
def test_fp16_weight_conv_packed(gpu, oracle, case):
    """kk_conv1d_packed / kk_conv_transpose1d_packed: the weights laid out
    once by kk_conv_pack give the per-call path's bits (the same kernel on
    the same layout) on two calls in a row with different activations, each
    within the oracle's bar."""
    kind, n, cin, cout, k, L, p0, p1, s, d, op, wdt = case
    r = rng(44)
    shape = (cin, cout, k) if kind == "convT" else (cout, cin, k)
    bshape = (1, cout, 1) if kind == "convT" else (cout, 1, 1)
    sc = zp = None
    if wdt == "f16":
        w = r.normal(0, 0.05, shape).astype(np.float16)
        wdeq = w
    elif wdt == "i8":
        w, sc = int8_weight(r, shape)
        wdeq = oracle.dequantize(w, sc)
    else:
        w = r.integers(0, 256, shape).astype(np.uint8)
        sc = r.uniform(1e-4, 1e-3, cout).astype(np.float32)
        zp = r.integers(100, 156, cout).astype(np.uint8)
        wdeq = oracle.dequantize(w, sc.reshape(bshape), zp.reshape(bshape))
    dv = gpu.to_device
    wd = dv(w)
    kw = dict(w_scale=dv(np.asarray(sc)) if sc is not None else None,
              w_zp=dv(zp) if zp is not None else None)
    packed = gpu.ops.conv_pack(wd, kw["w_zp"], kind == "convT", s)
    for call in range(2):
        x = r.normal(0, 1 + call, (n, cin, L)).astype(np.float32)
        b = r.normal(0, 0.1, cout).astype(np.float32)
        if kind == "convT":
            args = (dv(x), wd, dv(b), (p0, p1), s, d, 1, op)
            want = gpu.ops.conv_transpose1d(*args, **kw).numpy()
            got = gpu.ops.conv_transpose1d(*args, packed=packed, **kw).numpy()
            ref = oracle.conv_transpose1d(x, wdeq, b, (p0, p1), s, d, 1, op)
        else:
            args = (dv(x), wd, dv(b), (p0, p1), s, d)
            want = gpu.ops.conv1d(*args, **kw).numpy()
            got = gpu.ops.conv1d(*args, packed=packed, **kw).numpy()
            ref = oracle.conv1d(x, wdeq, b, (p0, p1), s, d)
        assert_bitexact(got, want, f"packed {wdt}-weight {case} call {call}")
        check(got, ref, f"packed {wdt}-weight {case} call {call}")


def test_fp16_weight_conv_packed_refuses_mismatch(gpu):
    """A packed Conv / ConvTranspose weight is used only with the tensor, zero
    point, operation and stride it was packed for."""
    r = rng(45)
    dv = gpu.to_device
    w = dv(r.integers(0, 256, (256, 128, 12)).astype(np.uint8))
    w2 = dv(r.integers(0, 256, (256, 128, 12)).astype(np.uint8))
    wz, wz2 = dv(np.array(120, np.uint8)), dv(np.array(121, np.uint8))
    sc = dv(np.array(0.002, np.float32))
    x = dv(r.normal(0, 1, (1, 256, 600)).astype(np.float32))
    packed = gpu.ops.conv_pack(w, wz, True, 6)
    ok = gpu.ops.conv_transpose1d(x, w, None, (3, 3), 6, w_scale=sc, w_zp=wz, packed=packed)
    assert ok.shape == (1, 128, 3600)
    E = gpu._lib.KKError
    with pytest.raises(E, match="another weight tensor"):
        gpu.ops.conv_transpose1d(x, w2, None, (3, 3), 6, w_scale=sc, w_zp=wz, packed=packed)
    with pytest.raises(E, match="another weight zero point"):
        gpu.ops.conv_transpose1d(x, w, None, (3, 3), 6, w_scale=sc, w_zp=wz2, packed=packed)
    with pytest.raises(E, match="another stride|packed must be"):
        gpu.ops.conv_transpose1d(x, w, None, (3, 3), 4, w_scale=sc, w_zp=wz, packed=packed)
    with pytest.raises(E, match="not made by kk_conv_pack"):
        gpu.ops.conv_transpose1d(x, w, None, (3, 3), 6, w_scale=sc, w_zp=wz,
                                 packed=gpu.DeviceTensor.empty(packed.shape, np.uint8))
    wc = dv(r.normal(0, 0.05, (128, 128, 3)).astype(np.float16))
    pc = gpu.ops.conv_pack(wc, None, False, 1)
    xc = dv(r.normal(0, 1, (1, 128, 900)).astype(np.float32))
    gpu.ops.conv1d(xc, wc, None, (1, 1), packed=pc)
    wt = dv(r.normal(0, 0.05, (128, 128, 3)).astype(np.float16))
    pt = gpu.ops.conv_pack(wt, None, True, 1)  # the same size as pc, packed for ConvTranspose
    with pytest.raises(E, match="another operation"):
        gpu.ops.conv1d(xc, wt, None, (1, 1), packed=pt)


# ------------------------------------------- packed dequant-GEMM weights
GEMM_PACKED = [  # (batch, m, k, n, weight kind, zero point)
    ((), 256, 768, 2048, "i8", None),      # the dequant GEMM configs (64-wide column tiles)
    ((), 256, 2048, 768, "i8", None),      # (32-wide)
    ((), 256, 768, 768, "f16", None),      # fp16 weights, two bf16 parts
    ((), 130, 100, 70, "u8", "col"),       # ragged K and N, per-column uint8 zero point
    ((), 37, 96, 333, "i8", "tensor"),     # a nonzero per-tensor int8 zero point
    ((2,), 64, 96, 80, "f16", None),       # batched activations, one weight
    ((), 50, 45, 40, "i8", None),          # K % 4 != 0: the fp32 kernels, w itself
]


@pytest.mark.parametrize("case", GEMM_PACKED, ids=[f"{c[4]}-{c[1]}x{c[2]}x{c[3]}" for c in GEMM_PACKED])
def test_gemm_packed(gpu, oracle, case):
    """kk_gemm_packed: the weights packed once by kk_gemm_pack give kk_gemm's
    bits (the same kernel on the same operand values) on two calls in a row
    with different activations, each within the oracle's bar."""
    batch, m, k, n, wdt, zpk = case
    r = rng(46)
    dv = gpu.to_device
    sc = zp = None
    if wdt == "f16":
        w = r.normal(0, 0.05, (k, n)).astype(np.float16)
        wdeq = w
    elif wdt == "i8":
        w, s = int8_weight(r, (k, n))
        sc = np.array(s, np.float32)
        zp = np.array(r.integers(-20, 20), np.int8) if zpk == "tensor" else None
        wdeq = oracle.dequantize(w, sc, zp)
    else:
        w = r.integers(0, 256, (k, n)).astype(np.uint8)
        sc = r.uniform(1e-4, 1e-3, n).astype(np.float32)
        zp = r.integers(100, 156, n).astype(np.uint8)
        wdeq = oracle.dequantize(w, sc, zp)
    wd = dv(w)
    kw = dict(w_scale=dv(sc) if sc is not None else None, w_zp=dv(zp) if zp is not None else None)
    packed = gpu.ops.gemm_pack(wd, kw["w_zp"])
    for call in range(2):
        a = r.normal(0, 1 + call, batch + (m, k)).astype(np.float32)
        want = gpu.ops.matmul(dv(a), wd, **kw).numpy()
        got = gpu.ops.matmul(dv(a), wd, packed=packed, **kw).numpy()
        assert_bitexact(got, want, f"packed {case} call {call}")
        check(got, oracle.matmul(a, wdeq), f"packed {case} call {call}")


def test_gemm_packed_refuses_mismatch(gpu):
    """A packed MatMul weight is used only with the tensor and zero point it
    was packed from."""
    r = rng(47)
    dv = gpu.to_device
    w = dv(r.integers(0, 256, (256, 512)).astype(np.uint8))
    w2 = dv(r.integers(0, 256, (256, 512)).astype(np.uint8))
    wz, wz2 = dv(np.array(120, np.uint8)), dv(np.array(121, np.uint8))
    sc = dv(np.array(0.002, np.float32))
    a = dv(r.normal(0, 1, (64, 256)).astype(np.float32))
    packed = gpu.ops.gemm_pack(w, wz)
    assert gpu.ops.matmul(a, w, sc, wz, packed=packed).shape == (64, 512)
    E = gpu._lib.KKError
    with pytest.raises(E, match="another weight tensor"):
        gpu.ops.matmul(a, w2, sc, wz, packed=packed)
    with pytest.raises(E, match="another weight zero point"):
        gpu.ops.matmul(a, w, sc, wz2, packed=packed)
    with pytest.raises(E, match="not made by kk_gemm_pack"):
        gpu.ops.matmul(a, w, sc, wz, packed=gpu.DeviceTensor.empty(packed.shape, np.uint8))
    with pytest.raises(E, match="packed must be"):
        gpu.ops.matmul(a, w, sc, wz, packed=gpu.DeviceTensor.empty((packed.shape[0] // 2,), np.uint8))
