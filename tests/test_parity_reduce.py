"""Parity of the reductions and normalisations (AdaIN, InstanceNorm,
LayerNorm/SkipLayerNorm, Softmax, ReduceMean/Sum) with the oracle.

Bar: |got - ref| <= 1e-4*|ref| + 1e-5 (rel 1e-4, abs 1e-5) on unit-scale
data; summation order differs from numpy's pairwise sums, nothing else."""
import numpy as np
import pytest

from conftest import assert_bitexact, assert_close, rng

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


def adain_inputs(c, t, seed=0):
    """x ~ N(0,1) [1,C,T]; style ~ N(0,0.1) [1,128]; W ~ N(0,0.05) [128,2C];
    b = 0 (the Linear's init is not fixed by the workload; recorded here)."""
    r = rng(seed)
    x = r.normal(0, 1, (1, c, t)).astype(np.float32)
    s = r.normal(0, 0.1, (1, 128)).astype(np.float32)
    w = r.normal(0, 0.05, (128, 2 * c)).astype(np.float32)
    b = np.zeros(2 * c, np.float32)
    return x, s, w, b


@pytest.mark.parametrize("t", [1200, 9600, 4100, 6000, 13000, 16384])
def test_adain_config(gpu, oracle, t):
    x, s, w, b = adain_inputs(512, t)
    got = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), gpu.to_device(w),
                        gpu.to_device(b), 1e-5).numpy()
    assert_close(got, oracle.adain(x, s, w, b, 1e-5), RTOL, ATOL, what=f"AdaIN T={t}")


@pytest.mark.parametrize("t,w8", [(1028, False), (1360, True), (1700, False), (2048, True)])
def test_adain_one_wave_rows(gpu, oracle, t, w8):
    """Rows of 257 .. 512 float4s (one wave a row; a last vector only some
    lanes hold), offset from zero, fp32 and int8 style weights."""
    r = rng(9)
    c = 96
    x = (3.0 + 2.0 * r.normal(0, 1, (1, c, t))).astype(np.float32)
    s = r.normal(0, 0.1, (1, 128)).astype(np.float32)
    b = r.normal(0, 0.05, 2 * c).astype(np.float32)
    if w8:
        q = r.integers(-127, 128, (128, 2 * c)).astype(np.int8)
        sc = r.uniform(1e-3, 1e-2, 2 * c).astype(np.float32)
        got = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), gpu.to_device(q),
                            gpu.to_device(b), 1e-5, w_scale=gpu.to_device(sc)).numpy()
        want = oracle.adain(x, s, oracle.dequantize(q, sc), b, 1e-5)
    else:
        w = r.normal(0, 0.05, (128, 2 * c)).astype(np.float32)
        got = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), gpu.to_device(w),
                            gpu.to_device(b), 1e-5).numpy()
        want = oracle.adain(x, s, w, b, 1e-5)
    assert_close(got, want, RTOL, ATOL, what=f"AdaIN T={t} int8 fc {w8}")


def test_adain_transposed_weight_and_dispatch(gpu, oracle):
    x, s, w, b = adain_inputs(256, 2400, seed=1)
    b = rng(2).normal(0, 0.05, 512).astype(np.float32)
    wt = gpu.to_device(np.ascontiguousarray(w.T)).transpose()  # W^T resident, viewed as W
    got = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), wt, gpu.to_device(b), 1e-5).numpy()
    assert_close(got, oracle.adain(x, s, w, b, 1e-5), RTOL, ATOL, what="AdaIN W^T")
    env = {"x": gpu.to_device(x), "s": gpu.to_device(s), "w": gpu.to_device(w),
           "b": gpu.to_device(b)}
    gpu.dispatch("AdaIN", ["x", "s", "w", "b"], ["y"], {"epsilon": 1.0013580322265625e-05}, env)
    assert_close(env["y"].numpy(), oracle.adain(x, s, w, b, 1.0013580322265625e-05), RTOL, ATOL,
                 what="AdaIN dispatch")


def test_adain_int8_weight(gpu, oracle):
    """The graph's fc is int8 with a per-column scale (MatMulInteger path
    in dequant form)."""
    r = rng(3)
    x = r.normal(0, 1, (1, 128, 700)).astype(np.float32)
    s = r.normal(0, 0.1, (1, 128)).astype(np.float32)
    q = r.integers(-127, 128, (128, 256)).astype(np.int8)
    sc = r.uniform(1e-3, 1e-2, 256).astype(np.float32)
    got = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), gpu.to_device(q), None, 1e-5,
                        w_scale=gpu.to_device(sc)).numpy()
    want = oracle.adain(x, s, oracle.dequantize(q, sc), None, 1e-5)
    assert_close(got, want, RTOL, ATOL, what="AdaIN int8 fc")


def test_adain_matches_node_chain(gpu, oracle):
    """Fused AdaIN equals the graph's nine dispatched norm nodes."""
    r = rng(4)
    c, t = 64, 1000
    x = r.normal(0, 1, (1, c, t)).astype(np.float32)
    g = r.normal(0, 0.3, (1, c, 1)).astype(np.float32)
    bt = r.normal(0, 0.3, (1, c, 1)).astype(np.float32)
    env = {"x": gpu.to_device(x), "g": gpu.to_device(g), "b": gpu.to_device(bt),
           "ax": np.array([2]), "eps": gpu.to_device(np.array(1e-5, np.float32)),
           "one": gpu.to_device(np.array(1.0, np.float32))}
    chain = [("ReduceMean", ["x", "ax"], "mu"), ("Sub", ["x", "mu"], "d"),
             ("Mul", ["d", "d"], "d2"), ("ReduceMean", ["d2", "ax"], "var"),
             ("Add", ["var", "eps"], "ve"), ("Sqrt", ["ve"], "sd"), ("Div", ["d", "sd"], "q"),
             ("Add", ["g", "one"], "g1"), ("Mul", ["q", "g1"], "y0"), ("Add", ["y0", "b"], "y")]
    for op, ins, out in chain:
        gpu.dispatch(op, ins, [out], {}, env)
    gb = np.concatenate([g.reshape(-1), bt.reshape(-1)]).astype(np.float32)
    fused = gpu.ops.instance_norm(env["x"], gpu.to_device(gb), 1e-5).numpy()
    assert_close(fused, env["y"].numpy(), RTOL, ATOL, what="fused vs chain")
    assert_close(fused, oracle.instance_norm_affine(x, g, bt, 1e-5), RTOL, ATOL, what="vs oracle")


@pytest.mark.parametrize("t", [5, 61, 257, 4097, 20000])
def test_instance_norm_lengths(gpu, oracle, t):
    r = rng(5)
    x = (3 + 2 * r.normal(0, 1, (2, 7, t))).astype(np.float32)
    zero = np.zeros((1, 7, 1), np.float32)
    got = gpu.ops.instance_norm(gpu.to_device(x), None, 1e-5).numpy()
    assert_close(got, oracle.instance_norm_affine(x, zero, zero, 1e-5), RTOL, ATOL,
                 what=f"instance norm T={t}")


def test_adain_invariants_full_size(gpu):
    """Zero style weights: every channel comes out with mean 0, variance 1."""
    x = (5 + 3 * rng(6).normal(0, 1, (1, 512, 9600))).astype(np.float32)
    w = np.zeros((128, 1024), np.float32)
    s = np.ones((1, 128), np.float32)
    y = gpu.ops.adain(gpu.to_device(x), gpu.to_device(s), gpu.to_device(w), None,
                      1e-5).numpy().astype(np.float64)
    assert np.abs(y.mean(-1)).max() < 1e-5
    assert np.abs(y.var(-1) - 1).max() < 1e-3


def test_layernorm_config(gpu, oracle):
    """x ~ N(0,1) [1,256,768]; gamma = 1 + 0.1 N, beta = 0.1 N; eps 1e-12
    (ALBERT) and the LayerNormalization default 1e-5."""
    r = rng(0)
    x = r.normal(0, 1, (1, 256, 768)).astype(np.float32)
    g = (1 + 0.1 * r.normal(0, 1, 768)).astype(np.float32)
    b = (0.1 * r.normal(0, 1, 768)).astype(np.float32)
    for eps in (1e-12, 1e-5):
        env = {"x": gpu.to_device(x), "g": gpu.to_device(g), "b": gpu.to_device(b)}
        gpu.dispatch("LayerNormalization", ["x", "g", "b"], ["y"], {"epsilon": eps}, env)
        assert_close(env["y"].numpy(), oracle.layernorm(x, g, b, -1, eps), RTOL, ATOL,
                     what=f"LayerNorm eps {eps}")


@pytest.mark.parametrize("rows,cols,with_bias", [(5, 260, False), (4, 512, True), (3, 1000, True),
                                                  (2, 2048, False), (7, 1996, True)])
def test_layernorm_row_lengths(gpu, oracle, rows, cols, with_bias):
    """Rows of 65 .. 512 float4s (one wave a row; a last vector only some
    lanes hold), with and without the bias, mean offset from zero."""
    r = rng(8)
    x = (3.0 + r.normal(0, 2, (rows, cols))).astype(np.float32)
    g = (1 + 0.1 * r.normal(0, 1, cols)).astype(np.float32)
    b = (0.1 * r.normal(0, 1, cols)).astype(np.float32) if with_bias else None
    env = {"x": gpu.to_device(x), "g": gpu.to_device(g)}
    ins = ["x", "g"]
    if with_bias:
        env["b"] = gpu.to_device(b)
        ins.append("b")
    gpu.dispatch("LayerNormalization", ins, ["y"], {"epsilon": 1e-5}, env)
    assert_close(env["y"].numpy(), oracle.layernorm(x, g, b, -1, 1e-5), RTOL, ATOL,
                 what=f"LayerNorm [{rows}, {cols}] bias {with_bias}")


def test_skip_layernorm(gpu, oracle):
    r = rng(7)
    x, skip = (r.normal(0, 1, (1, 130, 768)).astype(np.float32) for _ in range(2))
    g = (1 + 0.1 * r.normal(0, 1, 768)).astype(np.float16)
    b = (0.1 * r.normal(0, 1, 768)).astype(np.float16)
    bias = (0.1 * r.normal(0, 1, 768)).astype(np.float16)
    env = {k: gpu.to_device(v) for k, v in dict(x=x, s=skip, g=g, b=b, bb=bias).items()}
    gpu.dispatch("SkipLayerNormalization", ["x", "s", "g", "b", "bb"], ["y"], {}, env)
    want = oracle.skip_layernorm(x, skip, g, b, bias, 1e-12)
    assert_close(env["y"].numpy(), want, RTOL, ATOL, what="SkipLayerNorm")


@pytest.mark.parametrize("shape,axis", [((1, 12, 256, 256), -1), ((3, 77), -1), ((2, 5000), -1),
                                        ((4, 9, 33), 1), ((2, 3, 130, 130), -1)])
def test_softmax(gpu, oracle, shape, axis):
    r = rng(8)
    x = r.normal(0, 2, shape).astype(np.float32)  # std 2
    env = {"x": gpu.to_device(x)}
    gpu.dispatch("Softmax", ["x"], ["y"], {"axis": axis}, env)
    y = env["y"].numpy()
    assert_close(y, oracle.softmax(x, axis), RTOL, ATOL, what=f"softmax {shape} ax {axis}")
    assert np.allclose(y.astype(np.float64).sum(axis), 1.0, atol=1e-5)


def test_softmax_exp_range(gpu):
    """Rows spanning the whole range of exp below the row maximum (x - max
    from 0 to -87): every probability within rel 1e-5 of the float64 value,
    the smallest ones included."""
    r = rng(10)
    base = -np.linspace(0, 87, 256)
    x = np.stack([base + r.uniform(-5, 5) for _ in range(12)]).astype(np.float32)
    for row in x:
        r.shuffle(row)
    env = {"x": gpu.to_device(x)}
    gpu.dispatch("Softmax", ["x"], ["y"], {"axis": -1}, env)
    y = env["y"].numpy().astype(np.float64)
    xd = x.astype(np.float64)
    want = np.exp(xd - xd.max(-1, keepdims=True))
    want /= want.sum(-1, keepdims=True)
    keep = want > 2.0 ** -120  # (exp results below 2^-126 may flush to 0)
    rel = np.abs(y - want)[keep] / want[keep]
    assert rel.max() < 1e-5, rel.max()


@pytest.mark.parametrize("op", ["ReduceMean", "ReduceSum"])
@pytest.mark.parametrize("shape,axes,keep", [((1, 512, 2400), [2], 1), ((6, 40), [0], 1),
                                             ((3, 4, 50), [0, 2], 0), ((2, 3, 7), None, 1),
                                             ((1, 64, 9), [-1], 0), ((1, 128, 100000), [2], 1),
                                             ((1, 3, 40001), [-1], 1), ((3590, 1, 512), [0], 1),
                                             ((2, 14999), [1], 1), ((2, 15001), [1], 1),
                                             ((4, 8192), [1], 1), ((1, 7), [1], 1),
                                             ((5, 129), [1], 0), ((2, 16390), [1], 1)])
def test_reduce(gpu, oracle, op, shape, axes, keep):
    x = rng(9).normal(0, 1, shape).astype(np.float32)
    env = {"x": gpu.to_device(x)}
    ins = ["x"]
    if axes is not None:
        env["ax"] = np.array(axes)
        ins.append("ax")
    gpu.dispatch(op, ins, ["y"], {"keepdims": keep}, env)
    oenv = {"x": x}
    if axes is not None:
        oenv["ax"] = np.array(axes)
    oracle.dispatch(op, ins, ["y"], {"keepdims": keep}, oenv)
    got = env["y"].numpy()
    nd = len(shape)
    red = sorted(a % nd for a in (axes if axes is not None else range(nd)))
    if red == list(range(nd - len(red), nd)) or len(red) == 1:
        # One contiguous run of trailing axes (numpy's blocked pairwise order)
        # or a single outer axis (numpy's sequential order): same bits.
        assert_bitexact(got, oenv["y"], f"{op} {shape} {axes}")
    else:
        assert_close(got, oenv["y"], RTOL, ATOL, floor_rel=1e-6, what=f"{op} {shape} {axes}")
