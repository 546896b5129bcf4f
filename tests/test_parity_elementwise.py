"""Parity of libkk's elementwise family, casts and pure-indexing ops with the
oracle, on the GPU through the C ABI.

Bars: bit-exact for broadcast arithmetic whose ops IEEE rounds correctly
(+ - * / sqrt, LeakyRelu, floor, rint, casts) and for every indexing op;
rel 1e-5 for transcendental ops, with an absolute floor of 1e-6*max|ref|
where cancellation makes relative error meaningless (snake)."""
import json
import os

import numpy as np
import pytest

from conftest import assert_bitexact, assert_close, rng

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "elementwise_kats.json")))


def run_node(kk, op, inputs, attrs=None, nout=1):
    """Run one node through the drop-in dispatch; inputs are numpy (uploaded
    to the device) or ('host', array) for host shape data."""
    env, names = {}, []
    for i, v in enumerate(inputs):
        if v is None:
            names.append("")
            continue
        name = f"in{i}"
        if isinstance(v, tuple) and v[0] == "host":
            env[name] = v[1]
        else:
            env[name] = kk.to_device(np.asarray(v))
        names.append(name)
    outs = [f"out{i}" for i in range(nout)]
    kk.dispatch(op, names, outs, attrs or {}, env)
    res = [kk.to_host(env[o]) for o in outs]
    return res[0] if nout == 1 else res


def oracle_node(oracle, op, inputs, attrs=None, nout=1):
    env, names = {}, []
    for i, v in enumerate(inputs):
        if v is None:
            names.append("")
            continue
        env[f"in{i}"] = v[1] if isinstance(v, tuple) else np.asarray(v)
        names.append(f"in{i}")
    outs = [f"out{i}" for i in range(nout)]
    oracle.dispatch(op, names, outs, attrs or {}, env)
    res = [env[o] for o in outs]
    return res[0] if nout == 1 else res


# ----------------------------------------------- broadcast elementwise set
@pytest.fixture(scope="module")
def set1():
    """fp32 x [1,512,2400] ~ N(0,1), per-channel c [1,512,1] ~ N(0,1),
    alpha [1,512,1] ~ U(0.5,2), seed 0, drawn in that order."""
    r = rng(0)
    x = r.normal(0, 1, (1, 512, 2400)).astype(np.float32)
    c = r.normal(0, 1, (1, 512, 1)).astype(np.float32)
    alpha = r.uniform(0.5, 2, (1, 512, 1)).astype(np.float32)
    return x, c, alpha


@pytest.mark.parametrize("op", ["Add", "Mul", "Sub", "Div"])
def test_set1_binary_bitexact(gpu, oracle, set1, op):
    x, c, _ = set1
    got = run_node(gpu, op, [x, c])
    assert_bitexact(got, oracle.binary(op, x, c), op)


def test_set1_leaky_relu_bitexact(gpu, oracle, set1):
    x = set1[0]
    got = run_node(gpu, "LeakyRelu", [x], {"alpha": 0.2})
    assert_bitexact(got, oracle.unary("LeakyRelu", x, 0.2), "LeakyRelu")


def test_set1_snake(gpu, oracle, set1):
    x, _, alpha = set1
    got = gpu.ops.snake(gpu.to_device(x), gpu.to_device(alpha)).numpy()
    assert_close(got, oracle.snake(x, alpha), 1e-5, floor_rel=1e-6, what="snake")
    rec = (np.float32(1) / alpha).astype(np.float16)  # the graph's folded fp16 1/alpha
    got = run_node(gpu, "Snake", [x, alpha.astype(np.float16), rec])
    assert_close(got, oracle.snake(x, alpha.astype(np.float16), rec), 1e-5, floor_rel=1e-6,
                 what="snake fp16 recip")


def test_set1_snake_is_the_node_chain(gpu, oracle, set1):
    """The fused kernel equals the five dispatched nodes it replaces."""
    x, _, alpha = set1
    xs, al = x[:, :64], alpha[:, :64]
    rec = (np.float32(1) / al).astype(np.float32)
    env = {"x": gpu.to_device(xs), "a": gpu.to_device(al), "r": gpu.to_device(rec),
           "two": gpu.to_device(np.array(2.0, np.float32))}
    for op, ins, out in [("Mul", ["a", "x"], "t"), ("Sin", ["t"], "s"),
                         ("Pow", ["s", "two"], "p"), ("Mul", ["r", "p"], "q"),
                         ("Add", ["x", "q"], "y")]:
        gpu.dispatch(op, ins, [out], {}, env)
    chain = env["y"].numpy()
    fused = gpu.ops.snake(env["x"], env["a"], env["r"]).numpy()
    assert_bitexact(fused, chain, "fused snake vs node chain")


def test_snake_chain_edge_arguments(gpu):
    """Bit-exact against the node chain where the fused kernel's squared
    sine skips the sine's sign handling: signed zeros, tiny values, both
    parities of the multiple of pi taken off, and arguments past the
    reduction's range (the library sinf there)."""
    vals = np.array([0.0, -0.0, 1e-30, -1e-30, 1.5707964, -3.1415927, 4.712389, -7.8539815,
                     1e4, -1e4, 99999.0, -99999.0, 3e5, -3e5, 1e30, -1e30], np.float32)
    x = np.tile(vals, (4, 1))[None].astype(np.float32)          # [1, 4, 16]
    al = np.array([1.0, 0.5, 2.0, 1.3], np.float32).reshape(1, 4, 1)
    rec = (np.float32(1) / al).astype(np.float32)
    env = {"x": gpu.to_device(x), "a": gpu.to_device(al), "r": gpu.to_device(rec),
           "two": gpu.to_device(np.array(2.0, np.float32))}
    for op, ins, out in [("Mul", ["a", "x"], "t"), ("Sin", ["t"], "s"),
                         ("Pow", ["s", "two"], "p"), ("Mul", ["r", "p"], "q"),
                         ("Add", ["x", "q"], "y")]:
        gpu.dispatch(op, ins, [out], {}, env)
    fused = gpu.ops.snake(env["x"], env["a"], env["r"]).numpy()
    assert_bitexact(fused, env["y"].numpy(), "fused snake vs node chain, edge arguments")


# ------------------------------------------------------- reference KATs
@pytest.mark.parametrize("case", KATS["binary_shape_cases"], ids=lambda c: c[0])
def test_kat_binary_shapes(gpu, oracle, case):
    op, ashape, bshape = case
    r = rng(1)
    lo, hi = KATS["operand_range"]
    a = r.uniform(lo, hi, ashape).astype(np.float32)
    b = np.asarray(r.uniform(lo, hi, bshape)).astype(np.float32)
    got = run_node(gpu, op, [a, b])
    assert_bitexact(got, oracle.binary(op, a, b), f"{op} {ashape}x{bshape}")


@pytest.mark.parametrize("case", KATS["unary_shape_cases"], ids=lambda c: c[0])
def test_kat_unary_shapes(gpu, oracle, case):
    op, shape = case
    lo, hi = KATS["operand_range"]
    x = rng(3).uniform(lo, hi, shape).astype(np.float32)
    got = run_node(gpu, op, [x])
    want = oracle.unary(op, x)
    assert_close(got, want, 0, KATS["abs_tolerance"], what=op)
    if op in ("Sqrt", "Floor"):
        assert_bitexact(got, want, op)


def test_kat_leaky_where(gpu):
    k = KATS["leaky_relu"]
    got = run_node(gpu, "LeakyRelu", [np.array(k["x"], np.float32)], {"alpha": k["alpha"]})
    assert_bitexact(got, np.array(k["want"], np.float32), "LeakyRelu KAT")
    k = KATS["where"]
    cond = np.array(k["cond"], np.float32) != 0
    got = run_node(gpu, "Where", [cond, np.array(k["x"], np.float32), np.array(k["y"], np.float32)])
    assert_bitexact(got, np.array(k["want"], np.float32), "Where KAT")


# ----------------------------------------------------- broader coverage
SHAPES = [
    ((3, 5, 7), (5, 1)), ((1, 64, 123), (1, 64, 1)), ((4, 1, 6), (1, 5, 1)),
    ((1000,), ()), ((2, 3, 4, 5, 6), (3, 1, 5, 1)), ((0, 4), (4,)), ((7, 9), (7, 9)),
]


@pytest.mark.parametrize("ashape,bshape", SHAPES)
@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div"])
def test_broadcast_bitexact(gpu, oracle, op, ashape, bshape):
    r = rng(5)
    a = r.normal(0, 1, ashape).astype(np.float32)
    b = np.asarray(r.uniform(0.5, 2, bshape)).astype(np.float32)
    assert_bitexact(run_node(gpu, op, [a, b]), oracle.binary(op, a, b), f"{op} {ashape} {bshape}")
    # operands swapped
    assert_bitexact(run_node(gpu, op, [b, a]), oracle.binary(op, b, a), f"{op} swapped")


@pytest.mark.parametrize("op", ["Exp", "Sin", "Cos", "Atan", "Tanh", "Sigmoid", "Sqrt", "Floor",
                                "Round"])
def test_unary_ops(gpu, oracle, op):
    r = rng(6)
    x = r.normal(0, 3, (1, 37, 301)).astype(np.float32)
    if op == "Sqrt":
        x = np.abs(x)
    got = run_node(gpu, op, [x])
    want = oracle.unary(op, x)
    if op in ("Sqrt", "Floor", "Round"):
        assert_bitexact(got, want, op)
    else:
        assert_close(got, want, 1e-5, floor_rel=1e-7, what=op)


def test_pow_and_fp16_storage(gpu, oracle):
    r = rng(7)
    x = r.normal(0, 2, (64, 33)).astype(np.float32)
    two = np.array(2.0, np.float16)  # the graph's Pow exponent is an fp16 constant
    assert_close(run_node(gpu, "Pow", [x, two]), oracle.binary("Pow", x, two), 1e-6,
                 what="Pow 2")
    e = r.uniform(0.5, 3, (64, 33)).astype(np.float32)
    ax = np.abs(x)
    assert_close(run_node(gpu, "Pow", [ax, e]), oracle.binary("Pow", ax, e), 1e-5,
                 floor_rel=1e-7, what="Pow")
    # negative bases with integer exponents (elementwise.glsl:117-126)
    ints = np.array([3.0, 2.0, 1.0, 0.0, -1.0], np.float32)
    neg = -np.abs(r.normal(0, 2, 5)).astype(np.float32)
    assert_close(run_node(gpu, "Pow", [neg, ints]), oracle.binary("Pow", neg, ints), 1e-6,
                 what="Pow negative base")
    h = r.normal(0, 1, (8, 40)).astype(np.float16)
    assert_bitexact(run_node(gpu, "Add", [h, x[:8, :1]]), oracle.binary("Add", h, x[:8, :1]),
                    "fp16 + fp32")


def test_integer_arithmetic(gpu, oracle):
    a = np.array([[7, -7, 7, -7, 0, 9]], np.int64)
    b = np.array([[2, 2, -2, -2, 3, 1]], np.int64)
    for op in ("Add", "Sub", "Mul", "Div"):
        env = {"a": gpu.to_device(a), "b": gpu.to_device(b)}
        gpu.dispatch(op, ["a", "b"], ["c"], {}, env)
        assert_bitexact(env["c"].numpy(), oracle.binary(op, a, b), f"int64 {op}")


def test_comparisons_where_clip(gpu, oracle):
    r = rng(8)
    x = r.normal(0, 1, (5, 40)).astype(np.float32)
    y = r.normal(0, 1, (40,)).astype(np.float32)
    for op in ("Greater", "Less", "GreaterOrEqual", "Equal"):
        assert_bitexact(run_node(gpu, op, [x, y]), oracle_node(oracle, op, [x, y]), op)
    assert_bitexact(run_node(gpu, "Equal", [x, x]), np.ones_like(x, bool), "Equal self")
    c = x > 0
    assert_bitexact(run_node(gpu, "And", [c, y > 0]), np.logical_and(c, y > 0), "And")
    assert_bitexact(run_node(gpu, "Where", [c, x, y]), oracle.where(c, x, y), "Where")
    lo, hi = np.array(-0.5, np.float32), np.array(0.7, np.float32)
    assert_bitexact(run_node(gpu, "Clip", [x, lo, hi]), oracle_node(oracle, "Clip", [x, lo, hi]),
                    "Clip")
    assert_bitexact(run_node(gpu, "Clip", [x, None, hi]),
                    oracle_node(oracle, "Clip", [x, None, hi]), "Clip hi")


def test_strided_and_misaligned_inputs(gpu, oracle):
    r = rng(9)
    x = r.normal(0, 1, (6, 50)).astype(np.float32)
    y = r.normal(0, 1, (50, 6)).astype(np.float32)
    dx = gpu.to_device(x)
    dy = gpu.to_device(y)
    # transposed view operand
    out = gpu.ops.binary("Add", dx, dy.transpose()).numpy()
    assert_bitexact(out, x + y.T, "transposed operand")
    # view at an element offset (not 16-byte aligned): scalar path
    sub = dx.slice_axis(1, 1, 49)
    out = gpu.ops.binary("Mul", sub, sub).numpy()
    assert_bitexact(out, x[:, 1:49] * x[:, 1:49], "misaligned view")
    # reversed view
    rev = dx.slice_axis(1, 49, -1, -1)
    out = gpu.ops.unary("LeakyRelu", rev, np.float32(0.2)).numpy()
    assert_bitexact(out, oracle.unary("LeakyRelu", x[:, ::-1], 0.2), "reversed view")


def test_fast_gelu(gpu, oracle):
    r = rng(10)
    x = r.normal(0, 2, (1, 256, 2048)).astype(np.float32)
    b = r.normal(0, 0.5, (2048,)).astype(np.float32)
    assert_close(run_node(gpu, "FastGelu", [x, b]), oracle.fast_gelu(x, b), 1e-5, floor_rel=1e-7,
                 what="FastGelu bias")
    assert_close(run_node(gpu, "FastGelu", [x]), oracle.fast_gelu(x), 1e-5, floor_rel=1e-7,
                 what="FastGelu")


def test_dequantize(gpu, oracle):
    r = rng(11)
    q = r.integers(-127, 128, (768, 512)).astype(np.int8)
    s = r.uniform(1e-3, 1e-2, 512).astype(np.float32)
    zp = r.integers(-5, 5, 512).astype(np.int8)
    assert_bitexact(run_node(gpu, "DequantizeLinear", [q, s, zp]), oracle.dequantize(q, s, zp),
                    "dequant per column")
    u = r.integers(0, 256, (64, 64, 3)).astype(np.uint8)
    assert_bitexact(run_node(gpu, "DequantizeLinear", [u, np.float32(0.004), np.uint8(114)]),
                    oracle.dequantize(u, np.float32(0.004), np.uint8(114)), "dequant u8 zp")


# ------------------------------------------------------------- casts
def test_casts(gpu, oracle):
    r = rng(12)
    x = (r.normal(0, 50, (3, 333))).astype(np.float32)
    for to, name in ((7, "int64"), (6, "int32"), (9, "bool"), (1, "f32"), (10, "f16->f32")):
        got = run_node(gpu, "Cast", [x], {"to": to})
        assert_bitexact(got, oracle_node(oracle, "Cast", [x], {"to": to}), f"Cast {name}")
    i = r.integers(-1000, 1000, (7, 11)).astype(np.int64)
    assert_bitexact(run_node(gpu, "Cast", [i], {"to": 1}), i.astype(np.float32), "Cast i64->f32")
    h = r.normal(0, 1, (5, 9)).astype(np.float16)
    assert_bitexact(run_node(gpu, "Cast", [h], {"to": 1}), h.astype(np.float32), "Cast f16->f32")


# ------------------------------------------------------ indexing ops
def test_transpose_slice_concat_split(gpu, oracle):
    r = rng(13)
    x = r.normal(0, 1, (2, 12, 30)).astype(np.float32)
    t = run_node(gpu, "Transpose", [x], {"perm": [0, 2, 1]})
    assert_bitexact(t, np.transpose(x, (0, 2, 1)), "Transpose")
    for s, e, a, st in (([1, 3], [10, -2], [1, 2], [3, 2]), ([-1], [0], [2], [-1]),
                        ([5], [100], [1], [1]), ([0], [-100], [2], [-1])):
        ins = [x, ("host", np.array(s)), ("host", np.array(e)), ("host", np.array(a)),
               ("host", np.array(st))]
        got = run_node(gpu, "Slice", ins)
        assert_bitexact(got, oracle_node(oracle, "Slice", ins), f"Slice {s},{e},{a},{st}")
    y = r.normal(0, 1, (2, 5, 30)).astype(np.float32)
    h = r.normal(0, 1, (2, 3, 30)).astype(np.float16)
    got = run_node(gpu, "Concat", [x, y, h], {"axis": 1})
    assert_bitexact(got, oracle_node(oracle, "Concat", [x, y, h], {"axis": 1}), "Concat")
    parts = run_node(gpu, "Split", [x, ("host", np.array([5, 7]))], {"axis": 1}, nout=2)
    want = oracle_node(oracle, "Split", [x, ("host", np.array([5, 7]))], {"axis": 1}, nout=2)
    for g, w in zip(parts, want):
        assert_bitexact(g, w, "Split")
    parts = run_node(gpu, "Split", [x], {"axis": 2}, nout=4)
    want = oracle_node(oracle, "Split", [x], {"axis": 2}, nout=4)
    for g, w in zip(parts, want):
        assert_bitexact(g, w, "Split equal")


def test_gather_expand_reshape(gpu, oracle):
    r = rng(14)
    emb = r.integers(-127, 128, (178, 128)).astype(np.int8)
    ids = np.concatenate([[0], r.integers(1, 178, 128), [0]]).reshape(1, -1).astype(np.int64)
    got = run_node(gpu, "Gather", [emb, ("host", ids)], {"axis": 0})
    assert_bitexact(got, oracle_node(oracle, "Gather", [emb, ("host", ids)], {"axis": 0}),
                    "Gather embedding")
    x = r.normal(0, 1, (4, 6, 5)).astype(np.float32)
    idx = np.array([[-1, 0], [2, 5]], np.int64)
    got = run_node(gpu, "Gather", [x, ("host", idx)], {"axis": 1})
    assert_bitexact(got, np.take(x, idx, axis=1), "Gather negative index")
    with pytest.raises(IndexError):
        run_node(gpu, "Gather", [x, ("host", np.array([6]))], {"axis": 1})
    c = r.normal(0, 1, (1, 6, 1)).astype(np.float32)
    got = run_node(gpu, "Expand", [c, ("host", np.array([3, 6, 4]))])
    assert_bitexact(got, np.broadcast_to(c, (3, 6, 4)), "Expand")
    t = run_node(gpu, "Reshape", [x, ("host", np.array([0, -1]))])
    assert_bitexact(t, x.reshape(4, 30), "Reshape")
    u = run_node(gpu, "Unsqueeze", [x, ("host", np.array([0, 3]))])
    assert_bitexact(u, x.reshape(1, 4, 6, 1, 5), "Unsqueeze")
    fill = run_node(gpu, "ConstantOfShape", [("host", np.array([2, 3]))],
                    {"value": np.array([1.5], np.float32)})
    assert_bitexact(fill, np.full((2, 3), 1.5, np.float32), "ConstantOfShape")


def test_empty_and_scalar(gpu, oracle):
    e = np.zeros((0, 5), np.float32)
    assert run_node(gpu, "Add", [e, np.ones(5, np.float32)]).shape == (0, 5)
    s = np.array(3.0, np.float32)
    assert_bitexact(run_node(gpu, "Mul", [s, s]), np.array(9.0, np.float32), "scalar")


@pytest.mark.parametrize("case", ["add_per_channel", "mul_full", "snake", "rank1", "sub_scalar"])
def test_odd_rows_flat_path(gpu, oracle, case):
    """Rows whose length is not a multiple of 4 (the decoder's odd time axes)
    go through the flat float4 walk; items straddle row ends."""
    r = rng(31)
    if case == "add_per_channel":
        ins = [r.normal(0, 1, (1, 128, 4097)), r.normal(0, 1, (1, 128, 1))]
        op = "Add"
    elif case == "mul_full":
        ins = [r.normal(0, 1, (1, 3, 100003)), r.normal(0, 1, (1, 3, 100003))]
        op = "Mul"
    elif case == "snake":
        x = r.normal(0, 1, (1, 64, 5001)).astype(np.float32)
        a = r.uniform(0.5, 2, (1, 64, 1)).astype(np.float32)
        rec = (np.float32(1) / a).astype(np.float32)
        got = gpu.ops.snake(gpu.to_device(x), gpu.to_device(a), gpu.to_device(rec)).numpy()
        assert_close(got, oracle.snake(x, a, rec), 1e-5, floor_rel=1e-6, what="snake odd rows")
        return
    elif case == "rank1":
        ins = [r.normal(0, 1, 10007), r.normal(0, 1, 10007)]
        op = "Sub"
    else:
        ins = [r.normal(0, 1, (2, 9, 999)), np.array(1.5)]
        op = "Div"
    ins = [np.asarray(v, np.float32) for v in ins]
    got = gpu.ops.binary(op, *[gpu.to_device(v) for v in ins]).numpy()
    assert_bitexact(got, oracle.binary(op, *ins), f"{op} {case}")
