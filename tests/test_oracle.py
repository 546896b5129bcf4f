"""Pins the CPU oracle (oracle/ref_ops.py) against checks that do not
restate its formulas: the reference's known answers, brute-force loops,
float64 closed forms, torch's CPU ops, invariants and identities.  A few
tests plant a plausible mistake in a copy of an oracle function and show the
same check catches it.  CPU only."""
import json
import math
import os

import numpy as np
import pytest
import torch

from conftest import assert_bitexact, assert_close, rng

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "elementwise_kats.json")))


# --------------------------------------------------------- reference KATs
def _walk_expected(op, ashape, a, bshape, b, oshape):
    """Independent broadcast: unravel each output index and pick each operand
    element by coordinate (tests/test_gpu_elementwise.gd:64-95)."""
    n = int(np.prod(oshape)) if oshape else 1
    out = np.empty(n, dtype=np.float32)
    fa, fb = a.reshape(-1), b.reshape(-1)

    def pick(shape, data, coord):
        if not shape:
            return data[0]
        pad = len(coord) - len(shape)
        idx = 0
        for d, sd in enumerate(shape):
            c = 0 if sd == 1 else coord[pad + d]
            idx = idx * sd + c
        return data[idx]

    for i in range(n):
        coord, rem = [0] * len(oshape), i
        for d in range(len(oshape) - 1, -1, -1):
            coord[d] = rem % oshape[d]
            rem //= oshape[d]
        x, y = pick(ashape, fa, coord), pick(bshape, fb, coord)
        out[i] = {"Add": lambda: x + y, "Sub": lambda: x - y, "Mul": lambda: x * y,
                  "Div": lambda: x / y}[op]()
    return out.reshape(oshape)


@pytest.mark.parametrize("case", KATS["binary_shape_cases"], ids=lambda c: c[0])
def test_kat_broadcast_shapes(oracle, case):
    op, ashape, bshape = case
    r = rng(1)
    lo, hi = KATS["operand_range"]
    a = r.uniform(lo, hi, ashape).astype(np.float32)
    b = r.uniform(lo, hi, bshape).astype(np.float32)
    got = oracle.binary(op, a, b)
    oshape = list(np.broadcast_shapes(tuple(ashape), tuple(bshape)))
    want = _walk_expected(op, ashape, a, bshape, b, oshape)
    # np.float32 scalar ops are the same IEEE single operations: bit-exact.
    assert_bitexact(np.asarray(got, np.float32), want, f"{op} {ashape}x{bshape}")


def test_kat_leaky_relu(oracle):
    k = KATS["leaky_relu"]
    got = oracle.unary("LeakyRelu", np.array(k["x"], np.float32), k["alpha"])
    assert_close(got, np.array(k["want"], np.float32), 0, KATS["abs_tolerance"], what="LeakyRelu")
    assert_bitexact(got, np.array(k["want"], np.float32), "LeakyRelu")


def test_kat_where(oracle):
    k = KATS["where"]
    got = oracle.where(np.array(k["cond"], np.float32) != 0, np.array(k["x"], np.float32),
                       np.array(k["y"], np.float32))
    assert_bitexact(got.astype(np.float32), np.array(k["want"], np.float32), "Where")


# ------------------------------------------------------ float64 closed forms
UNARY64 = {
    "Sqrt": np.sqrt, "Exp": np.exp, "Sin": np.sin, "Cos": np.cos, "Atan": np.arctan,
    "Tanh": np.tanh, "Sigmoid": lambda v: 1.0 / (1.0 + np.exp(-v)),
}


@pytest.mark.parametrize("op", sorted(UNARY64))
def test_unary_float64(oracle, op):
    r = rng(2)
    x = r.normal(0, 3, 20000).astype(np.float32)
    if op == "Sqrt":
        x = np.abs(x)
    got = oracle.unary(op, x).astype(np.float64)
    want = UNARY64[op](x.astype(np.float64))
    # Within 4 ulp of the float32-rounded exact value.
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * ulp + 1e-45), op


def test_unary_exact_ops(oracle):
    x = np.array([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.7, -3.7], np.float32)
    # half-to-even, keeping the sign of zero
    want_round = np.array([-2.0, -2.0, -0.0, 0.0, 2.0, 2.0, 4.0, -4.0], np.float32)
    assert_bitexact(oracle.unary("Round", x), want_round, "Round")
    want_floor = np.array([-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0, -4.0], np.float32)
    assert_bitexact(oracle.unary("Floor", x), want_floor, "Floor")


def test_snake_closed_form(oracle):
    r = rng(3)
    x = r.normal(0, 1, (1, 64, 300)).astype(np.float32)
    alpha = r.uniform(0.5, 2, (1, 64, 1)).astype(np.float32)
    got = oracle.snake(x, alpha)
    xd, ad = x.astype(np.float64), alpha.astype(np.float64)
    want = xd + np.sin(ad * xd) ** 2 / ad
    # Cancellation near x = -sin^2(ax)/a needs an absolute floor.
    assert_close(got, want, 1e-5, floor_rel=1e-6, what="snake")
    # The recip form (the graph's folded 1/alpha constant) agrees too.
    rec = (1.0 / alpha).astype(np.float32)
    assert_close(oracle.snake(x, alpha, rec), want, 1e-5, floor_rel=1e-6, what="snake recip")


def test_fast_gelu_closed_form(oracle):
    r = rng(4)
    x = r.normal(0, 2, 5000).astype(np.float32)
    b = r.normal(0, 1, 5000).astype(np.float32)
    u = x.astype(np.float64) + b
    want = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
    assert_close(oracle.fast_gelu(x, b), want, 1e-5, floor_rel=1e-7, what="fast_gelu")


# ----------------------------------------------------------- reductions
def test_reduce_mean_float64(oracle):
    r = rng(5)
    x = r.normal(0, 1, (2, 64, 1000)).astype(np.float32)
    for axes in ([2], [0], [1, 2], None):
        got = oracle.reduce("ReduceMean", x, axes)
        want = x.astype(np.float64).mean(axis=None if axes is None else tuple(axes),
                                         keepdims=True)
        assert_close(got, want, 1e-5, floor_rel=1e-6, what=f"mean {axes}")
        got = oracle.reduce("ReduceSum", x, axes, keepdims=False)
        want = x.astype(np.float64).sum(axis=None if axes is None else tuple(axes))
        assert_close(got, want, 1e-5, floor_rel=1e-6, what=f"sum {axes}")


def test_softmax_torch_and_invariant(oracle):
    r = rng(6)
    x = r.normal(0, 2, (2, 3, 16, 64)).astype(np.float32)
    got = oracle.softmax(x, -1)
    want = torch.softmax(torch.from_numpy(x).double(), -1).numpy()
    assert_close(got, want, 1e-5, floor_rel=1e-7, what="softmax")
    assert np.allclose(got.sum(-1), 1.0, atol=1e-5)
    got1 = oracle.softmax(x, 1)
    want1 = torch.softmax(torch.from_numpy(x).double(), 1).numpy()
    assert_close(got1, want1, 1e-5, floor_rel=1e-7, what="softmax axis 1")


def test_layernorm_torch(oracle):
    r = rng(7)
    x = r.normal(0, 1, (1, 32, 768)).astype(np.float32)
    g = (1 + 0.1 * r.normal(0, 1, 768)).astype(np.float32)
    b = (0.1 * r.normal(0, 1, 768)).astype(np.float32)
    for eps in (1e-5, 1e-12):
        got = oracle.layernorm(x, g, b, -1, eps)
        want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,),
                                              torch.from_numpy(g).double(),
                                              torch.from_numpy(b).double(), eps).numpy()
        assert_close(got, want, 1e-4, 1e-5, what=f"layernorm eps={eps}")
    # invariant: gamma 1, beta 0 gives zero mean / unit variance rows
    y = oracle.layernorm(x, np.ones(768, np.float32), None, -1, 1e-12).astype(np.float64)
    assert np.abs(y.mean(-1)).max() < 1e-5 and np.abs(y.var(-1) - 1).max() < 1e-4


def test_skip_layernorm(oracle):
    r = rng(8)
    x, s = (r.normal(0, 1, (1, 8, 64)).astype(np.float32) for _ in range(2))
    g = np.ones(64, np.float32)
    bias = r.normal(0, 1, 64).astype(np.float32)
    got = oracle.skip_layernorm(x, s, g, None, bias, 1e-12)
    tot = x.astype(np.float64) + s + bias
    want = torch.nn.functional.layer_norm(torch.from_numpy(tot), (64,), eps=1e-12).numpy()
    assert_close(got, want, 1e-4, 1e-5, what="skip layernorm")


def test_instance_norm_torch(oracle):
    r = rng(9)
    c, t = 32, 1200
    x = r.normal(0, 1, (1, c, t)).astype(np.float32)
    gamma = r.normal(0, 0.2, (1, c, 1)).astype(np.float32)
    beta = r.normal(0, 0.2, (1, c, 1)).astype(np.float32)
    got = oracle.instance_norm_affine(x, gamma, beta, 1e-5)
    tx = torch.from_numpy(x).double()
    norm = torch.nn.functional.instance_norm(tx, eps=1e-5).numpy()
    want = norm * (1 + gamma.astype(np.float64)) + beta
    assert_close(got, want, 1e-4, 1e-5, what="instance norm")


def test_adain_matches_torch_linear(oracle):
    r = rng(10)
    c, t, s = 64, 600, 128
    x = r.normal(0, 1, (1, c, t)).astype(np.float32)
    style = r.normal(0, 0.1, (1, s)).astype(np.float32)
    w = r.normal(0, 0.05, (s, 2 * c)).astype(np.float32)
    b = r.normal(0, 0.05, 2 * c).astype(np.float32)
    got = oracle.adain(x, style, w, b, 1e-5)
    h = torch.from_numpy(style).double() @ torch.from_numpy(w).double() + torch.from_numpy(b).double()
    gamma = h[:, :c].reshape(1, c, 1)
    beta = h[:, c:].reshape(1, c, 1)
    norm = torch.nn.functional.instance_norm(torch.from_numpy(x).double(), eps=1e-5)
    want = (norm * (1 + gamma) + beta).numpy()
    assert_close(got, want, 1e-4, 1e-5, what="adain")


def _one_pass_instance_norm(x, eps):
    """A plausible mistake: variance as E[x^2] - E[x]^2."""
    x = x.astype(np.float32)
    mu = x.mean(-1, keepdims=True)
    var = (x * x).mean(-1, keepdims=True) - mu * mu
    return (x - mu) / np.sqrt(var + eps)


def test_variance_is_two_pass(oracle):
    """A large common offset: the two-pass oracle keeps unit variance, a
    one-pass E[x^2]-E[x]^2 does not -- so the check pins the two-pass form."""
    r = rng(11)
    x = (1e4 + r.normal(0, 1, (1, 8, 4096))).astype(np.float32)
    zero = np.zeros((1, 8, 1), np.float32)
    y = oracle.instance_norm_affine(x, zero, zero, 1e-5).astype(np.float64)
    assert np.abs(y.var(-1) - 1).max() < 1e-3
    bad = _one_pass_instance_norm(x, 1e-5).astype(np.float64)
    assert not (np.abs(bad.var(-1) - 1).max() < 1e-3)


# --------------------------------------------------------- contractions
def test_matmul_float64(oracle):
    r = rng(12)
    a = r.normal(0, 1, (3, 64, 96)).astype(np.float32)
    w = r.normal(0, 0.05, (96, 80)).astype(np.float16)
    got = oracle.matmul(a, w)
    want = a.astype(np.float64) @ w.astype(np.float64)
    assert_close(got, want, 1e-4, 1e-5, what="matmul f16 weight")
    got = oracle.fused_matmul(a, a, trans_b=1, alpha=0.125)
    want = (a.astype(np.float64) @ np.swapaxes(a, -1, -2).astype(np.float64)) * 0.125
    assert_close(got, want, 1e-4, 1e-5, what="fused matmul")


def test_dequantize_exact(oracle):
    q = np.arange(-127, 128, dtype=np.int8)
    s = np.float32(0.0037)
    got = oracle.dequantize(q, s)
    assert_bitexact(got, (q.astype(np.float64) * np.float64(s)).astype(np.float32), "dequant")
    zp = np.int8(3)
    got = oracle.dequantize(q, s, zp)
    assert_bitexact(got, ((q.astype(np.float64) - 3) * np.float64(s)).astype(np.float32), "dequant zp")


def _conv_loops(x, w, b, p0, p1, s, d, g):
    n, cin, L = x.shape
    cout, cing, k = w.shape
    lout = (L + p0 + p1 - d * (k - 1) - 1) // s + 1
    out = np.zeros((n, cout, lout))
    coutg = cout // g
    for bi in range(n):
        for co in range(cout):
            gi = co // coutg
            for l in range(lout):
                acc = 0.0
                for ci in range(cing):
                    for kk in range(k):
                        pos = l * s + kk * d - p0
                        if 0 <= pos < L:
                            acc += float(w[co, ci, kk]) * float(x[bi, gi * cing + ci, pos])
                out[bi, co, l] = acc + (float(b[co]) if b is not None else 0.0)
    return out


def _convt_loops(x, w, b, p0, p1, s, d, g, op):
    n, cin, L = x.shape
    _, coutg, k = w.shape
    cout = coutg * g
    cing = cin // g
    lfull = (L - 1) * s + d * (k - 1) + 1 + op
    acc = np.zeros((n, cout, lfull))
    for bi in range(n):
        for ci in range(cin):
            gi = ci // cing
            for co in range(coutg):
                for l in range(L):
                    for kk in range(k):
                        acc[bi, gi * coutg + co, l * s + kk * d] += float(x[bi, ci, l]) * float(w[ci, co, kk])
    out = acc[:, :, p0:lfull - p1]
    if b is not None:
        out = out + b.reshape(1, -1, 1)
    return out


CONV_CASES = [  # (cin, cout, k, L, p0, p1, s, d, g)
    (3, 4, 3, 11, 1, 1, 1, 1, 1),
    (4, 6, 5, 13, 2, 2, 1, 3, 1),
    (4, 4, 3, 12, 1, 0, 2, 1, 2),
    (6, 6, 3, 9, 1, 1, 1, 1, 6),
    (2, 3, 12, 30, 0, 0, 6, 1, 1),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv1d_loops_and_torch(oracle, case):
    cin, cout, k, L, p0, p1, s, d, g = case
    r = rng(13)
    x = r.normal(0, 1, (2, cin, L)).astype(np.float32)
    w = r.normal(0, 0.3, (cout, cin // g, k)).astype(np.float32)
    b = r.normal(0, 0.1, cout).astype(np.float32)
    got = oracle.conv1d(x, w, b, (p0, p1), s, d, g)
    assert_close(got, _conv_loops(x, w, b, p0, p1, s, d, g), 1e-5, 1e-6, what="conv loops")
    xt = torch.nn.functional.pad(torch.from_numpy(x).double(), (p0, p1))
    want = torch.nn.functional.conv1d(xt, torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                                      stride=s, dilation=d, groups=g).numpy()
    assert_close(got, want, 1e-5, 1e-6, what="conv torch")


CONVT_CASES = [  # (cin, cout, k, L, p0, p1, s, d, g, output_padding)
    (4, 3, 20, 7, 5, 5, 10, 1, 1, 0),
    (3, 2, 12, 9, 3, 3, 6, 1, 1, 0),
    (4, 4, 3, 8, 1, 1, 2, 1, 4, 1),
    (2, 3, 5, 6, 0, 0, 1, 2, 1, 0),
    (2, 1, 20, 5, 0, 0, 5, 1, 1, 0),
]


@pytest.mark.parametrize("case", CONVT_CASES)
def test_conv_transpose_loops_and_torch(oracle, case):
    cin, cout, k, L, p0, p1, s, d, g, op = case
    r = rng(14)
    x = r.normal(0, 1, (2, cin, L)).astype(np.float32)
    w = r.normal(0, 0.3, (cin, cout, k)).astype(np.float32)
    b = r.normal(0, 0.1, cout * g).astype(np.float32)
    got = oracle.conv_transpose1d(x, w, b, (p0, p1), s, d, g, op)
    assert_close(got, _convt_loops(x, w, b, p0, p1, s, d, g, op), 1e-5, 1e-6, what="convT loops")
    if p0 == p1:
        want = torch.nn.functional.conv_transpose1d(
            torch.from_numpy(x).double(), torch.from_numpy(w).double(),
            torch.from_numpy(b).double(), stride=s, padding=p0, output_padding=op, groups=g,
            dilation=d).numpy()
        assert_close(got, want, 1e-5, 1e-6, what="convT torch")


def test_conv_adjoint_identity(oracle):
    """<conv(x), y> == <x, convT(y)> with the same weights, stride, padding."""
    r = rng(15)
    cin, cout, k, L, s, p = 5, 7, 4, 23, 2, 1
    x = r.normal(0, 1, (1, cin, L)).astype(np.float32)
    w = r.normal(0, 0.3, (cout, cin, k)).astype(np.float32)
    cx = oracle.conv1d(x, w, None, (p, p), s)
    y = r.normal(0, 1, cx.shape).astype(np.float32)
    # convT of y with w viewed as [cout(in), cin(out), k]; output_padding
    # restores the input length lost to the stride.
    lfull = (cx.shape[2] - 1) * s + k - 2 * p
    op = L - lfull
    ty = oracle.conv_transpose1d(y, w, None, (p, p), s, 1, 1, op)
    lhs = float((cx.astype(np.float64) * y).sum())
    rhs = float((x.astype(np.float64) * ty).sum())
    assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs))


def test_delta_kernel_shifts(oracle):
    x = rng(16).normal(0, 1, (1, 1, 10)).astype(np.float32)
    w = np.zeros((1, 1, 3), np.float32)
    w[0, 0, 2] = 1.0
    got = oracle.conv1d(x, w, None, (1, 1))
    assert_bitexact(got[0, 0, :-1], x[0, 0, 1:], "delta shift")
    wt = np.zeros((1, 1, 4), np.float32)
    wt[0, 0, 0] = 1.0
    up = oracle.conv_transpose1d(x, wt, None, (0, 0), 4)
    assert_bitexact(up[0, 0, ::4], x[0, 0], "convT delta upsample")


def _convt_swapped_pads(x, w, pads, s):
    """A plausible mistake: crop with p0 and p1 exchanged."""
    from oracle import ref_ops
    return ref_ops.conv_transpose1d(x, w, None, (pads[1], pads[0]), s)


def test_planted_pad_swap_is_caught():
    r = rng(17)
    x = r.normal(0, 1, (1, 2, 6)).astype(np.float32)
    w = r.normal(0, 1, (2, 2, 8)).astype(np.float32)
    bad = _convt_swapped_pads(x, w, (1, 3), 4)
    good = _convt_loops(x, w, None, 1, 3, 4, 1, 1, 0)
    assert bad.shape == good.shape
    assert np.abs(bad - good).max() > 1e-3


# ------------------------------------------------------------------ pool
def test_bucket_properties(oracle):
    prev = 0
    for n in list(range(0, 20000, 7)) + [1 << 20, (1 << 20) + 1, 10 ** 8]:
        b = oracle.bucket(n)
        assert b >= max(n, 256) and b % 256 == 0
        assert b >= prev
        prev = b
        if b > 4096:
            m = b >> (b.bit_length() - 4)
            assert m << (b.bit_length() - 4) == b, "at most four significant bits"
            # Rounding to 2^(bits-4) granules costs under 1/8 of the size
            # (the reference's comment says ~6%; the rule itself allows 12.5%).
            assert b < max(n, 256) * 1.125 + 256


# -------------------------------------------------- dispatch conventions
def test_dispatch_slice_split_concat(oracle):
    x = np.arange(2 * 5 * 7, dtype=np.float32).reshape(2, 5, 7)
    env = {"x": x, "s": np.array([1, -1]), "e": np.array([4, 0]), "a": np.array([1, 2]),
           "st": np.array([2, -2])}
    oracle.dispatch("Slice", ["x", "s", "e", "a", "st"], ["y"], {}, env)
    assert_bitexact(env["y"], x[:, 1:4:2, 6:0:-2], "slice")
    # op_slice clamps a far negative end to -1 and hands it to a python
    # slice, where -1 means "the last element": the selection is empty
    # (ref_runtime.py:321-324).  The drop-in keeps that behaviour.
    env["e2"] = np.array([4, -100])
    oracle.dispatch("Slice", ["x", "s", "e2", "a", "st"], ["y2"], {}, env)
    assert env["y2"].shape == (2, 2, 0)
    env["sp"] = np.array([2, 5])
    oracle.dispatch("Split", ["x", "sp"], ["p0", "p1"], {"axis": 2}, env)
    assert_bitexact(env["p0"], x[:, :, :2], "split0")
    assert_bitexact(env["p1"], x[:, :, 2:], "split1")
    oracle.dispatch("Concat", ["p1", "p0"], ["c"], {"axis": 2}, env)
    assert_bitexact(env["c"], np.concatenate([x[:, :, 2:], x[:, :, :2]], 2), "concat")
