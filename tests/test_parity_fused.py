"""Parity of the fused graph chains with the node chains they replace, run
node by node through the oracle, at decoder sizes.

Each case builds the chain as graph nodes, lets the fusion pass rewrite it
(so the test covers the matcher as well as the kernel) and compares the
fused launch with the oracle's chain.  Bars: the quantised conv and
Linear tails bit-exact (integer arithmetic, then the chain's own Cast, Mul
and Add); the
InstanceNorm chain bit-exact (its sums follow numpy's summation order, the
rest are correctly rounded IEEE operations); the snake chain at the
elementwise bar rel 1e-5 (+1e-6 max|ref|: sin differs by ulps between numpy
and the device)."""
import importlib

import numpy as np
import pytest

from conftest import assert_bitexact, assert_close, rng

pytestmark = pytest.mark.gpu


def run_chain(gpu, oracle, nodes, inputs, weights, out):
    """Runs `nodes` (op, ins, outs, attrs) through the fusion pass and the
    device dispatch, and through the oracle unfused; returns (device result,
    oracle result, fused node list)."""
    fz = importlib.import_module("best-tts-godot_amd.fuse")
    dev_w = {}
    for k, v in weights.items():  # fp16 widened at upload, as PackedGraph does
        v = np.asarray(v)
        v = v.astype(np.float32) if v.dtype == np.float16 else v
        t = gpu.to_device(v)
        if v.size <= 16:
            t.host = v
        dev_w[k] = t
    fused, _groups = fz.fuse(nodes, dev_w, {out})
    env = dict(dev_w)
    env.update({k: gpu.to_device(np.asarray(v)) for k, v in inputs.items()})
    for op, ins, outs, at in fused:
        gpu.dispatch(op, ins, outs, at, env)
    oenv = {k: np.asarray(v) for k, v in {**weights, **inputs}.items()}
    for op, ins, outs, at in nodes:
        oracle.dispatch(op, ins, outs, at, oenv)
    return gpu.to_host(env[out]), oenv[out], fused


@pytest.mark.parametrize("cin,cout,k,L,pad,bias", [(128, 128, 7, 3000, 3, True),
                                                   (256, 256, 11, 900, 5, True),
                                                   (96, 40, 3, 257, 1, False)])
def test_qconv_tail(gpu, oracle, cin, cout, k, L, pad, bias):
    r = rng(21)
    x = r.integers(0, 256, (1, cin, L)).astype(np.uint8)
    w = r.integers(0, 256, (cout, cin, k)).astype(np.uint8)
    inputs = {"x": x, "xz": np.array(113, np.uint8),
              "b": r.integers(-3000, 3000, (1, cout, 1)).astype(np.int32),
              "s": np.array(3.1e-5, np.float32)}
    weights = {"w": w, "wz": np.array(71, np.uint8)}
    at = {"pads": [pad, pad], "dilations": [1], "strides": [1], "group": 1, "kernel_shape": [k]}
    nodes = [("ConvInteger", ["x", "w", "xz", "wz"], ["acc"], at)]
    last = "acc"
    if bias:
        nodes.append(("Add", ["acc", "b"], ["accb"], {}))
        last = "accb"
    nodes += [("Cast", [last], ["f"], {"to": 10}), ("Mul", ["f", "s"], ["y"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "y")
    assert [n[0] for n in fused] == ["QConvScaled"]
    assert_bitexact(got, want.astype(np.float32), f"QConvScaled {cin}->{cout} k{k}")


@pytest.mark.parametrize("M,K,N,wdt,per_col,bias", [(130, 768, 768, np.int8, True, True),
                                                    (130, 2048, 768, np.uint8, False, True),
                                                    (37, 100, 9, np.int8, True, False),
                                                    (256, 768, 2048, np.uint8, True, True)])
def test_qmatmul_tail(gpu, oracle, M, K, N, wdt, per_col, bias):
    """MatMulInteger -> Cast(float) -> Mul(scale) (-> Add(bias)), the
    quantised Linear of the text encoder and predictors, as one launch: the
    same bits as the chain (exact integer sums, then the chain's Mul and
    Add, each rounded once)."""
    r = rng(27)
    a = r.integers(0, 256, (1, M, K)).astype(np.uint8)
    w = (r.integers(-128, 128, (K, N)) if wdt == np.int8 else r.integers(0, 256, (K, N))).astype(wdt)
    s = (r.uniform(1e-4, 1e-3, (N,)) if per_col else np.array(3.7e-4)).astype(np.float32)
    inputs = {"a": a, "az": np.array(121, np.uint8), "s": s}
    weights = {"w": w, "wz": np.array(0 if wdt == np.int8 else 131, wdt),
               "b": r.normal(0, 1, (N,)).astype(np.float32)}
    nodes = [("MatMulInteger", ["a", "w", "az", "wz"], ["acc"], {}),
             ("Cast", ["acc"], ["f"], {"to": 1}), ("Mul", ["f", "s"], ["y"], {})]
    last = "y"
    if bias:
        nodes.append(("Add", ["y", "b"], ["z"], {}))
        last = "z"
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, last)
    assert [n[0] for n in fused] == ["QMatMulScaled"]
    assert_bitexact(got, want.astype(np.float32), f"QMatMulScaled {M}x{K}x{N}")


@pytest.mark.parametrize("per_col", [True, False])
def test_qmatmul_tail_scale_product(gpu, oracle, per_col):
    """The graph's form: the Linear's scale is Mul(activation scale, weight
    scale), read by the chain alone, and folds in with it; the epilogue forms
    the product (rounded once) before scaling, the same bits as the chain."""
    r = rng(29)
    M, K, N = 130, 512, 640
    a = r.integers(0, 256, (1, M, K)).astype(np.uint8)
    inputs = {"a": a, "az": np.array(117, np.uint8), "sa": np.array(0.0213, np.float32)}
    sw = r.uniform(1e-3, 1e-2, (N,) if per_col else ()).astype(np.float16)
    weights = {"w": r.integers(-128, 128, (K, N)).astype(np.int8), "wz": np.array(0, np.int8),
               "sw": sw, "b": r.normal(0, 1, (N,)).astype(np.float16)}
    nodes = [("Mul", ["sa", "sw"], ["s"], {}),
             ("MatMulInteger", ["a", "w", "az", "wz"], ["acc"], {}),
             ("Cast", ["acc"], ["f"], {"to": 1}), ("Mul", ["f", "s"], ["y"], {}),
             ("Add", ["y", "b"], ["z"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "z")
    assert [n[0] for n in fused] == ["QMatMulScaled"] and fused[0][3].get("scale_product")
    assert_bitexact(got, want.astype(np.float32), "QMatMulScaled with the scale product")


def test_qmatmul_tail_row_scale_runs_the_chain(gpu, oracle):
    """A scale that is not one value or one per column (here one per row)
    would change the product's shape handling: the fused node then runs the
    chain node by node, with the same result as the oracle."""
    r = rng(28)
    a = r.integers(0, 256, (1, 40, 64)).astype(np.uint8)
    inputs = {"a": a, "az": np.array(100, np.uint8),
              "s": r.uniform(1e-4, 1e-3, (40, 1)).astype(np.float32)}
    weights = {"w": r.integers(-128, 128, (64, 24)).astype(np.int8), "wz": np.array(0, np.int8),
               "b": r.normal(0, 1, (24,)).astype(np.float32)}
    nodes = [("MatMulInteger", ["a", "w", "az", "wz"], ["acc"], {}),
             ("Cast", ["acc"], ["f"], {"to": 1}), ("Mul", ["f", "s"], ["y"], {}),
             ("Add", ["y", "b"], ["z"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "z")
    assert [n[0] for n in fused] == ["QMatMulScaled"]
    assert_bitexact(got, want.astype(np.float32), "QMatMulScaled, per-row scale")


@pytest.mark.parametrize("cin,cout,k,L", [(128, 128, 5, 2000), (256, 96, 3, 777)])
def test_qconv_tail_with_bias_quantisation(gpu, oracle, cin, cout, k, L):
    """The graph's whole quantised-conv sequence: the activation's scale
    times the weight scale, the float bias divided by that, floored, cast
    to int32 and reshaped, then ConvInteger + bias -> Cast -> Mul(scale).
    The bias quantisation folds into the conv (one launch after the
    quantiser); the result is the chain's, bit for bit."""
    r = rng(30)
    xf = (r.normal(0.2, 1.5, (1, cin, L))).astype(np.float32)
    weights = {"w": r.integers(0, 256, (cout, cin, k)).astype(np.uint8),
               "wz": np.array(129, np.uint8), "sw": np.array(0.00371, np.float16),
               "b": r.normal(0, 0.5, (cout,)).astype(np.float16),
               "shp": np.array([1, cout, 1], np.int64)}
    at = {"pads": [k // 2, k // 2], "dilations": [1], "strides": [1], "group": 1,
          "kernel_shape": [k]}
    nodes = [("DynamicQuantizeLinear", ["xf"], ["q", "sa", "za"], {}),
             ("Cast", ["sa"], ["saf"], {"to": 10}), ("Mul", ["saf", "sw"], ["s"], {}),
             ("Div", ["b", "s"], ["bd"], {}), ("Floor", ["bd"], ["bf"], {}),
             ("Cast", ["bf"], ["bi"], {"to": 6}), ("Reshape", ["bi", "shp"], ["br"], {}),
             ("ConvInteger", ["q", "w", "za", "wz"], ["acc"], at),
             ("Add", ["acc", "br"], ["accb"], {}), ("Cast", ["accb"], ["f"], {"to": 10}),
             ("Mul", ["f", "s"], ["y"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, {"xf": xf}, weights, "y")
    assert [n[0] for n in fused] == ["DynamicQuantizeLinear", "Cast", "QConvScaled"]
    assert fused[-1][3].get("bias_quant")
    assert_bitexact(got, want.astype(np.float32), f"QConvScaled + bias quantisation {cin}->{cout}")


@pytest.mark.parametrize("cin,cout,k,L,side,rshape", [
    (128, 128, 5, 2000, 0, "full"), (256, 96, 3, 777, 1, "full"),
    # a residual the epilogue cannot take (broadcast over time, or over
    # channels): the Add runs after the conv, with its broadcasting
    (128, 64, 3, 500, 1, "channel"), (64, 64, 7, 300, 0, "time")])
def test_qconv_bias_quantisation_residual_add(gpu, oracle, cin, cout, k, L, side, rshape):
    """The decoder's residual sums: a quantised conv's output read only by
    an Add.  The Add folds into the conv (the residual added to the scaled
    result in the epilogue, fp32 x + y, which commutes), with the residual on
    either side of the Add; bit-exact to the chain."""
    r = rng(31)
    xf = (r.normal(0.1, 1.2, (1, cin, L))).astype(np.float32)
    shp = {"full": (1, cout, L), "channel": (1, cout, 1), "time": (1, 1, L)}[rshape]
    weights = {"w": r.integers(0, 256, (cout, cin, k)).astype(np.uint8),
               "wz": np.array(127, np.uint8), "sw": np.array(0.0029, np.float16),
               "b": r.normal(0, 0.5, (cout,)).astype(np.float16),
               "shp": np.array([1, cout, 1], np.int64)}
    at = {"pads": [k // 2, k // 2], "dilations": [1], "strides": [1], "group": 1,
          "kernel_shape": [k]}
    nodes = [("DynamicQuantizeLinear", ["xf"], ["q", "sa", "za"], {}),
             ("Cast", ["sa"], ["saf"], {"to": 10}), ("Mul", ["saf", "sw"], ["s"], {}),
             ("Div", ["b", "s"], ["bd"], {}), ("Floor", ["bd"], ["bf"], {}),
             ("Cast", ["bf"], ["bi"], {"to": 6}), ("Reshape", ["bi", "shp"], ["br"], {}),
             ("ConvInteger", ["q", "w", "za", "wz"], ["acc"], at),
             ("Add", ["acc", "br"], ["accb"], {}), ("Cast", ["accb"], ["f"], {"to": 10}),
             ("Mul", ["f", "s"], ["y"], {}),
             ("Add", ["y", "res"] if side == 0 else ["res", "y"], ["z"], {})]
    inputs = {"xf": xf, "res": r.normal(0, 2.0, shp).astype(np.float32)}
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "z")
    assert [n[0] for n in fused] == ["DynamicQuantizeLinear", "Cast", "QConvScaled"]
    assert fused[-1][3].get("bias_quant") and fused[-1][1][fused[-1][3]["resid"]] == "res"
    assert got.shape == want.shape
    assert_bitexact(got, want.astype(np.float32), f"QConvScaled + residual ({rshape}, side {side})")


@pytest.mark.parametrize("stride,dil,pad", [(1, 1, 2), (2, 1, 1), (1, 3, 6)])
def test_qconv_tail_residual_add(gpu, oracle, stride, dil, pad):
    """The plain quantised-conv tail (int32 bias given) followed by a residual
    Add, with strided and dilated convs (the residual sized to the output)."""
    r = rng(32)
    cin, cout, k, L = 96, 80, 5, 1501
    lout = (L + 2 * pad - dil * (k - 1) - 1) // stride + 1
    x = r.integers(0, 256, (1, cin, L)).astype(np.uint8)
    inputs = {"x": x, "xz": np.array(90, np.uint8),
              "b": r.integers(-3000, 3000, (1, cout, 1)).astype(np.int32),
              "s": np.array(2.7e-5, np.float32),
              "res": r.normal(0, 1.0, (1, cout, lout)).astype(np.float32)}
    weights = {"w": r.integers(0, 256, (cout, cin, k)).astype(np.uint8),
               "wz": np.array(140, np.uint8)}
    at = {"pads": [pad, pad], "dilations": [dil], "strides": [stride], "group": 1,
          "kernel_shape": [k]}
    nodes = [("ConvInteger", ["x", "w", "xz", "wz"], ["acc"], at),
             ("Add", ["acc", "b"], ["accb"], {}), ("Cast", ["accb"], ["f"], {"to": 1}),
             ("Mul", ["f", "s"], ["y"], {}), ("Add", ["res", "y"], ["z"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "z")
    assert [n[0] for n in fused] == ["QConvScaled"] and "resid" in fused[0][3]
    assert_bitexact(got, want.astype(np.float32), f"QConvScaled + residual s{stride} d{dil}")


def norm_chain(affine, leaky):
    nodes = [("ReduceMean", ["x", "ax"], ["m1"], {"keepdims": 1}),
             ("Sub", ["x", "m1"], ["d"], {}), ("Mul", ["d", "d"], ["sq"], {}),
             ("ReduceMean", ["sq", "ax"], ["m2"], {"keepdims": 1}),
             ("Add", ["m2", "eps"], ["ve"], {}), ("Sqrt", ["ve"], ["sd"], {}),
             ("Div", ["d", "sd"], ["n"], {})]
    out = "n"
    if affine:
        nodes += [("Mul", ["g", "n"], ["gn"], {}), ("Add", ["gn", "b"], ["y"], {})]
        out = "y"
        if leaky:
            nodes.append(("LeakyRelu", ["y"], ["z"], {"alpha": 0.2}))
            out = "z"
    return nodes, out


@pytest.mark.parametrize("C,T,affine,leaky", [(128, 40000, True, False), (128, 40001, True, True),
                                              (256, 700, True, True), (512, 279, False, False),
                                              (64, 20000, False, False),
                                              # long rows in 8192-blocks: two whole blocks;
                                              # three; three and 100 elements; four and 5;
                                              # 512 rows of five blocks
                                              (32, 16384, True, False), (32, 24576, False, False),
                                              (32, 24676, True, False), (16, 32773, False, True),
                                              (512, 40000, True, True),
                                              # rows held in registers: the decoder's
                                              # [1,256,71800]; eight blocks and 8188;
                                              # whole blocks only; a 4-element last
                                              # block (a leaf under eight); one block
                                              (256, 71800, True, True), (8, 73724, True, False),
                                              (16, 65536, False, False), (16, 65540, True, False),
                                              (40, 15004, False, True),
                                              # longer rows (statistics passes): a
                                              # partial last block of 1696, the
                                              # decoder's 430800 (2 and 128 rows),
                                              # nine whole blocks and no partial one,
                                              # sixteen, 63 of them and 100 elements,
                                              # a 6-element one
                                              (4, 100000, True, False), (2, 430800, True, True),
                                              (128, 430800, True, False), (40, 73728, False, False),
                                              (6, 131072, True, True), (2, 516196, True, False),
                                              (3, 81926, False, False)])
def test_instance_norm_chain(gpu, oracle, C, T, affine, leaky):
    r = rng(22)
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    inputs = {"x": x, "g": (1 + 0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32),
              "b": (0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32)}
    weights = {"ax": np.array([2], np.int64),
               "eps": np.array(1e-5, np.float16).astype(np.float32)}
    nodes, out = norm_chain(affine, leaky)
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, out)
    assert [n[0] for n in fused] == ["InstanceNormScaleShift"]
    # statistics in numpy's summation order, then the chain's own IEEE
    # operations: the same bits
    assert_bitexact(got, want, f"InstanceNorm chain C={C} T={T}")


@pytest.mark.parametrize("gshape,bshape,leaky,snake", [((64,), (1, 64, 1), False, False),
                                                      ((1, 64, 1), (64,), True, False),
                                                      ((), (1, 64, 1), False, False),
                                                      ((1, 64, 1), (1, 64, 1), False, True),
                                                      ((64,), (64,), False, True)])
def test_instance_norm_chain_operands_not_per_channel(gpu, oracle, gshape, bshape, leaky, snake):
    """A scale or shift of C values shaped [C] broadcasts along T, not along
    the channels; with T == C the graph is valid and the fused per-channel
    kernel would give a different result.  Such chains (and one-value
    scales) run past the statistics node by node and match the oracle's
    chain bit for bit; the snake's operands stay per channel."""
    C = T = 64
    r = rng(27)
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    inputs = {"x": x, "g": (1 + 0.1 * r.normal(0, 1, gshape)).astype(np.float32),
              "b": (0.1 * r.normal(0, 1, bshape)).astype(np.float32)}
    weights = {"ax": np.array([2], np.int64),
               "eps": np.array(1e-5, np.float16).astype(np.float32)}
    nodes, y = norm_chain(True, leaky)
    if snake:
        alpha = r.uniform(0.5, 2, (1, C, 1)).astype(np.float16)
        weights.update({"a": alpha, "two": np.array(2.0, np.float16),
                        "rc": (np.float32(1) / alpha.astype(np.float32)).astype(np.float16)})
        nodes += [("Mul", ["a", y], ["t"], {}), ("Sin", ["t"], ["s"], {}),
                  ("Pow", ["s", "two"], ["p"], {}), ("Mul", ["rc", "p"], ["q"], {}),
                  ("Add", [y, "q"], ["z"], {})]
        y = "z"
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, y)
    assert fused[0][0] in ("InstanceNormScaleShift", "InstanceNormSnake")
    if snake:
        assert_close(got, want, 1e-5, floor_rel=1e-6, what=f"{gshape} {bshape} + snake")
    else:
        assert_bitexact(got, want, f"InstanceNorm chain scale {gshape} shift {bshape}")


def test_instance_norm_resident_edge_values(gpu, oracle):
    """Rows held in registers divide by den with one reciprocal and two FMAs,
    exact only away from underflow and overflow; the values outside that
    range take the division itself.  Rows whose x - mean is exactly 0, tiny
    (1e-19), or whose variance overflows (den = inf), beside ordinary rows:
    the same bits as the oracle's chain."""
    r = rng(28)
    C, T = 6, 20000
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    x[0, 0] = 3.0                                                       # constant row
    x[0, 1] = (r.normal(0, 1, T) * 1e-19).astype(np.float32)            # tiny deviations
    x[0, 2] = (r.normal(0, 1, T) * 2e18).astype(np.float32)             # variance overflows
    x[0, 3, ::7] = np.float32(0.0)                                      # zeros among values
    x[0, 4, :T // 2] = np.float32(1.5)                                  # half the row constant
    inputs = {"x": x, "g": (1 + 0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32),
              "b": (0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32)}
    weights = {"ax": np.array([2], np.int64),
               "eps": np.array(1e-5, np.float16).astype(np.float32)}
    for affine in (False, True):
        nodes, out = norm_chain(affine, False)
        with np.errstate(over="ignore", invalid="ignore"):
            got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, out)
        assert [n[0] for n in fused] == ["InstanceNormScaleShift"]
        assert_bitexact(got, want, f"edge rows affine={affine}")


def test_instance_norm_long_rows_repeat(gpu, oracle):
    """The long-row instance norm leaves its per-row arrival counters at
    zero: three launches in a row, with one of another shape between each,
    give the same bits, and those of the oracle's chain."""
    r = rng(23)
    x = (r.normal(0, 2, (1, 64, 40000)) + r.normal(0, 3, (1, 64, 1))).astype(np.float32)
    x2 = r.normal(0, 1, (1, 200, 24676)).astype(np.float32)
    dx, dx2 = gpu.to_device(x), gpu.to_device(x2)
    first = gpu.ops.instance_norm(dx, None, 1e-5).numpy()
    for _ in range(2):
        gpu.ops.instance_norm(dx2, None, 1e-5)
        assert_bitexact(gpu.ops.instance_norm(dx, None, 1e-5).numpy(), first, "repeated launch")
    weights = {"ax": np.array([2], np.int64), "eps": np.array(1e-5, np.float32)}
    nodes, out = norm_chain(False, False)
    oenv = {"x": x, **weights}
    for op, ins, outs, at in nodes:
        oracle.dispatch(op, ins, outs, at, oenv)
    assert_bitexact(first, oenv[out], "long rows vs the oracle's chain")


@pytest.mark.parametrize("C,T,affine", [(128, 40000, True), (256, 7180, True), (64, 999, False)])
def test_instance_norm_snake_chain(gpu, oracle, C, T, affine):
    """The InstanceNorm chain with its output read only by a snake chain:
    one InstanceNormSnake launch (long rows and rows held in LDS)."""
    r = rng(24)
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    alpha = r.uniform(0.5, 2, (1, C, 1)).astype(np.float16)
    inputs = {"x": x, "g": (1 + 0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32),
              "b": (0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32)}
    weights = {"ax": np.array([2], np.int64),
               "eps": np.array(1e-5, np.float16).astype(np.float32), "a": alpha,
               "rc": (np.float32(1) / alpha.astype(np.float32)).astype(np.float16),
               "two": np.array(2.0, np.float16)}
    nodes, y = norm_chain(affine, False)
    nodes += [("Mul", ["a", y], ["t"], {}), ("Sin", ["t"], ["s"], {}),
              ("Pow", ["s", "two"], ["p"], {}), ("Mul", ["rc", "p"], ["q"], {}),
              ("Add", [y, "q"], ["z"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, inputs, weights, "z")
    assert [n[0] for n in fused] == ["InstanceNormSnake"]
    # the norm is bit-exact; sin differs from numpy's by ulps (the snake bar)
    assert_close(got, want, 1e-5, floor_rel=1e-6, what=f"InstanceNorm+snake C={C} T={T}")


@pytest.mark.parametrize("C,T,rc_mul,leaky", [(64, 20000, 1.0, None), (64, 20000, 5.0, None),
                                              (32, 24676, None, -0.5), (32, 24676, None, 0.2),
                                              (48, 3000, 5.0, None),
                                              # odd long rows: rows start at every
                                              # offset mod 4 (scalar head and tail)
                                              (24, 20001, 1.0, None), (16, 16386, None, 0.2),
                                              (24, 20003, 5.0, None),
                                              # rows held in registers (the decoder's
                                              # [1,256,71800]; a 4-element last block)
                                              (256, 71800, 1.0, None), (256, 71800, None, 0.2),
                                              (16, 65540, 5.0, None),
                                              # up to 2048 rows every quantising block
                                              # folds the rows' partials; beyond, a fold
                                              # launch does (with the fallback, both ways)
                                              (2048, 64, 5.0, None), (2100, 40, 5.0, None),
                                              (2100, 40, None, 0.2),
                                              # the fallback's partials (rows x 4 blocks)
                                              # beyond one block's fold: a fold launch
                                              (4200, 24580, 5.0, None)])
def test_instance_norm_quant_matches_unfused_device_path(gpu, C, T, rc_mul, leaky):
    """InstanceNormQuant gives the same bytes, scale and zero point as the
    device's own unfused chain: the float result stored, then
    DynamicQuantizeLinear's (min, max) over the stored values.  Long rows
    take the quantiser's range from each row's result at its x extremes
    (exact where y is monotonic in x); a snake with recip = 5 / alpha, or a
    LeakyRelu slope below 0, is not monotonic, so the quantising pass finds
    values outside that range and the exact fallback passes run.  Rows held
    in LDS form the exact range in one pass.  Scales of both signs."""
    r = rng(26)
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    g = r.normal(0, 1, (1, C, 1)).astype(np.float32)
    b = (0.3 * r.normal(0, 1, (1, C, 1))).astype(np.float32)
    D = gpu.to_device
    if rc_mul is not None:
        a = r.uniform(0.5, 2, (1, C, 1)).astype(np.float32)
        rc = (np.float32(rc_mul) / a).astype(np.float32)
        y = gpu.ops.instance_norm_scale_shift_snake(D(x), D(g), D(b), D(a), D(rc), 1e-5)
        fused = gpu.ops.instance_norm_quant(D(x), D(g), D(b), D(a), D(rc), 1e-5)
    else:
        y = gpu.ops.instance_norm_scale_shift(D(x), D(g), D(b), 1e-5, leaky)
        fused = gpu.ops.instance_norm_quant(D(x), D(g), D(b), eps=1e-5, leaky_alpha=leaky)
    want = gpu.ops.dynamic_quantize_linear(y)
    for got_t, want_t, what in zip(fused, want, ("bytes", "scale", "zero point")):
        assert_bitexact(gpu.to_host(got_t), gpu.to_host(want_t), f"{what} C={C} T={T}")


@pytest.mark.parametrize("C,T,kind", [(128, 40000, "affine"), (256, 7180, "leaky"),
                                      (128, 20000, "snake"), (64, 999, "snake"),
                                      (96, 2400, "plain"), (32, 24676, "leaky"),
                                      (512, 40000, "affine"),
                                      # long rows with T % 4 = 1, 2, 3
                                      (32, 24677, "snake"), (16, 16386, "affine"),
                                      (24, 20003, "leaky"),
                                      # rows held in registers
                                      (256, 71800, "snake"), (8, 73724, "affine"),
                                      (16, 15004, "leaky"),
                                      # longer rows (statistics passes)
                                      (4, 100000, "snake"), (2, 430800, "leaky"),
                                      (128, 430800, "leaky"), (40, 73732, "snake"),
                                      (3, 81926, "affine")])
def test_instance_norm_quant_chain(gpu, oracle, C, T, kind):
    """The InstanceNorm chain (plain, affine, + LeakyRelu, + snake) -> Cast
    -> DynamicQuantizeLinear: one InstanceNormQuant, its float result never
    stored.  Without the snake: the same bytes, scale and zero point as the
    oracle's chain; with it (sin differs from numpy's by ulps) a value on a
    rounding boundary may land one step away."""
    r = rng(25)
    x = (r.normal(0, 2, (1, C, T)) + r.normal(0, 3, (1, C, 1))).astype(np.float32)
    alpha = r.uniform(0.5, 2, (1, C, 1)).astype(np.float16)
    inputs = {"x": x, "g": (1 + 0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32),
              "b": (0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32)}
    weights = {"ax": np.array([2], np.int64),
               "eps": np.array(1e-5, np.float16).astype(np.float32), "a": alpha,
               "rc": (np.float32(1) / alpha.astype(np.float32)).astype(np.float16),
               "two": np.array(2.0, np.float16)}
    nodes, y = norm_chain(kind != "plain", kind == "leaky")
    if kind == "snake":
        nodes += [("Mul", ["a", y], ["t"], {}), ("Sin", ["t"], ["s"], {}),
                  ("Pow", ["s", "two"], ["p"], {}), ("Mul", ["rc", "p"], ["qq"], {}),
                  ("Add", [y, "qq"], ["z"], {})]
        y = "z"
    nodes += [("Cast", [y], ["f"], {"to": 1}),
              ("DynamicQuantizeLinear", ["f"], ["q", "qs", "qz"], {})]
    fz = importlib.import_module("best-tts-godot_amd.fuse")
    dev_w = {}
    for k, v in weights.items():
        v = np.asarray(v)
        v = v.astype(np.float32) if v.dtype == np.float16 else v
        t = gpu.to_device(v)
        if v.size <= 16:
            t.host = v
        dev_w[k] = t
    fused, _ = fz.fuse(nodes, dev_w, {"q", "qs", "qz"})
    assert [n[0] for n in fused] == ["InstanceNormQuant"]
    env = dict(dev_w)
    env.update({k: gpu.to_device(np.asarray(v)) for k, v in inputs.items()})
    for op, ins, outs, at in fused:
        gpu.dispatch(op, ins, outs, at, env)
    oenv = {k: np.asarray(v) for k, v in {**weights, **inputs}.items()}
    for op, ins, outs, at in nodes:
        oracle.dispatch(op, ins, outs, at, oenv)
    q, qs, qz = (gpu.to_host(env[n]) for n in ("q", "qs", "qz"))
    if kind != "snake":
        assert_bitexact(q, oenv["q"], f"quantised InstanceNorm ({kind})")
        assert_bitexact(np.asarray(qs, np.float32).reshape(()), np.asarray(oenv["qs"], np.float32),
                        "scale")
        assert_bitexact(np.asarray(qz).reshape(()), np.asarray(oenv["qz"]), "zero point")
    else:
        assert_close(np.asarray(qs, np.float32).reshape(()), np.asarray(oenv["qs"], np.float32),
                     1e-6, what="scale")
        assert abs(int(np.asarray(qz).reshape(())) - int(np.asarray(oenv["qz"]).reshape(()))) <= 1
        d = np.abs(q.astype(np.int64) - oenv["q"].astype(np.int64))
        assert d.max() <= 1 and (d > 0).mean() <= 1e-3, (d.max(), (d > 0).mean())


@pytest.mark.parametrize("C,T", [(128, 30000), (256, 5001)])
def test_snake_chain(gpu, oracle, C, T):
    r = rng(23)
    x = r.normal(0, 1, (1, C, T)).astype(np.float32)
    alpha = r.uniform(0.5, 2, (1, C, 1)).astype(np.float16)
    weights = {"a": alpha, "r": (np.float32(1) / alpha.astype(np.float32)).astype(np.float16),
               "two": np.array(2.0, np.float16)}
    nodes = [("Mul", ["a", "x"], ["t"], {}), ("Sin", ["t"], ["s"], {}),
             ("Pow", ["s", "two"], ["p"], {}), ("Mul", ["r", "p"], ["q"], {}),
             ("Add", ["x", "q"], ["y"], {})]
    got, want, fused = run_chain(gpu, oracle, nodes, {"x": x}, weights, "y")
    assert [n[0] for n in fused] == ["Snake"]
    assert_close(got, want, 1e-5, floor_rel=1e-6, what=f"snake chain C={C} T={T}")

