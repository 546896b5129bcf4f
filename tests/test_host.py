"""CPU-only checks of the host side: libkk loads and exports every entry
point include/kk.h declares, errors come back as statuses (no GPU work is
attempted), view arithmetic matches numpy's, and host shape ops match the
oracle's dispatch."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact, load_pkg


def header_symbols():
    text = open(os.path.join(ROOT, "include", "kk.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(kk_\w+)\(", text, re.M)))


def test_header_matches_binding():
    kk = load_pkg()
    assert header_symbols() == kk._lib.exported_symbols()


def test_library_exports_every_symbol():
    kk = load_pkg()
    lib = kk._lib.load()
    for name in header_symbols():
        assert hasattr(lib, name), name


def test_status_without_init():
    """Before kk_init every op reports KK_E_STATE instead of touching a GPU."""
    kk = load_pkg()
    lib = kk._lib.load()
    if kk.tensor._state["device"] is not None:
        pytest.skip("library already initialised in this process")
    p = ctypes.c_void_p()
    rc = lib.kk_alloc(16, ctypes.byref(p))
    assert rc == -4
    assert b"kk_init" in lib.kk_last_error()
    with pytest.raises(kk._lib.KKError):
        kk._lib.call("kk_sync")


class _FakeStorage:
    ptr = 1 << 20
    nbytes = 1 << 30


def _fake(shape, dtype=np.float32):
    kk = load_pkg()
    return kk.DeviceTensor(_FakeStorage(), shape, dtype)


def _np_view(a, t):
    """numpy array with the same element offset/strides as DeviceTensor t."""
    base = np.arange(a.size, dtype=np.float32)
    item = base.itemsize
    return np.lib.stride_tricks.as_strided(base[t.offset:], t.shape,
                                           [s * item for s in t.strides])


def test_view_arithmetic_matches_numpy():
    a = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    t = _fake(a.shape)
    cases = [
        (t.transpose([2, 0, 3, 1]), np.transpose(a, (2, 0, 3, 1))),
        (t.slice_axis(2, 1, 4, 2), a[:, :, 1:4:2]),
        (t.slice_axis(3, 4, -1, -1), a[:, :, :, ::-1]),
        (t.expand_dims(1), np.expand_dims(a, 1)),
        (t.expand_dims(4), np.expand_dims(a, 4)),
        (t.slice_axis(1, 1, 2).squeeze([1]), a[:, 1]),
        (t.reshape([6, -1]), a.reshape(6, -1)),
        (t.slice_axis(0, 1, 2).broadcast_to((3, 2, 3, 4, 5)),
         np.broadcast_to(a[1:2], (3, 2, 3, 4, 5))),
    ]
    for view, want in cases:
        got = _np_view(a, view)
        assert_bitexact(np.ascontiguousarray(got), np.ascontiguousarray(want), repr(view))


def test_slice_params_match_reference_rule():
    import importlib
    from oracle import ref_ops
    load_pkg()
    d = importlib.import_module("best-tts-godot_amd.dispatch")
    x = np.arange(11)
    for s, e, st in [(0, 11, 1), (-3, -1, 1), (9, -100, -1), (9, 0, -3), (100, 2, -2),
                     (-100, 100, 4), (5, 5, 1), (0, -1, -1)]:
        start, _, step, n = d._slice_params(11, s, e, st)
        want = ref_ops.slice_op(x, [s], [e], None, [st])
        got = x[start:start + n * step:step] if n else x[:0]
        if n and start + n * step < 0:
            got = x[start::step][:n]
        assert np.array_equal(got, want), (s, e, st)


def test_host_shape_ops_match_oracle():
    from oracle import ref_ops
    kk = load_pkg()
    shape = np.array([1, 130, 768], np.int64)
    cases = [
        ("Gather", [shape, np.array(1)], {"axis": 0}),
        ("Concat", [shape, np.array([2, 3])], {"axis": 0}),
        ("Unsqueeze", [np.array(5), np.array([0])], {}),
        ("Slice", [shape, np.array([1]), np.array([3])], {}),
        ("Mul", [shape, np.array(2)], {}),
        ("Div", [np.array([-7, 7]), np.array(2)], {}),
        ("Equal", [shape, np.array(130)], {}),
        ("Range", [np.array(0), np.array(10), np.array(3)], {}),
        ("Cast", [shape], {"to": 1}),
        ("ConstantOfShape", [np.array([2, 2])], {"value": np.array([7], np.int64)}),
        ("Reshape", [np.arange(6), np.array([2, -1])], {}),
    ]
    for op, ins, at in cases:
        names = [f"i{k}" for k in range(len(ins))]
        env = dict(zip(names, ins))
        oenv = dict(env)
        kk.dispatch(op, names, ["o"], at, env)
        if op == "Range":
            want = np.arange(0, 10, 3)
        else:
            ref_ops.dispatch(op, names, ["o"], at, oenv)
            want = oenv["o"]
        # np.take with a 0-d index gives a numpy scalar, as in the reference
        assert isinstance(env["o"], (np.ndarray, np.generic)), op
        assert np.array_equal(env["o"], want) and env["o"].dtype == want.dtype, op


def test_unknown_op_raises():
    kk = load_pkg()
    with pytest.raises(NotImplementedError):
        kk.dispatch("NoSuchOp", ["a"], ["b"], {}, {"a": np.zeros(1, np.float32)})


def _graph_nodes():
    import importlib
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    nodes = [(g["ops"][op], ["" if t < 0 else str(t) for t in ins],
              ["" if t < 0 else str(t) for t in outs], kkg._decode_attrs(at))
             for op, ins, outs, at, _pl in g["nodes"]]
    return g, nodes, {str(k): v for k, v in kkg.synth_weights(g, 0).items()}


def test_fusion_pass_on_the_kokoro_graph():
    """The fusion pass finds every quantised conv tail (87) and quantised
    Linear tail (148, 136 with their bias, each with its scale product),
    InstanceNorm
    chain (64 of 65: one has a Transpose inside) and snake (48) of the
    packed graph -- 42 norm chains feed a snake alone and merge with it, and
    59 norm chains (snake or not) feed only a Cast -> DynamicQuantizeLinear
    and merge with those -- keeps a valid topological order, and never drops
    a tensor that a node outside its group reads."""
    import importlib
    from collections import Counter
    fz = importlib.import_module("best-tts-godot_amd.fuse")
    g, nodes, weights = _graph_nodes()
    fused, groups = fz.fuse(nodes, weights, {str(g["output"])})
    kinds = Counter(n[0] for n in fused)
    assert (kinds["QConvScaled"], kinds["InstanceNormScaleShift"], kinds["Snake"],
            kinds["InstanceNormSnake"], kinds["InstanceNormQuant"]) == (87, 5, 6, 0, 59)
    assert kinds["QMatMulScaled"] == 148 and kinds["MatMulInteger"] == 0
    assert sum(1 for n in fused if n[0] == "QMatMulScaled" and n[1][5]) == 136
    # each Linear's scale is the Mul of the activation's and the weights'
    # scales, read by the chain alone: folded in as well
    assert sum(1 for n in fused if n[0] == "QMatMulScaled" and n[3].get("scale_product")) == 148
    # and each quantised conv whose int32 bias the graph forms per call
    # (Mul -> Div -> Floor -> Cast -> Reshape) takes those nodes in
    assert sum(1 for n in fused if n[0] == "QConvScaled" and n[3].get("bias_quant")) == 80
    # 35 of those feed a residual Add alone, which they take in (the sum in
    # the conv's epilogue); the residual is the merged node's last input
    res = [n for n in fused if n[0] == "QConvScaled" and "resid" in n[3]]
    assert len(res) == 35 and all(n[3]["resid"] == len(n[1]) - 1 for n in res)
    assert len(fused) == 1796
    covered = sorted(i for grp in groups for i in grp)
    assert covered == list(range(len(nodes)))  # every original node exactly once
    produced = {}
    for k, (_op, _ins, outs, _at) in enumerate(fused):
        for o in outs:
            if o:
                produced[o] = k
    for k, (_op, ins, _outs, _at) in enumerate(fused):
        for n in ins:
            if n and n in produced:
                assert produced[n] < k, (k, n)
    # tensors produced inside a group and read elsewhere must still be produced
    inner = {}
    for k, grp in enumerate(groups):
        for i in grp:
            for o in nodes[i][2]:
                if o:
                    inner[o] = k
    for k, (_op, ins, _outs, _at) in enumerate(fused):
        for n in ins:
            if n in inner and inner[n] != k:
                assert n in produced, n


def test_fusion_skips_chains_with_outside_readers():
    import importlib
    fz = importlib.import_module("best-tts-godot_amd.fuse")
    nodes = [("ReduceMean", ["x", "ax"], ["m1"], {"keepdims": 1}),
             ("Sub", ["x", "m1"], ["d"], {}), ("Mul", ["d", "d"], ["sq"], {}),
             ("ReduceMean", ["sq", "ax"], ["m2"], {"keepdims": 1}),
             ("Add", ["m2", "eps"], ["ve"], {}), ("Sqrt", ["ve"], ["sd"], {}),
             ("Div", ["d", "sd"], ["n"], {}), ("Mul", ["g", "n"], ["y"], {})]
    weights = {"ax": np.array([2], np.int64), "eps": np.array(1e-5, np.float32),
               "g": np.ones((1, 4, 1), np.float32)}
    fused, groups = fz.fuse(nodes, weights, {"y"})
    assert [n[0] for n in fused] == ["InstanceNormScaleShift"] and groups == [list(range(8))]
    extra = nodes + [("Mul", ["d", "x"], ["z"], {})]  # d gains a reader outside the chain
    fused, groups = fz.fuse(extra, weights, {"y", "z"})
    assert [n[0] for n in fused] == [n[0] for n in extra]
    fused, _ = fz.fuse(nodes, weights, {"y", "n"})  # a protected intermediate
    assert "InstanceNormScaleShift" in [n[0] for n in fused]
    assert any(n[2] == ["n"] for n in fused)
