"""The packed-graph walker's debugging aids on the GPU: strict mode (stop at
the first node with a non-finite float output and name it with its inputs'
ranges, tools/ref_runtime.py:378-418) and the node limit
(addons/best-tts/runtime/executor.gd:67-72, 306-307)."""
import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# The embeddings' LayerNormalization (node 30 of the packed graph) reads the
# fp16 scale [128] of tensor 53 (encoder.bert.embeddings.LayerNorm.weight).
LN_NODE, LN_SCALE = 30, 53


@pytest.fixture(scope="module")
def parts():
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    assert g["ops"][g["nodes"][LN_NODE][0]] == "LayerNormalization"
    assert LN_SCALE in g["nodes"][LN_NODE][1]
    return kkg, g, kkg.synth_weights(g, 0), kkg.synth_inputs(3, 1)


def test_strict_clean_run_matches_plain(gpu, parts):
    """On finite weights strict mode raises nothing and returns the same bits."""
    kkg, g, w, (ids, style, _) = parts
    pg = kkg.PackedGraph(g, w)
    plain = pg.run(ids, style, 2.0)
    strict = pg.run(ids, style, 2.0, strict=True)
    np.testing.assert_array_equal(strict, plain)


def test_strict_names_the_node_that_reads_a_nan_weight(gpu, parts):
    kkg, g, w, (ids, style, _) = parts
    planted = dict(w)
    scale = np.array(w[LN_SCALE], copy=True)
    scale[17] = np.nan
    planted[LN_SCALE] = scale
    pg = kkg.PackedGraph(g, planted)
    with pytest.raises(kkg.NonFiniteError) as info:
        pg.run(ids, style, 2.0, strict=True)
    err = info.value
    assert LN_NODE in pg.groups[err.node], (err.node, pg.groups[err.node])
    assert err.op == "LayerNormalization"
    names = [n for n, *_ in err.inputs]
    assert str(LN_SCALE) in names
    rng = dict((n, r) for n, _s, _d, r in err.inputs)[str(LN_SCALE)]
    assert rng is not None and np.isfinite(rng).all()  # nanmin/nanmax of the planted scale
    assert f"node {err.node} LayerNormalization" in str(err)
    # (The planted model is never run without strict mode: NaN durations
    # would reach the host's integer length arithmetic.)


def test_max_nodes_stops_the_walk(gpu, parts):
    """The walk stops after the first n nodes: the output is not reached
    (None) and the kept tensors hold the values of a full run."""
    kkg, g, w, (ids, style, _) = parts
    pg = kkg.PackedGraph(g, w, protect=[55])
    k = next(i for i, grp in enumerate(pg.groups) if LN_NODE in grp)
    assert pg.run(ids, style, 2.0, keep=[55], max_nodes=k + 1) is None
    partial = gpu.to_host(pg.last_env["55"])
    pg.run(ids, style, 2.0, keep=[55])
    np.testing.assert_array_equal(partial, gpu.to_host(pg.last_env["55"]))
    assert pg.run(ids, style, 2.0, max_nodes=0) is None
