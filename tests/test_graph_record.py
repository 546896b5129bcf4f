"""The text part of a run recorded as a HIP graph and replayed
(PackedGraph(record=True), kk_graph_begin_arena): every run's waveform
bit-identical to the node-by-node walk of the same inputs, for new ids,
style and speed of a recorded token count, for a second token count, after
a recorded token count is dropped, and when recording fails (an arena too
small: the run walks every node instead).  Ids outside the embedding table
raise the walk's error on a replay too."""
import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def graphs(gpu):
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    w = kkg.synth_weights(g, 0)
    return kkg, kkg.PackedGraph(g, w, record=False), kkg.PackedGraph(g, w)


def inputs(kkg, n, seed, speed):
    ids, style, _ = kkg.synth_inputs(n, seed)
    return ids, style, speed


def test_replay_matches_walk(graphs):
    kkg, walk, rec = graphs
    a = inputs(kkg, 6, 1, 1.0)
    b = inputs(kkg, 6, 2, 1.3)  # same length: new ids, style and speed
    c = inputs(kkg, 9, 3, 0.8)
    want = {k: walk.run(*v) for k, v in (("a", a), ("b", b), ("c", c))}
    for k, v in (("a", a), ("b", b), ("a", a), ("b", b), ("c", c), ("c", c), ("c", c), ("b", b)):
        np.testing.assert_array_equal(rec.run(*v), want[k], err_msg=k)
    for n in (a[0].size, c[0].size):
        end, kernels, arena, error = rec.recorded(n)
        assert error is None and kernels > 100 and end > 100 and arena > 0
    assert want["a"].size != want["b"].size  # speed moved the durations


def test_dropped_and_rerecorded(graphs):
    kkg, walk, rec = graphs
    keep, rec.RECORD_KEEP = rec.RECORD_KEEP, 1
    try:
        for n, seed in ((5, 4), (7, 5), (5, 6)):
            v = inputs(kkg, n, seed, 1.0)
            want = walk.run(*v)
            for _ in range(3):
                np.testing.assert_array_equal(rec.run(*v), want)
            assert list(rec._parts) == [v[0].size]
    finally:
        rec.RECORD_KEEP = keep


def test_failed_recording_walks(graphs):
    kkg, walk, rec = graphs
    v = inputs(kkg, 4, 7, 1.0)
    want = walk.run(*v)
    np.testing.assert_array_equal(rec.run(*v), want)  # finds the text part
    rec._parts[v[0].size].arena = 1 << 16
    for _ in range(2):
        np.testing.assert_array_equal(rec.run(*v), want)
    end, kernels, _arena, error = rec.recorded(v[0].size)
    assert kernels is None and "arena exhausted" in error


def test_replay_checks_ids(graphs):
    kkg, walk, rec = graphs
    ids, style, speed = inputs(kkg, 3, 8, 1.0)
    for _ in range(3):
        rec.run(ids, style, speed)
    assert rec.recorded(ids.size)[1] is not None
    bad = np.array(ids).reshape(-1)
    bad[1] = 100000
    with pytest.raises(RuntimeError, match="index out of bounds") as walked:
        walk.run(bad, style, speed)
    with pytest.raises(RuntimeError, match="index out of bounds") as replayed:
        rec.run(bad, style, speed)
    assert str(walked.value) == str(replayed.value)
