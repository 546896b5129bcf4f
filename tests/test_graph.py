"""HIP graph replay of recorded ops equals eager execution, on every replay,
with eager work and synchronisation between replays; recording refuses
allocation."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact, rng

pytestmark = pytest.mark.gpu


def test_graph_replay_matches_eager(gpu):
    r = rng(0)
    D = gpu.to_device
    x = D(r.normal(0, 1, (1, 256, 2400)).astype(np.float32))
    a = D(r.uniform(0.5, 2, (1, 256, 1)).astype(np.float32))
    s = D(r.normal(0, 0.1, (1, 128)).astype(np.float32))
    w = D(r.normal(0, 0.05, (128, 512)).astype(np.float32))
    q = D(r.integers(-127, 128, (256, 256, 3)).astype(np.int8))
    sc = D(np.array(0.005, np.float32))
    h1 = gpu.DeviceTensor.empty(x.shape)
    h2 = gpu.DeviceTensor.empty(x.shape)
    h3 = gpu.DeviceTensor.empty(x.shape)
    L = gpu._lib

    def record():
        L.call("kk_snake", h1.desc(), x.desc(), a.desc(), None)
        L.call("kk_adain", h2.desc(), h1.desc(), s.desc(), w.desc(), None, None, None, 1e-5)
        L.call("kk_conv1d", h3.desc(), h2.desc(), q.desc(), sc.desc(), None, None, 1, 1, 1, 1, 1)

    record()
    eager = h3.numpy()
    L.call("kk_graph_begin")
    record()
    with pytest.raises(L.KKError):  # no allocation while recording
        p = ctypes.c_void_p()
        L.call("kk_alloc", 64, ctypes.byref(p))
    gid = ctypes.c_int()
    L.call("kk_graph_end", ctypes.byref(gid))
    for rep in range(4):
        gpu.ops.fill(h3.shape, 0.0).numpy()  # unrelated eager work in between
        L.call("kk_fill", h3.desc(), -1.0)
        L.call("kk_graph_launch", gid.value)
        assert_bitexact(h3.numpy(), eager, f"replay {rep}")
    L.call("kk_graph_destroy", gid.value)
