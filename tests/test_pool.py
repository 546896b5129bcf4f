"""The device buffer pool (kk_alloc/kk_free): bucket reuse, no regrowth over
repeated runs, rejected double frees, trimming, and run-to-run identical
results (the reference gates drift at exactly 0, tests/test_repeat.gd:97-112;
its pool plateau check is tests/test_memory.gd:57-68)."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact, rng

pytestmark = pytest.mark.gpu


def test_alloc_free_reuse_and_double_free(gpu):
    lib = gpu._lib
    p = ctypes.c_void_p()
    lib.call("kk_alloc", 5000, ctypes.byref(p))
    first = p.value
    live0, pooled0, _ = gpu.pool_stats()
    lib.call("kk_free", ctypes.c_void_p(first))
    live1, pooled1, _ = gpu.pool_stats()
    assert live1 == live0 - 5120 and pooled1 == pooled0 + 5120  # bucket(5000) = 5120
    q = ctypes.c_void_p()
    lib.call("kk_alloc", 5100, ctypes.byref(q))  # same bucket: the same buffer comes back
    assert q.value == first
    lib.call("kk_free", ctypes.c_void_p(q.value))
    with pytest.raises(lib.KKError) as e:
        lib.call("kk_free", ctypes.c_void_p(q.value))
    assert e.value.code == -4
    with pytest.raises(lib.KKError):
        lib.call("kk_free", ctypes.c_void_p(0xdead000))


def _mini_stage(kk, x, style, w, alpha):
    h = kk.ops.snake(x, alpha)
    h = kk.ops.adain(h, style, w, None, 1e-5)
    return kk.ops.binary("Add", h, x)


def test_no_regrowth_and_zero_drift(gpu):
    r = rng(0)
    D = gpu.to_device
    style = D(r.normal(0, 0.1, (1, 128)).astype(np.float32))
    w = D(r.normal(0, 0.05, (128, 512)).astype(np.float32))
    alpha = D(r.uniform(0.5, 2, (1, 256, 1)).astype(np.float32))
    full = r.normal(0, 1, (1, 256, 2400)).astype(np.float32)
    short = full[:, :, :700].copy()
    outs, peaks = [], []
    for i in range(6):  # alternate long and short inputs like test_repeat.gd
        x = D(full if i % 2 == 0 else short)
        outs.append(_mini_stage(gpu, x, style, w, alpha).numpy())
        del x
        peaks.append(gpu.pool_stats()[2])
    for i in range(2, 6):
        assert_bitexact(outs[i], outs[i % 2], f"run {i} drifted")
    # peak live memory plateaus after the first long and short runs
    assert peaks[-1] == peaks[1], peaks


def test_trim(gpu):
    live, pooled, _ = gpu.pool_stats()
    gpu.pool_trim(0)
    live2, pooled2, _ = gpu.pool_stats()
    assert pooled2 == 0 and live2 == live


def test_async_uploads_capture_the_host_bytes(gpu):
    """kk_upload returns without waiting for the stream: the host buffer is
    overwritten right after each call, through both upload paths (kernel
    arguments for small uploads, the pinned staging ring for larger ones,
    enough of them to wrap the ring), and every device copy must still hold
    the bytes it was given."""
    import ctypes
    lib = gpu._lib
    host = np.zeros(1 << 20, np.float32)  # 4 MB, reused for every upload
    outs, want = [], []
    sizes = [1, 7, 512, 600, 3000, 1 << 18, 1 << 20] + [1 << 20] * 20
    for k, n in enumerate(sizes):
        host[:n] = np.arange(n, dtype=np.float32) * 0.5 + k
        t = gpu.DeviceTensor.empty((n,), np.float32)
        lib.call("kk_upload", ctypes.c_void_p(t.ptr), host.ctypes.data_as(ctypes.c_void_p), n * 4)
        outs.append(t)
        want.append(host[:n].copy())
        host[:n] = -1.0  # overwrite at once
    for t, w in zip(outs, want):
        assert np.array_equal(t.numpy(), w)
