import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libkk's HIP kernels)")


def load_pkg():
    """The product package (its directory name is not an identifier)."""
    return importlib.import_module("best-tts-godot_amd")


@pytest.fixture(scope="session")
def kk():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle():
    from oracle import ref_ops
    return ref_ops


@pytest.fixture(scope="session")
def gpu(kk):
    """Initialised libkk on device 0.  Fails (never skips) without a GPU, so
    a GPU run cannot pass silently."""
    kk._lib.load()
    n = kk.device_count()
    if n < 1:
        pytest.fail("no GPU visible to libkk (kk_device_count == 0)")
    kk.init(0)
    return kk


def rng(seed=0):
    return np.random.default_rng(seed)


def assert_close(got, want, rtol, atol=0.0, floor_rel=0.0, what=""):
    """|got - want| <= atol + rtol*|want| + floor_rel*max|want|, with
    non-finite values counted explicitly (NaN loses every comparison)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    nf_got = int((~np.isfinite(got)).sum())
    nf_want = int((~np.isfinite(want)).sum())
    assert nf_got == nf_want, f"{what}: {nf_got} non-finite values, expected {nf_want}"
    fin = np.isfinite(want)
    if not fin.any():
        return
    scale = float(np.abs(want[fin]).max()) if want.size else 0.0
    err = np.abs(got[fin] - want[fin])
    lim = atol + rtol * np.abs(want[fin]) + floor_rel * scale
    bad = err > lim
    if bad.any():
        i = int(np.argmax(err - lim))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{err.size} elements out of tolerance; worst "
            f"|err|={err[i]:.3e} vs limit {lim[i]:.3e} (want {want[fin][i]:.6e}, "
            f"got {got[fin][i]:.6e})")


def assert_bitexact(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert got.dtype == want.dtype, f"{what}: dtype {got.dtype} != {want.dtype}"
    if got.dtype.kind == "f":
        g = got.view(np.uint32 if got.dtype == np.float32 else np.uint16)
        w = want.view(np.uint32 if want.dtype == np.float32 else np.uint16)
        nd = int((g != w).sum())
        if nd:
            i = int(np.argmax((g != w).reshape(-1)))
            raise AssertionError(f"{what}: {nd}/{got.size} elements differ in bits; first at "
                                 f"{i}: got {got.reshape(-1)[i]!r} want {want.reshape(-1)[i]!r}")
    else:
        assert np.array_equal(got, want), f"{what}: values differ"
