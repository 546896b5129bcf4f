"""The allocation-free quantised convolution,
kk_conv_integer_scaled_qbias_noalloc, against the regular entry point
kk_conv_integer_scaled_qbias, both through the C ABI: bit-exact outputs on
two calls in a row, the second with a smaller input (the fixed scratch
still holds the first call's contents then); the device pool unchanged
across the allocation-free calls (the regular entry point takes its
workspace from the pool); a convolution whose workspace exceeds the
scratch rejected with a clear error."""
import numpy as np
import pytest

from conftest import assert_bitexact, rng

pytestmark = pytest.mark.gpu


def conv_case(kk, r, cin, cout, k, L, pad, dil, wdt):
    lo, hi = (-128, 128) if wdt == np.int8 else (0, 256)
    D = kk.to_device
    t = {
        "x": D(r.integers(0, 256, (1, cin, L)).astype(np.uint8)),
        "w": D(r.integers(lo, hi, (cout, cin, k)).astype(wdt)),
        "x_zp": D(np.array(r.integers(0, 256), np.uint8)),
        "w_zp": D(np.array(r.integers(lo, hi), wdt)),
        "bias": D(r.normal(0, 0.5, cout).astype(np.float32)),
        "sa": D(np.array(r.uniform(0.005, 0.02), np.float32)),
        "sw": D(np.array(r.uniform(0.001, 0.004), np.float32)),
    }
    lout = L + 2 * pad - dil * (k - 1)
    return t, (1, cout, lout), (1, dil, pad, pad, 1)


def call(kk, entry, out, t, attrs):
    kk._lib.call(entry, out.desc(), t["x"].desc(), t["w"].desc(), t["x_zp"].desc(),
                 t["w_zp"].desc(), t["bias"].desc(), t["sa"].desc(), t["sw"].desc(), *attrs)


def test_noalloc_conv_matches_regular_entry_point(gpu):
    kk = gpu
    r = rng(50)
    # the graph's largest convolution (3.4 MiB of workspace), then a smaller one
    cases = [(1090, 1024, 3, 300, 1, 1, np.uint8), (256, 130, 7, 999, 9, 3, np.int8)]
    for cin, cout, k, L, pad, dil, wdt in cases:
        t, oshape, attrs = conv_case(kk, r, cin, cout, k, L, pad, dil, wdt)
        ref = kk.DeviceTensor.empty(oshape, np.float32)
        call(kk, "kk_conv_integer_scaled_qbias", ref, t, attrs)
        got = kk.DeviceTensor.empty(oshape, np.float32)
        kk.sync()
        before = kk.pool_stats()
        call(kk, "kk_conv_integer_scaled_qbias_noalloc", got, t, attrs)
        kk.sync()
        assert kk.pool_stats() == before, "the allocation-free call changed the pool"
        assert_bitexact(kk.to_host(got), kk.to_host(ref), f"Cin {cin} Cout {cout} K {k}")


def test_noalloc_conv_rejects_a_workspace_beyond_the_scratch(gpu):
    kk = gpu
    r = rng(51)
    t, oshape, attrs = conv_case(kk, r, 2048, 2048, 3, 16, 1, 1, np.uint8)  # 12.6 MB of weights re-laid
    out = kk.DeviceTensor.empty(oshape, np.float32)
    with pytest.raises(kk._lib.KKError, match="allocation-free scratch"):
        call(kk, "kk_conv_integer_scaled_qbias_noalloc", out, t, attrs)
