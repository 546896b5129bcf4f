"""Parity of the output stage's kernels (kk_fir, kk_pcm16, kk_fir_pcm16)
with the oracle, through the C ABI (runtime/audio.gd:59-106,
kernels/fir.glsl:35-47, kernels/pcm16.glsl:28-46).

Bars: the FIR within fp32 summation rounding of the oracle -- both add the
taps in order, the device with a fused multiply-add per tap, the oracle with
a product and a sum rounded separately, so they differ by at most a few
units of 2^-24 * sum_k |h_k x_k| per output (held here to 4e-6 of that sum);
PCM16 of the same floats bit-exact (ties excepted: GLSL leaves them to the
implementation, the device rounds them away from zero, as the oracle
does); the fused kernel bit-exact with the two kernels in turn."""
import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def fir_bound(x, h, c):
    """sum_k |h_k x_k| per output, edges clamped, in float64."""
    n, t = x.size, h.size
    xp = np.abs(x.astype(np.float64))[np.clip(np.arange(-c, n - c + t - 1), 0, n - 1)]
    return np.correlate(xp, np.abs(h.astype(np.float64)), mode="valid")


@pytest.mark.parametrize("n,t,c", [
    (2154000, 1023, -1),   # the 128-id waveform's length, the notch filter
    (167400, 1023, -1),    # the 8-id waveform
    (1000, 1023, -1),      # shorter than the filter: clamped edges on both sides
    (1, 1023, -1), (9, 7, 0), (2049, 13, 12), (4100, 8, 3), (333, 1, 0), (12345, 4096, 2047),
])
def test_fir(gpu, oracle, n, t, c):
    r = rng(40)
    x = r.normal(0, 0.3, n).astype(np.float32)
    h = oracle.notch_taps() if t == 1023 else r.normal(0, 0.1, t).astype(np.float32)
    got = gpu.to_host(gpu.ops.fir(gpu.to_device(x.reshape(1, -1)), gpu.to_device(h), c)).reshape(-1)
    cc = (t - 1) // 2 if c < 0 else c
    want = oracle.fir(x, h, cc)
    err = np.abs(got.astype(np.float64) - want)
    bound = 4e-6 * fir_bound(x, h, cc) + 1e-30
    assert (err <= bound).all(), f"max err/bound {float((err / bound).max()):.3g}"


def test_fir_notch_removes_the_hop_tones(gpu, oracle):
    """A waveform carrying the iSTFT's 4800 / 9600 Hz ring: the device filter
    takes both tones down by at least 40 dB and leaves a 1 kHz tone within
    0.1 dB (away from the edges)."""
    t = np.arange(48000) / 24000.0
    ring = (0.1 * np.sin(2 * np.pi * 4800 * t) + 0.05 * np.sin(2 * np.pi * 9600 * t)).astype(np.float32)
    voice = (0.3 * np.sin(2 * np.pi * 1000 * t)).astype(np.float32)
    h = gpu.to_device(oracle.notch_taps())
    y_ring = gpu.to_host(gpu.ops.fir(gpu.to_device(ring), h))[2000:-2000]
    y_voice = gpu.to_host(gpu.ops.fir(gpu.to_device(voice), h))[2000:-2000]
    rms = lambda v: float(np.sqrt(np.mean(np.asarray(v, np.float64) ** 2)))
    assert 20 * np.log10(rms(y_ring) / rms(ring[2000:-2000])) < -40.0
    assert abs(20 * np.log10(rms(y_voice) / rms(voice[2000:-2000]))) < 0.1


@pytest.mark.parametrize("n", [2154000, 167400, 9, 8, 1, 7])
def test_pcm16(gpu, oracle, n):
    r = rng(41)
    x = r.normal(0, 0.6, n).astype(np.float32)  # ~10% beyond +-1: the clamp
    x[: min(n, 4)] = np.array([1.0, -1.0, 2.5, -7.0], np.float32)[: min(n, 4)]
    for gain in (1.0, 0.7):
        raw = gpu.to_host(gpu.ops.pcm16(gpu.to_device(x), gain))
        assert raw.dtype == np.uint8 and raw.size == 2 * n
        np.testing.assert_array_equal(raw.view("<i2"), oracle.pcm16(x, gain))


def test_pcm16_ties_round_away_from_zero(gpu, oracle):
    """Values whose scaled sample is an exact .5: the device (and the oracle)
    round away from zero; GLSL's round() may go either way there, so these
    are parity unpinned against the reference."""
    k = np.array([0, 1, 2, 100, 16383], np.float64)
    x = np.concatenate([(k + 0.5) / 32767.0, -(k + 0.5) / 32767.0]).astype(np.float32)
    s = x.astype(np.float64) * 32767.0
    ties = s == np.floor(s) + 0.5
    got = gpu.to_host(gpu.ops.pcm16(gpu.to_device(x))).view("<i2")
    np.testing.assert_array_equal(got, oracle.pcm16(x))
    assert ties.any()
    np.testing.assert_array_equal(got[ties], (np.sign(s) * np.ceil(np.abs(s)))[ties].astype(np.int16))


@pytest.mark.parametrize("n", [2154000, 1000, 3])
def test_fir_pcm16_fused(gpu, oracle, n):
    r = rng(42)
    x = gpu.to_device(r.normal(0, 0.8, n).astype(np.float32))
    h = gpu.to_device(oracle.notch_taps())
    fused = gpu.to_host(gpu.ops.fir_pcm16(x, h, -1, 0.9))
    two = gpu.to_host(gpu.ops.pcm16(gpu.ops.fir(x, h), 0.9))
    np.testing.assert_array_equal(fused, two)


def test_output_stage_errors(gpu, oracle):
    kk = gpu
    x = kk.to_device(np.zeros(100, np.float32))
    with pytest.raises(kk._lib.KKError, match="taps"):
        kk.ops.fir(x, kk.to_device(np.zeros(4097, np.float32)))
    with pytest.raises(kk._lib.KKError, match="center"):
        kk.ops.fir(x, kk.to_device(np.zeros(5, np.float32)), 5)
    with pytest.raises(kk._lib.KKError, match="fp32"):
        kk.ops.pcm16(kk.to_device(np.zeros(10, np.int32)))
