"""Pins the oracle's output stage (notch taps, FIR, PCM16) on the CPU without
retyping its formulas: the taps against scipy's window-method band-pass
design and the filter's own frequency response, the FIR against direct
convolution of the edge-clamped signal and a brute-force loop, PCM16
against known answers.  Also: the product's host-side taps equal the
oracle's bit for bit.  (runtime/audio.gd:30-106, kernels/fir.glsl:35-47,
kernels/pcm16.glsl:28-46.)"""
import importlib

import numpy as np
import pytest
from scipy import signal

from conftest import rng


def response_db(h, freq, sr=24000):
    k = np.arange(h.size)
    return 20 * np.log10(abs(np.sum(h.astype(np.float64) * np.exp(-2j * np.pi * freq / sr * k))))


def test_notch_taps_design(oracle):
    """Symmetric 1023 taps; equal to a unit impulse minus scipy's
    Blackman-window band-pass designs (unscaled) at 4800 +- 80 and 9600 +- 80
    Hz; a null of at least 40 dB at both tones (the design aims at 50) and
    less than 0.1 dB off unity at DC and away from the tones."""
    h = oracle.notch_taps()
    assert h.dtype == np.float32 and h.size == 1023
    np.testing.assert_array_equal(h, h[::-1])
    ref = np.zeros(1023)
    ref[511] = 1.0
    for f0 in (4800.0, 9600.0):
        ref -= signal.firwin(1023, [f0 - 80.0, f0 + 80.0], window="blackman", pass_zero=False,
                             scale=False, fs=24000.0)
    np.testing.assert_allclose(h.astype(np.float64), ref, rtol=0, atol=2e-7)
    for tone in (4800.0, 9600.0):
        assert response_db(h, tone) < -40.0
    for f in (0.0, 200.0, 1000.0, 3000.0, 4500.0, 7000.0, 9000.0, 11000.0):
        assert abs(response_db(h, f)) < 0.1, f


@pytest.mark.parametrize("mistake", ["hamming", "one_tone", "bw_halved"])
def test_notch_taps_planted_mistake(oracle, mistake):
    """Taps built with a plausible mistake -- a Hamming window for the
    Blackman, a tone left out, half the bandwidth -- fail the comparison of
    the design test above (its tolerance can tell them apart)."""
    h = oracle.notch_taps().astype(np.float64)
    bad = np.zeros(1023)
    bad[511] = 1.0
    tones = (4800.0,) if mistake == "one_tone" else (4800.0, 9600.0)
    bw = 40.0 if mistake == "bw_halved" else 80.0
    win = "hamming" if mistake == "hamming" else "blackman"
    for f0 in tones:
        bad -= signal.firwin(1023, [f0 - bw, f0 + bw], window=win, pass_zero=False, scale=False,
                             fs=24000.0)
    assert np.abs(bad - h).max() > 1e-5


def test_product_taps_equal_oracle(oracle):
    audio = importlib.import_module("best-tts-godot_amd.audio")
    np.testing.assert_array_equal(audio.notch_taps(), oracle.notch_taps())
    np.testing.assert_array_equal(audio.notch_taps(16000, (1000.0,), 50.0, 255),
                                  oracle.notch_taps(16000, (1000.0,), 50.0, 255))


def test_fir_against_convolution(oracle):
    r = rng(31)
    x = r.normal(0, 0.3, 5000).astype(np.float32)
    h = r.normal(0, 0.05, 63).astype(np.float32)
    c = 31
    got = oracle.fir(x, h, c).astype(np.float64)
    xp = np.concatenate([np.full(c, x[0]), x, np.full(h.size - 1 - c, x[-1])]).astype(np.float64)
    want = np.correlate(xp, h.astype(np.float64), mode="valid")
    assert want.size == x.size
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_fir_brute_force_edges_and_impulse(oracle):
    r = rng(32)
    for n, t, c in [(1, 5, 2), (7, 9, 0), (20, 4, 3), (50, 13, 6)]:
        x = r.normal(0, 1, n).astype(np.float32)
        h = r.normal(0, 1, t).astype(np.float32)
        want = np.zeros(n, np.float64)
        for i in range(n):
            for k in range(t):
                want[i] += float(h[k]) * float(x[min(max(i - c + k, 0), n - 1)])
        np.testing.assert_allclose(oracle.fir(x, h, c), want, rtol=1e-5, atol=1e-6)
    h = oracle.notch_taps()
    imp = np.zeros(4000, np.float32)
    imp[2000] = 1.0
    y = oracle.fir(imp, h)
    np.testing.assert_array_equal(y[2000 - 511:2000 + 512], h[::-1])  # the impulse response is the taps
    dc = oracle.fir(np.full(3000, 0.25, np.float32), h)
    np.testing.assert_allclose(dc, 0.25 * np.sum(h.astype(np.float64)), rtol=1e-5)


def test_pcm16_known_answers(oracle):
    x = np.array([0.0, 1.0, -1.0, 2.0, -3.0, 0.25, -0.25, 1 / 32767, -1 / 32767, 0.999, 1e-9],
                 np.float32)
    want = np.array([0, 32767, -32767, 32767, -32767, 8192, -8192, 1, -1, 32734, 0], np.int16)
    np.testing.assert_array_equal(oracle.pcm16(x), want)
    np.testing.assert_array_equal(oracle.pcm16(np.array([4.0, -0.5], np.float32), 0.25),
                                  np.array([32767, -4096], np.int16))
    # little-endian byte stream, as the reference reads it back
    assert oracle.pcm16(np.array([1.0], np.float32)).tobytes() == b"\xff\x7f"


@pytest.mark.parametrize("planted", ["no_clamp", "truncate"])
def test_pcm16_planted_mistakes(oracle, planted):
    """Versions with the clamp left out, or truncation for rounding, fail the
    known answers above."""
    x = np.array([2.0, 0.25 + 0.9 / 32767], np.float32)
    v = x.astype(np.float64) * 32767.0
    bad = v if planted == "no_clamp" else np.clip(x, -1, 1).astype(np.float64) * 32767.0
    bad = np.trunc(bad) if planted == "truncate" else np.rint(bad)
    assert not np.array_equal(bad.astype(np.int64), oracle.pcm16(x).astype(np.int64))
