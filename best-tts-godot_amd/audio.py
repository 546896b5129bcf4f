"""The waveform's output stage (KokoroAudio, addons/best-tts/runtime/audio.gd):
the notch filter's taps on the host, the FIR and the 16-bit PCM conversion
on the device.

Kokoro's iSTFT overlap-adds with hop 5, so the model's output carries a
steady tone at 24000 / 5 = 4800 Hz and its octave (audio.gd:11-14); the
reference removes both with a 1023-tap linear-phase notch filter before the
PCM conversion (audio.gd:59-106).
"""
import numpy as np

from . import ops

SAMPLE_RATE = 24000
TONE_HZ = (4800.0, 9600.0)
TONE_BW = 80.0
TONE_TAPS = 1023


def notch_taps(sample_rate=SAMPLE_RATE, tones=TONE_HZ, bw=TONE_BW, n=TONE_TAPS):
    """float32 taps of a filter flat except for a null at each tone: a unit
    centre tap minus a Blackman-windowed sinc band-pass [f - bw, f + bw] per
    tone (audio.gd:30-45), evaluated in double and rounded to float32 after
    each tone (GDScript's double arithmetic into a PackedFloat32Array)."""
    centre = (n - 1) // 2
    k = np.arange(n, dtype=np.float64)
    offset = k - centre
    phase = 2.0 * np.pi * k / (n - 1)
    blackman = 0.42 - 0.5 * np.cos(phase) + 0.08 * np.cos(2.0 * (2.0 * np.pi) * k / (n - 1))

    def lowpass(fc):  # 2 fc sinc(2 fc m), sinc(x) = sin(pi x) / (pi x), 1 near 0
        arg = 2.0 * fc * offset
        val = np.ones(n)
        nz = np.abs(arg) >= 1e-9
        val[nz] = np.sin(np.pi * arg[nz]) / (np.pi * arg[nz])
        return 2.0 * fc * val

    taps = np.zeros(n, np.float32)
    taps[centre] = 1.0
    for tone in tones:
        band = (lowpass((tone + bw) / sample_rate) - lowpass((tone - bw) / sample_rate)) * blackman
        taps = (taps.astype(np.float64) - band).astype(np.float32)
    return taps


def to_pcm16(wave, taps=None, gain=1.0):
    """Device waveform -> device PCM16 bytes (uint8 [2 * samples]): the notch
    FIR first when `taps` (a device tensor) is given, fused into the same
    pass."""
    if taps is None:
        return ops.pcm16(wave, gain)
    return ops.fir_pcm16(wave, taps, -1, gain)


__all__ = ["notch_taps", "to_pcm16", "SAMPLE_RATE", "TONE_HZ", "TONE_BW", "TONE_TAPS"]
