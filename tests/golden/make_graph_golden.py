"""Writes graph_golden_t8.npz: checkpoints of the synthetic Kokoro graph
(structure fixture kokoro_graph.json.gz + seeded random learned weights,
8 phoneme ids) computed by the CPU oracle (oracle/kpk_run.py).

Checkpoints (tensor ids of the packed graph):
  2430  pre-round durations  (/encoder/Div_output_0)
  2432  clipped durations    (/encoder/Clip_output_0)
  1165  text-encoder LSTM output
  3037  STFT of the harmonic source
  5092  the waveform -- stored as its length, its first 4096 samples and the
        RMS of every 1024-sample block.
Run from the repository root: python tests/golden/make_graph_golden.py
"""
import importlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

N_IDS = 8
CHECK = [2430, 2432, 1165, 3037]


def block_rms(w, block=1024):
    w = np.asarray(w, np.float64).reshape(-1)
    n = len(w) // block
    return np.sqrt((w[:n * block].reshape(n, block) ** 2).mean(1)).astype(np.float32)


def main():
    from oracle import kpk_run
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph(kkg.default_graph_path())
    w = kkg.synth_weights(g, 0)
    ids, style, speed = kkg.synth_inputs(N_IDS, 0)
    t = time.time()
    wav, cap = kpk_run.run(g, w, ids, style, speed, capture=CHECK)
    print(f"oracle graph: {time.time() - t:.1f} s, waveform {wav.shape}")
    out = {"ids": ids, "style": style, "wave_len": np.array(wav.size),
           "wave_head": wav.reshape(-1)[:4096].astype(np.float32),
           "wave_block_rms": block_rms(wav)}
    for k in CHECK:
        out[f"t{k}"] = np.asarray(cap[k])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"graph_golden_t{N_IDS}.npz")
    np.savez_compressed(path, **out)
    pre = np.asarray(cap[2430]).reshape(-1)
    print("durations", np.asarray(cap[2432]).reshape(-1), "min distance to .5:",
          float(np.abs(pre - np.floor(pre) - 0.5).min()))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
