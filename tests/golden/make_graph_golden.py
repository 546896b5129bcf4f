"""Writes graph_golden_t<N>.npz: checkpoints of the synthetic Kokoro graph
(the packaged structure + seeded random learned weights, N phoneme ids
(default 8; 128 for the graph the benchmark times), speed 1) computed by the
CPU oracle (oracle/kpk_run.py).

Checkpoints (tensor ids of the packed graph):
  2430  pre-round durations              (/encoder/Div_output_0)
  2432  clipped durations                (/encoder/Clip_output_0)
  1165  text-encoder LSTM output
  2892  F0 curve                         (/encoder/F0_proj/Conv_output_0)
  3037  STFT of the harmonic source      -- its first 1024 frames
  3304  decoder block decode.0 output    -- its first 16 frames
  5038  conv_post output (log-magnitude and phase logits) -- first 1024 frames
  5092  the waveform, whole, as float16 (its values are within +-2: float16
        holds them to 2^-11 relative, far inside the waveform gate).
With more than 8 ids the last frames of the three long checkpoints are kept
too (t<id>_tail), so the end of the utterance is checked as well as its
start, and so is every tensor the rest of the graph reads from the part up
to the durations (b<id>: the text encoder's output, the prosody features,
the rounded durations and the style projections, 0.8 MB at 128 ids), from
which a test runs the decoder part on its own.
Run from the repository root: python tests/golden/make_graph_golden.py [N]
(N = 128 takes about 22 minutes of CPU time on 2.7 GHz Xeon cores.)
"""
import importlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

N_IDS = int(sys.argv[1]) if len(sys.argv) > 1 else 8
CHECK = [2430, 2432, 1165, 2892, 3037, 3304, 5038]
HEAD = {3037: (1, 1024), 3304: (2, 16), 5038: (2, 1024)}  # tensor id: (time axis, frames kept)


def head(v, axis, n):
    return np.ascontiguousarray(np.take(np.asarray(v), np.arange(min(n, v.shape[axis])), axis=axis))


def tail(v, axis, n):
    m = v.shape[axis]
    return np.ascontiguousarray(np.take(np.asarray(v), np.arange(max(0, m - n), m), axis=axis))


def boundary(g, weights):
    """Non-weight tensors made up to the node that writes the rounded
    durations (2432) and read after it."""
    idx = next(i for i, n in enumerate(g["nodes"]) if 2432 in n[2])
    made = {int(v) for v in g["inputs"].values()}
    for n in g["nodes"][:idx + 1]:
        made |= {t for t in n[2] if t >= 0}
    read = set()
    for n in g["nodes"][idx + 1:]:
        read |= {t for t in n[1] if t >= 0}
    return sorted((made & read) - {int(k) for k in weights})


def main():
    from oracle import kpk_run
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    w = kkg.synth_weights(g, 0)
    ids, style, speed = kkg.synth_inputs(N_IDS, 0)
    bnd = boundary(g, w) if N_IDS > 8 else []
    t = time.time()
    wav, cap = kpk_run.run(g, w, ids, style, speed, capture=CHECK + bnd)
    print(f"oracle graph: {time.time() - t:.1f} s, waveform {wav.shape}")
    out = {"ids": ids, "style": style, "wave_len": np.array(wav.size),
           "wave_f16": np.asarray(wav, np.float32).reshape(-1).astype(np.float16)}
    for k in CHECK:
        v = np.asarray(cap[k])
        out[f"t{k}"] = head(v, *HEAD[k]) if k in HEAD else v
        if k in HEAD and N_IDS > 8:
            out[f"t{k}_tail"] = tail(v, *HEAD[k])
    for k in bnd:
        out[f"b{k}"] = np.asarray(cap[k])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"graph_golden_t{N_IDS}.npz")
    np.savez_compressed(path, **out)
    pre = np.asarray(cap[2430]).reshape(-1)
    print("durations", np.asarray(cap[2432]).reshape(-1), "min distance to .5:",
          float(np.abs(pre - np.floor(pre) - 0.5).min()))
    w64 = np.asarray(wav, np.float64).reshape(-1)
    print(f"waveform rms {np.sqrt((w64 ** 2).mean()):.4f}, max {np.abs(w64).max():.4f}")
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
