#!/usr/bin/env python3
"""Writes tests/golden/penalty.npz from the reference library built from its
own sources (oracle/_ref/libcmolref.so, `make -C oracle ref`): the
repetition penalty, alone and inside greedy generation.

- Vectors: cmol_apply_repeat_penalty (reference src/sampler.c:171-184) on
  seeded logits holding positives, negatives, +0 and -0, with windows that
  repeat ids and hold ids out of range, for penalties 0.9 (a no-op), 1.0
  (a no-op), 1.1, 1.3 and 2.0.
- Greedy ids: the reference's cmol_model_forward + cmol_apply_repeat_penalty
  + cmol_sample (temperature 0) through the generate loop's ring of recent
  tokens (reference src/api.c:465-507), for three synthetic models (at weight
  scales where the penalty changes the ids), penalty
  1.3 over a 64-token window and 1.15 over an 8-token window.  Q4_0 models
  go to the reference as their lossless Q8_0 re-encoding.

Run in the container that has /root/reference:
    python tests/golden/make_penalty_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libcmol_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

P = O.P
VOCAB = 512
PENALTIES = (0.9, 1.0, 1.1, 1.3, 2.0)
# (preset, weight std): scales at which the penalty changes the greedy ids
MODELS = (("micro-q8_0", 0.08), ("small-q5_0", 0.08), ("small-q4_0", 0.04))
RUNS = ((1.3, 64), (1.15, 8))
N_PROMPT, N_NEW = 24, 48


def penalty_cases():
    """(logits, window) pairs, seeded."""
    rng = np.random.default_rng(2024)
    cases = []
    for c in range(6):
        lg = (rng.standard_normal(VOCAB) * 3).astype(np.float32)
        lg[rng.integers(0, VOCAB, 40)] = 0.0
        lg[rng.integers(0, VOCAB, 40)] = -0.0
        n = [0, 1, 8, 64, 128, 100][c]
        win = rng.integers(-5, VOCAB + 5, n).astype(np.int32)
        if n > 4:
            win[1::3] = win[0]            # repeated ids are penalised once per occurrence
        cases.append((lg, win))
    return cases


def main():
    if not O.ref_available():
        raise SystemExit("build the reference first: make -C oracle ref")
    R = O.ref()
    R.cmol_apply_repeat_penalty.argtypes = [P, O.C.c_int, P, O.C.c_int, O.C.c_float]
    arrays = {}
    for ci, (lg, win) in enumerate(penalty_cases()):
        arrays[f"case{ci}_logits"] = lg
        arrays[f"case{ci}_window"] = win
        for pi, pen in enumerate(PENALTIES):
            out = lg.copy()
            R.cmol_apply_repeat_penalty(out.ctypes.data, VOCAB, win.ctypes.data, win.size, pen)
            arrays[f"case{ci}_p{pi}"] = out
    arrays["penalties"] = np.array(PENALTIES, np.float32)
    for name, wstd in MODELS:
        spec = synth.PRESETS[name].replace(wstd=wstd)
        arrays[f"{name}_wstd"] = np.float32(wstd)
        path = synth.model_file(spec.replace(transcode_q8=1) if spec.wtype == synth.Q4_0 else spec)
        prompt = synth.tokens(N_PROMPT, 61, spec.vocab)
        arrays[f"{name}_prompt"] = prompt
        for ri, (pen, last_n) in enumerate(RUNS):
            ref = O.RefModel(path, 128)
            arrays[f"{name}_run{ri}_ids"] = ref.generate(prompt, N_NEW, penalty=pen, last_n=last_n)
            ref.close()
    arrays["runs"] = np.array(RUNS, np.float32)
    np.savez_compressed(os.path.join(HERE, "penalty.npz"), **arrays)
    print("wrote penalty.npz")


if __name__ == "__main__":
    main()
