#!/usr/bin/env python3
"""Writes tests/golden/generate_edges.npz: the reference's generate-loop stop
rules (src/api.c:443-521) on synthetic models, from the reference library
built from its own sources (oracle/_ref/libcmolref.so):
  * EOS: a model whose tokenizer.ggml.eos_token_id is a token its own greedy
    continuation produces; the reference emits it and stops;
  * context full: a 24-position context after a 16-token prompt; the
    reference emits the token sampled at the last position and stops.
Run in the container that has /root/reference:
    python tests/golden/make_generate_golden.py
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libcmol_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

BASE = "small-q8_0-untied"
CTX_FULL = 24


def eos_spec(eos_id=-1):
    return synth.PRESETS[BASE].replace(wstd=0.08, eos_id=eos_id)


def main():
    arrays = {}
    with tempfile.TemporaryDirectory() as td:
        prompt = synth.tokens(16, 42, synth.PRESETS[BASE].vocab)
        arrays["prompt"] = prompt
        # EOS: the sixth token of the free continuation becomes the EOS id
        rm = O.RefModel(synth.model_file(eos_spec(), td), 128)
        free = rm.generate(prompt, 40)
        rm.close()
        eos = int(free[5])
        rm = O.RefModel(synth.model_file(eos_spec(eos), td), 128)
        arrays["eos_id"] = np.array([eos], np.int32)
        arrays["eos_ids"] = rm.generate(prompt, 40)
        rm.close()
        # context full: 24 positions, 16-token prompt, room for 64 tokens asked
        rm = O.RefModel(synth.model_file(eos_spec(), td), CTX_FULL)
        arrays["ctx_full_ids"] = rm.generate(prompt, 64)
        rm.close()
    out = os.path.join(HERE, "generate_edges.npz")
    np.savez_compressed(out, **arrays)
    print("wrote", out, {k: v.tolist() for k, v in arrays.items() if k != "prompt"})


if __name__ == "__main__":
    main()
