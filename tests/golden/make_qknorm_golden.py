#!/usr/bin/env python3
"""Writes tests/golden/qknorm.npz: synthetic models with QK-norm
(attn_q_norm / attn_k_norm, a per-head RMSNorm of q and k before RoPE,
reference src/attn.c:62-80) run by the reference library built from its own
sources (oracle/_ref/libcmolref.so): the greedy continuation of a prompt and
the logits after the prompt.  Run in the container that has /root/reference:
    python tests/golden/make_qknorm_golden.py
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

# name -> model (d_head 64 and 128; with and without NoPE layers)
MODELS = {
    "qkn_q8_0": ("small-q8_0-untied", {"qk_norm": 1}),
    "qkn_q5_0_nope": ("small-q5_0", {"qk_norm": 1, "nope_interval": 2}),
    "qkn_q4_k": ("small-q4_k", {"qk_norm": 1}),
    "qkn_q8_0_dh128": (None, {}),
    # SmolLM3 architecture key, NoPE, and a rope.scaling.type (YARN) key that
    # the reference records but does not apply (src/gguf.c:384-389)
    "qkn_smollm3_yarn": ("small-q8_0-untied", {"qk_norm": 1, "arch_smollm3": 1, "nope_interval": 2,
                                               "rope_scaling": 1}),
}


def spec_of(name):
    preset, kw = MODELS[name]
    if preset is None:
        return synth.ModelSpec(2, 256, 2, 1, 512, 1024, ctx_len=1024, wtype=synth.Q8_0,
                               embd_type=synth.Q8_0, qk_norm=1, wstd=0.08)
    return synth.PRESETS[preset].replace(wstd=0.08, **kw)


def main():
    arrays = {}
    with tempfile.TemporaryDirectory() as td:
        for name in MODELS:
            spec = spec_of(name)
            path = synth.model_file(spec, td)
            prompt = synth.tokens(16, 42, spec.vocab)
            rm = O.RefModel(path, 128)
            for p, t in enumerate(prompt):
                lg = rm.forward(int(t), p)
            arrays[f"{name}_prompt"] = prompt
            arrays[f"{name}_prompt_logits"] = lg
            rm.close()
            rm = O.RefModel(path, 128)
            arrays[f"{name}_ids"] = rm.generate(prompt, 40)
            rm.close()
    out = os.path.join(HERE, "qknorm.npz")
    np.savez_compressed(out, **arrays)
    print("wrote", out)


if __name__ == "__main__":
    main()
