#!/usr/bin/env python3
"""Writes tests/golden/kquant.npz: Q4_K / Q6_K vectors from the reference
library built from its own sources (oracle/_ref/libcmolref.so).

Every expected value is the reference's own output: cmol_dequant_row on
seeded random super-blocks (random codes and packed 6-bit / int8 scales;
fp16 super-block scales either in a normal range or drawn from the IEEE
special set: zeros, subnormals, max, inf, NaN), and cmol_matmul_scalar /
cmol_matmul_avx512 on seeded shapes with n = 1 and n = 3, and the greedy
continuation (cmol_load, forward, argmax) of synthetic models whose layers
are Q4_K or Q6_K.  Run in the container that has /root/reference:
    python tests/golden/make_kquant_golden.py
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
from tests.golden.make_golden import ref_dequant, ref_matmul  # noqa: E402
from tests.qdata import random_blocks  # noqa: E402

KTYPES = {"q4_k": 12, "q6_k": 14}
DEQ_SHAPE = (8, 1024)
MM_SHAPES = [(16, 512, 1), (24, 768, 3)]
MODEL_PRESETS = ["small-q4_k", "small-q6_k-untied", "small-q4_k_m"]


def main():
    arrays = {}
    for name, dt in KTYPES.items():
        for tag, special in (("rand", False), ("special", True)):
            rows, cols = DEQ_SHAPE
            raw = random_blocks(dt, rows, cols, seed=500 + dt + special, special=special)
            arrays[f"deq_{name}_{tag}_raw"] = raw
            arrays[f"deq_{name}_{tag}_out"] = ref_dequant(raw, cols, dt).view(np.uint32)
        for m, k, n in MM_SHAPES:
            raw = random_blocks(dt, m, k, seed=600 + dt + m)
            b = np.random.default_rng(700 + m).standard_normal((k, n)).astype(np.float32)
            key = f"mm_{name}_{m}x{k}x{n}"
            arrays[key + "_raw"] = raw
            arrays[key + "_b"] = b
            arrays[key + "_scalar"] = ref_matmul(0, raw, b, m, k, dt).view(np.uint32)
            arrays[key + "_avx512"] = ref_matmul(1, raw, b, m, k, dt).view(np.uint32)
    # whole models with K-quant layers: the reference's greedy continuation
    with tempfile.TemporaryDirectory() as td:
        for preset in MODEL_PRESETS:
            spec = synth.PRESETS[preset].replace(wstd=0.08)
            path = synth.model_file(spec, td)
            prompt = synth.tokens(16, 42, spec.vocab)
            rm = O.RefModel(path, 128)
            arrays[f"model_{preset}_prompt"] = prompt
            arrays[f"model_{preset}_ids"] = rm.generate(prompt, 48)
            rm.close()
    out = os.path.join(HERE, "kquant.npz")
    np.savez_compressed(out, **arrays)
    print("wrote", out, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
