#!/usr/bin/env python3
"""Writes tests/golden/golden.npz + golden.json from the reference library
built from its own sources (oracle/_ref/libcmolref.so, `make -C oracle ref`).

Every expected value in the fixtures is produced by the reference's code:
cmol_dequant_row, cmol_matmul_scalar / cmol_matmul_avx512, cmol_rms_norm,
cmol_softmax, cmol_swiglu, cmol_rope_apply, and cmol_load +
cmol_model_forward + cmol_apply_repeat_penalty + cmol_sample driven through
the reference's generate-loop semantics.  Q4_0 (absent from the reference)
is expressed as the bit-identical Q8_0 re-encoding (same fp16 scale, codes
nibble-8), so the reference computes the same dequantised values.

Inputs are seeded (numpy PCG64 for kernel vectors, libcmol_amd.synth for
models: integer-only generation, byte-identical on every host).  The SHA-256
of every model file is recorded so tests can check they regenerate the same
bytes.  Run in the container that has /root/reference:
    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libcmol_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests.qdata import SPECIAL_SCALES, random_blocks  # noqa: E402

P = O.P


def q4_to_q8(raw, rows, cols):
    """Lossless Q4_0 -> Q8_0 re-encoding of raw rows."""
    nb = cols // 32
    b4 = raw.reshape(rows, nb, 18)
    b8 = np.zeros((rows, nb, 34), np.uint8)
    b8[:, :, 0:2] = b4[:, :, 0:2]
    lo = (b4[:, :, 2:18] & 0xF).astype(np.int16) - 8
    hi = (b4[:, :, 2:18] >> 4).astype(np.int16) - 8
    b8[:, :, 2:18] = lo.astype(np.int8).view(np.uint8)
    b8[:, :, 18:34] = hi.astype(np.int8).view(np.uint8)
    return b8.reshape(rows, nb * 34)


def ref_dequant(raw, cols, dtype):
    R = O.ref()
    out = np.zeros((raw.shape[0], cols), np.float32)
    for r in range(raw.shape[0]):
        row = np.ascontiguousarray(raw[r])
        R.shim_dequant_row(row.ctypes.data, out[r].ctypes.data, cols, dtype)
    return out


def ref_matmul(kind, raw, b, m, k, dtype):
    R = O.ref()
    b = np.ascontiguousarray(b, np.float32)
    n = b.shape[1]
    out = np.zeros((m, n), np.float32)
    raw = np.ascontiguousarray(raw)
    assert R.shim_matmul(kind, out.ctypes.data, raw.ctypes.data, b.ctypes.data, m, k, n, dtype) == 0
    return out


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


MODEL_CASES = {
    # name: (preset, overrides, prompt_len, n_new, max_ctx)
    "micro_q8_0": ("micro-q8_0", {"wstd": 0.3}, 16, 32, 64),
    "micro_q4_0": ("micro-q4_0", {"wstd": 0.3}, 16, 32, 64),
    "small_q4_0": ("small-q4_0", {"wstd": 0.05}, 12, 24, 64),
    "small_q5_0": ("small-q5_0", {"wstd": 0.05}, 12, 24, 64),
    "small_q8_0_untied": ("small-q8_0-untied", {"wstd": 0.05}, 12, 24, 64),
}


def model_spec(name):
    preset, over, *_ = MODEL_CASES[name]
    return synth.PRESETS[preset].replace(**over)


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libcmolref.so missing: run `make -C oracle ref` first")
    arrays, meta = {}, {"reference_kernel": O.ref().shim_kernel_name().decode()}

    # fp16 -> fp32 of all 65536 halves
    h = np.arange(65536, dtype=np.uint16)
    f = np.zeros(65536, np.float32)
    O.ref().shim_dequant_row(h.ctypes.data, f.ctypes.data, 65536, 1)
    meta["f16_table_sha256"] = hashlib.sha256(f.view(np.uint32).tobytes()).hexdigest()
    arrays["f16_special_in"] = SPECIAL_SCALES
    arrays["f16_special_out"] = f[SPECIAL_SCALES.astype(np.int64)].view(np.uint32)

    # block dequantisation (random + special scales)
    for dt, name in ((8, "q8_0"), (6, "q5_0"), (2, "q4_0")):
        for tag, special in (("rand", False), ("special", True)):
            raw = random_blocks(dt, 24, 128, seed=100 + dt + special, special=special)
            want = ref_dequant(q4_to_q8(raw, 24, 128) if dt == 2 else raw, 128, 8 if dt == 2 else dt)
            arrays[f"deq_{name}_{tag}_in"] = raw
            arrays[f"deq_{name}_{tag}_out"] = want.view(np.uint32)

    # matmul in both reference orders
    rng = np.random.default_rng(7)
    for dt, name in ((8, "q8_0"), (6, "q5_0"), (2, "q4_0")):
        for (m, k, n) in ((16, 128, 1), (33, 256, 1), (8, 64, 3)):
            raw = random_blocks(dt, m, k, seed=m * 1000 + k + n + dt)
            b = rng.standard_normal((k, n)).astype(np.float32)
            key = f"mm_{name}_{m}x{k}x{n}"
            arrays[key + "_a"] = raw
            arrays[key + "_b"] = b
            src, sdt = (q4_to_q8(raw, m, k), 8) if dt == 2 else (raw, dt)
            arrays[key + "_scalar"] = ref_matmul(0, src, b, m, k, sdt).view(np.uint32)
            arrays[key + "_avx512"] = ref_matmul(1, src, b, m, k, sdt).view(np.uint32)
    a32 = rng.standard_normal((5, 37)).astype(np.float32)
    b32 = rng.standard_normal((37, 2)).astype(np.float32)
    arrays["mm_f32_5x37x2_a"], arrays["mm_f32_5x37x2_b"] = a32, b32
    arrays["mm_f32_5x37x2_scalar"] = ref_matmul(0, a32.view(np.uint8), b32, 5, 37, 0).view(np.uint32)
    arrays["mm_f32_5x37x2_avx512"] = ref_matmul(1, a32.view(np.uint8), b32, 5, 37, 0).view(np.uint32)

    # primitives
    R = O.ref()
    x = (rng.standard_normal(576) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(576)).astype(np.float32)
    o = np.zeros_like(x)
    R.shim_rms_norm(x.ctypes.data, w.ctypes.data, o.ctypes.data, 576, np.float32(1e-5))
    arrays["rms_x"], arrays["rms_w"], arrays["rms_out"] = x, w, o.view(np.uint32)
    sm = (rng.standard_normal(300) * 4).astype(np.float32)
    arrays["softmax_in"] = sm.copy()
    R.shim_softmax(sm.ctypes.data, 300)
    arrays["softmax_out"] = sm.view(np.uint32)
    g = (rng.standard_normal(1536) * 3).astype(np.float32)
    u = rng.standard_normal(1536).astype(np.float32)
    so = np.zeros_like(g)
    R.shim_swiglu(g.ctypes.data, u.ctypes.data, so.ctypes.data, 1536)
    arrays["swiglu_g"], arrays["swiglu_u"], arrays["swiglu_out"] = g, u, so.view(np.uint32)
    for pos in (0, 1, 37, 2047):
        q = rng.standard_normal(16 * 128).astype(np.float32)
        k = rng.standard_normal(4 * 128).astype(np.float32)
        arrays[f"rope_{pos}_q"], arrays[f"rope_{pos}_k"] = q.copy(), k.copy()
        R.shim_rope(q.ctypes.data, k.ctypes.data, pos, 16, 4, 128, np.float32(5e6))
        arrays[f"rope_{pos}_qo"], arrays[f"rope_{pos}_ko"] = q.view(np.uint32), k.view(np.uint32)

    # whole models through the reference's own load + forward + sampling
    tmp = os.environ.get("CMOL_MODEL_DIR", "/tmp/cmol_models")
    meta["models"] = {}
    for name, (preset, over, plen, n_new, max_ctx) in MODEL_CASES.items():
        spec = model_spec(name)
        path = synth.model_file(spec, tmp)
        # only Q4_0 needs the Q8_0 re-encoding; Q5_0/Q8_0 run natively
        ref_path = synth.model_file(spec.replace(transcode_q8=1), tmp) \
            if 2 in (spec.wtype, spec.embd_type) else path
        prompt = synth.tokens(plen, 42, spec.vocab)
        rm = O.RefModel(ref_path, max_ctx)
        toks = rm.generate(prompt, n_new)
        rm.close()
        rm = O.RefModel(ref_path, max_ctx)
        for p, t in enumerate(prompt):
            lg = rm.forward(int(t), p)
        rm.close()
        arrays[f"model_{name}_prompt"] = prompt
        arrays[f"model_{name}_tokens"] = toks
        arrays[f"model_{name}_last_prompt_logits"] = lg.view(np.uint32)
        meta["models"][name] = {"preset": preset, "overrides": over, "max_ctx": max_ctx,
                                "sha256": sha256(path), "n_new": n_new}
        print(name, toks[:12].tolist(), flush=True)

    # SmolLM2-135M shape, Q8_0: 32-token prompt, 128 greedy tokens (reference)
    spec = synth.PRESETS["smollm2-135m-q8_0"]
    path = synth.model_file(spec, tmp)
    prompt = synth.tokens(32, 42, spec.vocab)
    rm = O.RefModel(path, 256)
    toks = rm.generate(prompt, 128)
    rm.close()
    arrays["smollm2_135m_prompt"], arrays["smollm2_135m_tokens"] = prompt, toks
    meta["smollm2_135m_sha256"] = sha256(path)
    print("smollm2-135m", toks[:16].tolist(), flush=True)

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    with open(os.path.join(HERE, "golden.json"), "w") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)
    print("wrote", len(arrays), "arrays")


if __name__ == "__main__":
    main()
