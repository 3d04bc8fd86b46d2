"""Write tests/golden/c4_smollm3_3b.npz: the oracle's prefill of a
2048-token seeded prompt on the SmolLM3-3B-shaped Q4_0 model (Q8_0 tied
embedding, weights ~N(0, 0.02)), then 256 greedy tokens.

Kept: the logits after the prompt at a fixed index sample (every 64th entry
plus the 512 largest), the top-2 margin, the greedy ids with their margins,
and K/V rows of layers 0 and 35 at the prompt-chunk boundaries.

The oracle is the reference's arithmetic restated (oracle/); a full run on
this shape takes about 25 minutes on 8 cores, too long for a test, so its
result travels as this fixture.  Where the reference's own build
(oracle/_ref) exists, the script first checks the oracle against it on the
same weights transcoded losslessly to Q8_0 (the reference has no Q4_0): the
logits of the first prompt positions must be bit-identical.

Usage: python tests/golden/make_c4_golden.py [--threads N]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libcmol_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

PRESET = "smollm3-3b-q4_0"
PROMPT_SEED = 42
N_PROMPT = 2048
N_NEW = 256
KV_LAYERS = (0, 35)
KV_POS = (0, 1, 255, 256, 511, 512, 1023, 1024, 1535, 1536, 2046, 2047)
REF_CHECK_POS = 3


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    args = ap.parse_args()
    spec = synth.PRESETS[PRESET]
    path = synth.model_file(spec)
    prompt = synth.tokens(N_PROMPT, PROMPT_SEED, spec.vocab)
    max_ctx = N_PROMPT + N_NEW + 8
    om = O.Model(path, max_ctx, nthreads=args.threads)

    early = []
    t0 = time.time()
    for p, t in enumerate(prompt):
        lg = om.forward(int(t), p)
        if p < REF_CHECK_POS:
            early.append(lg.copy())
        if p % 128 == 0:
            print(f"prompt {p}/{N_PROMPT} {time.time() - t0:.0f}s", flush=True)
    last = lg.copy()

    if O.ref_available():
        q8 = synth.model_file(spec.replace(transcode_q8=1))
        ref = O.RefModel(q8, 64)
        for p in range(REF_CHECK_POS):
            want = ref.forward(int(prompt[p]), p)
            assert np.array_equal(want.view(np.uint32), early[p].view(np.uint32)), f"oracle != reference at {p}"
        ref.close()
        print("oracle logits bit-identical to the reference's on the first", REF_CHECK_POS, "positions")
        ref_checked = REF_CHECK_POS
    else:
        ref_checked = 0

    k, v = om.kv()
    kv_k = np.stack([k[l, list(KV_POS)] for l in KV_LAYERS]).copy()
    kv_v = np.stack([v[l, list(KV_POS)] for l in KV_LAYERS]).copy()

    order = np.argsort(last, kind="stable")
    top = order[-512:]
    idx = np.unique(np.concatenate([np.arange(0, spec.vocab, 64), top])).astype(np.int32)
    srt = np.sort(last)
    margin = float(srt[-1] - srt[-2])

    ids, margins = [], []
    cur = last
    for i in range(N_NEW):
        nxt = int(np.argmax(cur))   # first index of the maximum, as the reference
        s2 = np.sort(cur)
        ids.append(nxt)
        margins.append(float(s2[-1] - s2[-2]))
        if i + 1 < N_NEW:
            cur = om.forward(nxt, N_PROMPT + i)
        if i % 32 == 0:
            print(f"greedy {i}/{N_NEW} {time.time() - t0:.0f}s", flush=True)

    out = os.path.join(HERE, "c4_smollm3_3b.npz")
    np.savez_compressed(
        out, prompt=prompt, logit_idx=idx, logit_val=last[idx], argmax=np.int32(np.argmax(last)),
        top2_margin=np.float32(margin), ids=np.array(ids, np.int32), id_margins=np.array(margins, np.float32),
        kv_layers=np.array(KV_LAYERS, np.int32), kv_pos=np.array(KV_POS, np.int32), kv_k=kv_k, kv_v=kv_v,
        meta=np.array(json.dumps({"preset": PRESET, "prompt_seed": PROMPT_SEED, "n_prompt": N_PROMPT,
                                  "n_new": N_NEW, "ref_checked_positions": ref_checked,
                                  "threads": args.threads, "seconds": round(time.time() - t0)})))
    print("wrote", out, "min greedy margin", min(margins), "prompt margin", margin)


if __name__ == "__main__":
    main()
