"""Per-stage timeline of the persistent decode kernel (profiling aid).

    python3 -m libcmol_amd.persist_marks [preset] [context] [tokens]

Loads a synthetic model (libcmol_amd.synth preset, default
smollm3-3b-q4_0) with the persistent kernel and its stage marks switched on
(CMOL_PERSIST=1, CMOL_PERSIST_TRACE=1), fills one session's KV cache with
`context` synthetic positions and decodes `tokens` steps.  For the last
steps it reads cmolhip_persist_trace (work-group 0's start and end) and
cmolhip_persist_marks ([stage][work-group][8] wall-clock stamps, 100 MHz)
and prints, per stage kind, the mean over layers of:

  wait   io waves: start of polling the stage input -> input complete
  stage  io waves: input complete -> mac waves start the products
  mac    mac waves: products
  epi    mac waves: products done -> outputs issued
  lag    last output of the previous stage -> last work-group's input complete

plus the LM head and the whole token.  Times in microseconds.
"""
from __future__ import annotations

import os
import sys
import warnings

import numpy as np

STAGES = ("qkv", "attention", "merge", "wo", "gate_up", "down")
MARKS = 8
TICK_US = 0.01   # wall clock: 100 MHz


def _rel(m, t0):
    x = m.astype(np.float64)
    x[x <= 0] = np.nan
    return (x - t0) * TICK_US


def _nanmean(a):
    a = np.asarray(a, np.float64)
    return float(np.nanmean(a)) if np.isfinite(a).any() else float("nan")


def collect(preset="smollm3-3b-q4_0", context=2048, tokens=6, keep=4):
    os.environ["CMOL_PERSIST"] = "1"
    os.environ["CMOL_PERSIST_TRACE"] = "1"
    from libcmol_amd import native, synth
    spec = synth.PRESETS[preset]
    m = native.Model(synth.model_file(spec), max_ctx=context + tokens + 8, max_sessions=1)
    if not m.persistent:
        m.close()
        raise SystemExit(f"{preset}: the persistent kernel does not take this model")
    s = m.acquire()
    s.fill_kv(context, seed=3)
    ns = 2 + 6 * spec.n_layers
    marks = np.zeros(ns * 1024 * MARKS, np.uint64)
    trace = np.zeros(2, np.uint64)
    out = []
    tok = 1
    for i in range(tokens):
        marks[:] = 0
        tok, _ = s.forward(tok, context + i)
        native.lib().cmolhip_persist_trace(m.device, trace.ctypes.data, 2)
        nwg = native.lib().cmolhip_persist_marks(m.device, marks.ctypes.data, marks.size)
        if i >= tokens - keep and nwg > 0:
            out.append((trace.astype(np.int64).copy(),
                        marks[:ns * nwg * MARKS].reshape(ns, nwg, MARKS).astype(np.int64).copy()))
    m.close()
    return spec, out


def summarize(spec, runs):
    lines = []
    tok_us = [float(t[1] - t[0]) * TICK_US for t, _ in runs]
    lines.append(f"token: {np.mean(tok_us):.1f} us (work-group 0, {len(runs)} tokens)")
    rows = {k: [] for k in STAGES}
    head = []
    for t, M in runs:
        R = _rel(M, t[0])
        prev_last = np.nanmax(R[0][:, 0]) if np.isfinite(R[0][:, 0]).any() else 0.0
        for st in range(1, M.shape[0] - 1):
            r = R[st]
            name = STAGES[(st - 1) % 6]
            ready_last = np.nanmax(r[:, 1]) if np.isfinite(r[:, 1]).any() else np.nan
            out_last = np.nanmax(r[:, 2]) if np.isfinite(r[:, 2]).any() else np.nan
            rows[name].append([_nanmean(r[:, 1] - r[:, 0]), _nanmean(r[:, 3] - r[:, 1]), _nanmean(r[:, 4] - r[:, 3]),
                               _nanmean(r[:, 2] - r[:, 4]), ready_last - prev_last, out_last - prev_last])
            if np.isfinite(out_last):
                prev_last = out_last
        r = R[-1]
        head.append([np.nanmin(r[:, 0]), np.nanmax(r[:, 1]), np.nanmax(r[:, 2])])
    lines.append(f"{'stage':10s} {'wait':>7s} {'stage':>7s} {'mac':>7s} {'epi':>7s} {'lag':>7s} {'span':>7s}")
    total = 0.0
    for name in STAGES:
        a = np.nanmean(np.array(rows[name], np.float64), 0)
        total += a[5]
        lines.append(f"{name:10s} " + " ".join(f"{v:7.2f}" for v in a))
    lines.append(f"layer (sum of spans): {total:.1f} us x {spec.n_layers} layers")
    h = np.nanmean(np.array(head), 0)
    lines.append(f"lm head: input complete {h[1] - h[0]:.1f} us after its poll starts, outputs at +{h[2] - h[1]:.1f} us")
    return "\n".join(lines)


def main(argv):
    warnings.simplefilter("ignore", RuntimeWarning)   # stages without io or mac marks
    preset = argv[1] if len(argv) > 1 else "smollm3-3b-q4_0"
    context = int(argv[2]) if len(argv) > 2 else 2048
    tokens = int(argv[3]) if len(argv) > 3 else 6
    spec, runs = collect(preset, context, tokens)
    print(f"{preset}, context {context}")
    print(summarize(spec, runs))


if __name__ == "__main__":
    main(sys.argv)
