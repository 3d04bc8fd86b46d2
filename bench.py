#!/usr/bin/env python3
"""bench.py — decode throughput of libcmol's MI355X path on synthetic models.

Headline (`value`): single-session greedy decode tokens/s of the
SmolLM3-3B-shaped Q4_0 model (Q8_0 tied embedding/LM head) after a
2048-token prompt; one step = one decode token through the whole model.
Also reported on the same line:
  * 32-session lock-step decode tokens/s (fp16 KV, ragged contexts drawn
    log-uniformly from 512 to 16384, synthetic KV contents);
  * the isolated Q4_0 matvecs 11008x2048 and 2048x11008 at batch 1 and 8 with
    64 rotating weight copies (defeating the 256 MB Infinity Cache), timed with
    HIP events on the stream they run on -> `roofline`;
  * the SmolLM2-135M-shaped Q8_0 single session (32-token prompt + 128 greedy
    tokens, also as effective weight GB/s) and the SmolLM2-360M-shaped Q5_0
    16-session lock-step decode (contexts uniform in 64..1024);
  * the roofline kernel's HBM traffic from two rocprofv3 counter passes run
    by this script (FETCH_SIZE, WRITE_SIZE, scaled by a copy of known size);
  * the oracle's (CPU restatement of the reference) decode of the same
    configurations on bounded samples, one session per thread as the
    reference runs them -> `cpu_baseline`.
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import libcmol_amd.native as native  # noqa: E402
from libcmol_amd import hiprt, synth  # noqa: E402

METRIC = "decode tok/s SmolLM3-3B Q4_0 (1 & 32 sessions); matvec HBM GB/s % of peak"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense f16 MFMA, MI355X


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


BLOCK = {synth.Q4_0: (32, 18), synth.Q5_0: (32, 22), synth.Q8_0: (32, 34),
         synth.Q4_K: (256, 144), synth.Q6_K: (256, 210)}
DT_NAME = {synth.Q4_0: "Q4_0", synth.Q5_0: "Q5_0", synth.Q8_0: "Q8_0", synth.Q4_K: "Q4_K",
           synth.Q6_K: "Q6_K"}


def q4_bytes(m, k, n, dtype=synth.Q4_0):
    """Algorithmic HBM bytes of one matvec launch: the weight blocks in their
    GGUF size (Q4_0: 18 bytes per 32 weights; Q4_K 144 / Q6_K 210 per 256),
    the activation operand (an f16 high and an f16 low part per input and
    vector) and the fp32 outputs."""
    bv, bb = BLOCK[dtype]
    return m * (k // bv) * bb + 4 * k * n + 4 * m * n


def bench_matvec(rows, cols, n, copies, launches, fold=None, dtype=synth.Q4_0):
    """Average duration of the matvec kernel (Q4_0 unless `dtype`) over `copies` distinct
    weight buffers (defeating the 256 MB Infinity Cache): every launch records
    a pair of HIP events at the kernel's own start and end (on the stream it
    runs on).  The weights use the fold a model serving n sessions gives this
    shape unless `fold` is given.  More than 32 vectors run the tiled MFMA
    GEMM of the prompt pass."""
    if fold is None:
        fold = native.lib().cmolhip_pick_fold(rows, cols, n)
    w = synth.normal(rows * cols, seed=1234, stream=rows * 7 + cols, std=0.02)
    raw = synth.quantize(dtype, w).reshape(rows, -1)
    tensor_bytes = native.lib().cmolhip_qtensor_bytes(dtype, rows, cols, fold)
    arena = (copies * (tensor_bytes + 4096) + raw.nbytes + n * cols * 4 + n * rows * 4
             + native.lib().cmolhip_act_bytes(cols, n) + (64 << 20))
    ctx = native.Ctx(arena)
    stg = ctx.alloc(raw.nbytes)
    ts = [ctx.qtensor([raw], dtype, cols, [rows], staging_bytes=raw.nbytes, staging=stg, fold=fold)
          for _ in range(copies)]
    x = np.random.default_rng(1).standard_normal((n, cols)).astype(np.float32)
    dx = ctx.upload(x)
    dy = ctx.alloc(n * rows * 4)
    op, _ = ctx.act_prepare(ts[0], dx, n)
    L = native.lib()

    def launch(i, ev=None):
        native.check(L.cmolhip_gemm_prepared_timed(
            ctx.h, C.byref(ts[i % copies]), C.c_void_p(op), n, None, 0.0, C.c_void_p(dy),
            ev.a if ev else None, ev.b if ev else None), "gemm_prepared")

    for i in range(min(copies, 8)):
        launch(i)
    native.check(L.cmolhip_synchronize(ctx.h))
    # events recorded by each launch at the kernel's own start and end
    evs = [hiprt.EventTimer(ctx.stream()) for _ in range(launches)]
    for i, ev in enumerate(evs):
        launch(i, ev)
    native.check(L.cmolhip_synchronize(ctx.h))
    per_launch_s = sum(ev.elapsed() for ev in evs) / 1e3 / launches
    for ev in evs:
        ev.close()
    ctx.close()
    b = q4_bytes(rows, cols, n, dtype)
    flops = 2.0 * rows * cols * n
    out = {"shape": f"{rows}x{cols}", "dtype": DT_NAME[dtype], "n": n, "fold": fold,
           "us_per_launch": per_launch_s * 1e6,
           "bytes_per_launch": b, "GBps": b / per_launch_s / 1e9,
           "frac_of_peak": b / per_launch_s / 1e9 / HBM_PEAK_GBPS}
    if n > 32:
        # the tiled GEMM issues two f16 products per weight and vector (the
        # operand's high and low parts): useful and issued MFMA rates
        out.update(useful_TFLOPs=flops / per_launch_s / 1e12,
                   mfma_TFLOPs=2 * flops / per_launch_s / 1e12,
                   mfma_frac_of_peak=2 * flops / per_launch_s / 1e12 / MFMA_F16_PEAK_TFLOPS)
    return out


def bench_decode_1(path, spec, prompt_len, steps, warmup, synthetic_ctx=0, prefill_chunk=0):
    """Single-session greedy decode after a prompt_len-token prefill, or (with
    synthetic_ctx > 0) after filling the KV cache with that many synthetic
    positions instead of running a prefill.  The prompt goes through the
    prompt GEMMs in passes of prefill_chunk tokens (0: the whole prompt in
    one pass, M = prompt_len)."""
    ctx_len = synthetic_ctx or prompt_len
    max_ctx = ctx_len + warmup + steps + 8
    chunk = prefill_chunk or max(prompt_len, 1)
    m = native.Model(path, max_ctx=max_ctx, max_sessions=1, prefill_chunk=chunk)
    s = m.acquire()
    t0 = time.perf_counter()
    if synthetic_ctx:
        s.fill_kv(synthetic_ctx, seed=3)
        tok = 1
    else:
        prompt = synth.tokens(prompt_len, 42, spec.vocab)
        tok, _ = s.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    pos = ctx_len
    for _ in range(warmup):
        tok, _ = s.forward(tok, pos)
        pos += 1
    stream = native.lib().cmolhip_session_stream(m.device, s.slot)
    ev = hiprt.EventTimer(stream)
    hiprt.device_synchronize()
    ev.start()
    t0 = time.perf_counter()
    for _ in range(steps):
        tok, _ = s.forward(tok, pos)
        pos += 1
    ev.stop()
    hiprt.device_synchronize()
    wall = time.perf_counter() - t0
    dev_ms = ev.elapsed()
    ev.close()
    m.close()
    out = {"tok_s": steps / wall, "ms_per_step": wall * 1e3 / steps,
           "device_ms_per_step": dev_ms / steps, "context": ctx_len}
    if not synthetic_ctx:
        out.update(prefill_tok_s=prompt_len / prefill_s, prefill_s=prefill_s, prefill_chunk=chunk)
    return out


def bench_sampled_1(path, spec, new_tokens):
    """One session through cmol_generate's loop with the default sampling
    parameters (temperature 0.8, top-k 40, top-p 0.95, repeat penalty 1.1):
    the logits of every step go to the host sampler (vocabulary 128256).
    Timed with the sampler's worker pool and single-threaded."""
    m = native.Model(path, max_ctx=64 + 2 * new_tokens + 8, max_sessions=1)
    s = m.acquire()
    prompt = synth.tokens(32, 42, spec.vocab)
    prm = native.default_params(max_new_tokens=new_tokens, seed=5)
    out = {}
    L = native.lib()
    for label, threads in (("pool", -1), ("single_thread", 0)):
        prev = L.cmol__sampler_config(threads, 0)
        s.reset()
        s.generate_ids(prompt, prm, new_tokens)   # warm-up
        s.reset()
        t0 = time.perf_counter()
        got = s.generate_ids(prompt, prm, new_tokens)
        wall = time.perf_counter() - t0
        L.cmol__sampler_config(prev, 0)
        out[label] = {"tok_s": len(got) / wall, "tokens": int(len(got))}
    m.close()
    out["note"] = "wall clock includes the 32-token prompt pass"
    return out


def bench_decode_32(path, spec, sessions, steps, warmup, lo=512, hi=16384):
    lens = synth.log_uniform_lengths(sessions, lo, hi, seed=7)
    max_ctx = int(lens.max()) + warmup + steps + 8
    os.environ["CMOL_KV_F16"] = "1"
    try:
        m = native.Model(path, max_ctx=max_ctx, max_sessions=sessions)
    finally:
        os.environ.pop("CMOL_KV_F16", None)
    ss = [m.acquire() for _ in range(sessions)]
    for i, s in enumerate(ss):
        s.fill_kv(int(lens[i]), seed=100 + i)
    toks = synth.tokens(sessions, 5, spec.vocab)
    for _ in range(warmup):
        toks = native.decode_batch(ss, toks)
    hiprt.device_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = native.decode_batch(ss, toks)
    hiprt.device_synchronize()
    wall = time.perf_counter() - t0
    m.close()
    kv_bytes = float(np.sum(lens)) * spec.n_layers * 2 * spec.n_kv_heads * spec.d_head * 2
    return {"tok_s": sessions * steps / wall, "ms_per_step": wall * 1e3 / steps,
            "sessions": sessions, "mean_ctx": float(np.mean(lens)),
            "kv_bytes_per_step": kv_bytes}


def kv_bytes(spec, ctx_sum, elem_bytes):
    """Bytes of K and V one decode step reads over contexts summing to ctx_sum."""
    return float(ctx_sum) * spec.n_layers * 2 * spec.n_kv_heads * spec.d_head * elem_bytes


def with_roofline(r, step_bytes):
    """Adds the step's algorithmic bytes and its fraction of the HBM peak."""
    gbps = step_bytes / (r["ms_per_step"] * 1e-3) / 1e9
    r.update(bytes_per_step=step_bytes, GBps=round(gbps, 1), frac_of_hbm_peak=round(gbps / HBM_PEAK_GBPS, 4))
    return r


def bench_decode_small(steps=128, prompt_len=32):
    """SmolLM2-135M-shaped Q8_0 model, one session: a seeded 32-token prompt,
    then 128 greedy decode steps, timed (the same run once before, untimed).
    Its 142.9 MB of weights fit the 256 MB Infinity Cache, so the rate is
    reported as effective weight GB/s rather than against HBM."""
    spec = synth.PRESETS["smollm2-135m-q8_0"]
    path = synth.model_file(spec)
    m = native.Model(path, max_ctx=prompt_len + steps + 8, max_sessions=1)
    s = m.acquire()
    prompt = synth.tokens(prompt_len, 42, spec.vocab)
    wall = 0.0
    for _ in range(2):
        s.reset()
        tok, _ = s.prefill(prompt)
        hiprt.device_synchronize()
        t0 = time.perf_counter()
        pos = prompt_len
        for _ in range(steps):
            tok, _ = s.forward(tok, pos)
            pos += 1
        hiprt.device_synchronize()
        wall = time.perf_counter() - t0
    m.close()
    wb = spec.weight_bytes_per_token()
    r = {"model": "SmolLM2-135M-shaped Q8_0", "sessions": 1, "prompt": prompt_len, "new_tokens": steps,
         "tok_s": steps / wall, "ms_per_step": wall * 1e3 / steps, "weight_bytes_per_token": wb,
         "effective_weight_GBps": round(wb * steps / wall / 1e9, 1)}
    return with_roofline(r, wb + kv_bytes(spec, prompt_len + steps / 2, 4))


def bench_decode_16(steps=16, warmup=2, sessions=16, lo=64, hi=1024):
    """SmolLM2-360M-shaped Q5_0 model, 16 sessions decoding in lock-step over
    fp32 KV caches of lengths uniform in 64..1024 (synthetic contents)."""
    spec = synth.PRESETS["smollm2-360m-q5_0"]
    path = synth.model_file(spec)
    lens = synth.uniform_lengths(sessions, lo, hi, seed=5)
    m = native.Model(path, max_ctx=int(lens.max()) + warmup + steps + 8, max_sessions=sessions)
    ss = [m.acquire() for _ in range(sessions)]
    for i, s in enumerate(ss):
        s.fill_kv(int(lens[i]), seed=200 + i)
    toks = synth.tokens(sessions, 6, spec.vocab)
    for _ in range(warmup):
        toks = native.decode_batch(ss, toks)
    hiprt.device_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = native.decode_batch(ss, toks)
    hiprt.device_synchronize()
    wall = time.perf_counter() - t0
    m.close()
    r = {"model": "SmolLM2-360M-shaped Q5_0", "sessions": sessions, "tok_s": sessions * steps / wall,
         "ms_per_step": wall * 1e3 / steps, "mean_ctx": float(np.mean(lens))}
    return with_roofline(r, spec.weight_bytes_per_token() + kv_bytes(spec, np.sum(lens) + sessions * (warmup + steps / 2), 4))


def bench_generate_concurrent(path, spec, sessions, new_tokens, lo=512, hi=16384):
    """The public path with one thread per session: `sessions` concurrent
    cmol_generate callers (greedy, token ids) over the same log-uniform
    synthetic contexts as decode_32; the library's scheduler batches their
    decode steps.  Wall clock from the first call to the last return,
    including each caller's one-token prompt pass."""
    import threading
    lens = synth.log_uniform_lengths(sessions, lo, hi, seed=7)
    max_ctx = int(lens.max()) + new_tokens + 8
    os.environ["CMOL_KV_F16"] = "1"
    try:
        m = native.Model(path, max_ctx=max_ctx, max_sessions=sessions)
    finally:
        os.environ.pop("CMOL_KV_F16", None)
    ss = [m.acquire() for _ in range(sessions)]
    prm = native.greedy_params(new_tokens)
    prompts = [synth.tokens(1, 40 + i, spec.vocab) for i in range(sessions)]
    got = [0] * sessions

    def run(i):
        got[i] = len(ss[i].generate_ids(prompts[i], prm, new_tokens))

    def once():
        for i, s in enumerate(ss):
            s.reset()
            s.fill_kv(int(lens[i]), seed=100 + i)
        hiprt.device_synchronize()
        th = [threading.Thread(target=run, args=(i,)) for i in range(sessions)]
        t0 = time.perf_counter()
        for t in th:
            t.start()
        for t in th:
            t.join()
        return time.perf_counter() - t0

    once()   # warm-up: first batches of each size
    _, b0, s0, _ = m.sched_stats()
    wall = once()
    _, b1, s1, largest = m.sched_stats()
    m.close()
    tokens = sum(got)
    return {"tok_s": tokens / wall, "wall_s": wall, "sessions": sessions, "new_tokens": new_tokens,
            "tokens": tokens, "batches": b1 - b0, "mean_batch": (s1 - s0) / max(b1 - b0, 1),
            "largest_batch": largest, "mean_ctx": float(np.mean(lens))}


def recorded_traffic(name):
    """HBM bytes per launch of the roofline kernel from its counter summary
    under profiles/ (two rocprofv3 counter passes, FETCH_SIZE and WRITE_SIZE,
    scaled by a copy of known size); None when the summary is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def copy_calibration(mb, reps=4):
    """Device-to-device copies of a known size: under a counter run their
    read/write byte counters give the scale factor for FETCH_SIZE/WRITE_SIZE."""
    nbytes = mb << 20
    ctx = native.Ctx(2 * nbytes + (1 << 20))
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    L = native.lib()
    for _ in range(reps):
        native.check(L.cmolhip_memcpy_d2d(ctx.h, C.c_void_p(b), C.c_void_p(a), nbytes), "d2d")
    native.check(L.cmolhip_synchronize(ctx.h))
    ctx.close()
    return {"copy_bytes": nbytes, "copies": reps}


def cgroup_cpu_quota():
    """CPUs the process's cgroup allows (cpu.max quota / period; cgroup v1's
    cfs files), or None when unlimited or unreadable."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
            return None if q == "max" else int(q) / int(per)
    except (OSError, ValueError):
        pass
    try:
        with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f:
            q = int(f.read())
        with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
            per = int(f.read())
        return None if q <= 0 else q / per
    except (OSError, ValueError):
        return None


def cpu_cores():
    """Host threads the CPU baselines use: the CPUs this process may run on
    (its affinity mask and its cgroup's quota), at most OMP_NUM_THREADS and
    at most 16 (the CPU share of one GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    q = cgroup_cpu_quota()
    if q is not None:
        n = min(n, max(1, int(q)))
    e = os.environ.get("OMP_NUM_THREADS", "")
    if e.isdigit() and int(e) > 0:
        n = min(n, int(e))
    return max(1, min(n, 16))


ISA_FLAGS = ("sse4_2", "avx", "avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl", "avx512dq",
             "avx512_vnni", "avx512_bf16", "avx512_fp16", "amx_tile")


def oracle_build_flags():
    """The oracle's compiler flags, read from oracle/Makefile (OFLAGS)."""
    try:
        with open(os.path.join(ROOT, "oracle", "Makefile")) as f:
            for line in f:
                if line.startswith("OFLAGS"):
                    return "gcc " + line.split("=", 1)[1].strip()
    except OSError:
        pass
    return None


def host_cpu():
    """The host the CPU baselines ran on: CPU model, logical CPUs, the CPUs
    this process may use (affinity, cgroup quota) and the x86 ISA extensions
    /proc/cpuinfo reports."""
    model, flags = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "model name" and model is None:
                    model = v.strip()
                elif k == "flags" and not flags:
                    flags = set(v.split())
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": aff,
            "cgroup_cpu_quota": cgroup_cpu_quota(),
            "isa": [f for f in ISA_FLAGS if f in flags], "oracle_build": oracle_build_flags()}


def cpu_baseline(cores, c4_tokens=3):
    """The oracle (the reference's arithmetic restated in C, AVX-512
    accumulation order, `kind` "port") on bounded samples of each
    configuration, one session per thread as the reference runs them
    (min(sessions, cores) threads).  The top-level figure is the headline
    configuration: SmolLM3-3B-shaped single-session decode at context 2048
    (synthetic KV), the same context as the GPU figure."""
    from oracle import oracle as O
    out = {}
    spec3 = synth.PRESETS["smollm3-3b-q4_0"]
    path3 = synth.model_file(spec3)
    # C4: one session at context 2048, one thread
    S = O.Sessions(path3, [2048 + c4_tokens + 4])
    S.fill_kv(0, 2048, seed=1)
    S.step([1], [2048], 1)   # pages the weights in
    el = sum(S.step([5 + i], [2049 + i], 1) for i in range(c4_tokens))
    S.close()
    out["c4_decode_1"] = {"value": c4_tokens / el, "unit": "tok/s", "cores": 1,
                          "sample": f"{c4_tokens} decode steps at positions 2049.. over a synthetic "
                                    "2048-position fp32 KV cache"}
    # C5: 32 sessions at the GPU leg's log-uniform lengths, fp16-rounded KV
    lens = synth.log_uniform_lengths(32, 512, 16384, seed=7).astype(int)
    th = min(32, cores)
    S = O.Sessions(path3, [int(L) + 2 for L in lens], kv_f16=True)
    for i, L in enumerate(lens):
        S.fill_kv(i, int(L), seed=100 + i)
    el = S.step(synth.tokens(32, 5, spec3.vocab), lens, th)
    S.close()
    out["c5_decode_32"] = {"value": 32 / el, "unit": "tok/s", "cores": th,
                           "sample": "one lock-step decode step of 32 sessions at contexts drawn "
                                     "log-uniformly from 512 to 16384 (synthetic KV), "
                                     f"{th} threads"}
    # C1: SmolLM2-135M-shaped Q8_0, one session, 32-token prompt then 32 steps
    spec1 = synth.PRESETS["smollm2-135m-q8_0"]
    om = O.Model(synth.model_file(spec1), max_ctx=72, nthreads=1)
    toks = synth.tokens(64, 42, spec1.vocab)
    for p in range(32):
        om.forward(int(toks[p]), p)
    t0 = time.perf_counter()
    for p in range(32, 64):
        om.forward(int(toks[p]), p)
    el = time.perf_counter() - t0
    om.close()
    wb1 = spec1.weight_bytes_per_token()
    out["c1_decode_1"] = {"value": 32 / el, "unit": "tok/s", "cores": 1,
                          "effective_weight_GBps": round(wb1 * 32 / el / 1e9, 2),
                          "sample": "32 decode steps after a 32-token prompt"}
    # C1 through the reference itself (built from its own sources), when it
    # travelled with the tree: its runtime-selected AVX-512 / AVX2 kernels
    if O.ref_available():
        rm = O.RefModel(synth.model_file(spec1), max_ctx=72)
        for p in range(32):
            rm.forward(int(toks[p]), p)
        t0 = time.perf_counter()
        for p in range(32, 64):
            rm.forward(int(toks[p]), p)
        el = time.perf_counter() - t0
        rm.close()
        out["c1_decode_1_reference"] = {
            "value": 32 / el, "unit": "tok/s", "cores": 1, "kind": "reference",
            "kernel": O.ref().shim_kernel_name().decode(),
            "effective_weight_GBps": round(wb1 * 32 / el / 1e9, 2),
            "sample": "32 decode steps after a 32-token prompt, the reference's cmol_model_forward"}
    # C3: SmolLM2-360M-shaped Q5_0, 16 sessions at uniform lengths 64..1024
    spec_3 = synth.PRESETS["smollm2-360m-q5_0"]
    lens = synth.uniform_lengths(16, 64, 1024, seed=5).astype(int)
    th = min(16, cores)
    S = O.Sessions(synth.model_file(spec_3), [int(L) + 4 for L in lens])
    for i, L in enumerate(lens):
        S.fill_kv(i, int(L), seed=200 + i)
    toks = synth.tokens(16, 6, spec_3.vocab)
    S.step(toks, lens, th)
    el = S.step(toks, lens + 1, th) + S.step(toks, lens + 2, th)
    S.close()
    out["c3_decode_16"] = {"value": 32 / el, "unit": "tok/s", "cores": th,
                           "sample": f"two lock-step steps of 16 sessions, {th} threads"}
    # C2: the Q4_0 FFN matvec 11008x2048, one thread, n = 1 and 8
    rows, cols = 11008, 2048
    w = synth.normal(rows * cols, seed=1234, stream=rows * 7 + cols, std=0.02)
    raw = synth.quantize(synth.Q4_0, w).reshape(rows, -1)
    x = np.random.default_rng(1).standard_normal((8, cols)).astype(np.float32)
    c2 = {}
    for n, reps in ((1, 8), (8, 2)):
        b = np.ascontiguousarray(x[:n].T)   # [k][n]
        O.matmul(raw, b, rows, cols, synth.Q4_0)
        t0 = time.perf_counter()
        for _ in range(reps):
            O.matmul(raw, b, rows, cols, synth.Q4_0)
        el = (time.perf_counter() - t0) / reps
        c2[f"n{n}"] = {"ms_per_call": round(el * 1e3, 2), "GBps": round(q4_bytes(rows, cols, n) / el / 1e9, 2)}
    out["c2_gemv_q4_11008x2048"] = dict(c2, cores=1)
    head = out["c4_decode_1"]
    return {"value": round(head["value"], 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": "SmolLM3-3B-shaped Q4_0 single session, " + head["sample"]
                      + "; the oracle in the reference's AVX-512 accumulation order (the reference "
                        "has no Q4_0 kernel, so no reference figure exists for this model)",
            "threads_available": cores, "host": host_cpu(),
            "configs": out}


# ---- HBM traffic of the roofline kernel, measured in this run -----------------
TRAFFIC_SHAPE = (11008, 2048)


def traffic_child():
    """Run under rocprofv3 by measure_traffic and trace_pass: a device-to-device
    copy of known size (the counters' calibration kernel), then the roofline
    matvec exactly as the matvec leg times it (64 rotating weight copies,
    8 untimed + 256 event-timed launches)."""
    copy_calibration(64, reps=4)
    r = bench_matvec(TRAFFIC_SHAPE[0], TRAFFIC_SHAPE[1], 1, copies=64, launches=256)
    print(json.dumps(r), flush=True)


def trace_pass(workdir):
    """One rocprofv3 kernel-trace pass over traffic_child: mean, min and max
    duration (us) of the roofline matvec's dispatches, from the trace's own
    start and end timestamps, and the event-timed figure of the same run."""
    env = dict(os.environ, TMPDIR="/tmp")
    cmd = ["timeout", "-s", "KILL", "180", "rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv",
           "-d", workdir, "-o", "trace", "--", sys.executable, os.path.join(ROOT, "bench.py"), "--traffic-child"]
    res = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.DEVNULL,
                         check=True, text=True)
    ev = None
    for line in res.stdout.splitlines():
        if line.startswith("{"):
            ev = json.loads(line)
    path = None
    for root, _, files in os.walk(workdir):
        for f in files:
            if f.startswith("trace") and f.endswith("kernel_trace.csv"):
                path = os.path.join(root, f)
    durs = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Kernel_Name"].startswith("void k_gemv<"):
                durs.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return {"calls": len(durs), "avg_us": sum(durs) / len(durs), "min_us": min(durs), "max_us": max(durs),
            "event_us": ev["us_per_launch"] if ev else None}


def pmc_pass(counter, workdir):
    """One rocprofv3 counter pass over traffic_child: mean counter value (KiB)
    per dispatch of the largest copy and of the matvec kernel."""
    env = dict(os.environ, TMPDIR="/tmp")
    cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "--output-format", "csv",
           "-d", workdir, "-o", counter, "--", sys.executable, os.path.join(ROOT, "bench.py"), "--traffic-child"]
    subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, check=True)
    path = None
    for root, _, files in os.walk(workdir):
        for f in files:
            if f.startswith(counter) and f.endswith("counter_collection.csv"):
                path = os.path.join(root, f)
    copy, mv = {}, []
    with open(path) as f:
        for r in csv.DictReader(f):
            name, v = r["Kernel_Name"], float(r["Counter_Value"])
            if name.startswith("__amd_rocclr_copyBuffer"):
                g = int(r["Grid_Size"])
                copy.setdefault(g, []).append(v)
            elif name.startswith("void k_gemv<"):
                mv.append(v)
    big = copy[max(copy)]
    return sum(big) / len(big), sum(mv) / len(mv)


def measure_traffic():
    """The roofline matvec measured by rocprofv3 in this run: a kernel-trace
    pass (its dispatch durations) and HBM bytes per launch from FETCH_SIZE and
    WRITE_SIZE (two counter passes), each scaled by what it reads for the
    64 MiB copy.  Parts whose pass failed, or all of it without rocprofv3,
    are None."""
    if not shutil.which("rocprofv3"):
        return None, None
    errs = (subprocess.CalledProcessError, OSError, KeyError, ValueError, ZeroDivisionError, TypeError)
    work = tempfile.mkdtemp(prefix="cmol_pmc_", dir="/tmp")
    trace = traffic = None
    try:
        try:
            trace = trace_pass(os.path.join(work, "trace"))
        except errs:
            trace = None
        try:
            cf, mf = pmc_pass("FETCH_SIZE", work)
            cw, mw = pmc_pass("WRITE_SIZE", work)
            copy_kib = 64 * 1024
            fs, ws = copy_kib / cf, copy_kib / cw
            traffic = {"bytes": int((mf * fs + mw * ws) * 1024), "fetch_KiB": round(mf, 1),
                       "write_KiB": round(mw, 1), "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)}
        except errs:
            traffic = None
    finally:
        shutil.rmtree(work, ignore_errors=True)
    return trace, traffic


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--prefill-chunk", type=int, default=0,
                    help="prompt tokens per prefill pass (default: the whole prompt, M = --prompt)")
    ap.add_argument("--sessions", type=int, default=32)
    ap.add_argument("--multi-steps", type=int, default=16)
    ap.add_argument("--cpu-tokens", type=int, default=4)
    ap.add_argument("--generate-tokens", type=int, default=48)
    ap.add_argument("--skip", default="",
                    help="comma list of: decode,sampled,small,multi16,multi,generate,matvec,gemm,traffic,cpu")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--synthetic-context", type=int, default=0,
                    help="decode after filling the KV cache with this many synthetic positions "
                         "instead of a prefill (profiling runs)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run device-to-device copies of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.traffic_child:
        traffic_child()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              f"(every configuration fits one MI355X; sessions shard by data parallelism)",
              file=sys.stderr)
        sys.exit(2)
    skip = set(filter(None, args.skip.split(",")))
    if native.device_count() < 1:
        raise SystemExit("no GPU visible")
    spec = synth.PRESETS["smollm3-3b-q4_0"]
    t0 = time.perf_counter()
    path = synth.model_file(spec)
    log(f"model file ready in {time.perf_counter() - t0:.1f}s: {path}")

    d1 = None
    if "decode" not in skip:
        log("single-session decode")
        d1 = bench_decode_1(path, spec, args.prompt, args.steps, args.warmup, args.synthetic_context,
                            args.prefill_chunk)
        log(json.dumps(d1))
    s1 = None
    if "sampled" not in skip:
        log("single-session sampled generation")
        s1 = bench_sampled_1(path, spec, args.steps)
        log(json.dumps(s1))
    if args.copy_mb:
        log(json.dumps(copy_calibration(args.copy_mb)))
    mv = []
    if "matvec" not in skip:
        for rows, cols in ((11008, 2048), (2048, 11008)):
            for n in (1, 8, 32):
                r = bench_matvec(rows, cols, n, copies=64, launches=256)
                log(json.dumps(r))
                mv.append(r)
        # the K-quant formats of Q4_K_M files on the same shapes, one vector
        for dt in (synth.Q4_K, synth.Q6_K):
            for rows, cols in ((11008, 2048), (2048, 11008)):
                r = bench_matvec(rows, cols, 1, copies=64, launches=256, dtype=dt)
                log(json.dumps(r))
                mv.append(r)
    gm = []
    if "gemm" not in skip:
        # the prompt pass's GEMM at M = 2048 tokens on the FFN shapes
        for rows, cols in ((11008, 2048), (2048, 11008)):
            r = bench_matvec(rows, cols, 2048, copies=2, launches=16, fold=1)
            log(json.dumps(r))
            gm.append(r)
    c1 = None
    if "small" not in skip:
        log("SmolLM2-135M-shaped single-session decode")
        c1 = bench_decode_small()
        log(json.dumps(c1))
    c3 = None
    if "multi16" not in skip:
        log("SmolLM2-360M-shaped 16-session decode")
        c3 = bench_decode_16()
        log(json.dumps(c3))
    d32 = None
    if "multi" not in skip:
        log("32-session decode")
        d32 = bench_decode_32(path, spec, args.sessions, args.multi_steps, 2)
        log(json.dumps(d32))
    g32 = None
    if "generate" not in skip:
        log("32 concurrent cmol_generate callers")
        g32 = bench_generate_concurrent(path, spec, args.sessions, args.generate_tokens)
        log(json.dumps(g32))
    traffic = trace = None
    if mv and "traffic" not in skip:
        log("roofline kernel under rocprofv3 (a kernel-trace pass, then two counter passes)")
        trace, traffic = measure_traffic()
        log(json.dumps({"trace": trace, "traffic": traffic}))
    cpu = None
    if "cpu" not in skip:
        log("cpu baseline")
        cpu = cpu_baseline(cpu_cores(), args.cpu_tokens)
        log(json.dumps(cpu))

    weight_bytes = spec.weight_bytes_per_token()
    roof = None
    if mv:
        # achieved / frac from the rocprofv3 kernel trace of this run (the
        # profiler's dispatch durations), else from the HIP events
        r = mv[0]
        b = r["bytes_per_launch"]
        us = trace["avg_us"] if trace else r["us_per_launch"]
        roof = {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(b / us / 1e3 / HBM_PEAK_GBPS, 4),
                "traffic": traffic["bytes"] if traffic else recorded_traffic("gemv_q4_11008x2048_traffic.txt"),
                "traffic_source": ("rocprofv3 FETCH_SIZE + WRITE_SIZE passes in this run, scaled by a 64 MiB "
                                   "copy: " + json.dumps(traffic)) if traffic else
                                  "profiles/gemv_q4_11008x2048_traffic.txt (no counter pass in this run)",
                "kernel": "k_gemv<Q4_0> 11008x2048 n=1",
                "bytes_per_launch": b,
                "us_per_launch": round(us, 3),
                "us_source": ("rocprofv3 --kernel-trace pass in this run: mean of the dispatches' end - start "
                              "over the rotating-copy launches" if trace else
                              "HIP events (no kernel-trace pass in this run)"),
                "trace": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in trace.items()}
                if trace else None,
                "us_per_launch_events": round(r["us_per_launch"], 3),
                "frac_events": round(r["frac_of_peak"], 4)}
    if d1 is None:
        print(json.dumps({"metric": METRIC, "matvec": mv, "gemm": gm, "roofline": roof, "sampled_1": s1,
                          "decode_135m_1": c1, "decode_360m_16": c3, "decode_32": d32, "generate_32": g32,
                          "cpu_baseline": cpu}), flush=True)
        return
    ctx1 = d1["context"] + args.warmup + args.steps / 2
    with_roofline(d1, weight_bytes + kv_bytes(spec, ctx1, 4))
    if d32:
        with_roofline(d32, weight_bytes + d32["kv_bytes_per_step"])
    out = {
        "metric": METRIC,
        "value": round(d1["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 accumulate, hi/lo f16 operands",
        "data": "synthetic (seeded random weights ~N(0,0.02), seeded random prompt ids)",
        "config": {"workload": "SmolLM3-3B-shaped Q4_0 (Q8_0 tied embd/LM head), 1 session, "
                               + (f"greedy decode at a {args.synthetic_context}-position synthetic "
                                  "KV context" if args.synthetic_context else
                                  f"greedy decode after a {args.prompt}-token prompt"),
                   "sessions": 1, "prompt": 0 if args.synthetic_context else args.prompt,
                   "weight_bytes_per_token": weight_bytes,
                   "effective_weight_GBps": round(weight_bytes * d1["tok_s"] / 1e9, 1)},
        "decode_1": d1,
        "sampled_1": s1,
        "decode_135m_1": c1,
        "decode_360m_16": c3,
        "decode_32": d32,
        "generate_32": g32,
        "matvec": mv,
        "prefill_gemm": gm,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
