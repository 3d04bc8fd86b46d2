"""Concurrent cmol_generate callers on one model (one thread per session, the
reference's contract, src/api.c:309-334): the scheduler batches their decode
steps, and every session still produces what it produces alone."""
import ctypes as C
import threading

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run_concurrently(fns):
    """Runs each fn on its own thread (ctypes releases the GIL inside the
    library); returns their results in order."""
    out = [None] * len(fns)
    errs = []

    def call(i):
        try:
            out[i] = fns[i]()
        except Exception as e:   # reported on the main thread
            errs.append(e)

    th = [threading.Thread(target=call, args=(i,)) for i in range(len(fns))]
    for t in th:
        t.start()
    for t in th:
        t.join(120)
    assert not any(t.is_alive() for t in th), "a generate call did not return"
    if errs:
        raise errs[0]
    return out


@pytest.mark.parametrize("preset", ["small-q4_0", "small-q4_k_m"])
def test_concurrent_greedy_generate_matches_oracle(gpu, model_dir, preset):
    """Six callers with ragged prompts and ragged max_new_tokens: each
    session's ids equal the oracle's run of it alone, and the scheduler ran
    their steps in shared batches."""
    spec = synth.PRESETS[preset].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    lens = [3, 17, 1, 40, 8, 25]
    news = [20, 12, 24, 16, 5, 20]
    prompts = [synth.tokens(L, 200 + i, spec.vocab) for i, L in enumerate(lens)]
    m = native.Model(path, max_ctx=96, max_sessions=len(lens))
    ss = [m.acquire() for _ in lens]
    got = run_concurrently([
        (lambda s=s, p=p, k=k: s.generate_ids(p, native.greedy_params(k), k))
        for s, p, k in zip(ss, prompts, news)])
    on, batches, steps, largest = m.sched_stats()
    m.close()
    assert on
    # the first token of each comes from the prompt, which a 1-token prompt
    # takes as one more scheduled step
    assert steps == sum(k - 1 for k in news) + sum(L == 1 for L in lens)
    assert largest > 1 and batches < steps
    for i, p in enumerate(prompts):
        want = O.Model(path, 96).generate(p, news[i])
        assert got[i].tolist() == want.tolist(), f"session {i} (prompt {lens[i]})"


def test_concurrent_host_logits_generate(gpu, model_dir):
    """Callers whose parameters need the logits on the host (repeat penalty)
    next to greedy ones: each batch delivers every session's own logits, so
    every session continues exactly as when it runs alone."""
    spec = synth.PRESETS["small-q5_0"].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    prompts = [synth.tokens(L, 300 + i, spec.vocab) for i, L in enumerate([9, 30, 4, 17])]
    params = [native.default_params(temperature=0.0, max_new_tokens=18, seed=1, repeat_penalty=pen)
              for pen in (1.3, 1.0, 1.15, 1.3)]
    m = native.Model(path, max_ctx=96, max_sessions=4)
    ss = [m.acquire() for _ in prompts]
    alone = []
    for s, p, prm in zip(ss, prompts, params):   # one at a time: no batching
        alone.append(s.generate_ids(p, prm, 18))
        s.reset()
    _, b0, _, _ = m.sched_stats()
    together = run_concurrently([(lambda s=s, p=p, prm=prm: s.generate_ids(p, prm, 18))
                                 for s, p, prm in zip(ss, prompts, params)])
    _, b1, _, largest = m.sched_stats()
    m.close()
    assert largest > 1 and b1 > b0
    for i in range(len(prompts)):
        assert together[i].tolist() == alone[i].tolist(), f"session {i}"


def test_batch_each_logits_equal_batch_logits(gpu, model_dir):
    """cmolhip_decode_batch_each delivers row i of the batch's logits to
    session i's buffer (bit-identical to cmolhip_decode_batch's [n][vocab])
    and skips the sessions whose pointer is NULL."""
    spec = synth.PRESETS["small-q4_0"].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    n, V = 5, spec.vocab
    m = native.Model(path, max_ctx=64, max_sessions=n)
    ss = [m.acquire() for _ in range(n)]
    for i, s in enumerate(ss):
        s.prefill(synth.tokens(6 + 3 * i, 50 + i, V))
    slots = np.array([s.slot for s in ss], np.int32)
    pos = np.array([6 + 3 * i for i in range(n)], np.int32)
    toks = synth.tokens(n, 9, V)
    L = native.lib()
    # the same step twice (same positions: the cache rows are rewritten)
    whole = np.zeros((n, V), np.float32)
    am = np.zeros(n, np.int32)
    native.check(L.cmolhip_decode_batch(m.device, n, native.ptr(slots), native.ptr(toks), native.ptr(pos),
                                        native.ptr(whole), native.ptr(am)), "decode_batch")
    rows = [np.full(V, np.nan, np.float32) if i != 2 else None for i in range(n)]
    ptrs = (C.c_void_p * n)(*[(r.ctypes.data if r is not None else None) for r in rows])
    am2 = np.zeros(n, np.int32)
    native.check(L.cmolhip_decode_batch_each(m.device, n, native.ptr(slots), native.ptr(toks),
                                             native.ptr(pos), ptrs, native.ptr(am2)), "decode_batch_each")
    m.close()
    assert am2.tolist() == am.tolist()
    for i, r in enumerate(rows):
        if r is not None:
            assert np.array_equal(r.view(np.uint32), whole[i].view(np.uint32)), f"row {i}"


def test_batching_can_be_switched_off(gpu, model_dir, monkeypatch):
    """CMOL_BATCH=0: concurrent callers decode on their own streams, with the
    same results."""
    monkeypatch.setenv("CMOL_BATCH", "0")
    spec = synth.PRESETS["small-q4_0"].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    prompts = [synth.tokens(L, 400 + i, spec.vocab) for i, L in enumerate([5, 12, 20])]
    m = native.Model(path, max_ctx=64, max_sessions=3)
    ss = [m.acquire() for _ in prompts]
    got = run_concurrently([(lambda s=s, p=p: s.generate_ids(p, native.greedy_params(10), 10))
                            for s, p in zip(ss, prompts)])
    assert m.sched_stats() == (False, 0, 0, 0)
    m.close()
    for i, p in enumerate(prompts):
        assert got[i].tolist() == O.Model(path, 64).generate(p, 10).tolist()

