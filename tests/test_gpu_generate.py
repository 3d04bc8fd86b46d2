"""cmol_generate's stop rules on the GPU against the reference's generate loop
(src/api.c:443-521; ids in tests/golden/generate_edges.npz from the built
reference): EOS is emitted and ends the call; max_new_tokens 0 means no
limit; a full context ends the call after the token sampled at its last
position, and the next call on the session returns CMOL_ERR_CTX_FULL; the
same with two sessions generating at once through the scheduler."""
import os
import threading

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O
from tests.golden import make_generate_golden as ge

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GE = np.load(os.path.join(HERE, "golden", "generate_edges.npz"))


def test_eos_ends_generation(gpu, model_dir):
    path = synth.model_file(ge.eos_spec(int(GE["eos_id"][0])), model_dir)
    m = native.Model(path, max_ctx=128, max_sessions=1)
    s = m.acquire()
    got = s.generate_ids(GE["prompt"], native.greedy_params(40), 40)
    m.close()
    assert got.tolist() == GE["eos_ids"].tolist()
    assert int(got[-1]) == int(GE["eos_id"][0])


@pytest.mark.parametrize("max_new", [64, 0])
def test_full_context_ends_generation(gpu, model_dir, max_new):
    path = synth.model_file(ge.eos_spec(), model_dir)
    m = native.Model(path, max_ctx=ge.CTX_FULL, max_sessions=1)
    s = m.acquire()
    got = s.generate_ids(GE["prompt"], native.greedy_params(max_new), 64)
    assert got.tolist() == GE["ctx_full_ids"].tolist()
    with pytest.raises(RuntimeError, match=str(native.CMOL_ERR_CTX_FULL)):
        s.generate_ids(GE["prompt"][:1], native.greedy_params(4), 4)
    m.close()


def test_stop_rules_with_concurrent_sessions(gpu, model_dir):
    """A session that stops at EOS and one that stops at a full context,
    generating at the same time (their steps batched), each match the
    reference."""
    eos = int(GE["eos_id"][0])
    path = synth.model_file(ge.eos_spec(eos), model_dir)
    m = native.Model(path, max_ctx=ge.CTX_FULL, max_sessions=2)
    a, b = m.acquire(), m.acquire()
    out = {}

    def run(name, s, prompt, n):
        out[name] = s.generate_ids(prompt, native.greedy_params(n), 64)

    # a: the reference's EOS continuation (it fits in the 24 positions)
    # b: another prompt, no token limit
    ta = threading.Thread(target=run, args=("a", a, GE["prompt"], 40))
    tb = threading.Thread(target=run, args=("b", b, GE["prompt"][:-1], 0))
    ta.start(); tb.start(); ta.join(120); tb.join(120)
    m.close()
    assert out["a"].tolist() == GE["eos_ids"].tolist()
    # b stops at EOS or at the full context, as the oracle's loop does
    assert out["b"].tolist() == O.Model(path, ge.CTX_FULL).generate(GE["prompt"][:-1], 64).tolist()


# ---- the session pool contract (reference src/api.c:309-334,
# tests/test_threads.c:226-250, tests/test_generate.c:359-407) -------------
def test_pool_exhaustion_and_reuse(gpu, model_dir):
    """max_sessions acquires succeed, one more returns NULL; after a release
    the next acquire succeeds again (the freed slot)."""
    path = synth.model_file(synth.PRESETS["micro-q8_0"], model_dir)
    m = native.Model(path, max_ctx=64, max_sessions=3)
    held = [m.acquire() for _ in range(3)]
    assert all(h is not None for h in held)
    assert len({h.slot for h in held}) == 3
    assert m.acquire() is None
    held[1].release()
    again = m.acquire()
    assert again is not None and again.slot == held[1].slot
    assert m.acquire() is None
    for h in (held[0], again, held[2]):
        h.release()
    assert all(m.acquire() is not None for _ in range(3))
    m.close()


def test_release_keeps_the_session_context(gpu, model_dir):
    """Releasing a session does not reset it: the next owner of the slot
    continues after the tokens already in its cache (reset is explicit)."""
    spec = synth.PRESETS["small-q4_0"].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    m = native.Model(path, max_ctx=96, max_sessions=1)
    s = m.acquire()
    prompt = synth.tokens(10, 4, spec.vocab)
    first = s.generate_ids(prompt, native.greedy_params(6), 6)
    n = s.length
    assert n == 10 + 5   # the last sampled token is not yet in the cache
    s.release()
    t = m.acquire()
    assert t.slot == s.slot and t.length == n
    more = t.generate_ids(first[-1:], native.greedy_params(4), 4)
    om = O.Model(path, 96)
    want = om.generate(np.concatenate([prompt, first]), 4)
    assert more.tolist() == want.tolist()
    m.close()


def test_callback_abort_returns_ok(gpu, model_dir):
    """A callback that returns nonzero ends cmol_generate with CMOL_OK after
    exactly that callback (reference tests/test_generate.c:359-377)."""
    from tests.test_text import tokenizer_model, NAMES
    m = native.Model(tokenizer_model(NAMES[0], model_dir), max_ctx=128)
    s = m.acquire()
    calls = []

    def cb(piece, n, eos, ud):
        calls.append(n)
        return 1

    fn = native.TOKEN_CB(cb)
    prm = native.default_params(max_new_tokens=100, seed=1)
    rc = native.lib().cmol_generate(s.h, b"Hello", native.C.byref(prm), fn, None)
    assert rc == 0 and len(calls) == 1
    m.close()


def test_reset_reproduces_greedy_output(gpu, model_dir):
    """cmol_session_reset then the same prompt: the same greedy pieces
    (reference tests/test_generate.c:379-407)."""
    from tests.test_text import tokenizer_model, NAMES
    m = native.Model(tokenizer_model(NAMES[0], model_dir), max_ctx=128)
    s = m.acquire()
    prm = native.default_params(temperature=0.0, max_new_tokens=5)
    a, rc1 = s.generate_text(b"Hello", prm)
    s.reset()
    b, rc2 = s.generate_text(b"Hello", prm)
    assert rc1 == rc2 == 0 and len(a) == 5 and a == b
    m.close()


@pytest.mark.parametrize("name", ["micro-q8_0", "small-q5_0", "small-q4_0"])
def test_greedy_with_penalty_matches_reference(gpu, model_dir, name):
    """Greedy decoding with the repetition penalty (logits to the host, the
    penalty ring of the generate loop): the reference's ids
    (tests/golden/penalty.npz, written by the built reference)."""
    pen = np.load(os.path.join(HERE, "golden", "penalty.npz"))
    spec = synth.PRESETS[name].replace(wstd=float(pen[f"{name}_wstd"]))
    path = synth.model_file(spec, model_dir)
    m = native.Model(path, max_ctx=128, max_sessions=1)
    s = m.acquire()
    for ri, (p, last_n) in enumerate(pen["runs"]):
        s.reset()
        prm = native.greedy_params(48, repeat_penalty=float(p), repeat_last_n=int(last_n))
        got = s.generate_ids(pen[f"{name}_prompt"], prm, 48)
        assert got.tolist() == pen[f"{name}_run{ri}_ids"].tolist(), (name, ri)
    m.close()
