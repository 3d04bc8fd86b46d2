"""The persistent single-session decode kernel (one cooperative launch per
token; each stage's readers poll the vectors they consume) against the
oracle and against the per-kernel decode graph of the same model."""
import os

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def close_frac(got, want, atol=1e-4, rtol=1e-3):
    return np.mean(np.abs(got - want) <= atol + rtol * np.abs(want))


def load(path, max_ctx, persistent=True, kv_f16=False, **kw):
    """A single-session model decoding with the persistent kernel (opt-in) or
    with the decode graph."""
    env = {"CMOL_PERSIST": "1" if persistent else None, "CMOL_KV_F16": "1" if kv_f16 else None}
    old = {k: os.environ.get(k) for k in env}
    try:
        for k, v in env.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        m = native.Model(path, max_ctx=max_ctx, max_sessions=1, **kw)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    assert m.persistent == persistent
    return m


@pytest.mark.parametrize("preset", ["small-q5_0", "small-q8_0-untied", "smollm2-135m-q8_0"])
def test_persistent_greedy_matches_oracle(gpu, model_dir, preset):
    """Prompt, then greedy decode through the persistent kernel: the ids equal
    the oracle's, through prompts that cross the attention split size (the
    split-merge stage runs) and ones that do not."""
    spec = synth.PRESETS[preset].replace(wstd=0.08)
    if preset.startswith("smollm2"):
        spec = spec.replace(n_layers=4, vocab=4096)
    path = synth.model_file(spec, model_dir)
    for plen, n_new in ((9, 20), (140, 24)):
        prompt = synth.tokens(plen, 42 + plen, spec.vocab)
        m = load(path, 192)
        s = m.acquire()
        got = s.generate_ids(prompt, native.greedy_params(n_new), n_new)
        m.close()
        want = O.Model(path, 192).generate(prompt, n_new)
        assert got.tolist() == want.tolist(), f"prompt {plen}"


@pytest.mark.parametrize("preset", ["small-q5_0", "small-q8_0-untied"])
def test_persistent_logits_match_oracle(gpu, model_dir, preset):
    """Token by token through the persistent kernel: logits within
    1e-4 + 1e-3*|ref| of the oracle's at every position."""
    spec = synth.PRESETS[preset].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    toks = synth.tokens(30, 3, spec.vocab)
    m = load(path, 64)
    s = m.acquire()
    om = O.Model(path, 64)
    for p, t in enumerate(toks):
        am, lg = s.forward(int(t), p, spec.vocab)
        ref = om.forward(int(t), p)
        assert close_frac(lg, ref) == 1.0, f"position {p}"
        assert am == int(np.argmax(lg))
    m.close()


@pytest.mark.parametrize("preset,ctx,kv_f16", [("smollm2-360m-q5_0", 3000, False),
                                               ("smollm2-360m-q5_0", 900, True),
                                               ("smollm3-3b-q4_0", 2048, False),
                                               ("smollm3-3b-q4_0", 5000, True)])
def test_persistent_matches_graph_long_context(gpu, model_dir, preset, ctx, kv_f16):
    """Config-shaped models over synthetic KV caches of ctx positions (many
    attention splits, fp32 and fp16 caches): the persistent kernel's logits
    match the decode graph's within the matvec tolerance for a few steps, and
    the greedy token agrees unless the two best logits are that close."""
    spec = synth.PRESETS[preset]
    spec = spec.replace(ctx_len=max(spec.ctx_len, ctx + 16))
    path = synth.model_file(spec, model_dir)
    out = {}
    for persistent in (True, False):
        m = load(path, ctx + 16, persistent=persistent, kv_f16=kv_f16)
        s = m.acquire()
        s.fill_kv(ctx, seed=21)
        tok, res = 7, []
        for i in range(3):
            am, lg = s.forward(tok, ctx + i, spec.vocab)
            res.append((am, lg))
            tok = int(np.argmax(lg))
        out[persistent] = res
        m.close()
    for i, ((a1, l1), (a2, l2)) in enumerate(zip(out[True], out[False])):
        assert close_frac(l1, l2) == 1.0, f"step {i}"
        if a1 != a2:
            top = np.sort(l2)[-2:]
            assert top[1] - top[0] <= 1e-4 + 1e-3 * abs(top[1]), f"step {i}: {a1} vs {a2}"


def test_persistent_selection(gpu, model_dir, monkeypatch):
    """With CMOL_PERSIST=1 the persistent kernel serves single-session models
    with d_head 64/128 and uniform layer formats; pools of sessions, other
    head sizes and the default keep the decode graph."""
    spec = synth.PRESETS["small-q5_0"]
    path = synth.model_file(spec, model_dir)
    micro = synth.model_file(synth.PRESETS["micro-q4_0"], model_dir)   # d_head 16
    monkeypatch.delenv("CMOL_PERSIST", raising=False)
    m = native.Model(path, max_ctx=64, max_sessions=1)
    assert not m.persistent
    m.close()
    monkeypatch.setenv("CMOL_PERSIST", "1")
    m = native.Model(path, max_ctx=64, max_sessions=1)
    assert m.persistent
    m.close()
    m = native.Model(path, max_ctx=64, max_sessions=2)
    assert not m.persistent
    m.close()
    m = native.Model(micro, max_ctx=64, max_sessions=1)
    assert not m.persistent
    m.close()
