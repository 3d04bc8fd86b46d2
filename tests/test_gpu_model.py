"""Whole-model decode on the GPU against the oracle: identical greedy token
ids, logits within 1e-3 relative / 1e-4 absolute."""
import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def close_frac(got, want, atol=1e-4, rtol=1e-3):
    return np.mean(np.abs(got - want) <= atol + rtol * np.abs(want))


@pytest.mark.parametrize("preset", ["micro-q8_0", "micro-q4_0", "micro-q5_0", "small-q4_0",
                                    "small-q5_0", "small-q8_0-untied"])
def test_greedy_tokens_match_oracle(gpu, model_dir, preset):
    spec = synth.PRESETS[preset].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    prompt = synth.tokens(16, 42, spec.vocab)
    n_new = 48
    m = native.Model(path, max_ctx=128, max_sessions=2)
    s = m.acquire()
    got = s.generate_ids(prompt, native.greedy_params(n_new), n_new)
    om = O.Model(path, 128)
    want = om.generate(prompt, n_new)
    assert got.tolist() == want.tolist()
    m.close()


@pytest.mark.parametrize("preset", ["small-q4_0", "small-q5_0", "small-q8_0-untied"])
def test_forward_logits_match_oracle(gpu, model_dir, preset):
    spec = synth.PRESETS[preset]
    path = synth.model_file(spec, model_dir)
    toks = synth.tokens(40, 7, spec.vocab)
    m = native.Model(path, max_ctx=64, max_sessions=1)
    s = m.acquire()
    om = O.Model(path, 64)
    for pos, t in enumerate(toks):
        am, lg = s.forward(int(t), pos, spec.vocab)
        want = om.forward(int(t), pos)
        frac = close_frac(lg, want)
        assert frac == 1.0, f"pos {pos}: {1 - frac:.4%} of logits outside tolerance"
        assert am == int(np.argmax(lg))
    m.close()


def test_kv_cache_matches_oracle(gpu, model_dir):
    spec = synth.PRESETS["small-q4_0"]
    path = synth.model_file(spec, model_dir)
    toks = synth.tokens(20, 3, spec.vocab)
    m = native.Model(path, max_ctx=32, max_sessions=1)
    s = m.acquire()
    s.prefill(toks)
    om = O.Model(path, 32)
    for p, t in enumerate(toks):
        om.forward(int(t), p)
    ok, ov = om.kv()
    import ctypes as C
    kd = (spec.n_kv_heads * spec.d_head)
    for layer in range(spec.n_layers):
        k = np.zeros((20, kd), np.float32)
        v = np.zeros((20, kd), np.float32)
        native.check(native.lib().cmolhip_kv_download(m.device, s.slot, layer, 20,
                                                       native.ptr(k), native.ptr(v)), "kv")
        assert close_frac(k, ok[layer, :20].reshape(20, kd)) == 1.0
        assert close_frac(v, ov[layer, :20].reshape(20, kd)) == 1.0
    m.close()


def test_smollm2_135m_greedy_128(gpu, model_dir):
    """SmolLM2-135M shape, Q8_0, 32-token seeded prompt, 128 greedy tokens; the
    first 64 must be identical to the oracle's."""
    spec = synth.PRESETS["smollm2-135m-q8_0"]
    path = synth.model_file(spec, model_dir)
    prompt = synth.tokens(32, 42, spec.vocab)
    m = native.Model(path, max_ctx=256, max_sessions=1)
    s = m.acquire()
    got = s.generate_ids(prompt, native.greedy_params(128), 128)
    om = O.Model(path, 256)
    want, margins = om.generate(prompt, 128, margins=True)
    print("min top-2 margin over 128 steps:", float(margins.min()))
    assert got[:64].tolist() == want[:64].tolist()
    m.close()
