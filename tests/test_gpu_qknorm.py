"""QK-norm models (attn_q_norm / attn_k_norm: per-head RMSNorm of q and k
before RoPE, reference src/attn.c:62-80) on the GPU: the reference's own
prompt logits and greedy continuations (tests/golden/qknorm.npz, written by
tests/golden/make_qknorm_golden.py from the reference built from its
sources), and the decode matvec path, chunked prompt passes, lock-step
batches and the KV cache against the oracle."""
import os

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O
from tests.golden import make_qknorm_golden as qkn

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
QN = np.load(os.path.join(HERE, "golden", "qknorm.npz"))


def close_frac(got, want, atol=1e-4, rtol=1e-3):
    return np.mean(np.abs(got - want) <= atol + rtol * np.abs(want))


def kv_of(m, s, layer, n, kd):
    k = np.zeros((n, kd), np.float32)
    v = np.zeros((n, kd), np.float32)
    native.check(native.lib().cmolhip_kv_download(m.device, s.slot, layer, n, native.ptr(k), native.ptr(v)),
                 "kv")
    return k, v


@pytest.mark.parametrize("name", sorted(qkn.MODELS))
def test_qk_norm_models_match_reference(gpu, model_dir, name):
    """The prompt pass (GEMM + QK-norm stage) gives the reference's logits
    within 1e-3 relative / 1e-4 absolute, and prompt + greedy decode give the
    reference's 40 ids."""
    spec = qkn.spec_of(name)
    path = synth.model_file(spec, model_dir)
    prompt = QN[f"{name}_prompt"]
    m = native.Model(path, max_ctx=128, max_sessions=1)
    s = m.acquire()
    am, lg = s.prefill(prompt, spec.vocab)
    want = QN[f"{name}_prompt_logits"]
    assert close_frac(lg, want) == 1.0
    assert am == int(np.argmax(want))
    s.reset()
    got = s.generate_ids(prompt, native.greedy_params(40), 40)
    assert got.tolist() == QN[f"{name}_ids"].tolist()
    m.close()


@pytest.mark.parametrize("name", ["qkn_q8_0_dh128", "qkn_q5_0_nope", "qkn_q4_k"])
@pytest.mark.parametrize("kv_f16", [False, True])
def test_qk_norm_decode_matches_oracle(gpu, model_dir, monkeypatch, name, kv_f16):
    """Token-by-token decode (matvec + QK-norm stage): logits at every
    position and the whole KV cache match the oracle (fp32 cache); with an
    fp16 cache, layer 0's cache (whose inputs do not depend on the cache)
    matches the oracle's to fp16 rounding."""
    if kv_f16:
        monkeypatch.setenv("CMOL_KV_F16", "1")
    else:
        monkeypatch.delenv("CMOL_KV_F16", raising=False)
    spec = qkn.spec_of(name)
    path = synth.model_file(spec, model_dir)
    toks = synth.tokens(30, 8, spec.vocab)
    m = native.Model(path, max_ctx=64, max_sessions=1)
    s = m.acquire()
    om = O.Model(path, 64)
    for pos, t in enumerate(toks):
        am, lg = s.forward(int(t), pos, spec.vocab)
        want = om.forward(int(t), pos)
        if not kv_f16:
            assert close_frac(lg, want) == 1.0, f"pos {pos}"
            assert am == int(np.argmax(lg))
    ok, ov = om.kv()
    kd = spec.n_kv_heads * spec.d_head
    n = len(toks)
    for layer in range(1 if kv_f16 else spec.n_layers):
        k, v = kv_of(m, s, layer, n, kd)
        assert close_frac(k, ok[layer, :n].reshape(n, kd)) == 1.0, f"K layer {layer}"
        assert close_frac(v, ov[layer, :n].reshape(n, kd)) == 1.0, f"V layer {layer}"
    m.close()


@pytest.mark.parametrize("name,chunk", [("qkn_q8_0", 7), ("qkn_q4_k", 16), ("qkn_q8_0_dh128", 32)])
def test_qk_norm_chunked_prefill_matches_oracle(gpu, model_dir, name, chunk):
    """A prompt split into several passes: logits after the prompt and the
    KV cache of every layer match the oracle."""
    spec = qkn.spec_of(name)
    path = synth.model_file(spec, model_dir)
    prompt = synth.tokens(45, 11, spec.vocab)
    m = native.Model(path, max_ctx=64, max_sessions=1, prefill_chunk=chunk)
    s = m.acquire()
    am, lg = s.prefill(prompt, spec.vocab)
    om = O.Model(path, 64)
    for p, t in enumerate(prompt):
        want = om.forward(int(t), p)
    assert close_frac(lg, want) == 1.0
    assert am == int(np.argmax(want))
    ok, ov = om.kv()
    kd = spec.n_kv_heads * spec.d_head
    for layer in range(spec.n_layers):
        k, v = kv_of(m, s, layer, 45, kd)
        assert close_frac(k, ok[layer, :45].reshape(45, kd)) == 1.0, f"K layer {layer}"
        assert close_frac(v, ov[layer, :45].reshape(45, kd)) == 1.0, f"V layer {layer}"
    m.close()


@pytest.mark.parametrize("name", ["qkn_q8_0", "qkn_q5_0_nope"])
def test_qk_norm_decode_batch_matches_oracle(gpu, model_dir, name):
    """Lock-step decode of sessions with ragged prompts continues each one
    exactly as the oracle decodes it alone."""
    spec = qkn.spec_of(name)
    path = synth.model_file(spec, model_dir)
    lens = [3, 17, 1, 40, 8]
    prompts = [synth.tokens(L, 100 + i, spec.vocab) for i, L in enumerate(lens)]
    steps = 12
    m = native.Model(path, max_ctx=96, max_sessions=len(lens))
    ss = [m.acquire() for _ in lens]
    toks = np.array([s.prefill(p)[0] for s, p in zip(ss, prompts)], np.int32)
    got = [toks.copy()]
    for _ in range(steps):
        toks = native.decode_batch(ss, toks)
        got.append(toks.copy())
    got = np.stack(got, 1)
    m.close()
    for i, p in enumerate(prompts):
        want = O.Model(path, 96).generate(p, steps + 1)
        assert got[i].tolist() == want.tolist(), f"session {i} (prompt {lens[i]})"
