"""Text path against the reference: tokenizer encode and
decode, the sampler, and cmol_generate on text prompts.

Every expected value in tests/golden/text_golden.json was produced by the
reference library built from its own sources (tests/golden/make_text_golden.py):
cmol_encode / cmol_decode_token on two synthetic tokenizers (GPT-2 byte-level
BPE, SentencePiece-style BPE with <0xNN> byte tokens), cmol_sample draws with
cmol_rng_seed and cmol_apply_repeat_penalty, and cmol_generate's sampled ids.
The fixture carries the tokenizers, so the GGUFs are rebuilt here with the
synthetic-model writer.  Tokenizer and sampler checks run on the CPU (the
text-only load needs no device); generation runs on the GPU."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "text_golden.json")))
NAMES = sorted(GOLD["tokenizers"])


def tokenizer_model(name, directory):
    g = GOLD["tokenizers"][name]
    t = g["tokenizer"]
    tok = synth.Tokenizer(t["model"], tuple(t["tokens"]), tuple(t["types"]), tuple(t["merges"]),
                          bos_id=t["bos_id"], eos_id=t["eos_id"], unk_id=t["unk_id"],
                          add_bos=t["add_bos"])
    sp = g["spec"]
    spec = synth.ModelSpec(n_layers=sp["n_layers"], d_model=sp["d_model"], n_heads=sp["n_heads"],
                           n_kv_heads=sp["n_kv_heads"], d_ffn=sp["d_ffn"], vocab=len(t["tokens"]),
                           ctx_len=sp["ctx_len"], wtype=synth.Q8_0, embd_type=synth.Q8_0,
                           wstd=sp["wstd"], seed=sp["seed"])
    path = os.path.join(directory, f"text-{name}.gguf")
    if not os.path.exists(path):
        synth.write_gguf_tok(path, spec, tok)
    return path


@pytest.fixture(scope="module")
def text_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("text"))


@pytest.mark.parametrize("name", NAMES)
def test_encode_matches_reference(text_dir, name):
    """cmol_encode: the same ids (and return code) as the reference for every
    text, including empty, whitespace runs, unicode, control-token strings and
    characters that fall back to bytes or <unk>; a too-small buffer returns
    the reference's error."""
    m = native.TextModel(tokenizer_model(name, text_dir))
    for case in GOLD["tokenizers"][name]["encode"]:
        ids, rc = m.encode(case["text"].encode())
        assert rc == case["rc"], repr(case["text"])
        assert ids.tolist() == case["ids"], repr(case["text"])
    _, rc = m.encode(b"the quick brown fox", cap=2)
    assert rc == GOLD["tokenizers"][name]["encode_cap2_rc"]
    m.close()


@pytest.mark.parametrize("name", NAMES)
def test_decode_token_matches_reference(text_dir, name):
    """cmol_decode_token: the same bytes as the reference for every id (byte
    tokens, U+2581 prefixes, GPT-2 byte-level characters, control tokens), and
    NULL past the vocabulary."""
    m = native.TextModel(tokenizer_model(name, text_dir))
    pieces = GOLD["tokenizers"][name]["pieces"]
    for i, want in enumerate(pieces):
        got = m.decode_token(i)
        assert (got.hex() if got is not None else None) == want, f"id {i}"
    assert m.decode_token(len(pieces)) is None
    assert m.decode_token(-1) is None
    m.close()


def sampler_logits(case_seed, draw, vocab):
    """The fixture's logits: seeded, with exact ties every 7th entry."""
    rng = np.random.default_rng([case_seed, draw])
    x = (rng.standard_normal(vocab) * 3.0).astype(np.float32)
    x[7::7] = x[6:-1:7][: x[7::7].size]
    return x


@pytest.mark.parametrize("ci", range(len(GOLD["sampler"]["cases"])))
def test_sampler_matches_reference(ci):
    """cmol_sample with cmol_rng_seed / cmol_apply_repeat_penalty: the same
    draws as the reference for greedy, plain temperature, top-k (including
    k = 1, k past the 512-entry buffer and k >= vocab), top-p and penalties,
    on logits with exact ties."""
    case = GOLD["sampler"]["cases"][ci]
    V, L = GOLD["sampler"]["vocab"], native.lib()
    prm = native.GenParams(case["temperature"], case["top_p"], case["top_k"], 0, case["seed"],
                           case["penalty"], 64)
    st = np.zeros(4, np.uint64)
    L.cmol_rng_seed(st.ctypes.data, case["seed"])
    hist = list(case["history"])
    got = []
    for d in range(GOLD["sampler"]["draws"]):
        lg = sampler_logits(ci, d, V)
        h = np.array(hist[-64:], np.int32)
        L.cmol_apply_repeat_penalty(lg.ctypes.data, V, h.ctypes.data, h.size, case["penalty"])
        tid = L.cmol_sample(lg.ctypes.data, V, prm, st.ctypes.data)
        got.append(int(tid))
        hist.append(int(tid))
    assert got == case["ids"]


@pytest.mark.parametrize("ci", range(len(GOLD["sampler"]["cases"])))
def test_sampler_pool_matches_reference(ci):
    """The same reference draws with the softmax's element-wise parts on the
    worker pool (forced on for this small vocabulary)."""
    L = native.lib()
    assert L.cmol__sampler_pool(1) >= 1   # a hold, as cmol_load takes
    prev = L.cmol__sampler_config(4, 1)
    try:
        test_sampler_matches_reference(ci)
    finally:
        L.cmol__sampler_config(prev, 16384)
        L.cmol__sampler_pool(0)


@pytest.mark.parametrize("nan", [False, True])
@pytest.mark.parametrize("params", [dict(), dict(top_k=0, top_p=0.9), dict(temperature=1.0, top_k=0, top_p=1.0),
                                    dict(temperature=0.7, top_k=512, top_p=0.0)])
def test_sampler_pool_bit_identical(params, nan):
    """Vocabulary 128256 (SmolLM3): with and without the worker pool, the
    same draws and bit-identical probabilities left in the logits buffer, on
    logits with exact ties and -inf entries (and, separately, a NaN past the
    first entry, which makes every probability NaN in both)."""
    L, V = native.lib(), 128256
    rng = np.random.default_rng(11)
    base = (rng.standard_normal(V) * 4).astype(np.float32)
    base[1000:1100] = base[5]
    base[7::9001] = -np.inf
    if nan:
        base[12345] = np.nan
    prm = native.default_params(**params)
    out = {}
    assert L.cmol__sampler_pool(1) >= 1
    for threads in (0, 4):
        prev = L.cmol__sampler_config(threads, 16384)
        st = np.zeros(4, np.uint64)
        L.cmol_rng_seed(st.ctypes.data, 99)
        ids, probs = [], None
        for d in range(6):
            lg = np.roll(base, 1237 * d).copy()
            ids.append(int(L.cmol_sample(lg.ctypes.data, V, prm, st.ctypes.data)))
            probs = lg
        L.cmol__sampler_config(prev, 16384)
        out[threads] = (ids, probs.view(np.uint32))
    L.cmol__sampler_pool(0)
    assert out[0][0] == out[4][0]
    assert np.array_equal(out[0][1], out[4][1])
    if not nan:
        assert np.isfinite(out[0][1].view(np.float32)).all() and len(set(out[0][0])) > 1


def test_rng_stream_matches_closed_form():
    """xoshiro256** seeded by splitmix64 (src/sampler.c:37-60): the first
    outputs for seed 1 follow from the published recurrences, computed here
    in Python integers."""
    M = (1 << 64) - 1

    def splitmix(x):
        x = (x + 0x9E3779B97F4A7C15) & M
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return x, z ^ (z >> 31)

    def rotl(v, k):
        return ((v << k) | (v >> (64 - k))) & M

    x, s = 1, []
    for _ in range(4):
        x, z = splitmix(x)
        s.append(z)
    want = []
    for _ in range(6):
        want.append((rotl((s[1] * 5) & M, 7) * 9) & M)
        t = (s[1] << 17) & M
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t; s[3] = rotl(s[3], 45)
    st = np.zeros(4, np.uint64)
    native.lib().cmol_rng_seed(st.ctypes.data, 1)
    got = [int(native.lib().cmol_rng_next(st.ctypes.data)) for _ in range(6)]
    assert got == want


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_generate_text_matches_reference(gpu, text_dir, name):
    """Public cmol_generate on text prompts (encode -> prefill -> decode ->
    callback per piece), greedy with and without the repeat penalty: the
    callback receives the decoded pieces of the reference's sampled ids."""
    g = GOLD["tokenizers"][name]
    pieces = [bytes.fromhex(p) for p in g["pieces"]]
    m = native.Model(tokenizer_model(name, text_dir), max_ctx=128)
    s = m.acquire()
    for case in g["generate"]:
        s.reset()
        prm = native.default_params(temperature=0.0, max_new_tokens=case["max_new"], seed=0,
                                    repeat_penalty=case["penalty"])
        got, rc = s.generate_text(case["prompt"].encode(), prm)
        assert rc == 0
        assert [p for p, _ in got] == [pieces[i] for i in case["ids"]], case["prompt"]
    m.close()


@pytest.mark.skipif(not O.ref_available(), reason="reference library not built")
@pytest.mark.parametrize("k,p", [(40, 0.95), (512, 0.0), (7, 1.0)])
def test_sampler_top_k_matches_reference_full_vocab(k, p):
    """Vocabulary 128256: the top-k scan (which passes over runs of entries
    that cannot enter the heap) keeps the reference heap's order, checked on
    logits whose largest values are exact ties (so the draw depends on the
    heap's arrangement), over 16 seeded draws against the reference library
    built from its sources (src/sampler.c:171-268)."""
    L, R, V = native.lib(), O.ref(), 128256
    R.cmol_sample.restype = C.c_int32
    R.cmol_rng_seed.restype = None
    prm = native.default_params(temperature=0.8, top_k=k, top_p=p)
    rng = np.random.default_rng(5)
    st_a, st_b = np.zeros(4, np.uint64), np.zeros(4, np.uint64)
    L.cmol_rng_seed(st_a.ctypes.data, 77)
    R.cmol_rng_seed(C.c_void_p(st_b.ctypes.data), C.c_uint(77))
    for d in range(16):
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        top = np.sort(x)[-3 * k:]
        x[rng.choice(V, 2 * k, replace=False)] = top[rng.integers(0, 4, 2 * k)]   # ties near the top
        a, b = x.copy(), x.copy()
        ia = L.cmol_sample(a.ctypes.data, V, prm, st_a.ctypes.data)
        ib = R.cmol_sample(C.c_void_p(b.ctypes.data), C.c_int(V), C.byref(prm), C.c_void_p(st_b.ctypes.data))
        assert ia == ib, f"draw {d}"
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"draw {d}"


def test_sampler_pool_lifetime():
    """The worker pool exists only while held (cmol_load holds it until
    cmol_free): holds nest, the last release joins every worker, and a draw
    without the pool runs single-threaded with the same result."""
    L, V = native.lib(), 40000
    while L.cmol__sampler_pool(0) > 0:   # drop holds left by other tests
        pass
    rng = np.random.default_rng(3)
    base = rng.standard_normal(V).astype(np.float32)
    prm = native.default_params(temperature=1.0, top_k=0, top_p=1.0)

    def draw():
        st = np.zeros(4, np.uint64)
        L.cmol_rng_seed(st.ctypes.data, 5)
        lg = base.copy()
        return int(L.cmol_sample(lg.ctypes.data, V, prm, st.ctypes.data)), lg.view(np.uint32).copy()

    alone = draw()
    prev = L.cmol__sampler_config(3, 16384)   # size of the next pool
    n1 = L.cmol__sampler_pool(1)
    n2 = L.cmol__sampler_pool(1)
    assert n1 == n2 == 3
    pooled = draw()
    assert L.cmol__sampler_pool(0) == 3   # one hold left
    assert L.cmol__sampler_pool(0) == 0   # joined
    L.cmol__sampler_config(prev, 16384)
    assert pooled[0] == alone[0] and np.array_equal(pooled[1], alone[1])
    assert draw()[0] == alone[0]


def test_seed_zero_streams_differ():
    """Seed 0 asks for a fresh, non-reproducible stream on every call."""
    L = native.lib()
    firsts = set()
    for _ in range(8):
        st = np.zeros(4, np.uint64)
        L.cmol_rng_seed(st.ctypes.data, 0)
        firsts.add(int(L.cmol_rng_next(st.ctypes.data)))
    assert len(firsts) == 8
