"""The oracle (CPU restatement of the reference) against the reference's own
outputs (golden fixtures written by tests/golden/make_golden.py from the
reference built from its sources), the reference's own unit-test known
answers, and properties fixed by the mathematics."""
import hashlib
import json
import os

import numpy as np
import pytest

from libcmol_amd import synth
from oracle import oracle as O
from tests.golden import make_qknorm_golden as qkn
from tests.qdata import random_blocks

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "golden.npz"))
META = json.load(open(os.path.join(HERE, "golden", "golden.json")))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- fp16 -------------------------------------------------------------------
def test_f16_table_matches_reference():
    h = np.arange(65536, dtype=np.uint16)
    f = O.dequant_row(h, 65536, 1)
    assert hashlib.sha256(f.view(np.uint32).tobytes()).hexdigest() == META["f16_table_sha256"]
    assert np.array_equal(bits(f[G["f16_special_in"].astype(np.int64)]), G["f16_special_out"])


def test_f16_matches_numpy_for_all_non_nan():
    """numpy's half->float conversion is an independent implementation."""
    h = np.arange(65536, dtype=np.uint16)
    f = O.dequant_row(h, 65536, 1)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(bits(f[~nan]), bits(ref[~nan]))
    # NaN payload: mantissa << 13 under an all-ones exponent, sign kept
    exp_bits = (h[nan].astype(np.uint32) & 0x8000) << 16 | 0x7F800000 | \
        ((h[nan].astype(np.uint32) & 0x3FF) << 13)
    assert np.array_equal(bits(f[nan]), exp_bits)


# ---- dequantisation -----------------------------------------------------------
@pytest.mark.parametrize("name,dt", [("q8_0", 8), ("q5_0", 6), ("q4_0", 2)])
@pytest.mark.parametrize("tag", ["rand", "special"])
def test_dequant_matches_reference(name, dt, tag):
    raw = G[f"deq_{name}_{tag}_in"]
    want = G[f"deq_{name}_{tag}_out"]
    got = np.stack([O.dequant_row(raw[r], 128, dt) for r in range(raw.shape[0])])
    assert np.array_equal(bits(got), want)


def test_dequant_q8_0_reference_kats():
    """Reference tests/test_quant.c:97-127."""
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    b[2], b[3] = 3, np.uint8(np.int8(-1).view(np.uint8))
    out = O.dequant_row(b, 32, 8)
    assert out[0] == 6.0 and out[1] == -2.0 and out[2] == 0.0 and out[31] == 0.0
    b2 = np.zeros(68, np.uint8)
    b2[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8); b2[2] = 7
    b2[34:36] = np.frombuffer(np.float16(3.0).tobytes(), np.uint8); b2[36] = 2
    out2 = O.dequant_row(b2, 64, 8)
    assert out2[0] == 7.0 and out2[32] == 6.0


def test_dequant_edge_cases_are_noops():
    """Reference tests/test_quant.c:366-386: NULL src, n=0, unknown dtype."""
    dst = np.full(32, 9.9, np.float32)
    blk = np.zeros(34, np.uint8)
    O.lib().o_dequant_row(None, dst.ctypes.data, 32, 8)
    O.lib().o_dequant_row(blk.ctypes.data, dst.ctypes.data, 0, 8)
    O.lib().o_dequant_row(blk.ctypes.data, dst.ctypes.data, 32, 99)
    assert np.all(dst == np.float32(9.9))


def test_q4_0_closed_form():
    """Q4_0 value = fp16 scale * (nibble - 8); nibble j of block is the low
    half of byte j (j < 16) or the high half of byte j-16."""
    raw = random_blocks(2, 8, 256, seed=3)
    blk = raw.reshape(8, 8, 18)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    q = np.concatenate([(blk[:, :, 2:] & 0xF), (blk[:, :, 2:] >> 4)], axis=2).astype(np.float32) - 8
    want = (d[..., None] * q).reshape(8, 256)
    got = np.stack([O.dequant_row(raw[r], 256, 2) for r in range(8)])
    assert np.array_equal(bits(got), bits(want))


def test_q5_0_closed_form():
    raw = random_blocks(6, 4, 128, seed=4)
    blk = raw.reshape(4, 4, 22)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    qh = blk[:, :, 2:6].copy().view(np.uint32)[..., 0]
    j = np.arange(16)
    lo = (blk[:, :, 6:] & 0xF) | (((qh[..., None] >> j) & 1) << 4)
    hi = (blk[:, :, 6:] >> 4) | (((qh[..., None] >> (j + 16)) & 1) << 4)
    q = np.concatenate([lo, hi], axis=2).astype(np.float32) - 16
    want = (d[..., None] * q).reshape(4, 128)
    got = np.stack([O.dequant_row(raw[r], 128, 6) for r in range(4)])
    assert np.array_equal(bits(got), bits(want))


# ---- K-quants (tests/golden/make_kquant_golden.py) ---------------------------
KQ = np.load(os.path.join(HERE, "golden", "kquant.npz"))


@pytest.mark.parametrize("name,dt", [("q4_k", 12), ("q6_k", 14)])
@pytest.mark.parametrize("tag", ["rand", "special"])
def test_kquant_dequant_matches_reference(name, dt, tag):
    raw = KQ[f"deq_{name}_{tag}_raw"]
    want = KQ[f"deq_{name}_{tag}_out"]
    cols = want.shape[1]
    got = np.stack([O.dequant_row(raw[r], cols, dt) for r in range(raw.shape[0])])
    assert np.array_equal(bits(got), want)


@pytest.mark.parametrize("name,dt", [("q4_k", 12), ("q6_k", 14)])
@pytest.mark.parametrize("shape", [(16, 512, 1), (24, 768, 3)])
def test_kquant_matmul_matches_reference_orders(name, dt, shape):
    m, k, n = shape
    key = f"mm_{name}_{m}x{k}x{n}"
    a, b = KQ[key + "_raw"], KQ[key + "_b"]
    for order, suffix in ((O.SCALAR, "_scalar"), (O.AVX512, "_avx512")):
        assert np.array_equal(bits(O.matmul(a, b, m, k, dt, order)), KQ[key + suffix]), suffix


@pytest.mark.parametrize("preset", ["small-q4_k", "small-q6_k-untied", "small-q4_k_m"])
def test_kquant_models_match_reference(preset, model_dir):
    """Whole models with Q4_K / Q6_K layers (and K-quant embedding / LM
    head): the oracle's greedy continuation equals the reference's."""
    spec = synth.PRESETS[preset].replace(wstd=0.08)
    path = synth.model_file(spec, model_dir)
    prompt = KQ[f"model_{preset}_prompt"]
    assert np.array_equal(prompt, synth.tokens(16, 42, spec.vocab))
    got = O.Model(path, 128).generate(prompt, 48)
    assert got.tolist() == KQ[f"model_{preset}_ids"].tolist()


# ---- QK-norm (tests/golden/make_qknorm_golden.py) ---------------------------
QN = np.load(os.path.join(HERE, "golden", "qknorm.npz"))


@pytest.mark.parametrize("name", sorted(qkn.MODELS))
def test_qk_norm_models_match_reference(name, model_dir):
    """Models with attn_q_norm / attn_k_norm (per-head RMSNorm of q and k
    before RoPE; d_head 64 and 128, with NoPE layers, Q8_0 / Q5_0 / Q4_K):
    the oracle's logits after the prompt and its greedy continuation equal
    the reference's."""
    spec = qkn.spec_of(name)
    path = synth.model_file(spec, model_dir)
    prompt = QN[f"{name}_prompt"]
    om = O.Model(path, 128)
    for p, t in enumerate(prompt):
        lg = om.forward(int(t), p)
    want = QN[f"{name}_prompt_logits"]
    assert np.all(np.abs(lg - want) <= 1e-5 + 1e-4 * np.abs(want))
    got = O.Model(path, 128).generate(prompt, 40)
    assert got.tolist() == QN[f"{name}_ids"].tolist()


def test_yarn_key_is_not_applied(model_dir):
    """A rope.scaling.type key is recorded and ignored by the reference
    (src/gguf.c:384-389): the SmolLM3-shaped fixture model decodes exactly as
    the same weights without the key."""
    spec = qkn.spec_of("qkn_smollm3_yarn")
    prompt = QN["qkn_smollm3_yarn_prompt"]
    plain = synth.model_file(spec.replace(rope_scaling=0), model_dir)
    assert O.Model(plain, 128).generate(prompt, 40).tolist() == QN["qkn_smollm3_yarn_ids"].tolist()


# ---- generate-loop stop rules (tests/golden/make_generate_golden.py) --------
GE = np.load(os.path.join(HERE, "golden", "generate_edges.npz"))


def test_generate_stop_rules_match_reference(model_dir):
    """The oracle's greedy loop stops as the reference's: after emitting the
    EOS id, and after the token sampled at the last context position."""
    from tests.golden import make_generate_golden as ge
    prompt = GE["prompt"]
    path = synth.model_file(ge.eos_spec(int(GE["eos_id"][0])), model_dir)
    assert O.Model(path, 128).generate(prompt, 40).tolist() == GE["eos_ids"].tolist()
    path = synth.model_file(ge.eos_spec(), model_dir)
    assert O.Model(path, ge.CTX_FULL).generate(prompt, 64).tolist() == GE["ctx_full_ids"].tolist()


def test_q4_k_closed_form():
    """Q4_K: sub-block j of a super-block with d = 1, dmin = 0.5, scale
    j + 1 and min 2j (the six-bit packing spelled out by hand, bits 4-5 of
    scales/mins 4..7 in the top bits of bytes 0..7) and codes q = (k + j) % 16
    dequantises to (j + 1) q - j."""
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    q = np.array([[(k + j) % 16 for k in range(32)] for j in range(8)], np.uint8)
    qs = np.zeros(128, np.uint8)
    for p in range(4):
        qs[32 * p:32 * p + 32] = q[2 * p] | (q[2 * p + 1] << 4)
    blk = np.concatenate([np.frombuffer(np.float16(1.0).tobytes(), np.uint8),
                          np.frombuffer(np.float16(0.5).tobytes(), np.uint8), s, qs])
    got = O.dequant_row(blk, 256, 12).reshape(8, 32)
    want = np.array([[(j + 1) * q[j, k] - 0.5 * (2 * j) for k in range(32)] for j in range(8)], np.float32)
    assert np.array_equal(got, want)


def test_q6_k_closed_form():
    """Q6_K: value i of a super-block with d = 0.25 and int8 scale
    (i//16) - 8 holds code c = (7 i) % 64 split into ql nibbles and qh bit
    pairs as the reference lays them out; it dequantises to
    0.25 (i//16 - 8)(c - 32)."""
    c = np.array([(7 * i) % 64 for i in range(256)])
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for i in range(256):
        g, j = divmod(i, 32)
        li = (0 if g < 4 else 64) + 32 * (g & 1) + j
        ql[li] |= (c[i] & 0xF) << (4 if g & 2 else 0)
        qh[(0 if g < 4 else 32) + j] |= (c[i] >> 4) << (2 * (g & 3))
    scales = np.array([k - 8 for k in range(16)], np.int8).view(np.uint8)
    blk = np.concatenate([ql, qh, scales, np.frombuffer(np.float16(0.25).tobytes(), np.uint8)])
    got = O.dequant_row(blk, 256, 14)
    want = np.array([0.25 * (i // 16 - 8) * (c[i] - 32) for i in range(256)], np.float32)
    assert np.array_equal(got, want)


# ---- matmul -------------------------------------------------------------------
@pytest.mark.parametrize("name,dt", [("q8_0", 8), ("q5_0", 6), ("q4_0", 2)])
@pytest.mark.parametrize("shape", [(16, 128, 1), (33, 256, 1), (8, 64, 3)])
def test_matmul_matches_reference_orders(name, dt, shape):
    m, k, n = shape
    key = f"mm_{name}_{m}x{k}x{n}"
    a, b = G[key + "_a"], G[key + "_b"]
    for order, suffix in ((O.SCALAR, "_scalar"), (O.AVX512, "_avx512")):
        got = O.matmul(a, b, m, k, dt, order)
        assert np.array_equal(bits(got), G[key + suffix]), suffix


def test_matmul_f32_with_tail_matches_reference():
    a, b = G["mm_f32_5x37x2_a"], G["mm_f32_5x37x2_b"]
    for order, suffix in ((O.SCALAR, "_scalar"), (O.AVX512, "_avx512")):
        assert np.array_equal(bits(O.matmul(a.view(np.uint8), b, 5, 37, 0, order)),
                              G["mm_f32_5x37x2" + suffix])


def test_matmul_reference_kats():
    """Reference tests/test_quant.c:217-320."""
    A = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0]], np.float32)
    assert O.matmul(A.view(np.uint8), np.array([5, 7, 0, 0], np.float32), 3, 4, 0)[:, 0].tolist() == [5, 7, 12]
    A2 = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    B2 = np.array([[1, 2], [3, 4], [0, 0], [0, 0]], np.float32)
    assert O.matmul(A2.view(np.uint8), B2, 2, 4, 0).tolist() == [[1, 2], [3, 4]]
    def blk(d, qs):
        b = np.zeros(34, np.uint8)
        b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
        for i, v in qs.items():
            b[2 + i] = np.uint8(np.int8(v).view(np.uint8))
        return b
    x = np.zeros(32, np.float32); x[0], x[1] = 1, 2
    assert O.matmul(np.stack([blk(1, {0: 1}), blk(3, {1: 1})]), x, 2, 32, 8)[:, 0].tolist() == [1, 6]
    x2 = np.zeros(64, np.float32); x2[0] = x2[32] = 1
    assert O.matmul(np.concatenate([blk(1, {0: 5}), blk(2, {0: 3})]), x2, 1, 64, 8)[0, 0] == 11


def test_matmul_matches_float64_dot():
    """Independent: float64 dot of the dequantised rows, within fp32 rounding."""
    raw = random_blocks(2, 64, 2048, seed=5)
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    w = np.stack([O.dequant_row(raw[r], 2048, 2) for r in range(64)]).astype(np.float64)
    want = w @ x.astype(np.float64)
    for order in (O.SCALAR, O.AVX512):
        got = O.matmul(raw, x, 64, 2048, 2, order)[:, 0]
        assert np.allclose(got, want, rtol=1e-4, atol=1e-5)


# ---- primitives -----------------------------------------------------------------
def test_primitives_match_reference():
    assert np.array_equal(bits(O.rms_norm(G["rms_x"], G["rms_w"], 1e-5)), G["rms_out"])
    assert np.array_equal(bits(O.softmax(G["softmax_in"])), G["softmax_out"])
    assert np.array_equal(bits(O.swiglu(G["swiglu_g"], G["swiglu_u"])), G["swiglu_out"])
    for pos in (0, 1, 37, 2047):
        q, k = O.rope(G[f"rope_{pos}_q"], G[f"rope_{pos}_k"], pos, 16, 4, 128, 5e6)
        assert np.array_equal(bits(q), G[f"rope_{pos}_qo"])
        assert np.array_equal(bits(k), G[f"rope_{pos}_ko"])


def test_primitive_reference_kats():
    """Reference tests/test_model.c:45-166."""
    o = O.rms_norm(np.array([3, 4], np.float32), np.ones(2, np.float32), 0.0)
    assert abs(o[0] - 3 / np.sqrt(12.5)) < 1e-4 and abs(o[1] - 4 / np.sqrt(12.5)) < 1e-4
    s = O.softmax(np.array([1, 2, 3], np.float32))
    assert abs(s.sum() - 1) < 1e-6 and s[2] > s[1] > s[0]
    assert np.allclose(O.softmax(np.full(4, 5.0)), 0.25)
    g = O.swiglu(np.array([0, 1], np.float32), np.array([3, 2], np.float32))
    assert g[0] == 0 and abs(g[1] - 2 / (1 + np.exp(-1))) < 1e-3
    q, k = O.rope(np.array([1, 2, 3, 4], np.float32), np.array([1, 2, 3, 4], np.float32), 1, 1, 1, 4, 10000.0)
    assert abs(q[0] - (np.cos(1) - 2 * np.sin(1))) < 1e-3 and abs(q[1] - (np.sin(1) + 2 * np.cos(1))) < 1e-3
    q0, _ = O.rope(np.arange(8, dtype=np.float32), np.arange(4, dtype=np.float32), 0, 2, 1, 4, 10000.0)
    assert np.array_equal(q0, np.arange(8, dtype=np.float32))


def test_rope_is_a_rotation_of_adjacent_pairs():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    qo, _ = O.rope(q, k, 123, 1, 1, 128, 10000.0)
    nb = np.hypot(q[0::2], q[1::2]); na = np.hypot(qo[0::2], qo[1::2])
    assert np.allclose(na, nb, rtol=1e-5)
    # angle of pair i is pos / base^(2i/d) (adjacent pairs, not split halves)
    ang = np.arctan2(qo[1::2], qo[0::2]) - np.arctan2(q[1::2], q[0::2])
    theta = 123 / 10000.0 ** (np.arange(64) * 2 / 128)
    d = np.angle(np.exp(1j * (ang - theta)))
    assert np.max(np.abs(d)) < 1e-3


def test_attention_matches_float64_bruteforce():
    rng = np.random.default_rng(9)
    nh, nkv, dh, L = 6, 2, 16, 13
    q = rng.standard_normal(nh * dh).astype(np.float32)
    kc = rng.standard_normal((L, nkv, dh)).astype(np.float32)
    vc = rng.standard_normal((L, nkv, dh)).astype(np.float32)
    got = O.attention(q, kc, vc, L, nh, nkv, dh)
    want = np.zeros(nh * dh)
    for h in range(nh):
        hk = h * nkv // nh
        s = kc[:, hk, :].astype(np.float64) @ q[h * dh:(h + 1) * dh].astype(np.float64) / np.sqrt(dh)
        p = np.exp(s - s.max()); p /= p.sum()
        want[h * dh:(h + 1) * dh] = p @ vc[:, hk, :].astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


# ---- whole model -------------------------------------------------------------------
MODEL_CASES = META["models"]


@pytest.mark.parametrize("name", sorted(MODEL_CASES))
def test_model_matches_reference(name, model_dir):
    info = MODEL_CASES[name]
    spec = synth.PRESETS[info["preset"]].replace(**info["overrides"])
    path = synth.model_file(spec, model_dir)
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == info["sha256"]
    prompt = G[f"model_{name}_prompt"]
    om = O.Model(path, info["max_ctx"])
    toks = om.generate(prompt, info["n_new"])
    assert toks.tolist() == G[f"model_{name}_tokens"].tolist()
    om.close()
    om = O.Model(path, info["max_ctx"])
    for p, t in enumerate(prompt):
        lg = om.forward(int(t), p)
    assert np.array_equal(bits(lg), G[f"model_{name}_last_prompt_logits"])
    om.close()


def test_smollm2_135m_matches_reference(model_dir):
    spec = synth.PRESETS["smollm2-135m-q8_0"]
    path = synth.model_file(spec, model_dir)
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == META["smollm2_135m_sha256"]
    om = O.Model(path, 256)
    toks = om.generate(G["smollm2_135m_prompt"], 128)
    assert toks.tolist() == G["smollm2_135m_tokens"].tolist()
    om.close()


# ---- repetition penalty (reference src/sampler.c:171-184, src/api.c:465-507) --
PEN = np.load(os.path.join(HERE, "golden", "penalty.npz"))


@pytest.mark.parametrize("ci", range(6))
def test_repeat_penalty_matches_reference(ci):
    """o_apply_repeat_penalty is bit-identical to the reference's on logits
    with +0 / -0 / negatives and windows that repeat ids or hold ids out of
    range, for penalties at and below 1 (no-ops) and above."""
    lg, win = PEN[f"case{ci}_logits"], PEN[f"case{ci}_window"]
    for pi, pen in enumerate(PEN["penalties"]):
        got = O.apply_repeat_penalty(lg, win, float(pen))
        assert np.array_equal(bits(got), bits(PEN[f"case{ci}_p{pi}"])), (ci, float(pen))


def test_repeat_penalty_closed_form():
    """Each occurrence of an in-range id divides a positive logit by the
    penalty and multiplies a non-positive one by it."""
    lg = np.array([2.0, -3.0, 0.0, 5.0], np.float32)
    got = O.apply_repeat_penalty(lg, [0, 1, 2, 0, 9, -1], 2.0)
    assert got.tolist() == [0.5, -6.0, 0.0, 5.0]


@pytest.mark.parametrize("name", ["micro-q8_0", "small-q5_0", "small-q4_0"])
def test_greedy_with_penalty_matches_reference(name, model_dir):
    """The oracle's generate loop with the penalty ring gives the reference's
    greedy ids (penalty 1.3 over 64 tokens, 1.15 over 8), and the penalty
    changes the ids (the fixture would catch a loop that ignored it)."""
    spec = synth.PRESETS[name].replace(wstd=float(PEN[f"{name}_wstd"]))
    path = synth.model_file(spec, model_dir)
    prompt = PEN[f"{name}_prompt"]
    plain = O.Model(path, 128).generate(prompt, 48)
    for ri, (pen, last_n) in enumerate(PEN["runs"]):
        got = O.Model(path, 128).generate(prompt, 48, penalty=float(pen), last_n=int(last_n))
        want = PEN[f"{name}_run{ri}_ids"]
        assert got.tolist() == want.tolist(), (name, ri)
        assert got.tolist() != plain.tolist()


# ---- fp16 KV cache rounding (the multi-session configuration's cache) --------
def test_f32_to_f16_matches_numpy():
    """Round-to-nearest-even float->half, against numpy's independent
    conversion: every half's neighbourhood (exact values, the midpoints to
    the next half, one ulp either side), overflow and random floats."""
    h = np.arange(0x7C00, dtype=np.uint32)
    lo = h.astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    mid = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    xs = np.concatenate([lo, mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9)),
                         np.float32([65504, 65519.99, 65520, 70000, 1e30, np.inf, 0.0, 2.0**-25,
                                     2.0**-25 * 1.0001, 2.0**-26]),
                         np.random.default_rng(5).standard_normal(20000).astype(np.float32) * 100])
    xs = np.concatenate([xs, -xs])
    got = O.f32_to_f16_bits(xs)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nan = O.f32_to_f16_bits(np.float32([np.nan]))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_kv_f16_session_rounds_each_write(model_dir):
    """With the fp16 cache, layer 0's K/V at the first position are the fp32
    session's rounded once to half (later layers see the rounded values of
    the layers before them, so only their representability is fixed)."""
    spec = synth.PRESETS["small-q4_0"]
    path = synth.model_file(spec, model_dir)
    a, b = O.Model(path, 8), O.Model(path, 8, kv_f16=True)
    a.forward(17, 0)
    b.forward(17, 0)
    ka, va = a.kv()
    kb, vb = b.kv()
    assert np.array_equal(bits(kb[0, 0]), bits(ka[0, 0].astype(np.float16).astype(np.float32)))
    assert np.array_equal(bits(vb[0, 0]), bits(va[0, 0].astype(np.float16).astype(np.float32)))
    assert not np.array_equal(bits(kb[0, 0]), bits(ka[0, 0]))
    for c in (kb, vb):
        assert np.array_equal(bits(c[:, 0]), bits(c[:, 0].astype(np.float16).astype(np.float32)))
