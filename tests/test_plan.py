"""Launch planning on the CPU: the k-split scratch a model reserves for its
lock-step batch covers every matvec launch of a decode step at every batch
size.  The launch list is spelled out here from the model's shape (q, k and
v launch once per run of consecutive parts that share a format), not taken
from the library, and each launch's need comes from the library's own
planner (cmolhip_gemv_scratch_floats)."""
import ctypes as C

import pytest

import libcmol_amd.native as native

F32, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K = 0, 2, 6, 8, 12, 14


def hparams(layers, d, heads, kv, ffn, vocab, sessions):
    return native.HParams(layers, heads, kv, d, d // heads, ffn, vocab, 4096, sessions, 4, 1, 512, 1e4,
                          1e-6)


# (name, hparams, q, k, v, o, gate/up, down, embedding, lm head or None)
SHAPES = [
    ("smollm3-3b q4_k_m", hparams(36, 2048, 16, 4, 11008, 128256, 32), Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q6_K,
     Q6_K, None),
    ("smollm3-3b q4_0", hparams(36, 2048, 16, 4, 11008, 128256, 32), Q4_0, Q4_0, Q4_0, Q4_0, Q4_0, Q4_0,
     Q8_0, None),
    ("smollm3-3b q4_0, q5_0 v", hparams(36, 2048, 16, 4, 11008, 128256, 32), Q4_0, Q4_0, Q5_0, Q4_0, Q4_0,
     Q5_0, Q8_0, None),
    ("smollm3-3b q5_0 k", hparams(36, 2048, 16, 4, 11008, 128256, 24), Q4_0, Q5_0, Q4_0, Q4_0, Q4_0, Q4_0,
     Q8_0, Q8_0),
    ("smollm2-360m q5_0", hparams(32, 960, 15, 5, 2560, 49152, 16), Q5_0, Q5_0, Q5_0, Q5_0, Q5_0, Q5_0,
     Q5_0, None),
    ("smollm2-360m q4_k_m", hparams(32, 1024, 16, 4, 2816, 49152, 32), Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q6_K,
     Q6_K, Q6_K),
    ("smollm2-135m q8_0", hparams(30, 576, 9, 3, 1536, 49152, 32), Q8_0, Q8_0, Q8_0, Q8_0, Q8_0, Q8_0, Q8_0,
     None),
    # hidden 4096: the operand slice of every projection is split in k
    ("hidden-4096 q4_k_m", hparams(4, 4096, 32, 8, 14336, 32000, 32), Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q6_K,
     Q6_K, Q6_K),
]


def step_launches(hp, q, k, v, o, gu, dn, embd, lm):
    """(dtype, rows, cols) of every matvec of one decode step."""
    d, kvd = hp.d_model, hp.n_kv_heads * hp.d_head
    runs = []
    for dt, rows in ((q, d), (k, kvd), (v, kvd)):
        if runs and runs[-1][0] == dt:
            runs[-1][1] += rows
        else:
            runs.append([dt, rows])
    layer = [(dt, rows, d) for dt, rows in runs] + [(o, d, d), (gu, 2 * hp.d_ffn, d), (dn, d, hp.d_ffn)]
    return layer * hp.n_layers + [(lm if lm is not None else embd, hp.vocab, d)]


def need(L, hp, launches, n):
    best = 0
    for dt, rows, cols in launches:
        fold = L.cmolhip_pick_fold(rows, cols, hp.max_sessions)
        best = max(best, L.cmolhip_gemv_scratch_floats(dt, rows, cols, fold, n))
    return best


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_batch_scratch_covers_every_launch(shape):
    name, hp, *fmts = shape
    L = native.lib()
    desc, keep = native.shape_desc(hp, *fmts)
    have = C.c_size_t()
    assert L.cmolhip_batch_scratch_floats(C.byref(desc), hp.max_sessions, C.byref(have)) == 0
    launches = step_launches(hp, *fmts)
    needs = [need(L, hp, launches, n) for n in range(1, hp.max_sessions + 1)]
    assert max(needs) <= have.value, (name, max(needs), have.value)
    # the reservation is the largest need, not more
    assert max(needs) == have.value
    del keep


def test_mixed_qkv_runs_need_more_than_the_whole_matrix():
    """The case the per-run launch list exists for: q|k Q4_K (2560 rows) and
    v Q6_K split k more finely than one 3072-row matrix would, so a batch of
    24 needs more scratch than the whole q|k|v matrix would suggest."""
    L = native.lib()
    whole = L.cmolhip_gemv_scratch_floats(Q4_K, 3072, 2048, 1, 24)
    qk_run = L.cmolhip_gemv_scratch_floats(Q4_K, 2560, 2048, 1, 24)
    assert qk_run > whole
    _, hp, *fmts = SHAPES[0]
    desc, keep = native.shape_desc(hp, *fmts)
    have = C.c_size_t()
    assert L.cmolhip_batch_scratch_floats(C.byref(desc), 32, C.byref(have)) == 0
    assert have.value >= qk_run


def test_scratch_planner_rejects_bad_shapes():
    L = native.lib()
    assert L.cmolhip_gemv_scratch_floats(Q4_0, 2048, 2048, 1, 0) == 0
    assert L.cmolhip_gemv_scratch_floats(Q4_0, 2048, 2048, 1, 33) == 0
    assert L.cmolhip_gemv_scratch_floats(Q4_0, 2048, 2000, 1, 16) == 0
    assert L.cmolhip_gemv_scratch_floats(F32, 2048, 2048, 1, 16) == 0
    # batches of up to 8 vectors never split k
    assert all(L.cmolhip_gemv_scratch_floats(Q4_0, 2048, 11008, 1, n) == 0 for n in range(1, 9))
    hp = SHAPES[1][1]
    desc, keep = native.shape_desc(hp, *SHAPES[1][2:])
    out = C.c_size_t()
    assert L.cmolhip_batch_scratch_floats(C.byref(desc), 0, C.byref(out)) == native.CMOL_ERR_ARGS
    assert L.cmolhip_batch_scratch_floats(None, 4, C.byref(out)) == native.CMOL_ERR_ARGS
