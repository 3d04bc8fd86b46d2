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
