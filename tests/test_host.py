"""Host side of the drop-in, on the CPU: the C-ABI library loads and exports
every entry point its headers declare; public utilities and load-time error
paths behave like the reference's (src/api.c:24-41,139-206,356-398)."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

import libcmol_amd.native as native
from libcmol_amd import synth
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cmol\w*)\s*\(", text)) - {"cmol_token_cb_t", "cmol_log_fn_t"})


@pytest.mark.parametrize("header", ["cmol.h", "cmol_hip.h", "cmol_ext.h"])
def test_library_exports_every_declared_entry_point(header):
    lib = C.CDLL(native.lib_path())
    names = declared_functions(header)
    assert names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_every_declared_entry_point():
    bound = {n for n, _, _ in native.SIGNATURES}
    for h in ("cmol.h", "cmol_hip.h", "cmol_ext.h"):
        assert set(declared_functions(h)) <= bound


def ref_lib():
    if not O.ref_available():
        pytest.skip("reference library not built here (oracle/_ref)")
    L = C.CDLL(O.REF_SO)
    L.cmol_strerror.restype = C.c_char_p
    L.cmol_version.restype = C.c_char_p
    L.cmol_format_chatml.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, C.c_size_t]
    L.cmol_format_chatml_turn.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    return L


def test_strerror_and_version_match_reference():
    R, L = ref_lib(), native.lib()
    for code in range(-9, 2):
        assert L.cmol_strerror(code) == R.cmol_strerror(code)
    assert L.cmol_version() == R.cmol_version() == b"0.1.0"


@pytest.mark.parametrize("system", [None, b"", b"You are terse."])
@pytest.mark.parametrize("cap", [0, 5, 40, 400])
def test_chatml_matches_reference(system, cap):
    R, L = ref_lib(), native.lib()
    user = b"hello \xc3\xa9"
    ba, bb = C.create_string_buffer(max(cap, 1)), C.create_string_buffer(max(cap, 1))
    ra = L.cmol_format_chatml(system, user, ba if cap else None, cap)
    rb = R.cmol_format_chatml(system, user, bb if cap else None, cap)
    assert ra == rb and ba.raw == bb.raw
    ra = L.cmol_format_chatml_turn(user, ba if cap else None, cap)
    rb = R.cmol_format_chatml_turn(user, bb if cap else None, cap)
    assert ra == rb and ba.raw == bb.raw
    assert L.cmol_format_chatml(system, None, None, 0) == native.CMOL_ERR_ARGS


def load_rc(path, **cfg):
    c = native.Config(cfg.get("max_ctx", 64), cfg.get("max_sessions", 1), 512, native.LOG_FN(), None)
    err = C.c_int(99)
    h = native.lib().cmol_load(path, C.byref(c), C.byref(err))
    if h:
        native.lib().cmol_free(h)
    return err.value, h


def test_load_error_paths(tmp_path):
    assert load_rc(None)[0] == native.CMOL_ERR_ARGS
    assert load_rc(str(tmp_path / "missing.gguf").encode())[0] == native.CMOL_ERR_IO
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOPE" + b"\0" * 60)
    assert load_rc(str(bad).encode())[0] == native.CMOL_ERR_INVALID
    v4 = tmp_path / "v4.gguf"
    v4.write_bytes(struct.pack("<IIQQ", 0x46554747, 4, 0, 0))
    assert load_rc(str(v4).encode())[0] == native.CMOL_ERR_INVALID
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(struct.pack("<IIQQ", 0x46554747, 3, 1, 1)[:20])
    assert load_rc(str(trunc).encode())[0] == native.CMOL_ERR_INVALID


def test_load_without_gpu_is_unsupported(model_dir):
    if native.device_count() > 0:
        pytest.skip("a GPU is visible")
    path = synth.model_file(synth.PRESETS["micro-q8_0"], model_dir)
    rc, h = load_rc(path.encode())
    assert rc == native.CMOL_ERR_UNSUPPORTED and not h


def test_arena_estimate(model_dir):
    spec = synth.PRESETS["micro-q4_0"]
    path = synth.model_file(spec, model_dir).encode()
    c = native.Config(64, 2, 512, native.LOG_FN(), None)
    est = native.lib().cmol_arena_estimate(path, C.byref(c))
    # covers at least two sessions of fp32 KV and the quantised weights
    kv = 2 * spec.n_layers * 64 * spec.n_kv_heads * spec.d_head * 4 * 2
    assert est > kv + spec.weight_bytes_per_token()
    assert native.lib().cmol_arena_estimate(b"/nonexistent", C.byref(c)) == 0


def test_null_handles_are_safe():
    L = native.lib()
    L.cmol_free(None)
    L.cmol_session_release(None)
    L.cmol_session_reset(None)
    assert L.cmol_session_acquire(None) is None
    assert L.cmol_generate(None, b"x", None, native.TOKEN_CB(), None) == native.CMOL_ERR_ARGS
    assert L.cmol_encode(None, b"x", None, 0) == native.CMOL_ERR_ARGS
    assert L.cmol_decode_token(None, 0) is None


def test_synthetic_models_are_deterministic(tmp_path):
    spec = synth.PRESETS["micro-q5_0"]
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    synth.write_gguf(str(a), spec, nthreads=1)
    synth.write_gguf(str(b), spec, nthreads=3)
    assert a.read_bytes() == b.read_bytes()


def test_quantisers_round_trip_error_bounds():
    """Q8_0 rounds to the nearest of 255 levels (half a step); Q4_0/Q5_0 map
    the signed extreme to -8/-16, so the opposite extreme clamps at +7/+15
    (at most one step).  The scale is stored in fp16 after the codes were
    chosen with the fp32 scale: up to levels * 2^-11 steps more."""
    x = synth.normal(32 * 64, seed=3, std=0.02)
    for dt, levels, bound in ((8, 127, 0.5), (2, 8, 1.0), (6, 16, 1.0)):
        raw = synth.quantize(dt, x)
        y = O.dequant_row(raw, x.size, dt)
        amax = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
        step = amax / levels
        err = np.abs((y - x).reshape(-1, 32))
        assert np.all(err <= step * (bound + levels * 2.0 ** -11) * (1 + 1e-6))


# ---- cross-session scheduler (host/sched.c), no device ----------------------
@pytest.mark.parametrize("threads,steps,wait_us,device_us,host_us", [
    (1, 40, 2000, 200, 0),      # a lone caller never waits for others
    (8, 40, 2000, 300, 0),      # callers that return at once rejoin every batch
    (8, 40, 0, 300, 400),       # no window, jittery host work: batches form anyway
    (32, 20, 500, 200, 300),    # the full pool, ragged exits
])
def test_scheduler_rendezvous(threads, steps, wait_us, device_us, host_us):
    """Posters on their own threads (thread i leaves after steps + i steps)
    against a stand-in batch: every poster gets its own answer, no batch holds
    one session twice, and concurrent posters share batches."""
    st = np.zeros(3, np.uint64)
    bad = native.lib().cmol__sched_selftest(threads, steps, wait_us, device_us, host_us, native.ptr(st))
    assert bad == 0
    batches, total, largest = (int(x) for x in st)
    assert total == sum(steps + i for i in range(threads))
    assert largest <= threads
    if threads == 1:
        assert batches == total and largest == 1
    else:
        assert largest > 1
        assert batches < total


def test_scheduler_window_gathers_returning_callers():
    """With a window longer than the host work between steps, callers that a
    batch releases rejoin the next one: batches stay close to the count of
    steps of the longest-lived caller rather than one per step."""
    threads, steps = 8, 30
    st = np.zeros(3, np.uint64)
    assert native.lib().cmol__sched_selftest(threads, steps, 20000, 300, 200, native.ptr(st)) == 0
    batches = int(st[0])
    assert batches <= steps + threads + 4


def test_scheduler_posts_wake_no_waiter_early():
    """32 callers, a short window and long device steps: a posted step must
    not wake the other waiters (each would re-check, and a leader woken
    before the set is complete runs a partial batch). Batches stay near the
    step count of the longest-lived caller (91 here); waking every waiter on
    each post gave about 160."""
    threads, steps = 32, 60
    st = np.zeros(3, np.uint64)
    assert native.lib().cmol__sched_selftest(threads, steps, 200, 4500, 0, native.ptr(st)) == 0
    batches, total = int(st[0]), int(st[1])
    assert total == sum(steps + i for i in range(threads))
    assert batches <= steps + threads - 1 + 25
