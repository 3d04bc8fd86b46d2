"""ctypes bindings of libcmol.so: the public C API (include/cmol.h), the gfx950
backend C ABI (include/cmol_hip.h) and the harness entry points
(include/cmol_ext.h).

The library is required: nothing here falls back to a CPU path.  Loading fails
loudly when the in-tree build is missing.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _paths

P = C.c_void_p
I32 = C.c_int32
CMOL_OK, CMOL_ERR_OOM, CMOL_ERR_IO, CMOL_ERR_INVALID, CMOL_ERR_UNSUPPORTED = 0, -1, -2, -3, -4
CMOL_ERR_NO_SESSION, CMOL_ERR_ARGS, CMOL_ERR_CTX_FULL, CMOL_ERR_TRUNC = -5, -6, -7, -8

LOG_FN = C.CFUNCTYPE(None, C.c_int, C.c_char_p, C.c_void_p)
TOKEN_CB = C.CFUNCTYPE(C.c_int, C.c_char_p, C.c_size_t, C.c_int, C.c_void_p)


class Config(C.Structure):
    _fields_ = [("max_ctx", C.c_int), ("max_sessions", C.c_int), ("prefill_chunk", C.c_int),
                ("log_fn", LOG_FN), ("log_ud", C.c_void_p)]


class GenParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("max_new_tokens", C.c_int), ("seed", C.c_uint), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_int)]


def default_params(**kw) -> GenParams:
    p = GenParams(0.8, 0.95, 40, 256, 0, 1.1, 64)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def greedy_params(max_new: int, **kw) -> GenParams:
    return default_params(**{"temperature": 0.0, "repeat_penalty": 1.0, "max_new_tokens": max_new, **kw})


class QTensor(C.Structure):
    _fields_ = [("qs", P), ("d", P), ("qh", P), ("dtype", I32), ("rows", I32), ("cols", I32),
                ("row_tiles", I32), ("block_quads", I32), ("fold", I32)]


# (name, restype, argtypes) of every exported entry point declared in include/*.h
SIGNATURES = [
    # cmol.h
    ("cmol_load", P, [C.c_char_p, C.POINTER(Config), C.POINTER(C.c_int)]),
    ("cmol_free", None, [P]),
    ("cmol_session_acquire", P, [P]),
    ("cmol_session_release", None, [P]),
    ("cmol_session_reset", None, [P]),
    ("cmol_generate", C.c_int, [P, C.c_char_p, C.POINTER(GenParams), TOKEN_CB, P]),
    ("cmol_encode", C.c_int, [P, C.c_char_p, P, C.c_int]),
    ("cmol_decode_token", C.c_char_p, [P, I32]),
    ("cmol_strerror", C.c_char_p, [C.c_int]),
    ("cmol_version", C.c_char_p, []),
    ("cmol_arena_estimate", C.c_size_t, [C.c_char_p, C.POINTER(Config)]),
    ("cmol_format_chatml", C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_size_t]),
    ("cmol_format_chatml_turn", C.c_int, [C.c_char_p, C.c_char_p, C.c_size_t]),
    # cmol_hip.h
    ("cmolhip_device_count", C.c_int, []),
    ("cmolhip_ctx_create", C.c_int, [C.c_int, C.c_size_t, C.POINTER(P)]),
    ("cmolhip_ctx_destroy", None, [P]),
    ("cmolhip_alloc", C.c_int, [P, C.c_size_t, C.c_size_t, C.POINTER(P)]),
    ("cmolhip_arena_used", C.c_size_t, [P]),
    ("cmolhip_arena_size", C.c_size_t, [P]),
    ("cmolhip_memcpy_h2d", C.c_int, [P, P, P, C.c_size_t]),
    ("cmolhip_memcpy_d2h", C.c_int, [P, P, P, C.c_size_t]),
    ("cmolhip_memcpy_d2d", C.c_int, [P, P, P, C.c_size_t]),
    ("cmolhip_synchronize", C.c_int, [P]),
    ("cmolhip_stream", P, [P]),
    ("cmolhip_qtensor_bytes", C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    ("cmolhip_pick_fold", C.c_int, [C.c_int, C.c_int, C.c_int]),
    ("cmolhip_qtensor_upload", C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(P),
                                         C.POINTER(I32), C.c_int, P, C.c_size_t,
                                         C.POINTER(QTensor)]),
    ("cmolhip_dequant", C.c_int, [P, C.POINTER(QTensor), P]),
    ("cmolhip_gemm", C.c_int, [P, C.POINTER(QTensor), P, P, C.c_int, P, C.c_float]),
    ("cmolhip_act_bytes", C.c_size_t, [C.c_int, C.c_int]),
    ("cmolhip_act_prepare", C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P, P]),
    ("cmolhip_gemm_prepared", C.c_int, [P, C.POINTER(QTensor), P, C.c_int, P, C.c_float, P]),
    ("cmolhip_gemm_prepared_timed", C.c_int, [P, C.POINTER(QTensor), P, C.c_int, P, C.c_float, P,
                                              P, P]),
    ("cmolhip_matmul_host", C.c_int, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int]),
    ("cmolhip_gemm_noalloc", C.c_int, [P, C.POINTER(QTensor), P, P, C.c_int, P, C.c_float]),
    ("cmolhip_noalloc_scratch_bytes", C.c_size_t, []),
    ("cmolhip_attn_decode", C.c_int, [P, C.c_int, P, P, P, P, C.c_int, C.c_int, C.c_int,
                                      C.c_int, C.c_int, C.c_int, P]),
    ("cmolhip_model_plan", C.c_int, [P, C.POINTER(C.c_size_t)]),
    ("cmolhip_gemv_scratch_floats", C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    ("cmolhip_batch_scratch_floats", C.c_int, [P, C.c_int, C.POINTER(C.c_size_t)]),
    ("cmolhip_model_create", C.c_int, [P, C.c_int, C.POINTER(P)]),
    ("cmolhip_model_destroy", None, [P]),
    ("cmolhip_model_ctx", P, [P]),
    ("cmolhip_decode", C.c_int, [P, C.c_int, I32, I32, P, P]),
    ("cmolhip_decode_batch", C.c_int, [P, C.c_int, P, P, P, P, P]),
    ("cmolhip_decode_batch_each", C.c_int, [P, C.c_int, P, P, P, P, P]),
    ("cmolhip_prefill", C.c_int, [P, C.c_int, P, C.c_int, I32, P, P]),
    ("cmolhip_kv_download", C.c_int, [P, C.c_int, C.c_int, C.c_int, P, P]),
    ("cmolhip_kv_upload", C.c_int, [P, C.c_int, C.c_int, C.c_int, P, P]),
    ("cmolhip_kv_fill_synthetic", C.c_int, [P, C.c_int, C.c_int, C.c_uint64]),
    ("cmolhip_session_stream", P, [P, C.c_int]),
    ("cmolhip_model_persistent", C.c_int, [P]),
    ("cmolhip_persist_trace", C.c_int, [P, P, C.c_int]),
    ("cmolhip_persist_marks", C.c_int, [P, P, C.c_size_t]),
    # cmol_ext.h
    ("cmol__forward", C.c_int, [P, I32, C.c_int, P]),
    ("cmol__prefill", C.c_int, [P, P, C.c_int, P]),
    ("cmol__generate_ids", C.c_int, [P, P, C.c_int, C.POINTER(GenParams), P, C.c_int]),
    ("cmol__decode_batch", C.c_int, [P, P, C.c_int, P]),
    ("cmol__session_fill_kv", C.c_int, [P, C.c_int, C.c_uint64]),
    ("cmol__load_text", P, [C.c_char_p, C.POINTER(C.c_int)]),
    ("cmol_sample", I32, [P, C.c_int, C.POINTER(GenParams), P]),
    ("cmol_rng_seed", None, [P, C.c_uint]),
    ("cmol_rng_next", C.c_uint64, [P]),
    ("cmol_apply_repeat_penalty", None, [P, C.c_int, P, C.c_int, C.c_float]),
    ("cmol__sampler_config", C.c_int, [C.c_int, C.c_int]),
    ("cmol__sampler_pool", C.c_int, [C.c_int]),
    ("cmol__sched_stats", C.c_int, [P, P]),
    ("cmol__sched_selftest", C.c_int, [C.c_int, C.c_int, C.c_long, C.c_long, C.c_uint, P]),
    ("cmol__session_length", C.c_int, [P]),
    ("cmol__session_slot", C.c_int, [P]),
    ("cmol__device", P, [P]),
]



class HParams(C.Structure):
    """cmolhip_hparams_t"""
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "n_heads", "n_kv_heads", "d_model", "d_head", "d_ffn", "vocab",
        "max_ctx", "max_sessions", "no_rope_interval", "kv_f16", "prefill_chunk")] + [
        ("rope_base", C.c_float), ("rms_eps", C.c_float)]


class HostTensor(C.Structure):
    """cmolhip_host_tensor_t"""
    _fields_ = [("data", P), ("dtype", I32), ("rows", I32), ("cols", I32)]


class LayerTensors(C.Structure):
    """cmolhip_layer_tensors_t"""
    _fields_ = [(n, HostTensor) for n in (
        "attn_norm", "q", "k", "v", "o", "q_norm", "k_norm", "ffn_norm", "gate", "up", "down")]


class ModelDesc(C.Structure):
    """cmolhip_model_desc_t"""
    _fields_ = [("hp", HParams), ("embd", HostTensor), ("out_norm", HostTensor),
                ("lm_head", HostTensor), ("layers", C.POINTER(LayerTensors)),
                ("rope_table", P)]


def shape_desc(hp: HParams, q, k, v, o, gate, down, embd, lm=None):
    """A model description with shapes and formats only, for the device-free
    planning calls (the data pointers point at a dummy byte: planning never
    reads weights).  Returns (desc, keepalive)."""
    dummy = (C.c_uint8 * 16)()
    addr = C.cast(dummy, P)
    d, kvd = hp.d_model, hp.n_kv_heads * hp.d_head

    def t(dt, rows, cols):
        return HostTensor(addr, dt, rows, cols)

    layers = (LayerTensors * hp.n_layers)()
    for L in layers:
        L.attn_norm = t(0, 1, d)
        L.ffn_norm = t(0, 1, d)
        L.q, L.k, L.v = t(q, d, d), t(k, kvd, d), t(v, kvd, d)
        L.o = t(o, d, d)
        L.gate, L.up = t(gate, hp.d_ffn, d), t(gate, hp.d_ffn, d)
        L.down = t(down, d, hp.d_ffn)
    desc = ModelDesc()
    desc.hp = hp
    desc.embd = t(embd, hp.vocab, d)
    desc.out_norm = t(0, 1, d)
    desc.lm_head = t(lm, hp.vocab, d) if lm is not None else HostTensor(None, 0, 0, 0)
    desc.layers = layers
    desc.rope_table = addr
    return desc, (dummy, layers)


_lib = None


def lib_path() -> str:
    return _paths.lib_path("libcmol.so")


def lib():
    """The loaded libcmol.so (raises when the in-tree build is missing)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(path)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "call"):
    if rc < 0:
        msg = lib().cmol_strerror(rc).decode()
        raise RuntimeError(f"{what} failed: {rc} ({msg})")
    return rc


def device_count() -> int:
    return lib().cmolhip_device_count()


def ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


# ---------------------------------------------------------------------------
# Device context helpers (kernel-level tests and benches)
# ---------------------------------------------------------------------------
class Ctx:
    def __init__(self, arena_bytes: int, device: int = 0):
        h = C.c_void_p()
        check(lib().cmolhip_ctx_create(device, arena_bytes, C.byref(h)), "cmolhip_ctx_create")
        self.h = h

    def close(self):
        if self.h:
            lib().cmolhip_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def alloc(self, nbytes: int, align: int = 256) -> int:
        p = C.c_void_p()
        check(lib().cmolhip_alloc(self.h, nbytes, align, C.byref(p)), "cmolhip_alloc")
        return p.value

    def h2d(self, dptr: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        check(lib().cmolhip_memcpy_h2d(self.h, C.c_void_p(dptr), ptr(a), a.nbytes), "h2d")

    def d2h(self, dptr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(lib().cmolhip_memcpy_d2h(self.h, ptr(out), C.c_void_p(dptr), out.nbytes), "d2h")
        return out

    def upload(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        d = self.alloc(max(a.nbytes, 1))
        self.h2d(d, a)
        return d

    def qtensor(self, raw_parts, dtype: int, cols: int, rows, mode: int = 0,
                staging_bytes: int | None = None, staging: int | None = None,
                fold: int = 1) -> QTensor:
        parts = [np.ascontiguousarray(p, np.uint8) for p in raw_parts]
        staging_bytes = staging_bytes or max(p.nbytes for p in parts)
        stg = staging if staging is not None else self.alloc(staging_bytes)
        arr_p = (C.c_void_p * len(parts))(*[p.ctypes.data for p in parts])
        arr_r = (I32 * len(parts))(*rows)
        t = QTensor()
        check(lib().cmolhip_qtensor_upload(self.h, dtype, cols, fold, len(parts), arr_p, arr_r, mode,
                                           C.c_void_p(stg), staging_bytes, C.byref(t)), "upload")
        return t

    def dequant(self, t: QTensor) -> np.ndarray:
        d = self.alloc(t.rows * t.cols * 4)
        check(lib().cmolhip_dequant(self.h, C.byref(t), C.c_void_p(d)), "dequant")
        return self.d2h(d, (t.rows, t.cols), np.float32)

    def gemm(self, t: QTensor, x: np.ndarray, norm_w: np.ndarray | None = None,
             eps: float = 1e-5) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1, t.cols)
        n = x.shape[0]
        dx = self.upload(x)
        dy = self.alloc(n * t.rows * 4)
        dn = self.upload(np.ascontiguousarray(norm_w, np.float32)) if norm_w is not None else None
        check(lib().cmolhip_gemm(self.h, C.byref(t), C.c_void_p(dx), C.c_void_p(dy), n,
                                 C.c_void_p(dn) if dn else None, eps), "gemm")
        check(lib().cmolhip_synchronize(self.h), "sync")
        return self.d2h(dy, (n, t.rows), np.float32)

    def act_prepare(self, t: QTensor, dx: int, n: int, norm_w: int | None = None):
        """Device operand (and sum-of-squares partials when norm_w is given)
        for n fp32 vectors at device address dx; returns (op, ss)."""
        op = self.alloc(lib().cmolhip_act_bytes(t.cols, n))
        ss = self.alloc(n * (t.cols // 32) * 4) if norm_w else None
        check(lib().cmolhip_act_prepare(self.h, C.c_void_p(dx), n, t.cols, t.dtype,
                                        C.c_void_p(norm_w) if norm_w else None, C.c_void_p(op),
                                        C.c_void_p(ss) if ss else None), "act_prepare")
        return op, ss

    def gemm_prepared(self, t: QTensor, op: int, n: int, ss: int | None, dy: int,
                      eps: float = 1e-5):
        check(lib().cmolhip_gemm_prepared(self.h, C.byref(t), C.c_void_p(op), n,
                                          C.c_void_p(ss) if ss else None, eps, C.c_void_p(dy)),
              "gemm_prepared")

    def stream(self):
        return lib().cmolhip_stream(self.h)


# ---------------------------------------------------------------------------
# Model / sessions (public API + harness entry points)
# ---------------------------------------------------------------------------
class Model:
    def __init__(self, path: str, max_ctx: int = 0, max_sessions: int = 1, log: bool = False,
                 prefill_chunk: int = 512):
        self._logs = []
        self._logfn = LOG_FN(lambda lvl, msg, ud: self._logs.append(msg.decode()))
        cfg = Config(max_ctx, max_sessions, prefill_chunk, self._logfn if log else LOG_FN(), None)
        err = C.c_int(0)
        self.h = lib().cmol_load(path.encode(), C.byref(cfg), C.byref(err))
        if not self.h:
            raise RuntimeError(f"cmol_load({path}) failed: {err.value} "
                               f"({lib().cmol_strerror(err.value).decode()})")
        self.path = path

    def close(self):
        if self.h:
            lib().cmol_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sched_stats(self):
        """(batching on, batches, steps, largest batch) of the scheduler that
        batches concurrent decode steps."""
        out = np.zeros(3, np.uint64)
        on = check(lib().cmol__sched_stats(self.h, ptr(out)), "sched_stats")
        return bool(on), int(out[0]), int(out[1]), int(out[2])

    def acquire(self) -> "Session":
        s = lib().cmol_session_acquire(self.h)
        return Session(self, s) if s else None

    @property
    def device(self):
        return lib().cmol__device(self.h)

    @property
    def persistent(self) -> bool:
        """Single-session decode runs the persistent kernel."""
        return bool(lib().cmolhip_model_persistent(self.device))


class Session:
    def __init__(self, model: Model, handle):
        self.model = model
        self.h = handle

    def release(self):
        lib().cmol_session_release(self.h)

    def reset(self):
        lib().cmol_session_reset(self.h)

    @property
    def length(self) -> int:
        return lib().cmol__session_length(self.h)

    @property
    def slot(self) -> int:
        return lib().cmol__session_slot(self.h)

    def forward(self, token: int, pos: int, vocab: int | None = None):
        logits = np.zeros(vocab, np.float32) if vocab else None
        r = check(lib().cmol__forward(self.h, int(token), int(pos),
                                      ptr(logits) if logits is not None else None), "forward")
        return r, logits

    def prefill(self, tokens, vocab: int | None = None):
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.zeros(vocab, np.float32) if vocab else None
        r = check(lib().cmol__prefill(self.h, ptr(t), t.size,
                                      ptr(logits) if logits is not None else None), "prefill")
        return r, logits

    def generate_ids(self, prompt, params: GenParams, cap: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(cap, np.int32)
        n = check(lib().cmol__generate_ids(self.h, ptr(p), p.size, C.byref(params), ptr(out), cap),
                  "generate_ids")
        return out[:n]

    def fill_kv(self, n_tokens: int, seed: int = 7):
        check(lib().cmol__session_fill_kv(self.h, n_tokens, seed), "fill_kv")

    def generate_text(self, prompt: bytes, params: GenParams):
        """Public cmol_generate on a text prompt: the (piece, eos) pairs the
        callback received, and the return code."""
        got = []
        cb = TOKEN_CB(lambda piece, n, eos, ud: got.append((C.string_at(piece, n), bool(eos))) or 0)
        rc = lib().cmol_generate(self.h, prompt, C.byref(params), cb, None)
        return got, rc


def encode(h, text: bytes, cap: int = 8192):
    """cmol_encode on model handle h: (ids, return code)."""
    out = np.zeros(max(cap, 1), np.int32)
    rc = lib().cmol_encode(h, text, ptr(out), cap)
    return (out[:rc].copy() if rc >= 0 else None), rc


def decode_token(h, tid: int) -> bytes | None:
    return lib().cmol_decode_token(h, tid)


class TextModel:
    """A GGUF's tokenizer without a device (cmol__load_text)."""

    def __init__(self, path: str):
        err = C.c_int(0)
        self.h = lib().cmol__load_text(path.encode(), C.byref(err))
        if not self.h:
            raise RuntimeError(f"cmol__load_text({path}) failed: {err.value}")

    def encode(self, text: bytes, cap: int = 8192):
        return encode(self.h, text, cap)

    def decode_token(self, tid: int) -> bytes | None:
        return decode_token(self.h, tid)

    def close(self):
        if self.h:
            lib().cmol_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def decode_batch(sessions, tokens) -> np.ndarray:
    n = len(sessions)
    arr = (C.c_void_p * n)(*[s.h for s in sessions])
    t = np.ascontiguousarray(tokens, np.int32)
    out = np.zeros(n, np.int32)
    check(lib().cmol__decode_batch(arr, ptr(t), n, ptr(out)), "decode_batch")
    return out


def decode_batch_logits(model: Model, sessions, tokens, pos, vocab: int):
    """One lock-step step of `sessions` at their own positions through
    cmolhip_decode_batch: (next ids, logits [n][vocab]).  Session lengths are
    the caller's to track."""
    n = len(sessions)
    slots = np.array([s.slot for s in sessions], np.int32)
    t = np.ascontiguousarray(tokens, np.int32)
    p = np.ascontiguousarray(pos, np.int32)
    lg = np.zeros((n, vocab), np.float32)
    out = np.zeros(n, np.int32)
    check(lib().cmolhip_decode_batch(model.device, n, ptr(slots), ptr(t), ptr(p), ptr(lg), ptr(out)),
          "decode_batch")
    return out, lg


def kv_download(model: Model, slot: int, layer: int, n: int, kvd: int):
    """K and V rows [n][kvd] of one layer of a session's cache, as fp32."""
    k = np.zeros((n, kvd), np.float32)
    v = np.zeros((n, kvd), np.float32)
    check(lib().cmolhip_kv_download(model.device, slot, layer, n, ptr(k), ptr(v)), "kv_download")
    return k, v
