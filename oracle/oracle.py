"""ctypes view of the oracle (CPU restatement of the reference hot path).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libcmolref.so")
P = C.c_void_p
SCALAR, AVX512 = 0, 1

_o = None


def lib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run __graft_entry__.build()")
        L = C.CDLL(ORACLE_SO)
        L.o_f16_to_f32.argtypes = [C.c_uint16]; L.o_f16_to_f32.restype = C.c_float
        L.o_dequant_row.argtypes = [P, P, C.c_int, C.c_int]
        L.o_matmul.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        L.o_rms_norm.argtypes = [P, P, P, C.c_int, C.c_float]
        L.o_softmax.argtypes = [P, C.c_int]
        L.o_swiglu.argtypes = [P, P, P, C.c_int]
        L.o_rope_apply.argtypes = [P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.o_argmax.argtypes = [P, C.c_int]; L.o_argmax.restype = C.c_int
        L.o_f32_to_f16.argtypes = [C.c_float]; L.o_f32_to_f16.restype = C.c_uint16
        L.o_apply_repeat_penalty.argtypes = [P, C.c_int, P, C.c_int, C.c_float]
        L.o_sess_kv_f16.argtypes = [P, C.c_int]
        L.o_attention.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P, P]
        L.o_model_load.argtypes = [C.c_char_p, C.c_int, C.c_int]; L.o_model_load.restype = P
        L.o_model_free.argtypes = [P]
        L.o_model_hparams.argtypes = [P, P, P]
        L.o_sess_new.argtypes = [P, C.c_int]; L.o_sess_new.restype = P
        L.o_sess_free.argtypes = [P]
        L.o_forward.argtypes = [P, P, C.c_int32, C.c_int]; L.o_forward.restype = P
        L.o_generate_greedy.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, P, P]
        L.o_generate_greedy.restype = C.c_int
        L.o_sess_k.argtypes = [P]; L.o_sess_k.restype = P
        L.o_sess_v.argtypes = [P]; L.o_sess_v.restype = P
        L.o_sess_logits.argtypes = [P]; L.o_sess_logits.restype = P
        _o = L
    return _o


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def dequant_row(src: np.ndarray, n: int, dtype: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    src = np.ascontiguousarray(src)
    lib().o_dequant_row(src.ctypes.data, out.ctypes.data, n, dtype)
    return out


def matmul(a_bytes: np.ndarray, b: np.ndarray, m: int, k: int, dtype: int, order: int = AVX512) -> np.ndarray:
    """out[m, n] = A[m, k] . B where B is given as [k, n] (k-major)."""
    b = _f32(b)
    n = 1 if b.ndim == 1 else b.shape[1]
    out = np.zeros((m, n), np.float32)
    a_bytes = np.ascontiguousarray(a_bytes)
    lib().o_matmul(out.ctypes.data, a_bytes.ctypes.data, b.ctypes.data, m, k, n, dtype, order)
    return out


def apply_repeat_penalty(logits, window, penalty):
    out = _f32(logits).copy()
    w = np.ascontiguousarray(window, np.int32)
    lib().o_apply_repeat_penalty(out.ctypes.data, out.size, w.ctypes.data, w.size, penalty)
    return out


def f32_to_f16_bits(x):
    x = _f32(x).ravel()
    return np.array([lib().o_f32_to_f16(float(v)) for v in x], np.uint16)


def rms_norm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    lib().o_rms_norm(x.ctypes.data, w.ctypes.data, out.ctypes.data, x.size, eps)
    return out


def softmax(x):
    x = _f32(x).copy()
    lib().o_softmax(x.ctypes.data, x.size)
    return x


def swiglu(g, u):
    g, u = _f32(g), _f32(u)
    out = np.zeros_like(g)
    lib().o_swiglu(g.ctypes.data, u.ctypes.data, out.ctypes.data, g.size)
    return out


def rope(q, k, pos, n_heads, n_kv, head_dim, base):
    q, k = _f32(q).copy(), _f32(k).copy()
    lib().o_rope_apply(q.ctypes.data, k.ctypes.data, pos, n_heads, n_kv, head_dim, base)
    return q, k


def attention(q, kc, vc, seqlen, n_heads, n_kv, d_head):
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    scores = np.zeros(max(seqlen, 1), np.float32)
    out = np.zeros(n_heads * d_head, np.float32)
    lib().o_attention(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, seqlen, n_heads, n_kv, d_head,
                      scores.ctypes.data, out.ctypes.data)
    return out


class Model:
    """Oracle model + one session (fp32 KV [layer][pos][n_kv][d_head])."""

    def __init__(self, path: str, max_ctx: int, order: int = AVX512, nthreads: int = 0, kv_f16: bool = False):
        nthreads = nthreads or min(16, os.cpu_count() or 1)
        self.h = lib().o_model_load(path.encode(), order, nthreads)
        if not self.h:
            raise RuntimeError(f"oracle failed to load {path}")
        hp = np.zeros(11, np.int32); hf = np.zeros(2, np.float32)
        lib().o_model_hparams(self.h, hp.ctypes.data, hf.ctypes.data)
        (self.n_layers, self.n_heads, self.n_kv, self.d_model, self.d_head, self.d_ffn,
         self.vocab, self.model_max_ctx, self.nope, self.tie, self.eos) = map(int, hp)
        self.rope_base, self.eps = float(hf[0]), float(hf[1])
        self.max_ctx = max_ctx
        self.s = lib().o_sess_new(self.h, max_ctx)
        if not self.s:
            raise MemoryError("oracle session")
        lib().o_sess_kv_f16(self.s, int(kv_f16))

    def close(self):
        if self.s:
            lib().o_sess_free(self.s); self.s = None
        if self.h:
            lib().o_model_free(self.h); self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, token: int, pos: int) -> np.ndarray:
        p = lib().o_forward(self.h, self.s, int(token), int(pos))
        if not p:
            raise RuntimeError("oracle forward failed")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.vocab,)).copy()

    def generate(self, prompt, n_new, pos0=0, penalty=1.0, last_n=64, margins=False):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_new, np.int32)
        mg = np.zeros(n_new, np.float32)
        n = lib().o_generate_greedy(self.h, self.s, prompt.ctypes.data, prompt.size, pos0, n_new,
                                    penalty, last_n, out.ctypes.data, mg.ctypes.data)
        if n < 0:
            raise RuntimeError("oracle generate failed")
        return (out[:n], mg[:n]) if margins else out[:n]

    def kv(self):
        n = self.n_layers * self.max_ctx * self.n_kv * self.d_head
        k = np.ctypeslib.as_array(C.cast(lib().o_sess_k(self.s), C.POINTER(C.c_float)), (n,))
        v = np.ctypeslib.as_array(C.cast(lib().o_sess_v(self.s), C.POINTER(C.c_float)), (n,))
        shp = (self.n_layers, self.max_ctx, self.n_kv, self.d_head)
        return k.reshape(shp), v.reshape(shp)


class Sessions:
    """One oracle model shared by several sessions (CPU baselines): the
    reference's concurrency model, one session per thread (its
    tests/test_threads.c:153-172), each forward single-threaded.  KV caches
    are filled with a synthetic pattern up to each session's length."""

    def __init__(self, path: str, max_ctxs, kv_f16: bool = False):
        self.h = lib().o_model_load(path.encode(), AVX512, 1)
        if not self.h:
            raise RuntimeError(f"oracle failed to load {path}")
        hp = np.zeros(11, np.int32); hf = np.zeros(2, np.float32)
        lib().o_model_hparams(self.h, hp.ctypes.data, hf.ctypes.data)
        self.n_layers, self.n_kv, self.d_head = int(hp[0]), int(hp[2]), int(hp[4])
        self.max_ctxs = [int(c) for c in max_ctxs]
        self.ss = []
        for c in self.max_ctxs:
            s = lib().o_sess_new(self.h, c)
            if not s:
                self.close()
                raise MemoryError("oracle session")
            lib().o_sess_kv_f16(s, int(kv_f16))
            self.ss.append(s)

    def fill_kv(self, i, n, seed=0):
        """Positions 0..n-1 of session i (every layer) get a repeated seeded
        pattern (the pages are written, so the attention reads real memory)."""
        c = self.max_ctxs[i]
        row = self.n_kv * self.d_head
        pat = (np.random.default_rng(seed).standard_normal(1 << 14) * 0.5).astype(np.float32)
        for get in (lib().o_sess_k, lib().o_sess_v):
            buf = np.ctypeslib.as_array(C.cast(get(self.ss[i]), C.POINTER(C.c_float)),
                                        (self.n_layers * c * row,)).reshape(self.n_layers, c * row)
            flat = buf[:, :n * row]
            reps = -(-flat.shape[1] // pat.size)
            flat[:] = np.tile(pat, reps)[:flat.shape[1]]

    def step(self, tokens, positions, threads):
        """One forward of every session (token i at position i), sessions
        spread over `threads` threads; returns the wall seconds."""
        import threading
        import time
        nxt = [0]
        lock = threading.Lock()
        err = []

        def work():
            while True:
                with lock:
                    i = nxt[0]
                    nxt[0] += 1
                if i >= len(self.ss):
                    return
                if not lib().o_forward(self.h, self.ss[i], int(tokens[i]), int(positions[i])):
                    err.append(i)

        th = [threading.Thread(target=work) for _ in range(max(1, threads))]
        t0 = time.perf_counter()
        for t in th:
            t.start()
        for t in th:
            t.join()
        el = time.perf_counter() - t0
        if err:
            raise RuntimeError(f"oracle forward failed for sessions {err}")
        return el

    def close(self):
        for s in getattr(self, "ss", []):
            lib().o_sess_free(s)
        self.ss = []
        if getattr(self, "h", None):
            lib().o_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- the reference itself, built from its sources (only where it exists) ----
_r = None


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    global _r
    if _r is None:
        L = C.CDLL(REF_SO)
        L.shim_dequant_row.argtypes = [P, P, C.c_int, C.c_int]
        L.shim_matmul.argtypes = [C.c_int, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int]
        L.shim_kernel_name.restype = C.c_char_p
        L.shim_rms_norm.argtypes = [P, P, P, C.c_int, C.c_float]
        L.shim_softmax.argtypes = [P, C.c_int]
        L.shim_swiglu.argtypes = [P, P, P, C.c_int]
        L.shim_rope.argtypes = [P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.shim_load.argtypes = [C.c_char_p, C.c_int, C.c_int, P]; L.shim_load.restype = P
        L.shim_free.argtypes = [P]
        L.shim_acquire.argtypes = [P]; L.shim_acquire.restype = P
        L.shim_release.argtypes = [P]
        L.shim_forward.argtypes = [P, P, C.c_int, C.c_int, P]; L.shim_forward.restype = C.c_int
        L.shim_vocab.argtypes = [P]; L.shim_vocab.restype = C.c_int
        L.shim_generate_greedy.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, P]
        L.shim_generate_greedy.restype = C.c_int
        L.shim_kv.argtypes = [P, C.c_int]; L.shim_kv.restype = P
        _r = L
    return _r


class RefModel:
    """The reference library's own load + forward (public cmol_load)."""

    def __init__(self, path: str, max_ctx: int, sessions: int = 1):
        err = C.c_int(0)
        self.m = ref().shim_load(path.encode(), max_ctx, sessions, C.byref(err))
        if not self.m:
            raise RuntimeError(f"reference cmol_load failed: {err.value}")
        self.s = ref().shim_acquire(self.m)
        self.vocab = ref().shim_vocab(self.m)

    def close(self):
        if self.m:
            ref().shim_free(self.m); self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, token, pos):
        out = np.zeros(self.vocab, np.float32)
        if ref().shim_forward(self.m, self.s, int(token), int(pos), out.ctypes.data) != 0:
            raise RuntimeError("reference forward failed")
        return out

    def generate(self, prompt, n_new, pos0=0, penalty=1.0, last_n=64):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_new, np.int32)
        n = ref().shim_generate_greedy(self.m, self.s, prompt.ctypes.data, prompt.size, pos0, n_new,
                                       penalty, last_n, out.ctypes.data)
        if n < 0:
            raise RuntimeError("reference generate failed")
        return out[:n]
