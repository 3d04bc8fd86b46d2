"""Deterministic synthetic GGUF models and inputs (ctypes over libcmolsynth.so).

Model presets mirror the SmolLM2/SmolLM3 shapes the decode path is measured on.
Weights are ~N(0, 0.02) from a counter-based integer generator, quantised with
GGML's reference quantisers, so every host writes byte-identical files.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import hashlib
import math
import os

import numpy as np

from . import _paths

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 6, 8, 12, 14


class _Spec(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "d_model", "n_heads", "n_kv_heads", "d_ffn", "vocab", "ctx_len",
        "wtype", "embd_type", "out_type", "nope_interval", "eos_id", "qk_norm",
        "arch_smollm3", "transcode_q8", "v_type", "down_type", "rope_scaling")] + [
        ("rope_base", C.c_float), ("rms_eps", C.c_float), ("wstd", C.c_float),
        ("norm_jitter", C.c_float), ("seed", C.c_uint64)]


class _Tok(C.Structure):
    _fields_ = [("model", C.c_char_p), ("n_tokens", C.c_int32), ("tokens", C.POINTER(C.c_char_p)),
                ("types", C.POINTER(C.c_int32)), ("n_merges", C.c_int32),
                ("merges", C.POINTER(C.c_char_p)), ("bos_id", C.c_int32), ("eos_id", C.c_int32),
                ("unk_id", C.c_int32), ("add_bos", C.c_int32)]


@dataclasses.dataclass(frozen=True)
class Tokenizer:
    """Tokenizer metadata of a synthetic GGUF (tokenizer.ggml.* keys); ids and
    add_bos < 0 are left out of the file."""
    model: str
    tokens: tuple
    types: tuple | None = None
    merges: tuple = ()
    bos_id: int = -1
    eos_id: int = -1
    unk_id: int = -1
    add_bos: int = -1


@dataclasses.dataclass(frozen=True)
class ModelSpec:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    d_ffn: int
    vocab: int
    ctx_len: int = 8192
    wtype: int = Q8_0
    embd_type: int = Q8_0
    out_type: int = -1            # -1: tied embeddings (no output.weight)
    nope_interval: int = 0
    eos_id: int = -1              # -1: no EOS key, generation never stops early
    qk_norm: int = 0
    arch_smollm3: int = 0
    transcode_q8: int = 0         # write Q4_0/Q5_0 tensors as lossless Q8_0
    v_type: int = -1              # attn_v format (-1: wtype)
    down_type: int = -1           # ffn_down format (-1: wtype)
    rope_scaling: int = 0         # 1: a rope.scaling.type = "yarn" key (recorded, not applied)
    rope_base: float = 10000.0
    rms_eps: float = 1e-5
    wstd: float = 0.02
    norm_jitter: float = 0.1      # norm weights are 1 + N(0, jitter)
    seed: int = 1234

    @property
    def d_head(self) -> int:
        return self.d_model // self.n_heads

    def replace(self, **kw) -> "ModelSpec":
        return dataclasses.replace(self, **kw)

    def weight_bytes_per_token(self) -> int:
        """Bytes of quantised weights one decode token streams (embedding row
        excluded, LM head included)."""
        def rb(dt, k):
            return {F32: 4 * k, F16: 2 * k, Q4_0: k // 32 * 18, Q5_0: k // 32 * 22,
                    Q8_0: k // 32 * 34}[dt]
        d, kv, f = self.d_model, self.n_kv_heads * self.d_head, self.d_ffn
        per_layer = (rb(self.wtype, d) * (2 * d + 2 * kv) + rb(self.wtype, d) * 2 * f
                     + rb(self.wtype, f) * d + 2 * 4 * d)
        head_t = self.embd_type if self.out_type < 0 else self.out_type
        return self.n_layers * per_layer + rb(head_t, d) * self.vocab + 4 * d


PRESETS = {
    # reference's own CPU-runnable case: SmolLM2-135M shape, Q8_0, tied
    "smollm2-135m-q8_0": ModelSpec(30, 576, 9, 3, 1536, 49152, wtype=Q8_0, embd_type=Q8_0),
    # SmolLM2-360M shape, Q5_0 everywhere
    "smollm2-360m-q5_0": ModelSpec(32, 960, 15, 5, 2560, 49152, wtype=Q5_0, embd_type=Q5_0),
    # SmolLM3-3B shape: Q4_0 projections, Q8_0 tied embedding/LM head, NoPE every 4th layer
    "smollm3-3b-q4_0": ModelSpec(36, 2048, 16, 4, 11008, 128256, ctx_len=65536, wtype=Q4_0,
                                 embd_type=Q8_0, nope_interval=4, arch_smollm3=1,
                                 rope_base=5e6, rms_eps=1e-6),
    # small shapes for fast tests
    "micro-q8_0": ModelSpec(2, 64, 4, 2, 128, 512, ctx_len=512, wtype=Q8_0, embd_type=Q8_0),
    "micro-q4_0": ModelSpec(2, 64, 4, 2, 128, 512, ctx_len=512, wtype=Q4_0, embd_type=Q8_0),
    "micro-q5_0": ModelSpec(2, 64, 4, 2, 128, 512, ctx_len=512, wtype=Q5_0, embd_type=Q5_0),
    "small-q4_0": ModelSpec(4, 256, 8, 2, 704, 2048, ctx_len=4096, wtype=Q4_0, embd_type=Q8_0,
                            nope_interval=4, arch_smollm3=1, rope_base=5e6, rms_eps=1e-6),
    "small-q5_0": ModelSpec(3, 320, 5, 1, 640, 1024, ctx_len=4096, wtype=Q5_0, embd_type=Q5_0),
    "small-q8_0-untied": ModelSpec(2, 192, 3, 3, 512, 1024, ctx_len=1024, wtype=Q8_0,
                                   embd_type=Q8_0, out_type=Q8_0),
    # K-quant layers (every matrix dimension a multiple of 256)
    "small-q4_k": ModelSpec(3, 256, 4, 2, 768, 1024, ctx_len=4096, wtype=Q4_K, embd_type=Q6_K),
    "small-q6_k-untied": ModelSpec(2, 512, 8, 2, 1536, 1024, ctx_len=1024, wtype=Q6_K,
                                   embd_type=Q4_K, out_type=Q6_K),
    # the Q4_K_M mix: Q4_K projections, Q6_K attn_v / ffn_down / embedding
    "small-q4_k_m": ModelSpec(3, 512, 8, 2, 1536, 1024, ctx_len=4096, wtype=Q4_K, embd_type=Q6_K,
                              v_type=Q6_K, down_type=Q6_K),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        path = _paths.lib_path("libcmolsynth.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run __graft_entry__.build() first")
        L = C.CDLL(path)
        L.cmolsynth_write_gguf.argtypes = [C.c_char_p, C.POINTER(_Spec), C.c_int]
        L.cmolsynth_write_gguf.restype = C.c_int
        L.cmolsynth_write_gguf_tok.argtypes = [C.c_char_p, C.POINTER(_Spec), C.c_int, C.POINTER(_Tok)]
        L.cmolsynth_write_gguf_tok.restype = C.c_int
        L.cmolsynth_normal.argtypes = [C.c_void_p, C.c_int64, C.c_uint64, C.c_uint64, C.c_float]
        L.cmolsynth_tokens.argtypes = [C.c_void_p, C.c_int, C.c_uint64, C.c_int]
        L.cmolsynth_uniform.argtypes = [C.c_uint64, C.c_uint64]
        L.cmolsynth_uniform.restype = C.c_double
        L.cmolsynth_quantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        L.cmolsynth_quantize.restype = C.c_int64
        L.cmolsynth_f32_to_f16.argtypes = [C.c_float]
        L.cmolsynth_f32_to_f16.restype = C.c_uint16
        _lib = L
    return _lib


def write_gguf(path: str, spec: ModelSpec, nthreads: int | None = None) -> str:
    s = _Spec(**{f.name: getattr(spec, f.name) for f in dataclasses.fields(spec)})
    nt = nthreads or min(16, os.cpu_count() or 1)
    rc = lib().cmolsynth_write_gguf(path.encode(), C.byref(s), nt)
    if rc != 0:
        raise RuntimeError(f"cmolsynth_write_gguf({path}) failed: {rc}")
    return path


def write_gguf_tok(path: str, spec: ModelSpec, tok: Tokenizer, nthreads: int | None = None) -> str:
    """A synthetic model of `spec` whose tokenizer is `tok` (spec.vocab must be
    len(tok.tokens))."""
    enc = lambda xs: (C.c_char_p * len(xs))(*[x.encode("utf-8") for x in xs])
    toks = enc(tok.tokens)
    merges = enc(tok.merges) if tok.merges else None
    types = (C.c_int32 * len(tok.types))(*tok.types) if tok.types is not None else None
    t = _Tok(tok.model.encode(), len(tok.tokens), toks, types, len(tok.merges), merges,
             tok.bos_id, tok.eos_id, tok.unk_id, tok.add_bos)
    s = _Spec(**{f.name: getattr(spec, f.name) for f in dataclasses.fields(spec)})
    nt = nthreads or min(16, os.cpu_count() or 1)
    rc = lib().cmolsynth_write_gguf_tok(path.encode(), C.byref(s), nt, C.byref(t))
    if rc != 0:
        raise RuntimeError(f"cmolsynth_write_gguf_tok({path}) failed: {rc}")
    return path


def model_file(spec: ModelSpec, directory: str | None = None) -> str:
    """Write (once) and return the path of the GGUF for `spec`, cached by a hash
    of the spec under `directory` (default $CMOL_MODEL_DIR or /tmp/cmol_models)."""
    directory = directory or os.environ.get("CMOL_MODEL_DIR", "/tmp/cmol_models")
    os.makedirs(directory, exist_ok=True)
    h = hashlib.sha1(repr(spec).encode()).hexdigest()[:16]
    path = os.path.join(directory, f"synth-{h}.gguf")
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write_gguf(tmp, spec)
        os.replace(tmp, path)
    return path


def normal(n: int, seed: int, stream: int = 0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().cmolsynth_normal(out.ctypes.data, n, seed, stream, std)
    return out


def tokens(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().cmolsynth_tokens(out.ctypes.data, n, seed, vocab)
    return out


def log_uniform_lengths(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    u = np.array([lib().cmolsynth_uniform(seed, i) for i in range(n)])
    return np.floor(np.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))).astype(np.int64).clip(lo, hi)


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    u = np.array([lib().cmolsynth_uniform(seed, i) for i in range(n)])
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64).clip(lo, hi)


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    bb = {F32: 4, F16: 2, Q4_0: 18, Q5_0: 22, Q8_0: 34, Q4_K: 144, Q6_K: 210}[dtype]
    bv = 256 if dtype in (Q4_K, Q6_K) else 32
    nbytes = x.size * bb if dtype in (F32, F16) else x.size // bv * bb
    out = np.empty(nbytes, np.uint8)
    if lib().cmolsynth_quantize(dtype, x.ctypes.data, x.size, out.ctypes.data) < 0:
        raise ValueError("quantize failed")
    return out
