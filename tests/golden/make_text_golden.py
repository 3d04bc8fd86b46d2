#!/usr/bin/env python3
"""Writes tests/golden/text_golden.json: text-path vectors from the reference
library built from its own sources (oracle/_ref/libcmolref.so).

Two tokenizers are built here (a GPT-2 byte-level BPE and a SentencePiece
style BPE with <0xNN> byte tokens), each from a fixed corpus by a small
deterministic BPE trainer, and written into synthetic GGUF models.  The
reference then produces every expected value:
  * cmol_encode of a list of texts (empty, spaces, tabs, newlines, digits,
    unicode, control-token strings, text past the merges), and the return
    code for a too-small output buffer;
  * cmol_decode_token of every id;
  * cmol_sample draws (with cmol_rng_seed / cmol_apply_repeat_penalty) over
    a grid of temperature / top-k / top-p / penalty / seed on seeded logits
    that include exact ties;
  * cmol_generate on text prompts (greedy, with and without repeat penalty):
    the sampled ids.
The fixture holds the tokenizers themselves (tokens, types, merges, special
ids), so tests rebuild the same GGUFs without this script.  Run in the
container that has /root/reference:
    python tests/golden/make_text_golden.py
"""
import ctypes as C
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libcmol_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

P = C.c_void_p

CORPUS = (
    "the quick brown fox jumps over the lazy dog. the dog sleeps; the fox runs. " * 3
    + "hello world! hello there, world of tokens. token tokens tokenizer tokenize. "
    + "numbers 12345 67890 2024-12-01 3.14159 "
    + "def main():\n    return 0\n"
)

TEXTS = [
    "",
    "the quick brown fox",
    "The Quick Brown Fox!",
    "  leading spaces",
    "trailing spaces   ",
    "multiple   spaces\tand\ttabs\nnew\nlines",
    "hello world",
    "tokenizer tokens token",
    "12345 67890 3.14159",
    "def main():\n    return 0\n",
    "unicode: café naïve 漢字 🙂",
    "<|im_start|>user\nhello<|im_end|>\n<|im_start|>assistant\n",
    "<s>hi</s> there",
    "<|endoftext|>",
    "a" * 300,
    "zzzz qqqq",
    "\x01\x02 control bytes",
    "ÿþ",
    CORPUS[:1500],
]


def gpt2_byte_chars():
    """GPT-2's byte -> printable code point map: bytes 0x21-0x7E, 0xA1-0xAC
    and 0xAE-0xFF map to themselves, the other 68 bytes to U+0100.. in order."""
    keep = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cp, extra = {}, 0
    for b in range(256):
        if b in keep:
            cp[b] = b
        else:
            cp[b] = 0x100 + extra
            extra += 1
    return [chr(cp[b]) for b in range(256)]


def train_bpe(symbols, n_merges):
    """Greedy BPE: repeatedly merge the most frequent adjacent pair (ties:
    the lexicographically smallest pair), left to right."""
    seq = list(symbols)
    merges = []
    for _ in range(n_merges):
        counts = {}
        for a, b in zip(seq, seq[1:]):
            counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        best = max(counts.values())
        if best < 2:
            break
        pair = min(p for p, c in counts.items() if c == best)
        merges.append(pair)
        out, i = [], 0
        while i < len(seq):
            if i + 1 < len(seq) and (seq[i], seq[i + 1]) == pair:
                out.append(seq[i] + seq[i + 1])
                i += 2
            else:
                out.append(seq[i])
                i += 1
        seq = out
    return merges


def add_unique(tokens, s):
    if s not in tokens:
        tokens.append(s)


def gpt2_tokenizer():
    chars = gpt2_byte_chars()
    merges = train_bpe([chars[b] for b in CORPUS.encode()], 160)
    tokens = list(chars)
    for a, b in merges:
        add_unique(tokens, a + b)
    controls = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    n_plain = len(tokens)
    tokens += controls
    types = [1] * n_plain + [3] * len(controls)
    return synth.Tokenizer("gpt2", tuple(tokens), tuple(types), tuple(f"{a} {b}" for a, b in merges),
                           bos_id=n_plain, eos_id=n_plain + 2, unk_id=-1, add_bos=0)


def spm_tokenizer():
    text = "▁" + CORPUS.replace(" ", "▁")
    merges = train_bpe(list(text), 160)
    tokens = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    types = [2, 3, 3] + [6] * 256
    for ch in sorted(set(text)):
        add_unique(tokens, ch)
    for a, b in merges:
        add_unique(tokens, a + b)
    types += [1] * (len(tokens) - len(types))
    return synth.Tokenizer("llama", tuple(tokens), tuple(types), tuple(f"{a} {b}" for a, b in merges),
                           bos_id=1, eos_id=2, unk_id=0, add_bos=1)


def model_spec(vocab):
    return synth.ModelSpec(n_layers=1, d_model=64, n_heads=4, n_kv_heads=2, d_ffn=128, vocab=vocab,
                           ctx_len=256, wtype=synth.Q8_0, embd_type=synth.Q8_0, wstd=0.08, seed=77)


def tok_dict(t):
    return {"model": t.model, "tokens": list(t.tokens), "types": list(t.types), "merges": list(t.merges),
            "bos_id": t.bos_id, "eos_id": t.eos_id, "unk_id": t.unk_id, "add_bos": t.add_bos}


class GenParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("max_new_tokens", C.c_int), ("seed", C.c_uint), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_int)]


def sampler_logits(case_seed, draw, vocab):
    """Seeded logits with exact ties (every 7th value repeats its neighbour)."""
    rng = np.random.default_rng([case_seed, draw])
    x = (rng.standard_normal(vocab) * 3.0).astype(np.float32)
    x[7::7] = x[6:-1:7][: x[7::7].size]
    return x


SAMPLER_GRID = [
    # temperature, top_k, top_p, penalty, seed (seed 0 seeds from the clock: greedy only)
    (0.0, 40, 0.95, 1.0, 0), (0.7, 0, 0.0, 1.0, 1), (1.0, 0, 1.0, 1.0, 2), (1.3, 0, 0.0, 1.0, 3),
    (0.8, 1, 0.0, 1.0, 4), (0.8, 10, 0.0, 1.0, 5), (0.8, 64, 0.9, 1.0, 6), (0.8, 40, 0.95, 1.1, 7),
    (1.0, 512, 0.0, 1.0, 8), (1.0, 1000, 0.0, 1.0, 9), (0.9, 0, 0.5, 1.0, 10), (0.9, 0, 0.3, 1.3, 11),
    (0.6, 600, 0.99, 1.2, 13), (1.1, 3, 0.6, 1.0, 123456789),
]
SAMPLER_VOCAB, SAMPLER_DRAWS = 3000, 24


def sampler_cases(R):
    R.cmol_sample.argtypes = [P, C.c_int, C.POINTER(GenParams), P]
    R.cmol_sample.restype = C.c_int32
    R.cmol_rng_seed.argtypes = [P, C.c_uint]
    R.cmol_apply_repeat_penalty.argtypes = [P, C.c_int, P, C.c_int, C.c_float]
    cases = []
    for ci, (t, k, p, pen, seed) in enumerate(SAMPLER_GRID):
        prm = GenParams(t, p, k, 0, seed, pen, 64)
        st = np.zeros(4, np.uint64)
        R.cmol_rng_seed(st.ctypes.data, seed)
        hist = list(range(0, 60, 3))   # prior tokens the penalty sees
        ids = []
        for d in range(SAMPLER_DRAWS):
            lg = sampler_logits(ci, d, SAMPLER_VOCAB)
            h = np.array(hist[-64:], np.int32)
            R.cmol_apply_repeat_penalty(lg.ctypes.data, SAMPLER_VOCAB, h.ctypes.data, h.size, pen)
            tid = R.cmol_sample(lg.ctypes.data, SAMPLER_VOCAB, C.byref(prm), st.ctypes.data)
            ids.append(int(tid))
            hist.append(int(tid))
        cases.append({"temperature": t, "top_k": k, "top_p": p, "penalty": pen, "seed": seed,
                      "history": list(range(0, 60, 3)), "ids": ids})
    return cases


def main():
    R = O.ref()
    R.cmol_encode.argtypes = [P, C.c_char_p, P, C.c_int]
    R.cmol_encode.restype = C.c_int
    R.cmol_decode_token.argtypes = [P, C.c_int32]
    R.cmol_decode_token.restype = C.c_char_p
    R.shim_generate_text.argtypes = [P, P, C.c_char_p, C.c_int, C.c_float, C.c_uint, C.c_float, P, C.c_int]
    R.shim_generate_text.restype = C.c_int
    R.cmol_session_reset.argtypes = [P]
    out = {"tokenizers": {}, "sampler": {"vocab": SAMPLER_VOCAB, "draws": SAMPLER_DRAWS}}
    with tempfile.TemporaryDirectory() as td:
        for name, tok in (("gpt2", gpt2_tokenizer()), ("spm", spm_tokenizer())):
            spec = model_spec(len(tok.tokens))
            path = os.path.join(td, f"{name}.gguf")
            synth.write_gguf_tok(path, spec, tok)
            m = O.RefModel(path, 256)
            enc = []
            for text in TEXTS:
                buf = np.zeros(8192, np.int32)
                n = R.cmol_encode(m.m, text.encode(), buf.ctypes.data, 8192)
                enc.append({"text": text, "rc": int(n), "ids": buf[:max(n, 0)].tolist()})
            small = np.zeros(2, np.int32)
            rc_small = R.cmol_encode(m.m, b"the quick brown fox", small.ctypes.data, 2)
            pieces = []
            for i in range(len(tok.tokens)):
                s = R.cmol_decode_token(m.m, i)
                pieces.append(None if s is None else s.hex())
            gens = []
            for prompt, pen in (("the quick brown", 1.0), ("hello world", 1.3), ("<|im_start|>user\nhi", 1.0)):
                ids = np.zeros(64, np.int32)
                R.cmol_session_reset(m.s)
                n = R.shim_generate_text(m.m, m.s, prompt.encode(), 20, 0.0, 0, pen, ids.ctypes.data, 64)
                gens.append({"prompt": prompt, "penalty": pen, "max_new": 20, "rc": int(n),
                             "ids": ids[:max(n, 0)].tolist()})
            m.close()
            out["tokenizers"][name] = {"tokenizer": tok_dict(tok), "spec": {
                "n_layers": spec.n_layers, "d_model": spec.d_model, "n_heads": spec.n_heads,
                "n_kv_heads": spec.n_kv_heads, "d_ffn": spec.d_ffn, "ctx_len": spec.ctx_len,
                "wstd": spec.wstd, "seed": spec.seed},
                "encode": enc, "encode_cap2_rc": int(rc_small), "pieces": pieces, "generate": gens}
    out["sampler"]["cases"] = sampler_cases(R)
    with open(os.path.join(HERE, "text_golden.json"), "w") as f:
        json.dump(out, f, ensure_ascii=True, separators=(",", ":"))
    print("wrote", os.path.join(HERE, "text_golden.json"))


if __name__ == "__main__":
    main()
