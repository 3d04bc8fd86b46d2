/*
 * gguf.c — GGUF v2/v3 reader for libcmol (MI355X build).
 *
 * Same acceptance rules as the reference loader (src/gguf.c:299-518):
 *   - "general.architecture" sets the prefix of arch keys (default "llama");
 *   - hparams are read only from UINT32 / FLOAT32 values (src/gguf.c:321-353);
 *   - tokenizer arrays tokens / scores / token_type / merges, bos/eos/unk ids,
 *     add_bos flag, tokenizer model name;
 *   - tensor data starts at align32(end of tensor infos) + offset, alignment
 *     fixed at 32 (src/gguf.c:505);
 *   - tied LM head when "output.weight" is absent (src/gguf.c:512-513).
 * Added here: Q4_0 tensor sizes (18-byte blocks), which the reference's
 * tensor_nbytes (src/gguf.c:401-411) lacks.
 */
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define GGUF_MAGIC 0x46554747u
#define GGUF_ALIGN 32u

enum { GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR,
       GV_U64, GV_I64, GV_F64 };
static const uint8_t gv_width[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

typedef struct {
    const uint8_t *p;
    size_t size, pos;
    int err;               /* sticky: once set every read yields 0 */
} cur_t;

static int cur_has(cur_t *c, size_t n)
{
    if (c->err || n > c->size - c->pos) { c->err = 1; return 0; }
    return 1;
}
static uint64_t cur_uint(cur_t *c, size_t w)
{
    uint64_t v = 0;
    if (!cur_has(c, w)) return 0;
    memcpy(&v, c->p + c->pos, w);
    c->pos += w;
    return v;
}
static uint32_t cur_u32(cur_t *c) { return (uint32_t)cur_uint(c, 4); }
static uint64_t cur_u64(cur_t *c) { return cur_uint(c, 8); }
static float cur_f32(cur_t *c)
{
    uint32_t u = cur_u32(c);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Length-prefixed string: pointer into the file plus its length. */
static const char *cur_strn(cur_t *c, size_t *len)
{
    uint64_t n = cur_u64(c);
    if (c->err || n > ((uint64_t)128 << 20) || !cur_has(c, (size_t)n)) { c->err = 1; return NULL; }
    const char *src = (const char *)c->p + c->pos;
    c->pos += (size_t)n;
    *len = (size_t)n;
    return src;
}

/* Copy a length-prefixed string into a bounded NUL-terminated buffer. */
static int cur_str_buf(cur_t *c, char *dst, size_t cap)
{
    size_t n;
    const char *s = cur_strn(c, &n);
    if (!s) return 0;
    if (n >= cap) { dst[0] = 0; return 0; }
    memcpy(dst, s, n);
    dst[n] = 0;
    return 1;
}

/* Length-prefixed string copied into the arena (NUL-terminated). */
static const char *cur_str(cur_t *c, cmol_arena_t *a)
{
    size_t n;
    const char *src = cur_strn(c, &n);
    if (!src) return NULL;
    if (!a) return src;
    char *s = (char *)cmol_arena_alloc(a, (size_t)n + 1, 1);
    if (!s) { c->err = 2; return NULL; }
    memcpy(s, src, (size_t)n);
    s[n] = 0;
    return s;
}

static void skip_scalar(cur_t *c, uint32_t t)
{
    size_t n;
    if (t == GV_STR) { (void)cur_strn(c, &n); return; }
    if (t < 13 && gv_width[t]) { if (cur_has(c, gv_width[t])) c->pos += gv_width[t]; }
    else c->err = 1;
}
static void skip_value(cur_t *c, uint32_t t)
{
    if (t != GV_ARR) { skip_scalar(c, t); return; }
    uint32_t et = cur_u32(c);
    uint64_t n = cur_u64(c);
    for (uint64_t i = 0; i < n && !c->err; i++) skip_scalar(c, et);
}

/* key == arch + "." + suffix */
static int arch_key(const char *key, const char *arch, const char *suffix)
{
    size_t la = strlen(arch);
    return strncmp(key, arch, la) == 0 && key[la] == '.' && strcmp(key + la + 1, suffix) == 0;
}

/* Apply one arch-prefixed UINT32 value; returns 1 if the key was known. */
static int apply_u32(cmol_hparams_t *hp, const char *arch, const char *key, uint32_t v)
{
    static const struct { const char *suffix; size_t off; } map[] = {
        {"context_length", offsetof(cmol_hparams_t, model_max_ctx)},
        {"embedding_length", offsetof(cmol_hparams_t, d_model)},
        {"block_count", offsetof(cmol_hparams_t, n_layers)},
        {"feed_forward_length", offsetof(cmol_hparams_t, d_ffn)},
        {"attention.head_count", offsetof(cmol_hparams_t, n_heads)},
        {"attention.head_count_kv", offsetof(cmol_hparams_t, n_kv_heads)},
        {"vocab_size", offsetof(cmol_hparams_t, vocab_size)},
        {"attention.no_rope_layer_interval", offsetof(cmol_hparams_t, no_rope_layer_interval)},
    };
    for (size_t i = 0; i < sizeof map / sizeof map[0]; i++)
        if (arch_key(key, arch, map[i].suffix)) {
            *(int *)((char *)hp + map[i].off) = (int)v;
            return 1;
        }
    return 0;
}

static void apply_f32(cmol_hparams_t *hp, const char *arch, const char *key, float v)
{
    if (arch_key(key, arch, "rope.freq_base")) hp->rope_freq_base = v;
    else if (arch_key(key, arch, "attention.layer_norm_rms_epsilon")) hp->rms_norm_eps = v;
}

size_t cmol_tensor_nbytes(cmol_dtype_t dtype, int64_t n)
{
    switch (dtype) {
    case CMOL_DTYPE_F32: return (size_t)n * 4;
    case CMOL_DTYPE_F16: return (size_t)n * 2;
    case CMOL_DTYPE_Q4_0: return (size_t)(n / 32) * 18;
    case CMOL_DTYPE_Q5_0: return (size_t)(n / 32) * 22;
    case CMOL_DTYPE_Q8_0: return (size_t)(n / 32) * 34;
    case CMOL_DTYPE_Q4_K: return (size_t)(n / 256) * 144;
    case CMOL_DTYPE_Q6_K: return (size_t)(n / 256) * 210;
    default: return 0;
    }
}

/* ---- merges: "left right" strings -> vocab id pairs -------------------- */
static const char **g_sort_vocab; /* load is single-threaded (qsort) */
static int cmp_vocab(const void *a, const void *b)
{
    return strcmp(g_sort_vocab[*(const int32_t *)a], g_sort_vocab[*(const int32_t *)b]);
}
static int32_t vocab_find(const int32_t *idx, const char **vocab, int n, const char *s)
{
    int lo = 0, hi = n - 1;
    while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        int c = strcmp(vocab[idx[mid]], s);
        if (!c) return idx[mid];
        if (c < 0) lo = mid + 1;
        else hi = mid - 1;
    }
    return -1;
}

static cmol_err_t resolve_merges(cmol_arena_t *a, cmol_tokenizer_t *tok, const char **raw, int n)
{
    if (!n || !tok->vocab || !tok->vocab_size) return CMOL_OK;
    int32_t *idx = (int32_t *)cmol_arena_alloc_n(a, (size_t)tok->vocab_size, 4);
    tok->merge_left = (int32_t *)cmol_arena_alloc_n(a, (size_t)n, 4);
    tok->merge_right = (int32_t *)cmol_arena_alloc_n(a, (size_t)n, 4);
    if (!idx || !tok->merge_left || !tok->merge_right) return CMOL_ERR_OOM;
    for (int i = 0; i < tok->vocab_size; i++) idx[i] = i;
    g_sort_vocab = tok->vocab;
    qsort(idx, (size_t)tok->vocab_size, 4, cmp_vocab);
    tok->n_merges = n;
    char left[512];
    for (int i = 0; i < n; i++) {
        const char *sp = strchr(raw[i], ' ');
        size_t ll = sp ? (size_t)(sp - raw[i]) : 0;
        if (!sp || ll >= sizeof left) { tok->merge_left[i] = tok->merge_right[i] = -1; continue; }
        memcpy(left, raw[i], ll);
        left[ll] = 0;
        tok->merge_left[i] = vocab_find(idx, tok->vocab, tok->vocab_size, left);
        tok->merge_right[i] = vocab_find(idx, tok->vocab, tok->vocab_size, sp + 1);
    }
    return CMOL_OK;
}

static cmol_err_t cur_status(const cur_t *c) { return c->err == 2 ? CMOL_ERR_OOM : CMOL_ERR_INVALID; }

static cmol_err_t read_kv(cur_t *c, cmol_arena_t *a, char *arch, cmol_hparams_t *hp,
                          cmol_tokenizer_t *tok, const char ***merges, int *n_merges)
{
    char k[256];
    int have = cur_str_buf(c, k, sizeof k);   /* over-long keys match nothing */
    uint32_t t = cur_u32(c);
    if (c->err) return cur_status(c);
    if (!have) { skip_value(c, t); return c->err ? CMOL_ERR_INVALID : CMOL_OK; }

    if (!strcmp(k, "general.architecture") && t == GV_STR) {
        const char *s = cur_str(c, a);
        if (s) {
            snprintf(arch, 32, "%s", s);
            snprintf(hp->arch, sizeof hp->arch, "%s", s);
        }
        return c->err ? cur_status(c) : CMOL_OK;
    }
    if (t == GV_U32) {
        uint32_t v = cur_u32(c);
        if (c->err) return CMOL_ERR_INVALID;
        if (apply_u32(hp, arch, k, v)) return CMOL_OK;
        if (!strcmp(k, "tokenizer.ggml.bos_token_id")) tok->bos_id = (int32_t)v;
        else if (!strcmp(k, "tokenizer.ggml.eos_token_id")) tok->eos_id = (int32_t)v;
        else if (!strcmp(k, "tokenizer.ggml.unknown_token_id")) tok->unk_id = (int32_t)v;
        return CMOL_OK;
    }
    if (t == GV_BOOL) {
        uint8_t v = (uint8_t)cur_uint(c, 1);
        if (c->err) return CMOL_ERR_INVALID;
        if (!strcmp(k, "tokenizer.ggml.add_bos_token")) tok->add_bos = v ? 1 : 0;
        return CMOL_OK;
    }
    if (t == GV_F32) {
        float v = cur_f32(c);
        if (c->err) return CMOL_ERR_INVALID;
        apply_f32(hp, arch, k, v);
        return CMOL_OK;
    }
    if (t == GV_ARR) {
        uint32_t et = cur_u32(c);
        uint64_t n = cur_u64(c);
        if (c->err || n > ((uint64_t)1 << 26)) return CMOL_ERR_INVALID;
        if (!strcmp(k, "tokenizer.ggml.tokens") && et == GV_STR) {
            tok->vocab = (const char **)cmol_arena_alloc_n(a, (size_t)n, sizeof(char *));
            if (!tok->vocab) return CMOL_ERR_OOM;
            tok->vocab_size = (int)n;
            for (uint64_t i = 0; i < n; i++) {
                tok->vocab[i] = cur_str(c, a);
                if (!tok->vocab[i]) return cur_status(c);
            }
            return CMOL_OK;
        }
        if (!strcmp(k, "tokenizer.ggml.scores") && et == GV_F32) {
            tok->scores = (float *)cmol_arena_alloc_n(a, (size_t)n, 4);
            if (!tok->scores) return CMOL_ERR_OOM;
            for (uint64_t i = 0; i < n; i++) tok->scores[i] = cur_f32(c);
            return c->err ? CMOL_ERR_INVALID : CMOL_OK;
        }
        if (!strcmp(k, "tokenizer.ggml.token_type") && et == GV_I32) {
            tok->token_type = (uint8_t *)cmol_arena_alloc_n(a, (size_t)n, 1);
            if (!tok->token_type) return CMOL_ERR_OOM;
            for (uint64_t i = 0; i < n; i++) tok->token_type[i] = (uint8_t)cur_u32(c);
            return c->err ? CMOL_ERR_INVALID : CMOL_OK;
        }
        if (!strcmp(k, "tokenizer.ggml.merges") && et == GV_STR) {
            *merges = (const char **)cmol_arena_alloc_n(a, (size_t)n, sizeof(char *));
            if (!*merges) return CMOL_ERR_OOM;
            *n_merges = (int)n;
            for (uint64_t i = 0; i < n; i++) {
                (*merges)[i] = cur_str(c, a);
                if (!(*merges)[i]) return cur_status(c);
            }
            return CMOL_OK;
        }
        for (uint64_t i = 0; i < n && !c->err; i++) skip_scalar(c, et);
        return c->err ? CMOL_ERR_INVALID : CMOL_OK;
    }
    if (t == GV_STR && !strcmp(k, "tokenizer.ggml.model")) {
        size_t n;
        const char *s = cur_strn(c, &n);
        if (s) tok->tok_model = (n == 5 && !memcmp(s, "llama", 5)) ? CMOL_TOK_LLAMA : CMOL_TOK_GPT2;
        return c->err ? CMOL_ERR_INVALID : CMOL_OK;
    }
    if (t == GV_STR && arch_key(k, arch, "rope.scaling.type")) {
        size_t n;
        (void)cur_strn(c, &n);
        hp->yarn_factor_x100 = -1; /* present, not applied (as the reference) */
        return c->err ? CMOL_ERR_INVALID : CMOL_OK;
    }
    skip_value(c, t);
    return c->err ? CMOL_ERR_INVALID : CMOL_OK;
}

static void hp_defaults(cmol_hparams_t *hp)
{
    memset(hp, 0, sizeof *hp);
    hp->rope_freq_base = 10000.0f;
    hp->rms_norm_eps = 1e-5f;
    snprintf(hp->arch, sizeof hp->arch, "llama");
}

static void hp_derive(cmol_hparams_t *hp)
{
    if (!hp->n_kv_heads) hp->n_kv_heads = hp->n_heads;
    if (hp->n_heads > 0) hp->d_head = hp->d_model / hp->n_heads;
}

cmol_err_t cmol_gguf_parse(const cmol_mmap_t *mm, cmol_arena_t *a, cmol_hparams_t *hp,
                           cmol_tensor_t **tensors_out, int *n_tensors_out,
                           cmol_tokenizer_t *tok)
{
    cur_t c = {(const uint8_t *)mm->data, mm->size, 0, 0};
    uint32_t magic = cur_u32(&c), ver = cur_u32(&c);
    if (c.err || magic != GGUF_MAGIC) return CMOL_ERR_INVALID;
    if (ver < 2 || ver > 3) return CMOL_ERR_UNSUPPORTED;
    uint64_t nt = cur_u64(&c), nkv = cur_u64(&c);
    if (c.err || nt > 65536 || nkv > 65536) return CMOL_ERR_INVALID;
    hp_defaults(hp);
    memset(tok, 0, sizeof *tok);
    tok->bos_id = tok->eos_id = tok->unk_id = -1;
    tok->add_bos = 1;
    char arch[32] = "llama";
    const char **merges = NULL;
    int n_merges = 0;
    for (uint64_t i = 0; i < nkv; i++) {
        cmol_err_t e = read_kv(&c, a, arch, hp, tok, &merges, &n_merges);
        if (e != CMOL_OK) return e;
    }
    hp_derive(hp);
    if (!hp->vocab_size) hp->vocab_size = tok->vocab_size;
    if (!tok->vocab_size) tok->vocab_size = hp->vocab_size;
    hp->bos_token_id = tok->bos_id;
    hp->eos_token_id = tok->eos_id;
    if (n_merges) {
        cmol_err_t e = resolve_merges(a, tok, merges, n_merges);
        if (e != CMOL_OK) return e;
    }
    cmol_tensor_t *t = (cmol_tensor_t *)cmol_arena_alloc_n(a, (size_t)(nt ? nt : 1), sizeof *t);
    if (!t) return CMOL_ERR_OOM;
    for (uint64_t i = 0; i < nt; i++) {
        size_t nl;
        const char *nm = cur_strn(&c, &nl);
        if (!nm) return cur_status(&c);
        size_t cl = nl < CMOL_MAX_TENSOR_NAME - 1 ? nl : CMOL_MAX_TENSOR_NAME - 1;
        memcpy(t[i].name, nm, cl);
        t[i].name[cl] = 0;
        uint32_t nd = cur_u32(&c);
        if (c.err || nd < 1 || nd > CMOL_MAX_DIMS) return CMOL_ERR_INVALID;
        t[i].n_dims = (int)nd;
        int64_t ne = 1;
        for (int d = 0; d < CMOL_MAX_DIMS; d++) t[i].shape[d] = 1;
        for (uint32_t d = 0; d < nd; d++) {
            t[i].shape[d] = (int64_t)cur_u64(&c);
            if (t[i].shape[d] < 0 || t[i].shape[d] > ((int64_t)1 << 40)) return CMOL_ERR_INVALID;
            ne *= t[i].shape[d];
        }
        t[i].dtype = (cmol_dtype_t)cur_u32(&c);
        t[i].file_offset = cur_u64(&c);
        t[i].n_bytes = cmol_tensor_nbytes(t[i].dtype, ne);
        if (c.err) return CMOL_ERR_INVALID;
    }
    size_t data0 = (c.pos + GGUF_ALIGN - 1u) & ~(size_t)(GGUF_ALIGN - 1u);
    for (uint64_t i = 0; i < nt; i++) {
        size_t off = data0 + (size_t)t[i].file_offset;
        if (off < data0 || off > mm->size || t[i].n_bytes > mm->size - off) return CMOL_ERR_INVALID;
        t[i].data = (uint8_t *)mm->data + off;
    }
    hp->tie_embeddings = cmol_gguf_find_tensor(t, (int)nt, "output.weight") == NULL;
    *tensors_out = t;
    *n_tensors_out = (int)nt;
    return CMOL_OK;
}

cmol_tensor_t *cmol_gguf_find_tensor(cmol_tensor_t *tensors, int n, const char *name)
{
    for (int i = 0; i < n; i++)
        if (!strcmp(tensors[i].name, name)) return &tensors[i];
    return NULL;
}

/* Header-only read of hparams and the tensor count (reference
 * src/gguf.c:535-626); no arena. */
cmol_err_t cmol_gguf_peek(const char *path, cmol_hparams_t *hp_out, size_t *n_tensors_out)
{
    if (!path || !hp_out || !n_tensors_out) return CMOL_ERR_ARGS;
    cmol_mmap_t mm;
    cmol_err_t e = cmol_mmap_open(path, &mm);
    if (e != CMOL_OK) return e;
    cur_t c = {(const uint8_t *)mm.data, mm.size, 0, 0};
    cmol_hparams_t hp;
    hp_defaults(&hp);
    e = CMOL_ERR_INVALID;
    uint32_t magic = cur_u32(&c), ver = cur_u32(&c);
    uint64_t nt = cur_u64(&c), nkv = cur_u64(&c);
    if (!c.err && magic == GGUF_MAGIC && ver >= 2 && ver <= 3) {
        char arch[32] = "llama";
        for (uint64_t i = 0; i < nkv && !c.err; i++) {
            char k[128];
            int have = cur_str_buf(&c, k, sizeof k);
            uint32_t t = cur_u32(&c);
            if (c.err) break;
            if (have && !strcmp(k, "general.architecture") && t == GV_STR) {
                char s[32];
                if (cur_str_buf(&c, s, sizeof s)) {
                    snprintf(arch, sizeof arch, "%s", s);
                    snprintf(hp.arch, sizeof hp.arch, "%s", s);
                }
            } else if (have && t == GV_U32) {
                (void)apply_u32(&hp, arch, k, cur_u32(&c));
            } else if (have && t == GV_F32) {
                apply_f32(&hp, arch, k, cur_f32(&c));
            } else {
                skip_value(&c, t);
            }
        }
        if (!c.err) {
            hp_derive(&hp);
            *hp_out = hp;
            *n_tensors_out = (size_t)nt;
            e = CMOL_OK;
        }
    }
    cmol_mmap_close(&mm);
    return e;
}
