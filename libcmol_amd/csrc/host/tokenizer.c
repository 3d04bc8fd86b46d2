/*
 * tokenizer.c — BPE tokenizer behind cmol_encode / cmol_generate.
 *
 * Same behaviour as the reference tokenizer (src/tokenizer.c):
 *   build   sorted vocab index for string -> id, merges sorted by the packed
 *           (left, right) pair for pair -> rank, merge results, and decoded
 *           pieces (<0xNN> byte tokens -> the byte, U+2581 prefix -> space,
 *           GPT-2 byte-level vocab decoded back to bytes) (src/tokenizer.c:189-343);
 *   encode  optional BOS; longest verbatim match of control tokens; for the
 *           SentencePiece model a U+2581 prefix at each text segment and
 *           spaces mapped to U+2581, each UTF-8 character looked up with a
 *           lowercase "<0x%02x>" byte fallback; GPT-2 byte-level lookup for
 *           other models; then repeated merging of the adjacent pair of
 *           lowest rank (src/tokenizer.c:359-558);
 *   decode  decoded piece of an id (src/tokenizer.c:564-571).
 * Model loading is single-threaded, so the qsort comparators use statics.
 */
#include "internal.h"

#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define TOKEN_CONTROL 3
#define TOKEN_BYTE 6
#define WORK_MAX 4096

static const char **s_vocab;
static const int32_t *s_ml, *s_mr;

static int cmp_vocab_idx(const void *a, const void *b)
{
    return strcmp(s_vocab[*(const int32_t *)a], s_vocab[*(const int32_t *)b]);
}

static uint64_t pair_key(int32_t l, int32_t r) { return ((uint64_t)(uint32_t)l << 32) | (uint32_t)r; }

static int cmp_merge_idx(const void *a, const void *b)
{
    int32_t i = *(const int32_t *)a, j = *(const int32_t *)b;
    uint64_t x = pair_key(s_ml[i], s_mr[i]), y = pair_key(s_ml[j], s_mr[j]);
    return x < y ? -1 : x > y;
}

static int32_t token_id(const cmol_tokenizer_t *t, const char *s)
{
    int lo = 0, hi = t->vocab_size - 1;
    while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        int32_t id = t->vocab_sort_idx[mid];
        int c = strcmp(t->vocab[id], s);
        if (!c) return id;
        if (c < 0) lo = mid + 1;
        else hi = mid - 1;
    }
    return -1;
}

static int32_t merge_rank(const cmol_tokenizer_t *t, int32_t l, int32_t r)
{
    if (!t->msort_idx || !t->n_merges || l < 0 || r < 0) return -1;
    uint64_t want = pair_key(l, r);
    int lo = 0, hi = t->n_merges - 1;
    while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        int32_t id = t->msort_idx[mid];
        uint64_t k = pair_key(t->merge_left[id], t->merge_right[id]);
        if (k == want) return id;
        if (k < want) lo = mid + 1;
        else hi = mid - 1;
    }
    return -1;
}

static int utf8_len(unsigned char c)
{
    if (c < 0x80) return 1;
    if ((c & 0xE0) == 0xC0) return 2;
    if ((c & 0xF0) == 0xE0) return 3;
    if ((c & 0xF8) == 0xF0) return 4;
    return 1;
}

static unsigned utf8_decode(const char **p)
{
    const unsigned char *u = (const unsigned char *)*p;
    if (!*u) return 0;
    if (u[0] >= 0x80 && u[0] < 0xC0) { (*p)++; return 0xFFFDu; }
    int n = u[0] < 0x80 ? 1 : u[0] < 0xE0 ? 2 : u[0] < 0xF0 ? 3 : 4;
    unsigned cp = n == 1 ? u[0] : n == 2 ? (u[0] & 0x1Fu) : n == 3 ? (u[0] & 0x0Fu) : (u[0] & 0x07u);
    for (int i = 1; i < n; i++) {
        if ((u[i] & 0xC0) != 0x80) break;
        cp = (cp << 6) | (u[i] & 0x3Fu);
    }
    *p += n;
    return cp;
}

static int utf8_encode(unsigned cp, char *b)
{
    if (cp < 0x80) { b[0] = (char)cp; return 1; }
    if (cp < 0x800) { b[0] = (char)(0xC0 | (cp >> 6)); b[1] = (char)(0x80 | (cp & 0x3F)); return 2; }
    if (cp < 0x10000) {
        b[0] = (char)(0xE0 | (cp >> 12));
        b[1] = (char)(0x80 | ((cp >> 6) & 0x3F));
        b[2] = (char)(0x80 | (cp & 0x3F));
        return 3;
    }
    b[0] = (char)(0xF0 | (cp >> 18));
    b[1] = (char)(0x80 | ((cp >> 12) & 0x3F));
    b[2] = (char)(0x80 | ((cp >> 6) & 0x3F));
    b[3] = (char)(0x80 | (cp & 0x3F));
    return 4;
}

/* GPT-2 byte <-> printable code point map (bytes 0x21-0x7E, 0xA1-0xAC and
 * 0xAE-0xFF map to themselves, the other 68 bytes to U+0100.. in order). */
static unsigned byte_to_cp(unsigned char b)
{
    if (b <= 0x20) return 0x100u + b;
    if (b <= 0x7E) return b;
    if (b == 0x7F) return 0x121u;
    if (b <= 0xA0) return 0x122u + (b - 0x80u);
    if (b == 0xAD) return 0x143u;
    return b;
}

static unsigned char cp_to_byte(unsigned cp)
{
    if (cp >= 0x100 && cp <= 0x120) return (unsigned char)(cp - 0x100);
    if (cp == 0x121) return 0x7F;
    if (cp >= 0x122 && cp <= 0x142) return (unsigned char)(0x80 + (cp - 0x122));
    if (cp == 0x143) return 0xAD;
    return (unsigned char)(cp & 0xFF);
}

cmol_err_t cmol_tokenizer_build(cmol_tokenizer_t *t, cmol_arena_t *a)
{
    if (!t || !a) return CMOL_ERR_ARGS;
    if (t->vocab_size == 0 || !t->vocab) return CMOL_ERR_INVALID;
    const int V = t->vocab_size, M = t->n_merges;
    t->vocab_sort_idx = (int32_t *)cmol_arena_alloc_n(a, (size_t)V, 4);
    if (!t->vocab_sort_idx) return CMOL_ERR_OOM;
    for (int i = 0; i < V; i++) t->vocab_sort_idx[i] = i;
    s_vocab = t->vocab;
    qsort(t->vocab_sort_idx, (size_t)V, 4, cmp_vocab_idx);
    if (M > 0) {
        t->msort_idx = (int32_t *)cmol_arena_alloc_n(a, (size_t)M, 4);
        t->merge_result = (int32_t *)cmol_arena_alloc_n(a, (size_t)M, 4);
        if (!t->msort_idx || !t->merge_result) return CMOL_ERR_OOM;
        for (int i = 0; i < M; i++) t->msort_idx[i] = i;
        s_ml = t->merge_left;
        s_mr = t->merge_right;
        qsort(t->msort_idx, (size_t)M, 4, cmp_merge_idx);
        char cat[256];
        for (int i = 0; i < M; i++) {
            int32_t l = t->merge_left[i], r = t->merge_right[i];
            t->merge_result[i] = t->unk_id;
            if (l < 0 || l >= V || r < 0 || r >= V) continue;
            size_t ll = strlen(t->vocab[l]), rl = strlen(t->vocab[r]);
            if (ll + rl >= sizeof cat) continue;
            memcpy(cat, t->vocab[l], ll);
            memcpy(cat + ll, t->vocab[r], rl + 1);
            int32_t id = token_id(t, cat);
            if (id >= 0) t->merge_result[i] = id;
        }
    }
    t->decoded_vocab = (const char **)cmol_arena_alloc_n(a, (size_t)V, sizeof(char *));
    if (!t->decoded_vocab) return CMOL_ERR_OOM;
    for (int i = 0; i < V; i++) {
        const char *s = t->vocab[i];
        t->decoded_vocab[i] = s;
        if (t->tok_model == CMOL_TOK_GPT2) {
            if (t->token_type && t->token_type[i] == TOKEN_CONTROL) continue;
            char buf[256];
            int n = 0;
            const char *p = s;
            while (*p && n < (int)sizeof buf - 1) {
                unsigned cp = utf8_decode(&p);
                if (!cp) break;
                buf[n++] = (char)cp_to_byte(cp);
            }
            if (n > 0) {
                char *d = (char *)cmol_arena_alloc(a, (size_t)n + 1, 1);
                if (!d) return CMOL_ERR_OOM;
                memcpy(d, buf, (size_t)n);
                d[n] = 0;
                t->decoded_vocab[i] = d;
            }
            continue;
        }
        int is_byte = t->token_type && t->token_type[i] == TOKEN_BYTE;
        if (!is_byte && strlen(s) == 6 && s[0] == '<' && s[1] == '0' && s[2] == 'x' && s[5] == '>')
            is_byte = 1;
        unsigned bv;
        if (is_byte && sscanf(s, "<0x%02x>", &bv) == 1) {
            char *d = (char *)cmol_arena_alloc(a, 2, 1);
            if (!d) return CMOL_ERR_OOM;
            d[0] = (char)(unsigned char)bv;
            t->decoded_vocab[i] = d;
            continue;
        }
        if ((unsigned char)s[0] == 0xE2 && (unsigned char)s[1] == 0x96 && (unsigned char)s[2] == 0x81) {
            size_t rest = strlen(s + 3);
            char *d = (char *)cmol_arena_alloc(a, rest + 2, 1);
            if (!d) return CMOL_ERR_OOM;
            d[0] = ' ';
            memcpy(d + 1, s + 3, rest + 1);
            t->decoded_vocab[i] = d;
        }
    }
    return CMOL_OK;
}

/* Upper bound of the arena bytes build + parse need for the tables beyond
 * the raw strings (sizing helper for cmol_load). */
size_t cmol_tokenizer_arena_bytes(int vocab, int n_merges)
{
    return (size_t)vocab * 80u + (size_t)n_merges * 16u;
}

typedef struct {
    int32_t *w;
    int n;
    int overflow;
} work_t;

static void push(work_t *k, int32_t id)
{
    if (k->n < WORK_MAX) k->w[k->n++] = id;
    else k->overflow = 1;
}

/* One character: its vocab id, else one byte token per byte (or unk). */
static void emit_char(const cmol_tokenizer_t *t, work_t *k, const char *p, int len)
{
    char c[8];
    memcpy(c, p, (size_t)len);
    c[len] = 0;
    int32_t id = token_id(t, c);
    if (id >= 0) { push(k, id); return; }
    for (int b = 0; b < len && !k->overflow; b++) {
        char bt[8];
        snprintf(bt, sizeof bt, "<0x%02x>", (unsigned char)p[b]);
        int32_t bid = token_id(t, bt);
        if (bid < 0) bid = t->unk_id;
        if (bid >= 0) push(k, bid);
    }
}

/* Longest control token matching verbatim at p, or -1. */
static int32_t control_at(const cmol_tokenizer_t *t, const char *p, size_t *len)
{
    int32_t best = -1;
    size_t bl = 0;
    if (!t->token_type) return -1;
    for (int v = 0; v < t->vocab_size; v++) {
        if (t->token_type[v] != TOKEN_CONTROL) continue;
        size_t tl = strlen(t->vocab[v]);
        if (tl > bl && !strncmp(p, t->vocab[v], tl)) { bl = tl; best = v; }
    }
    *len = bl;
    return best;
}

int cmol_tokenizer_encode(const cmol_tokenizer_t *t, const char *text, int32_t *out, int cap,
                          int add_bos)
{
    if (!t || !text || !out || cap <= 0) return CMOL_ERR_ARGS;
    if (!t->vocab_sort_idx || !t->decoded_vocab) return CMOL_ERR_UNSUPPORTED;
    int n = 0;
    if (add_bos && t->bos_id >= 0) out[n++] = t->bos_id;
    int32_t wbuf[WORK_MAX];
    work_t k = {wbuf, 0, 0};
    static const char spiece[] = "\xe2\x96\x81";
    const char *p = text;
    int prefixed = 0;
    while (*p && !k.overflow) {
        size_t cl;
        int32_t ctl = control_at(t, p, &cl);
        if (ctl >= 0) {
            push(&k, ctl);
            p += cl;
            prefixed = 0;
            continue;
        }
        if (t->tok_model == CMOL_TOK_GPT2) {
            char v[5];
            int vl = utf8_encode(byte_to_cp((unsigned char)*p++), v);
            v[vl] = 0;
            int32_t id = token_id(t, v);
            if (id < 0) id = t->unk_id;
            if (id >= 0) push(&k, id);
            continue;
        }
        if (!prefixed) {
            emit_char(t, &k, spiece, 3);
            prefixed = 1;
        }
        if (*p == ' ') {
            emit_char(t, &k, spiece, 3);
            p++;
        } else {
            int len = utf8_len((unsigned char)*p);
            emit_char(t, &k, p, len);
            p += len;
        }
    }
    if (t->n_merges > 0 && t->merge_result && t->msort_idx) {
        while (k.n > 1) {
            int at = -1;
            int32_t best = INT32_MAX;
            for (int i = 0; i < k.n - 1; i++) {
                int32_t r = merge_rank(t, k.w[i], k.w[i + 1]);
                if (r >= 0 && r < best) { best = r; at = i; }
            }
            if (at < 0) break;
            k.w[at] = t->merge_result[best];
            memmove(k.w + at + 1, k.w + at + 2, (size_t)(k.n - at - 2) * 4);
            k.n--;
        }
    }
    int trunc = k.overflow;
    for (int i = 0; i < k.n; i++) {
        if (n >= cap) { trunc = 1; break; }
        out[n++] = k.w[i];
    }
    return trunc ? CMOL_ERR_TRUNC : n;
}

const char *cmol_tokenizer_decode_token(const cmol_tokenizer_t *t, int32_t id)
{
    if (!t || id < 0 || id >= t->vocab_size) return NULL;
    if (t->decoded_vocab) return t->decoded_vocab[id];
    return t->vocab ? t->vocab[id] : NULL;
}
