/*
 * synth_gguf.c — deterministic synthetic GGUF models and inputs.
 *
 * Writes SmolLM-shaped GGUF v3 files that libcmol's loader accepts
 * (reference src/gguf.c:299-518): arch-prefixed UINT32/FLOAT32 hparams,
 * a tokenizer.ggml.tokens array, F32 norm weights, 32-byte data alignment,
 * output.weight omitted for tied embeddings.  cmolsynth_write_gguf_tok adds a
 * full tokenizer description (model, tokens, token types, merges, special
 * ids, add-BOS flag) with the key types the reference reads
 * (src/gguf.c:71-79,299-395).
 *
 * Weights are ~N(0, std) from a counter-based integer generator (sum of four
 * 16-bit uniforms from a splitmix64 hash, an Irwin-Hall approximation), so
 * every host produces identical bytes.  Quantisers follow GGML's published
 * reference quantisers (quantize_row_q8_0/q4_0/q5_0_ref): Q8_0 d=amax/127,
 * q=round(x/d); Q4_0 d=max/-8, q=min(15,(int8)(x/d+8.5)); Q5_0 d=max/-16,
 * q=min(31,(int8)(x/d+16.5)); scales rounded to fp16 (round-to-nearest-even).
 * The K-quants use a plain min/max quantiser (not GGML's iterative search,
 * which only changes which valid encoding a weight gets): Q4_K per 32-value
 * sub-block scale (max - min')/15 with min' = min(0, min), super-block
 * d = max scale / 63 and dmin = max |min'| / 63, six-bit codes of both;
 * Q6_K per 16-value group scale max|x|/31, super-block d = max |scale| / 127,
 * int8 group scales, codes q + 32 in 0..63.
 */
#define _DEFAULT_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

typedef struct {
    int32_t n_layers, d_model, n_heads, n_kv_heads, d_ffn, vocab, ctx_len;
    int32_t wtype, embd_type, out_type;   /* out_type < 0: tied embeddings */
    int32_t nope_interval, eos_id, qk_norm, arch_smollm3, transcode_q8;
    int32_t v_type, down_type;            /* attn_v / ffn_down format (< 0: wtype) */
    int32_t rope_scaling;                 /* 1: write <arch>.rope.scaling.type = "yarn" */
    float rope_base, rms_eps, wstd, norm_jitter;
    uint64_t seed;
} cmolsynth_spec_t;

/* ---- generator ---------------------------------------------------------- */
static inline uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline float normal_at(uint64_t key, uint64_t i, float scale)
{
    uint64_t h = mix64(key ^ mix64(i));
    int32_t s = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) +
                (int32_t)((h >> 32) & 0xFFFF) + (int32_t)(h >> 48);
    return (float)(s - 131070) * scale;
}

/* sd of a sum of four uniform 16-bit integers */
#define IH4_SD 37837.2264f

static uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return mix64(seed * 0xD1B54A32D192ED03ull + mix64(stream + 0x632BE59BD9B4E019ull));
}

void cmolsynth_normal(float *out, int64_t n, uint64_t seed, uint64_t stream, float std)
{
    uint64_t key = stream_key(seed, stream);
    float sc = std / IH4_SD;
    for (int64_t i = 0; i < n; i++) out[i] = normal_at(key, (uint64_t)i, sc);
}

void cmolsynth_tokens(int32_t *out, int n, uint64_t seed, int vocab)
{
    uint64_t key = stream_key(seed, 0x70C3ull);
    for (int i = 0; i < n; i++)
        out[i] = (int32_t)((mix64(key ^ mix64((uint64_t)i)) >> 11) % (uint64_t)vocab);
}

/* uniform double in [0,1) for seeded length draws */
double cmolsynth_uniform(uint64_t seed, uint64_t i)
{
    return (double)(mix64(stream_key(seed, 0x1E6ull) ^ mix64(i)) >> 11) * (1.0 / 9007199254740992.0);
}

/* ---- fp16 ---------------------------------------------------------------- */
uint16_t cmolsynth_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
    if (ax < 0x38800000u) {                                      /* subnormal half */
        if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: zero */
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                                /* 14..24 */
        uint32_t v = m >> shift, rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (v & 1u))) v++;
        return (uint16_t)(sign | v);
    }
    uint32_t v = ((ax >> 13) - (112u << 10));
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v++;
    return (uint16_t)(sign | v);
}

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ---- quantisers (GGML reference algorithms) ----------------------------- */
static void q8_0_block(const float *x, uint8_t *o)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
    float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(o, cmolsynth_f32_to_f16(d));
    for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

static void q4_0_block(const float *x, uint8_t *o)
{
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
    float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(o, cmolsynth_f32_to_f16(d));
    for (int j = 0; j < 16; j++) {
        int a = (int8_t)(x[j] * id + 8.5f), b = (int8_t)(x[j + 16] * id + 8.5f);
        if (a > 15) a = 15;
        if (b > 15) b = 15;
        o[2 + j] = (uint8_t)(a | (b << 4));
    }
}

static void q5_0_block(const float *x, uint8_t *o)
{
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
    float d = mx / -16.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(o, cmolsynth_f32_to_f16(d));
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        int a = (int8_t)(x[j] * id + 16.5f), b = (int8_t)(x[j + 16] * id + 16.5f);
        if (a > 31) a = 31;
        if (b > 31) b = 31;
        o[6 + j] = (uint8_t)((a & 0xF) | ((b & 0xF) << 4));
        qh |= (uint32_t)((a >> 4) & 1) << j;
        qh |= (uint32_t)((b >> 4) & 1) << (j + 16);
    }
    memcpy(o + 2, &qh, 4);
}

/* Lossless re-encoding of a Q4_0 / Q5_0 block as Q8_0 (same fp16 scale,
 * integer codes centred).  Lets the Q8_0-only reference consume the exact
 * same dequantised weights. */
static void to_q8_0(int dtype, const uint8_t *b, uint8_t *o)
{
    o[0] = b[0]; o[1] = b[1];
    if (dtype == T_Q4_0) {
        for (int j = 0; j < 16; j++) {
            o[2 + j] = (uint8_t)(int8_t)((b[2 + j] & 0xF) - 8);
            o[2 + j + 16] = (uint8_t)(int8_t)((b[2 + j] >> 4) - 8);
        }
    } else {
        uint32_t qh;
        memcpy(&qh, b + 2, 4);
        for (int j = 0; j < 16; j++) {
            int lo = (b[6 + j] & 0xF) | (int)(((qh >> j) & 1u) << 4);
            int hi = (b[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            o[2 + j] = (uint8_t)(int8_t)(lo - 16);
            o[2 + j + 16] = (uint8_t)(int8_t)(hi - 16);
        }
    }
}

/* IEEE half -> float for finite values (the quantisers' rounded scales). */
static float f16_value(uint16_t h)
{
    int e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float v = e ? ldexpf((float)(m | 0x400), e - 25) : ldexpf((float)m, -24);
    return (h & 0x8000) ? -v : v;
}

static float f16_round(float v) { return f16_value(cmolsynth_f32_to_f16(v)); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* Q4_K super-block of 256 values (layout src/quant.c:92-97,113-132,172-195). */
static void q4_k_block(const float *x, uint8_t *o)
{
    float scale[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int k = 0; k < 32; k++) {
            float v = x[32 * j + k];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        scale[j] = (hi - lo) / 15.0f;
        mins[j] = -lo;
        if (scale[j] > smax) smax = scale[j];
        if (mins[j] > mmax) mmax = mins[j];
    }
    float d = f16_round(smax / 63.0f), dmin = f16_round(mmax / 63.0f);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.0f ? clampi((int)lrintf(scale[j] / d), 0, 63) : 0;
        mn[j] = dmin > 0.0f ? clampi((int)lrintf(mins[j] / dmin), 0, 63) : 0;
    }
    memset(o, 0, 144);
    put16(o, cmolsynth_f32_to_f16(d));
    put16(o + 2, cmolsynth_f32_to_f16(dmin));
    uint8_t *s = o + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    for (int j = 0; j < 8; j++) {
        float db = d * (float)sc[j], mb = dmin * (float)mn[j];
        for (int k = 0; k < 32; k++) {
            int q = db > 0.0f ? clampi((int)lrintf((x[32 * j + k] + mb) / db), 0, 15) : 0;
            o[16 + 32 * (j / 2) + k] |= (uint8_t)(q << ((j & 1) ? 4 : 0));
        }
    }
}

/* Q6_K super-block of 256 values (layout src/quant.c:99-105,197-231). */
static void q6_k_block(const float *x, uint8_t *o)
{
    float gs[16], gmax = 0.0f;
    for (int g = 0; g < 16; g++) {
        float a = 0.0f;
        for (int k = 0; k < 16; k++) {
            float v = fabsf(x[16 * g + k]);
            if (v > a) a = v;
        }
        gs[g] = a / 31.0f;
        if (gs[g] > gmax) gmax = gs[g];
    }
    float d = f16_round(gmax / 127.0f);
    memset(o, 0, 210);
    for (int g = 0; g < 16; g++) {
        int sc = d > 0.0f ? clampi((int)lrintf(gs[g] / d), -128, 127) : 0;
        o[192 + g] = (uint8_t)(int8_t)sc;
        float ds = d * (float)sc;
        for (int k = 0; k < 16; k++) {
            int i = 16 * g + k;
            int q = ds != 0.0f ? clampi((int)lrintf(x[i] / ds), -32, 31) : 0;
            int u = q + 32, g8 = i / 32, j32 = i % 32;
            o[(g8 < 4 ? 0 : 64) + (g8 & 1) * 32 + j32] |= (uint8_t)((u & 0xF) << ((g8 & 2) ? 4 : 0));
            o[128 + (g8 < 4 ? 0 : 32) + j32] |= (uint8_t)(((u >> 4) & 3) << ((g8 & 3) * 2));
        }
    }
    put16(o + 208, cmolsynth_f32_to_f16(d));
}

static size_t block_bytes(int dtype)
{
    switch (dtype) {
    case T_Q4_K: return 144;
    case T_Q6_K: return 210;
    case T_Q4_0: return 18;
    case T_Q5_0: return 22;
    case T_Q8_0: return 34;
    case T_F16: return 2;
    case T_F32: return 4;
    default: return 0;
    }
}

static int block_values(int dtype) { return (dtype == T_Q4_K || dtype == T_Q6_K) ? 256 : 32; }

static size_t row_bytes(int dtype, int64_t k)
{
    if (dtype == T_F32 || dtype == T_F16) return (size_t)k * block_bytes(dtype);
    return (size_t)(k / block_values(dtype)) * block_bytes(dtype);
}

/* Quantise n values (n % 32 == 0 for block formats); returns bytes written. */
int64_t cmolsynth_quantize(int dtype, const float *x, int64_t n, void *out)
{
    uint8_t *o = (uint8_t *)out;
    if (dtype == T_F32) { memcpy(o, x, (size_t)n * 4); return n * 4; }
    if (dtype == T_F16) {
        for (int64_t i = 0; i < n; i++) put16(o + 2 * i, cmolsynth_f32_to_f16(x[i]));
        return n * 2;
    }
    size_t bb = block_bytes(dtype);
    const int bv = block_values(dtype);
    if (!bb || n % bv) return -1;
    for (int64_t b = 0; b < n / bv; b++) {
        if (dtype == T_Q8_0) q8_0_block(x + b * 32, o + b * bb);
        else if (dtype == T_Q4_0) q4_0_block(x + b * 32, o + b * bb);
        else if (dtype == T_Q5_0) q5_0_block(x + b * 32, o + b * bb);
        else if (dtype == T_Q4_K) q4_k_block(x + b * 256, o + b * bb);
        else q6_k_block(x + b * 256, o + b * bb);
    }
    return (n / bv) * (int64_t)bb;
}

/* ---- tensor generation --------------------------------------------------- */
typedef struct {
    char name[96];
    int dtype;        /* dtype written to the file */
    int gen_dtype;    /* dtype the values are quantised with */
    int64_t ne0, ne1; /* ne0 = in features (row length), ne1 = rows */
    int kind;         /* 0 = weight ~N(0,std), 1 = norm 1+N(0,jitter) */
    uint64_t stream;
    uint64_t offset;
} tdesc_t;

typedef struct {
    const tdesc_t *t;
    uint8_t *buf;
    int64_t r0, r1;
    uint64_t key;
    float sc;
} gen_job_t;

static void *gen_rows(void *p)
{
    gen_job_t *j = (gen_job_t *)p;
    const tdesc_t *t = j->t;
    float *row = (float *)malloc((size_t)t->ne0 * 4);
    uint8_t *tmp = (uint8_t *)malloc(row_bytes(t->gen_dtype, t->ne0) + 64);
    size_t orb = row_bytes(t->dtype, t->ne0);
    for (int64_t r = j->r0; r < j->r1; r++) {
        for (int64_t c = 0; c < t->ne0; c++) {
            float v = normal_at(j->key, (uint64_t)(r * t->ne0 + c), j->sc);
            row[c] = t->kind == 1 ? 1.0f + v : v;
        }
        if (t->gen_dtype == t->dtype) {
            cmolsynth_quantize(t->dtype, row, t->ne0, j->buf + (size_t)r * orb);
        } else {
            cmolsynth_quantize(t->gen_dtype, row, t->ne0, tmp);
            size_t gb = block_bytes(t->gen_dtype);
            for (int64_t b = 0; b < t->ne0 / 32; b++)
                to_q8_0(t->gen_dtype, tmp + b * gb, j->buf + (size_t)r * orb + b * 34);
        }
    }
    free(row);
    free(tmp);
    return NULL;
}

static int gen_tensor(const cmolsynth_spec_t *s, const tdesc_t *t, uint8_t *buf, int nthreads)
{
    uint64_t key = stream_key(s->seed, t->stream);
    float sc = (t->kind == 1 ? s->norm_jitter : s->wstd) / IH4_SD;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    gen_job_t jb[64];
    int64_t per = (t->ne1 + nthreads - 1) / nthreads;
    int used = 0;
    for (int i = 0; i < nthreads; i++) {
        int64_t a = i * per, b = a + per > t->ne1 ? t->ne1 : a + per;
        if (a >= b) break;
        jb[i] = (gen_job_t){t, buf, a, b, key, sc};
        if (pthread_create(&th[i], NULL, gen_rows, &jb[i]) != 0) return -1;
        used++;
    }
    for (int i = 0; i < used; i++) pthread_join(th[i], NULL);
    return 0;
}

/* ---- GGUF writing --------------------------------------------------------- */
static void w_u32(FILE *f, uint32_t v) { fwrite(&v, 4, 1, f); }
static void w_u64(FILE *f, uint64_t v) { fwrite(&v, 8, 1, f); }
static void w_str(FILE *f, const char *s) { uint64_t n = strlen(s); w_u64(f, n); fwrite(s, 1, n, f); }
static void kv_u32(FILE *f, const char *k, uint32_t v) { w_str(f, k); w_u32(f, 4); w_u32(f, v); }
static void kv_f32(FILE *f, const char *k, float v) { w_str(f, k); w_u32(f, 6); fwrite(&v, 4, 1, f); }
static void kv_str(FILE *f, const char *k, const char *v) { w_str(f, k); w_u32(f, 8); w_str(f, v); }

static void vocab_string(int i, char *buf)
{
    if (i < 256) snprintf(buf, 16, "<0x%02X>", i);
    else snprintf(buf, 16, "t%d", i);
}

/* Tokenizer of a synthetic model (all arrays of n_tokens entries; types and
 * merges may be null; ids < 0 and add_bos < 0 are left out). */
typedef struct {
    const char *model;
    int32_t n_tokens;
    const char *const *tokens;
    const int32_t *types;
    int32_t n_merges;
    const char *const *merges;
    int32_t bos_id, eos_id, unk_id, add_bos;
} cmolsynth_tok_t;

static int write_gguf(const char *path, const cmolsynth_spec_t *s, int nthreads, const cmolsynth_tok_t *tk);

int cmolsynth_write_gguf(const char *path, const cmolsynth_spec_t *s, int nthreads)
{
    return write_gguf(path, s, nthreads, NULL);
}

int cmolsynth_write_gguf_tok(const char *path, const cmolsynth_spec_t *s, int nthreads,
                             const cmolsynth_tok_t *tk)
{
    if (!tk || !tk->model || !tk->tokens || tk->n_tokens != s->vocab) return -1;
    return write_gguf(path, s, nthreads, tk);
}

static int write_gguf(const char *path, const cmolsynth_spec_t *s, int nthreads, const cmolsynth_tok_t *tk)
{
    if (!path || !s || s->n_layers < 1 || s->d_model % 32 || s->d_ffn % 32 ||
        s->n_heads < 1 || s->d_model % s->n_heads || s->vocab < 1)
        return -1;
    int L = s->n_layers, d = s->d_model, dh = d / s->n_heads, kvd = s->n_kv_heads * dh;
    int nt_max = 2 + L * 11 + 1;
    tdesc_t *td = (tdesc_t *)calloc((size_t)nt_max, sizeof(tdesc_t));
    int nt = 0;
#define ADD(nm, dt, a, b, kd)                                                    \
    do {                                                                         \
        tdesc_t *t_ = &td[nt];                                                   \
        snprintf(t_->name, sizeof t_->name, "%s", nm);                           \
        t_->gen_dtype = (dt);                                                    \
        t_->dtype = (s->transcode_q8 && ((dt) == T_Q4_0 || (dt) == T_Q5_0)) ? T_Q8_0 : (dt); \
        t_->ne0 = (a); t_->ne1 = (b); t_->kind = (kd);                           \
        t_->stream = (uint64_t)nt + 1;                                           \
        nt++;                                                                    \
    } while (0)
    char nm[96];
    ADD("token_embd.weight", s->embd_type, d, s->vocab, 0);
    for (int l = 0; l < L; l++) {
        snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l);   ADD(nm, T_F32, d, 1, 1);
        snprintf(nm, sizeof nm, "blk.%d.attn_q.weight", l);      ADD(nm, s->wtype, d, d, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_k.weight", l);      ADD(nm, s->wtype, d, kvd, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_v.weight", l);      ADD(nm, s->v_type >= 0 ? s->v_type : s->wtype, d, kvd, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_output.weight", l); ADD(nm, s->wtype, d, d, 0);
        if (s->qk_norm) {
            snprintf(nm, sizeof nm, "blk.%d.attn_q_norm.weight", l); ADD(nm, T_F32, dh, 1, 1);
            snprintf(nm, sizeof nm, "blk.%d.attn_k_norm.weight", l); ADD(nm, T_F32, dh, 1, 1);
        }
        snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l);    ADD(nm, T_F32, d, 1, 1);
        snprintf(nm, sizeof nm, "blk.%d.ffn_gate.weight", l);    ADD(nm, s->wtype, d, s->d_ffn, 0);
        snprintf(nm, sizeof nm, "blk.%d.ffn_up.weight", l);      ADD(nm, s->wtype, d, s->d_ffn, 0);
        snprintf(nm, sizeof nm, "blk.%d.ffn_down.weight", l);    ADD(nm, s->down_type >= 0 ? s->down_type : s->wtype, s->d_ffn, d, 0);
    }
    ADD("output_norm.weight", T_F32, d, 1, 1);
    if (s->out_type >= 0) ADD("output.weight", s->out_type, d, s->vocab, 0);
#undef ADD
    uint64_t off = 0;
    for (int i = 0; i < nt; i++) {
        td[i].offset = off;
        off += (row_bytes(td[i].dtype, td[i].ne0) * (uint64_t)td[i].ne1 + 31u) & ~(uint64_t)31u;
    }

    FILE *f = fopen(path, "wb");
    if (!f) { free(td); return -2; }
    const char *arch = s->arch_smollm3 ? "smollm3" : "llama";
    int n_kv = 12 + (s->nope_interval > 0) + (s->rope_scaling > 0);
    if (tk)
        n_kv += (tk->types != NULL) + (tk->n_merges > 0) + (tk->bos_id >= 0) + (tk->eos_id >= 0) +
                (tk->unk_id >= 0) + (tk->add_bos >= 0);
    else
        n_kv += s->eos_id >= 0;
    w_u32(f, 0x46554747u);
    w_u32(f, 3);
    w_u64(f, (uint64_t)nt);
    w_u64(f, (uint64_t)n_kv);
    char key[128];
    kv_str(f, "general.architecture", arch);
#define AKEY(suffix) (snprintf(key, sizeof key, "%s.%s", arch, suffix), key)
    kv_u32(f, AKEY("context_length"), (uint32_t)s->ctx_len);
    kv_u32(f, AKEY("embedding_length"), (uint32_t)d);
    kv_u32(f, AKEY("block_count"), (uint32_t)L);
    kv_u32(f, AKEY("feed_forward_length"), (uint32_t)s->d_ffn);
    kv_u32(f, AKEY("attention.head_count"), (uint32_t)s->n_heads);
    kv_u32(f, AKEY("attention.head_count_kv"), (uint32_t)s->n_kv_heads);
    kv_f32(f, AKEY("rope.freq_base"), s->rope_base);
    kv_f32(f, AKEY("attention.layer_norm_rms_epsilon"), s->rms_eps);
    kv_u32(f, AKEY("vocab_size"), (uint32_t)s->vocab);
    if (s->nope_interval > 0) kv_u32(f, AKEY("attention.no_rope_layer_interval"), (uint32_t)s->nope_interval);
    if (s->rope_scaling > 0) kv_str(f, AKEY("rope.scaling.type"), "yarn");
#undef AKEY
    if (!tk) {
        kv_str(f, "tokenizer.ggml.model", "llama");
        if (s->eos_id >= 0) kv_u32(f, "tokenizer.ggml.eos_token_id", (uint32_t)s->eos_id);
        /* token list */
        w_str(f, "tokenizer.ggml.tokens");
        w_u32(f, 9);
        w_u32(f, 8);
        w_u64(f, (uint64_t)s->vocab);
        for (int i = 0; i < s->vocab; i++) { char vb[16]; vocab_string(i, vb); w_str(f, vb); }
    } else {
        kv_str(f, "tokenizer.ggml.model", tk->model);
        if (tk->bos_id >= 0) kv_u32(f, "tokenizer.ggml.bos_token_id", (uint32_t)tk->bos_id);
        if (tk->eos_id >= 0) kv_u32(f, "tokenizer.ggml.eos_token_id", (uint32_t)tk->eos_id);
        if (tk->unk_id >= 0) kv_u32(f, "tokenizer.ggml.unknown_token_id", (uint32_t)tk->unk_id);
        if (tk->add_bos >= 0) {   /* BOOL */
            w_str(f, "tokenizer.ggml.add_bos_token");
            w_u32(f, 7);
            uint8_t b = tk->add_bos ? 1 : 0;
            fwrite(&b, 1, 1, f);
        }
        w_str(f, "tokenizer.ggml.tokens");   /* ARRAY of STRING */
        w_u32(f, 9);
        w_u32(f, 8);
        w_u64(f, (uint64_t)tk->n_tokens);
        for (int i = 0; i < tk->n_tokens; i++) w_str(f, tk->tokens[i]);
        if (tk->types) {                     /* ARRAY of INT32 */
            w_str(f, "tokenizer.ggml.token_type");
            w_u32(f, 9);
            w_u32(f, 5);
            w_u64(f, (uint64_t)tk->n_tokens);
            for (int i = 0; i < tk->n_tokens; i++) w_u32(f, (uint32_t)tk->types[i]);
        }
        if (tk->n_merges > 0) {              /* ARRAY of STRING */
            w_str(f, "tokenizer.ggml.merges");
            w_u32(f, 9);
            w_u32(f, 8);
            w_u64(f, (uint64_t)tk->n_merges);
            for (int i = 0; i < tk->n_merges; i++) w_str(f, tk->merges[i]);
        }
    }
    /* tensor infos: shape[0] is the innermost (in-features) dimension */
    for (int i = 0; i < nt; i++) {
        w_str(f, td[i].name);
        int nd = td[i].ne1 > 1 ? 2 : 1;
        w_u32(f, (uint32_t)nd);
        w_u64(f, (uint64_t)td[i].ne0);
        if (nd == 2) w_u64(f, (uint64_t)td[i].ne1);
        w_u32(f, (uint32_t)td[i].dtype);
        w_u64(f, td[i].offset);
    }
    long pos = ftell(f);
    static const uint8_t zeros[64] = {0};
    long pad = ((pos + 31) & ~31L) - pos;
    fwrite(zeros, 1, (size_t)pad, f);
    int rc = 0;
    for (int i = 0; i < nt && rc == 0; i++) {
        size_t bytes = row_bytes(td[i].dtype, td[i].ne0) * (size_t)td[i].ne1;
        size_t padded = (bytes + 31u) & ~(size_t)31u;
        uint8_t *buf = (uint8_t *)calloc(padded ? padded : 1, 1);
        if (!buf) { rc = -3; break; }
        if (gen_tensor(s, &td[i], buf, nthreads) != 0) rc = -4;
        if (rc == 0 && fwrite(buf, 1, padded, f) != padded) rc = -5;
        free(buf);
    }
    if (fclose(f) != 0 && rc == 0) rc = -5;
    free(td);
    return rc;
}
