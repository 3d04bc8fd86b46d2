/*
 * o_model.c — oracle: transformer primitives, GQA attention, GGUF reader
 * and the single-token forward pass.  TEST INFRASTRUCTURE ONLY (see
 * oracle.h).  Compiled with -ffp-contract=off: every expression rounds
 * where the reference's C rounds it.
 */
#define _DEFAULT_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ---- primitives ------------------------------------------------------- */

/* RMSNorm, sequential sum of squares.  Reference src/model.c:90-97. */
void o_rms_norm(const float *x, const float *w, float *out, int n, float eps)
{
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss = ss + x[i] * x[i];
    float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = w[i] * (x[i] * s);
}

/* In-place softmax: max, expf(x-max) with a running sum, times 1/sum.
 * Reference src/model.c:102-110. */
void o_softmax(float *x, int n)
{
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum = sum + x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* SiLU(gate)*up.  Reference src/model.c:117-123. */
void o_swiglu(const float *gate, const float *up, float *out, int n)
{
    for (int i = 0; i < n; i++) {
        float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* Adjacent-pair rotary embedding on n_heads query heads and n_kv_heads key
 * heads; theta_i = pos / powf(base, 2i/head_dim).
 * Reference src/model.c:137-166. */
void o_rope_apply(float *q, float *k, int pos, int n_heads, int n_kv_heads,
                  int head_dim, float freq_base)
{
    int half = head_dim / 2;
    for (int pass = 0; pass < 2; pass++) {
        float *base = pass ? k : q;
        int nh = pass ? n_kv_heads : n_heads;
        for (int h = 0; h < nh; h++) {
            float *v = base + (size_t)h * head_dim;
            for (int i = 0; i < half; i++) {
                float theta = (float)pos /
                    powf(freq_base, (float)(2 * i) / (float)head_dim);
                float c = cosf(theta), s = sinf(theta);
                float a = v[2 * i], b = v[2 * i + 1];
                v[2 * i] = a * c - b * s;
                v[2 * i + 1] = a * s + b * c;
            }
        }
    }
}

/* Greedy pick, first index wins ties.  Reference src/sampler.c:199-204. */
int o_argmax(const float *logits, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++) if (logits[i] > logits[best]) best = i;
    return best;
}

/* Reference src/sampler.c:171-184: one application per occurrence. */
void o_apply_repeat_penalty(float *logits, int vocab, const int32_t *tokens,
                            int n_tokens, float penalty)
{
    if (penalty <= 1.0f || !logits || !tokens || n_tokens <= 0) return;
    for (int i = 0; i < n_tokens; i++) {
        int32_t id = tokens[i];
        if (id < 0 || id >= vocab) continue;
        if (logits[id] > 0.0f) logits[id] = logits[id] / penalty;
        else logits[id] = logits[id] * penalty;
    }
}

/* Per query head h (kv head h*n_kv/n_heads): scores over t<seqlen scaled
 * by 1/sqrtf(d_head), softmax, then out_h = sum_t p_t V_t accumulated in
 * t order from zero.  Reference src/attn.c:103-137. */
void o_attention(const float *q, const float *kc, const float *vc,
                 int seqlen, int n_heads, int n_kv, int d_head,
                 float *scores, float *out)
{
    float scale = 1.0f / sqrtf((float)d_head);
    int stride = n_kv * d_head;
    memset(out, 0, (size_t)n_heads * d_head * sizeof(float));
    for (int h = 0; h < n_heads; h++) {
        int hk = h * n_kv / n_heads;
        const float *qh = q + (size_t)h * d_head;
        float *oh = out + (size_t)h * d_head;
        for (int t = 0; t < seqlen; t++) {
            const float *kt = kc + (size_t)t * stride + (size_t)hk * d_head;
            float dot = 0.0f;
            for (int i = 0; i < d_head; i++) dot = dot + qh[i] * kt[i];
            scores[t] = dot * scale;
        }
        o_softmax(scores, seqlen);
        for (int t = 0; t < seqlen; t++) {
            const float *vt = vc + (size_t)t * stride + (size_t)hk * d_head;
            float p = scores[t];
            for (int i = 0; i < d_head; i++) oh[i] = oh[i] + p * vt[i];
        }
    }
}

/* ---- GGUF reader (subset needed by the oracle) --------------------------
 * Follows reference src/gguf.c:299-518: arch-prefixed UINT32/FLOAT32 keys,
 * tensor infos, data = align32(end of infos) + offset, tied output when
 * output.weight is absent.  Only what the forward pass needs is kept. */

typedef struct {
    char name[96];
    int dtype;
    int64_t shape[4];
    const uint8_t *data;
} o_tensor_t;

typedef struct {
    const uint8_t *p;
    size_t size, pos;
    int err;
} rd_t;

static int rd_need(rd_t *r, size_t n)
{
    if (r->err || r->pos + n > r->size) { r->err = 1; return 0; }
    return 1;
}
static uint64_t rd_u(rd_t *r, int w)
{
    uint64_t v = 0;
    if (!rd_need(r, (size_t)w)) return 0;
    memcpy(&v, r->p + r->pos, (size_t)w);
    r->pos += (size_t)w;
    return v;
}
static void rd_str(rd_t *r, char *dst, size_t cap)
{
    uint64_t n = rd_u(r, 8);
    if (!rd_need(r, (size_t)n)) return;
    if (dst && cap) {
        size_t c = n < cap - 1 ? (size_t)n : cap - 1;
        memcpy(dst, r->p + r->pos, c);
        dst[c] = 0;
    }
    r->pos += (size_t)n;
}
static const int gv_width[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
static void rd_skip(rd_t *r, uint32_t t)
{
    if (t == 8) { rd_str(r, NULL, 0); return; }
    if (t == 9) {
        uint32_t et = (uint32_t)rd_u(r, 4);
        uint64_t n = rd_u(r, 8);
        for (uint64_t i = 0; i < n && !r->err; i++) rd_skip(r, et);
        return;
    }
    if (t < 13 && gv_width[t]) { if (rd_need(r, (size_t)gv_width[t])) r->pos += (size_t)gv_width[t]; }
    else r->err = 1;
}
static int key_is(const char *key, const char *arch, const char *suffix)
{
    size_t la = strlen(arch);
    return strncmp(key, arch, la) == 0 && key[la] == '.' && strcmp(key + la + 1, suffix) == 0;
}

struct o_model {
    void *map;
    size_t map_size;
    int n_layers, n_heads, n_kv, d_model, d_head, d_ffn, vocab, max_ctx;
    int nope, tie, eos;
    float rope_base, eps;
    int n_tensors;
    o_tensor_t *t;
    int order, nthreads;
    /* per-layer tensor pointers resolved once */
    o_tensor_t *embd, *out_norm, *lm_head;
    o_tensor_t **lt; /* [n_layers][11] */
};

enum { L_ATTN_NORM, L_Q, L_K, L_V, L_O, L_FFN_NORM, L_GATE, L_UP, L_DOWN, L_QN, L_KN, L_COUNT };
static const char *l_suffix[L_COUNT] = {
    "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
    "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
    "ffn_down.weight", "attn_q_norm.weight", "attn_k_norm.weight"};

static o_tensor_t *find_t(o_model_t *m, const char *name)
{
    for (int i = 0; i < m->n_tensors; i++)
        if (strcmp(m->t[i].name, name) == 0) return &m->t[i];
    return NULL;
}

o_model_t *o_model_load(const char *path, int order, int nthreads)
{
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) < 0) { close(fd); return NULL; }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return NULL;
    o_model_t *m = (o_model_t *)calloc(1, sizeof *m);
    m->map = map;
    m->map_size = (size_t)st.st_size;
    m->order = order;
    m->nthreads = nthreads > 0 ? nthreads : 1;
    m->rope_base = 10000.0f;
    m->eps = 1e-5f;
    m->eos = -1;
    rd_t r = {(const uint8_t *)map, (size_t)st.st_size, 0, 0};
    uint32_t magic = (uint32_t)rd_u(&r, 4);
    uint32_t ver = (uint32_t)rd_u(&r, 4);
    uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
    if (r.err || magic != 0x46554747u || ver < 2 || ver > 3 || nt > 65536) goto fail;
    char arch[32] = "llama";
    for (uint64_t i = 0; i < nkv && !r.err; i++) {
        char key[128];
        rd_str(&r, key, sizeof key);
        uint32_t t = (uint32_t)rd_u(&r, 4);
        if (!strcmp(key, "general.architecture") && t == 8) {
            rd_str(&r, arch, sizeof arch);
        } else if (t == 4) {
            int v = (int)(uint32_t)rd_u(&r, 4);
            if (key_is(key, arch, "context_length")) m->max_ctx = v;
            else if (key_is(key, arch, "embedding_length")) m->d_model = v;
            else if (key_is(key, arch, "block_count")) m->n_layers = v;
            else if (key_is(key, arch, "feed_forward_length")) m->d_ffn = v;
            else if (key_is(key, arch, "attention.head_count")) m->n_heads = v;
            else if (key_is(key, arch, "attention.head_count_kv")) m->n_kv = v;
            else if (key_is(key, arch, "vocab_size")) m->vocab = v;
            else if (key_is(key, arch, "attention.no_rope_layer_interval")) m->nope = v;
            else if (!strcmp(key, "tokenizer.ggml.eos_token_id")) m->eos = v;
        } else if (t == 6) {
            uint32_t u = (uint32_t)rd_u(&r, 4);
            float f;
            memcpy(&f, &u, 4);
            if (key_is(key, arch, "rope.freq_base")) m->rope_base = f;
            else if (key_is(key, arch, "attention.layer_norm_rms_epsilon")) m->eps = f;
        } else if (t == 9 && !strcmp(key, "tokenizer.ggml.tokens")) {
            uint32_t et = (uint32_t)rd_u(&r, 4);
            uint64_t n = rd_u(&r, 8);
            if (!m->vocab) m->vocab = (int)n;
            for (uint64_t j = 0; j < n && !r.err; j++) rd_skip(&r, et);
        } else {
            rd_skip(&r, t);
        }
    }
    if (r.err) goto fail;
    if (!m->n_kv) m->n_kv = m->n_heads;
    m->d_head = m->d_model / m->n_heads;
    m->n_tensors = (int)nt;
    m->t = (o_tensor_t *)calloc(nt ? nt : 1, sizeof(o_tensor_t));
    uint64_t *offs = (uint64_t *)calloc(nt ? nt : 1, 8);
    for (uint64_t i = 0; i < nt && !r.err; i++) {
        rd_str(&r, m->t[i].name, sizeof m->t[i].name);
        uint32_t nd = (uint32_t)rd_u(&r, 4);
        for (int d = 0; d < 4; d++) m->t[i].shape[d] = 1;
        for (uint32_t d = 0; d < nd && d < 4; d++) m->t[i].shape[d] = (int64_t)rd_u(&r, 8);
        m->t[i].dtype = (int)(uint32_t)rd_u(&r, 4);
        offs[i] = rd_u(&r, 8);
    }
    if (r.err) { free(offs); goto fail; }
    size_t data0 = (r.pos + 31u) & ~(size_t)31u;
    for (uint64_t i = 0; i < nt; i++) m->t[i].data = (const uint8_t *)map + data0 + offs[i];
    free(offs);
    m->embd = find_t(m, "token_embd.weight");
    m->out_norm = find_t(m, "output_norm.weight");
    m->lm_head = find_t(m, "output.weight");
    m->tie = m->lm_head == NULL;
    if (!m->lm_head) m->lm_head = m->embd;
    m->lt = (o_tensor_t **)calloc((size_t)m->n_layers * L_COUNT, sizeof(o_tensor_t *));
    for (int l = 0; l < m->n_layers; l++)
        for (int j = 0; j < L_COUNT; j++) {
            char nm[96];
            snprintf(nm, sizeof nm, "blk.%d.%s", l, l_suffix[j]);
            m->lt[l * L_COUNT + j] = find_t(m, nm);
        }
    return m;
fail:
    munmap(map, (size_t)st.st_size);
    free(m->t);
    free(m);
    return NULL;
}

void o_model_free(o_model_t *m)
{
    if (!m) return;
    munmap(m->map, m->map_size);
    free(m->t);
    free(m->lt);
    free(m);
}

void o_model_hparams(const o_model_t *m, int32_t o[11], float f[2])
{
    o[0] = m->n_layers; o[1] = m->n_heads; o[2] = m->n_kv; o[3] = m->d_model;
    o[4] = m->d_head; o[5] = m->d_ffn; o[6] = m->vocab; o[7] = m->max_ctx;
    o[8] = m->nope; o[9] = m->tie; o[10] = m->eos;
    f[0] = m->rope_base; f[1] = m->eps;
}

/* ---- threaded matmul (row split; per-output order unchanged) ------------ */
typedef struct {
    float *out; const void *a; const float *b;
    int m0, m1, k, dtype, order;
} mm_job_t;

static void *mm_run(void *p)
{
    mm_job_t *j = (mm_job_t *)p;
    size_t rb = o_row_bytes(j->k, j->dtype);
    o_matmul(j->out + j->m0, (const uint8_t *)j->a + rb * (size_t)j->m0, j->b,
             j->m1 - j->m0, j->k, 1, j->dtype, j->order);
    return NULL;
}

static void mm(o_model_t *m, float *out, const o_tensor_t *t, const float *x, int rows, int k)
{
    int nt = m->nthreads;
    if (nt <= 1 || rows < 256) {
        o_matmul(out, t->data, x, rows, k, 1, t->dtype, m->order);
        return;
    }
    if (nt > 64) nt = 64;
    pthread_t th[64];
    mm_job_t jb[64];
    int per = (rows + nt - 1) / nt;
    int used = 0;
    for (int i = 0; i < nt; i++) {
        int a = i * per, b = a + per > rows ? rows : a + per;
        if (a >= b) break;
        jb[i] = (mm_job_t){out, t->data, x, a, b, k, t->dtype, m->order};
        pthread_create(&th[i], NULL, mm_run, &jb[i]);
        used++;
    }
    for (int i = 0; i < used; i++) pthread_join(th[i], NULL);
}

/* ---- session + forward -------------------------------------------------- */
struct o_sess {
    o_model_t *m;
    int max_ctx;
    int kv_f16;              /* round K/V to fp16 on write */
    float *k, *v;            /* [L][max_ctx][n_kv][d_head] */
    float *x, *xn, *q, *kb, *vb, *sc, *ao, *g, *u, *logits;
};

o_sess_t *o_sess_new(o_model_t *m, int max_ctx)
{
    o_sess_t *s = (o_sess_t *)calloc(1, sizeof *s);
    size_t kvn = (size_t)m->n_layers * max_ctx * m->n_kv * m->d_head;
    s->m = m;
    s->max_ctx = max_ctx;
    s->k = (float *)calloc(kvn ? kvn : 1, 4);
    s->v = (float *)calloc(kvn ? kvn : 1, 4);
    int d = m->d_model, kv = m->n_kv * m->d_head;
    s->x = (float *)calloc((size_t)d, 4);
    s->xn = (float *)calloc((size_t)d, 4);
    s->q = (float *)calloc((size_t)d, 4);
    s->kb = (float *)calloc((size_t)kv, 4);
    s->vb = (float *)calloc((size_t)kv, 4);
    s->sc = (float *)calloc((size_t)max_ctx, 4);
    s->ao = (float *)calloc((size_t)d, 4);
    s->g = (float *)calloc((size_t)m->d_ffn, 4);
    s->u = (float *)calloc((size_t)m->d_ffn, 4);
    s->logits = (float *)calloc((size_t)m->vocab, 4);
    if (!s->k || !s->v) { o_sess_free(s); return NULL; }
    return s;
}

void o_sess_free(o_sess_t *s)
{
    if (!s) return;
    free(s->k); free(s->v); free(s->x); free(s->xn); free(s->q); free(s->kb);
    free(s->vb); free(s->sc); free(s->ao); free(s->g); free(s->u); free(s->logits);
    free(s);
}

void o_sess_kv_f16(o_sess_t *s, int on) { s->kv_f16 = on != 0; }

float *o_sess_k(o_sess_t *s) { return s->k; }
float *o_sess_v(o_sess_t *s) { return s->v; }
const float *o_sess_logits(o_sess_t *s) { return s->logits; }

/* One token through embedding, L x (norm, attention, residual, norm,
 * SwiGLU FFN, residual), final norm and LM head.
 * Reference src/model.c:176-276 and src/attn.c:27-146. */
const float *o_forward(o_model_t *m, o_sess_t *s, int32_t token, int pos)
{
    if (pos < 0 || pos >= s->max_ctx || token < 0 || token >= m->vocab) return NULL;
    int d = m->d_model, dh = m->d_head, nkv = m->n_kv, nh = m->n_heads;
    int kvd = nkv * dh, ffn = m->d_ffn;
    o_dequant_row(m->embd->data + o_row_bytes(d, m->embd->dtype) * (size_t)token,
                  s->x, d, m->embd->dtype);
    for (int l = 0; l < m->n_layers; l++) {
        o_tensor_t **t = m->lt + (size_t)l * L_COUNT;
        o_rms_norm(s->x, (const float *)t[L_ATTN_NORM]->data, s->xn, d, m->eps);
        mm(m, s->q, t[L_Q], s->xn, d, d);
        mm(m, s->kb, t[L_K], s->xn, kvd, d);
        mm(m, s->vb, t[L_V], s->xn, kvd, d);
        if (t[L_QN])
            for (int h = 0; h < nh; h++)
                o_rms_norm(s->q + h * dh, (const float *)t[L_QN]->data, s->q + h * dh, dh, m->eps);
        if (t[L_KN])
            for (int h = 0; h < nkv; h++)
                o_rms_norm(s->kb + h * dh, (const float *)t[L_KN]->data, s->kb + h * dh, dh, m->eps);
        int nope = m->nope > 0 && (l + 1) % m->nope == 0;
        if (!nope) o_rope_apply(s->q, s->kb, pos, nh, nkv, dh, m->rope_base);
        float *kc = s->k + (size_t)l * s->max_ctx * kvd;
        float *vc = s->v + (size_t)l * s->max_ctx * kvd;
        memcpy(kc + (size_t)pos * kvd, s->kb, (size_t)kvd * 4);
        memcpy(vc + (size_t)pos * kvd, s->vb, (size_t)kvd * 4);
        if (s->kv_f16)
            for (int i = 0; i < kvd; i++) {
                kc[(size_t)pos * kvd + i] = o_f16_to_f32(o_f32_to_f16(s->kb[i]));
                vc[(size_t)pos * kvd + i] = o_f16_to_f32(o_f32_to_f16(s->vb[i]));
            }
        o_attention(s->q, kc, vc, pos + 1, nh, nkv, dh, s->sc, s->ao);
        memcpy(s->q, s->ao, (size_t)d * 4);
        mm(m, s->ao, t[L_O], s->q, d, d);
        for (int i = 0; i < d; i++) s->x[i] = s->x[i] + s->ao[i];
        o_rms_norm(s->x, (const float *)t[L_FFN_NORM]->data, s->xn, d, m->eps);
        mm(m, s->g, t[L_GATE], s->xn, ffn, d);
        mm(m, s->u, t[L_UP], s->xn, ffn, d);
        o_swiglu(s->g, s->u, s->g, ffn);
        mm(m, s->ao, t[L_DOWN], s->g, d, ffn);
        for (int i = 0; i < d; i++) s->x[i] = s->x[i] + s->ao[i];
    }
    o_rms_norm(s->x, (const float *)m->out_norm->data, s->xn, d, m->eps);
    mm(m, s->logits, m->lm_head, s->xn, m->vocab, d);
    return s->logits;
}

static float top2_margin(const float *lg, int n)
{
    float a = -INFINITY, b = -INFINITY;
    for (int i = 0; i < n; i++) {
        if (lg[i] > a) { b = a; a = lg[i]; }
        else if (lg[i] > b) b = lg[i];
    }
    return a - b;
}

/* Token-by-token prefill then greedy decode with the optional repetition
 * penalty ring; stops early on EOS.  Reference src/api.c:443-521. */
int o_generate_greedy(o_model_t *m, o_sess_t *s, const int32_t *prompt,
                      int n_prompt, int pos0, int n_new, float penalty,
                      int last_n, int32_t *out_tokens, float *margins)
{
    int pos = pos0;
    const float *lg = NULL;
    for (int i = 0; i < n_prompt; i++) {
        lg = o_forward(m, s, prompt[i], pos++);
        if (!lg) return -1;
    }
    if (!lg) return -1;
    enum { RB = 128 };
    int32_t ring[RB];
    int head = 0, fill = 0;
    if (last_n <= 0 || last_n > RB) last_n = RB;
    int seed_n = n_prompt < last_n ? n_prompt : last_n;
    for (int i = 0; i < seed_n; i++) ring[i] = prompt[n_prompt - seed_n + i];
    head = seed_n % RB;
    fill = seed_n;
    int produced = 0;
    for (;;) {
        float *lgw = s->logits;
        if (penalty > 1.0f && fill > 0) o_apply_repeat_penalty(lgw, m->vocab, ring, fill, penalty);
        if (margins) margins[produced] = top2_margin(lgw, m->vocab);
        int32_t next = o_argmax(lgw, m->vocab);
        out_tokens[produced++] = next;
        if (m->eos >= 0 && next == m->eos) break;
        ring[head] = next;
        head = (head + 1) % RB;
        if (fill < RB) fill++;
        if (produced >= n_new) break;
        if (pos >= s->max_ctx) break;
        if (!o_forward(m, s, next, pos++)) return -1;
    }
    return produced;
}
