/*
 * api.c — public API of libcmol (MI355X build) and the internal harness
 * entry points (include/cmol_ext.h).
 *
 * Host side of the drop-in: loads and validates the GGUF exactly as the
 * reference does (src/api.c:139-291), keeps its single host allocation, its
 * 32-slot mutex-guarded session pool (src/api.c:309-334) and its generate
 * loop (src/api.c:412-524), and hands the forward pass to the gfx950 backend
 * (include/cmol_hip.h): weights, KV caches and activations are placed in one
 * device arena inside cmol_load; nothing is allocated after cmol_load.
 */
#ifndef _DEFAULT_SOURCE
#define _DEFAULT_SOURCE
#endif
#include "internal.h"
#include "../../../include/cmol_ext.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

const char *cmol_strerror(cmol_err_t err)
{
    switch (err) {
    case CMOL_OK: return "success";
    case CMOL_ERR_OOM: return "out of memory";
    case CMOL_ERR_IO: return "I/O error";
    case CMOL_ERR_INVALID: return "invalid or corrupt GGUF file";
    case CMOL_ERR_UNSUPPORTED: return "unsupported quantisation type or architecture";
    case CMOL_ERR_NO_SESSION: return "session pool exhausted — retry later";
    case CMOL_ERR_ARGS: return "invalid argument (NULL or out of range)";
    case CMOL_ERR_CTX_FULL: return "KV cache full — call cmol_session_reset()";
    case CMOL_ERR_TRUNC: return "output buffer too small (result truncated)";
    default: return "unknown error";
    }
}

const char *cmol_version(void) { return CMOL_VERSION_STRING; }

void cmol_log(const cmol_model_t *m, int level, const char *fmt, ...)
{
    if (!m || !m->cfg.log_fn) return;
    char buf[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    m->cfg.log_fn(level, buf, m->cfg.log_ud);
}

/* ---- configuration and sizing ------------------------------------------- */

static void resolve_cfg(cmol_config_t *c, const cmol_hparams_t *hp)
{
    /* reference src/api.c:155-160 */
    if (c->max_ctx <= 0 || c->max_ctx > hp->model_max_ctx) c->max_ctx = hp->model_max_ctx;
    if (c->max_sessions <= 0) c->max_sessions = 4;
    if (c->max_sessions > CMOL_MAX_SESSIONS) c->max_sessions = CMOL_MAX_SESSIONS;
    if (c->prefill_chunk <= 0) c->prefill_chunk = 512;
}

/* Host arena: tensor descriptors, tokenizer tables, session structs, per
 * session logits + token buffer, the layer table and RoPE table handed to
 * the device backend at load. */
static size_t host_arena_size(const cmol_hparams_t *hp, const cmol_config_t *c, size_t n_tensors)
{
    size_t s = n_tensors * sizeof(cmol_tensor_t);
    s += cmol_tokenizer_arena_bytes(hp->vocab_size, 0) + ((size_t)1 << 20);
    s += (size_t)c->max_sessions * sizeof(struct cmol_session);
    s += (size_t)c->max_sessions * ((size_t)hp->vocab_size * 4 + (size_t)c->max_ctx * 4);
    s += (size_t)(hp->n_layers > 0 ? hp->n_layers : 0) * sizeof(cmolhip_layer_tensors_t);
    s += (size_t)c->max_ctx * (size_t)(hp->d_head > 0 ? hp->d_head : 0) * 4;
    s += (size_t)(c->max_sessions + 16) * 64 + 4096;
    return s;
}

static int env_kv_f16(void)
{
    const char *e = getenv("CMOL_KV_F16");
    return e && e[0] == '1';
}

/* Cross-session batching of concurrent decode steps (sched.c): on unless
 * CMOL_BATCH=0; CMOL_BATCH_WAIT_US sets how long a posted step waits for the
 * other active sessions (default 2000 µs, about one decode step of a 3B
 * model). */
static int env_batch(void)
{
    const char *e = getenv("CMOL_BATCH");
    return !(e && e[0] == '0');
}

static long env_batch_wait_us(void)
{
    const char *e = getenv("CMOL_BATCH_WAIT_US");
    long v = e ? atol(e) : 2000;
    return v < 0 ? 0 : v > 1000000 ? 1000000 : v;
}

/* The scheduler's batch: one session through its own decode graph, more as
 * one lock-step batch (each session's logits to its own buffer). */
static int run_steps(void *ctx, cmol_step_t *const *st, int n)
{
    cmol_model_t *m = (cmol_model_t *)ctx;
    int rc;
    if (n == 1) {
        int32_t next = 0;
        rc = cmolhip_decode(m->dev, st[0]->slot, st[0]->token, st[0]->pos, st[0]->logits, &next);
        st[0]->next = next;
        st[0]->rc = rc;
        return rc;
    }
    int32_t slots[CMOL_MAX_SESSIONS] = {0}, tokens[CMOL_MAX_SESSIONS] = {0}, pos[CMOL_MAX_SESSIONS] = {0},
            next[CMOL_MAX_SESSIONS] = {0};
    float *lg[CMOL_MAX_SESSIONS] = {0};
    for (int i = 0; i < n; i++) {
        slots[i] = st[i]->slot;
        tokens[i] = st[i]->token;
        pos[i] = st[i]->pos;
        lg[i] = st[i]->logits;
    }
    rc = cmolhip_decode_batch_each(m->dev, n, slots, tokens, pos, lg, next);
    for (int i = 0; i < n; i++) {
        st[i]->next = rc ? 0 : next[i];
        st[i]->rc = rc;
    }
    return rc;
}

static cmolhip_host_tensor_t host_tensor(const cmol_tensor_t *t)
{
    cmolhip_host_tensor_t h;
    memset(&h, 0, sizeof h);
    if (!t) return h;
    h.data = t->data;
    h.dtype = (int32_t)t->dtype;
    h.cols = (int32_t)t->shape[0];
    h.rows = (int32_t)(t->n_dims > 1 ? t->shape[1] : 1);
    return h;
}

static cmol_tensor_t *blk(cmol_model_t *m, int l, const char *suffix)
{
    char nm[CMOL_MAX_TENSOR_NAME];
    snprintf(nm, sizeof nm, "blk.%d.%s", l, suffix);
    return cmol_gguf_find_tensor(m->tensors, m->n_tensors, nm);
}

/* Fill the device description from the parsed GGUF.  The RoPE table is
 * computed with the host libm exactly as the reference computes each angle
 * (src/model.c:146-148): theta = pos / powf(base, 2i/d_head). */
static cmol_err_t make_desc(cmol_model_t *m, cmolhip_model_desc_t *d, cmol_arena_t *a)
{
    const cmol_hparams_t *hp = &m->hparams;
    memset(d, 0, sizeof *d);
    if (hp->n_layers < 1 || hp->n_heads < 1 || hp->d_model < 1 || hp->vocab_size < 1)
        return CMOL_ERR_INVALID;
    d->hp.n_layers = hp->n_layers;
    d->hp.n_heads = hp->n_heads;
    d->hp.n_kv_heads = hp->n_kv_heads;
    d->hp.d_model = hp->d_model;
    d->hp.d_head = hp->d_head;
    d->hp.d_ffn = hp->d_ffn;
    d->hp.vocab = hp->vocab_size;
    d->hp.max_ctx = m->cfg.max_ctx;
    d->hp.max_sessions = m->cfg.max_sessions;
    d->hp.no_rope_interval = hp->no_rope_layer_interval;
    d->hp.kv_f16 = m->kv_f16;
    d->hp.prefill_chunk = m->cfg.prefill_chunk;
    d->hp.rope_base = hp->rope_freq_base;
    d->hp.rms_eps = hp->rms_norm_eps;
    cmol_tensor_t *embd = cmol_gguf_find_tensor(m->tensors, m->n_tensors, "token_embd.weight");
    cmol_tensor_t *onorm = cmol_gguf_find_tensor(m->tensors, m->n_tensors, "output_norm.weight");
    cmol_tensor_t *out = cmol_gguf_find_tensor(m->tensors, m->n_tensors, "output.weight");
    if (!embd || !onorm) return CMOL_ERR_INVALID;
    d->embd = host_tensor(embd);
    d->out_norm = host_tensor(onorm);
    d->lm_head = host_tensor(out);
    cmolhip_layer_tensors_t *L = (cmolhip_layer_tensors_t *)cmol_arena_alloc_n(
        a, (size_t)hp->n_layers, sizeof(cmolhip_layer_tensors_t));
    if (!L) return CMOL_ERR_OOM;
    for (int l = 0; l < hp->n_layers; l++) {
        L[l].attn_norm = host_tensor(blk(m, l, "attn_norm.weight"));
        L[l].q = host_tensor(blk(m, l, "attn_q.weight"));
        L[l].k = host_tensor(blk(m, l, "attn_k.weight"));
        L[l].v = host_tensor(blk(m, l, "attn_v.weight"));
        L[l].o = host_tensor(blk(m, l, "attn_output.weight"));
        L[l].q_norm = host_tensor(blk(m, l, "attn_q_norm.weight"));
        L[l].k_norm = host_tensor(blk(m, l, "attn_k_norm.weight"));
        L[l].ffn_norm = host_tensor(blk(m, l, "ffn_norm.weight"));
        L[l].gate = host_tensor(blk(m, l, "ffn_gate.weight"));
        L[l].up = host_tensor(blk(m, l, "ffn_up.weight"));
        L[l].down = host_tensor(blk(m, l, "ffn_down.weight"));
    }
    d->layers = L;
    const int half = hp->d_head / 2, ctx = m->cfg.max_ctx;
    float *rope = (float *)cmol_arena_alloc_n(a, (size_t)ctx * (size_t)(half > 0 ? half : 1) * 2, 4);
    if (!rope) return CMOL_ERR_OOM;
    for (int pos = 0; pos < ctx; pos++)
        for (int i = 0; i < half; i++) {
            float theta = (float)pos / powf(hp->rope_freq_base, (float)(2 * i) / (float)hp->d_head);
            rope[((size_t)pos * half + i) * 2 + 0] = cosf(theta);
            rope[((size_t)pos * half + i) * 2 + 1] = sinf(theta);
        }
    d->rope_table = rope;
    return CMOL_OK;
}

size_t cmol_arena_estimate(const char *path, const cmol_config_t *cfg)
{
    static const cmol_config_t def = CMOL_DEFAULT_CONFIG;
    if (!path) return 0;
    if (!cfg) cfg = &def;
    cmol_hparams_t hp;
    size_t nt;
    if (cmol_gguf_peek(path, &hp, &nt) != CMOL_OK) return 0;
    cmol_config_t c = *cfg;
    resolve_cfg(&c, &hp);
    size_t host = sizeof(struct cmol_model) + host_arena_size(&hp, &c, nt);
    /* device arena: needs the tensor table, so parse into a scratch arena */
    size_t dev = 0;
    uint8_t *buf = (uint8_t *)malloc(host);
    if (buf) {
        cmol_model_t *m = (cmol_model_t *)calloc(1, sizeof *m);
        if (m) {
            m->cfg = c;
            m->kv_f16 = env_kv_f16();
            cmol_arena_init(&m->arena, buf, host);
            if (cmol_mmap_open(path, &m->mmap) == CMOL_OK) {
                cmolhip_model_desc_t d;
                if (cmol_gguf_parse(&m->mmap, &m->arena, &m->hparams, &m->tensors, &m->n_tensors,
                                    &m->tokenizer) == CMOL_OK &&
                    make_desc(m, &d, &m->arena) == CMOL_OK)
                    (void)cmolhip_model_plan(&d, &dev);
                cmol_mmap_close(&m->mmap);
            }
            free(m);
        }
        free(buf);
    }
    return host + dev;
}

/* ---- load / free --------------------------------------------------------- */

/* The load of cmol_load; with_device 0 stops after the tokenizer (no
 * sessions, no device), for cmol__load_text. */
static cmol_model_t *load_model(const char *path, const cmol_config_t *cfg, cmol_err_t *err, int with_device)
{
    static const cmol_config_t def = CMOL_DEFAULT_CONFIG;
    cmol_err_t rc;
    if (err) *err = CMOL_OK;
    if (!path) { if (err) *err = CMOL_ERR_ARGS; return NULL; }
    if (!cfg) cfg = &def;
    cmol_hparams_t hp;
    size_t nt;
    rc = cmol_gguf_peek(path, &hp, &nt);
    if (rc != CMOL_OK) { if (err) *err = rc; return NULL; }
    cmol_config_t c = *cfg;
    resolve_cfg(&c, &hp);
    if (c.max_ctx <= 0) { if (err) *err = CMOL_ERR_INVALID; return NULL; }

    const size_t hdr = (sizeof(struct cmol_model) + 63u) & ~(size_t)63u;
    const size_t need = host_arena_size(&hp, &c, nt);
    uint8_t *buf = (uint8_t *)malloc(hdr + need); /* the only host allocation */
    if (!buf) { if (err) *err = CMOL_ERR_OOM; return NULL; }
    memset(buf, 0, hdr + need);
    cmol_model_t *m = (cmol_model_t *)(void *)buf;
    m->arena_buf = buf;
    cmol_arena_init(&m->arena, buf + hdr, need);
    m->cfg = c;
    m->kv_f16 = env_kv_f16();
#define FAIL(code)                            \
    do {                                      \
        if (m->dev) cmolhip_model_destroy(m->dev); \
        cmol_mmap_close(&m->mmap);            \
        free(buf);                            \
        if (err) *err = (code);               \
        return NULL;                          \
    } while (0)
    rc = cmol_mmap_open(path, &m->mmap);
    if (rc != CMOL_OK) FAIL(rc);
    rc = cmol_gguf_parse(&m->mmap, &m->arena, &m->hparams, &m->tensors, &m->n_tensors, &m->tokenizer);
    if (rc != CMOL_OK) FAIL(rc);
    rc = cmol_tokenizer_build(&m->tokenizer, &m->arena);
    if (rc != CMOL_OK) FAIL(rc);
    if (!with_device) {
        if (pthread_mutex_init(&m->pool_lock, NULL) != 0) FAIL(CMOL_ERR_OOM);
        return m;
    }
    m->session_slots = (struct cmol_session *)cmol_arena_alloc_n(&m->arena, (size_t)c.max_sessions,
                                                                 sizeof(struct cmol_session));
    if (!m->session_slots) FAIL(CMOL_ERR_OOM);
    for (int i = 0; i < c.max_sessions; i++) {
        struct cmol_session *s = &m->session_slots[i];
        s->model = m;
        s->slot = i;
        s->max_tokens = c.max_ctx;
        s->n_tokens = 0;
        s->logits = (float *)cmol_arena_alloc_n(&m->arena, (size_t)m->hparams.vocab_size, 4);
        s->token_buf = (int32_t *)cmol_arena_alloc_n(&m->arena, (size_t)c.max_ctx, 4);
        s->token_buf_cap = c.max_ctx;
        if (!s->logits || !s->token_buf) FAIL(CMOL_ERR_OOM);
    }
    cmolhip_model_desc_t desc;
    rc = make_desc(m, &desc, &m->arena);
    if (rc != CMOL_OK) FAIL(rc);
    int drc = cmolhip_model_create(&desc, 0, &m->dev);
    if (drc != 0) {
        m->dev = NULL;
        FAIL((cmol_err_t)drc);
    }
    m->pool_free = c.max_sessions == 32 ? 0xFFFFFFFFu : (1u << c.max_sessions) - 1u;
    if (pthread_mutex_init(&m->pool_lock, NULL) != 0) FAIL(CMOL_ERR_OOM);
    cmol_sampler_pool_start();   /* the sampler's threads exist before the first draw */
    m->sampler_held = 1;
    if (c.max_sessions > 1 && env_batch()) {
        if (cmol_sched_init(&m->sched, run_steps, m, env_batch_wait_us()) != CMOL_OK) {
            pthread_mutex_destroy(&m->pool_lock);
            cmol_sampler_pool_stop();
            FAIL(CMOL_ERR_OOM);
        }
        m->sched_on = 1;
    }
#undef FAIL
    cmol_log(m, CMOL_LOG_INFO,
             "cmol_load: arch=%s layers=%d heads=%d/%d d=%d ffn=%d vocab=%d ctx=%d sessions=%d "
             "backend=gfx950 kv=%s device_arena=%zu",
             m->hparams.arch, m->hparams.n_layers, m->hparams.n_heads, m->hparams.n_kv_heads,
             m->hparams.d_model, m->hparams.d_ffn, m->hparams.vocab_size, c.max_ctx,
             c.max_sessions, m->kv_f16 ? "f16" : "f32",
             cmolhip_arena_size(cmolhip_model_ctx(m->dev)));
    return m;
}

cmol_model_t *cmol_load(const char *path, const cmol_config_t *cfg, cmol_err_t *err)
{
    return load_model(path, cfg, err, 1);
}

cmol_model_t *cmol__load_text(const char *path, cmol_err_t *err)
{
    return load_model(path, NULL, err, 0);
}

void cmol_free(cmol_model_t *m)
{
    if (!m) return;
    pthread_mutex_destroy(&m->pool_lock);
    if (m->sched_on) cmol_sched_destroy(&m->sched);
    if (m->sampler_held) cmol_sampler_pool_stop();
    cmolhip_model_destroy(m->dev);
    cmol_mmap_close(&m->mmap);
    free(m->arena_buf);
}

/* ---- session pool (reference src/api.c:309-334) ------------------------- */

cmol_session_t *cmol_session_acquire(cmol_model_t *m)
{
    if (!m) return NULL;
    pthread_mutex_lock(&m->pool_lock);
    if (!m->pool_free) {
        pthread_mutex_unlock(&m->pool_lock);
        return NULL;
    }
    int slot = __builtin_ctz(m->pool_free);
    m->pool_free &= ~(1u << slot);
    pthread_mutex_unlock(&m->pool_lock);
    return &m->session_slots[slot];
}

void cmol_session_release(cmol_session_t *s)
{
    if (!s) return;
    cmol_model_t *m = s->model;
    pthread_mutex_lock(&m->pool_lock);
    m->pool_free |= 1u << s->slot;
    pthread_mutex_unlock(&m->pool_lock);
}

void cmol_session_reset(cmol_session_t *s)
{
    if (!s) return;
    s->n_tokens = 0;
}

/* ---- tokenizer wrappers ---------------------------------------------------- */

int cmol_encode(cmol_model_t *m, const char *text, int32_t *out, int out_cap)
{
    if (!m || !text || !out || out_cap <= 0) return CMOL_ERR_ARGS;
    return cmol_tokenizer_encode(&m->tokenizer, text, out, out_cap, m->tokenizer.add_bos);
}

const char *cmol_decode_token(cmol_model_t *m, int32_t id)
{
    if (!m) return NULL;
    return cmol_tokenizer_decode_token(&m->tokenizer, id);
}

/* ---- ChatML helpers (reference src/api.c:356-398) -------------------------- */

int cmol_format_chatml(const char *system, const char *user, char *buf, size_t cap)
{
    if (!user) return (int)CMOL_ERR_ARGS;
    const char *sys = system ? system : "";
    int n = sys[0] ? snprintf(buf, cap,
                              "<|im_start|>system\n%s<|im_end|>\n<|im_start|>user\n%s<|im_end|>\n"
                              "<|im_start|>assistant\n",
                              sys, user)
                   : snprintf(buf, cap, "<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n",
                              user);
    if (n < 0) return (int)CMOL_ERR_ARGS;
    if (buf && cap > 0 && (size_t)n >= cap) return (int)CMOL_ERR_TRUNC;
    return n;
}

int cmol_format_chatml_turn(const char *user, char *buf, size_t cap)
{
    if (!user) return (int)CMOL_ERR_ARGS;
    int n = snprintf(buf, cap, "<|im_end|>\n<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n",
                     user);
    if (n < 0) return (int)CMOL_ERR_ARGS;
    if (buf && cap > 0 && (size_t)n >= cap) return (int)CMOL_ERR_TRUNC;
    return n;
}

/* ---- generation ------------------------------------------------------------ */

/* Device-side selection is exact for greedy without penalty: the argmax over
 * the logits is taken in the LM-head kernel.  Any other parameters need the
 * logits on the host (penalty and sampling run on the host). */
static int wants_host_logits(const cmol_gen_params_t *p)
{
    return !(p->temperature == 0.0f && !(p->repeat_penalty > 1.0f));
}

typedef int (*emit_fn)(void *ud, int32_t id, int is_eos);

/* The generate loop shared by cmol_generate (text) and cmol__generate_ids.
 * Order of operations follows reference src/api.c:443-521. */
static cmol_err_t generate_core(cmol_session_t *s, int n_prompt, const cmol_gen_params_t *params,
                                emit_fn emit, void *ud)
{
    cmol_model_t *m = s->model;
    const int V = m->hparams.vocab_size;
    const int host_logits = wants_host_logits(params);
    int avail = s->max_tokens - s->n_tokens;
    if (n_prompt > avail) n_prompt = avail;
    int pos = s->n_tokens;
    int32_t dev_next = 0;
    int drc;
    /* A caller joins the scheduler's batches once its prompt is in (a long
     * prompt pass would hold the others' steps); a one-token prompt is a
     * decode step and joins at once. */
    const int batch_prompt = m->sched_on && n_prompt == 1;
    if (batch_prompt) {
        cmol_sched_enter(&m->sched);
        cmol_step_t st = {s->slot, s->token_buf[0], pos, host_logits ? s->logits : NULL, 0, 0, 0};
        drc = cmol_sched_step(&m->sched, &st);
        dev_next = st.next;
        if (drc != 0) cmol_sched_leave(&m->sched);
    } else {
        drc = cmolhip_prefill(m->dev, s->slot, s->token_buf, n_prompt, pos, host_logits ? s->logits : NULL,
                              &dev_next);
    }
    if (drc != 0) return (cmol_err_t)drc;
    pos += n_prompt;
    s->n_tokens = pos;

    int max_new = params->max_new_tokens;
    if (max_new < 0) max_new = s->max_tokens;
    uint64_t rng[4];
    cmol_rng_seed(rng, params->seed);
    int32_t ring[CMOL_REPEAT_BUF];
    int head, fill;
    {
        int last_n = params->repeat_last_n;
        if (last_n <= 0 || last_n > CMOL_REPEAT_BUF) last_n = CMOL_REPEAT_BUF;
        int seed_n = n_prompt < last_n ? n_prompt : last_n;
        for (int i = 0; i < seed_n; i++) ring[i] = s->token_buf[n_prompt - seed_n + i];
        head = seed_n % CMOL_REPEAT_BUF;
        fill = seed_n;
    }
    int produced = 0;
    cmol_err_t out = CMOL_OK;
    if (m->sched_on && !batch_prompt) cmol_sched_enter(&m->sched);
    for (;;) {
        int32_t next;
        if (host_logits) {
            if (params->repeat_penalty > 1.0f && fill > 0)
                cmol_apply_repeat_penalty(s->logits, V, ring, fill, params->repeat_penalty);
            next = cmol_sample(s->logits, V, params, rng);
        } else {
            next = dev_next;
        }
        int is_eos = m->tokenizer.eos_id >= 0 && next == m->tokenizer.eos_id;
        if (emit(ud, next, is_eos)) break;
        if (is_eos) break;
        ring[head] = next;
        head = (head + 1) % CMOL_REPEAT_BUF;
        if (fill < CMOL_REPEAT_BUF) fill++;
        produced++;
        if (max_new > 0 && produced >= max_new) break;
        if (pos >= s->max_tokens) break;
        if (m->sched_on) {   /* batched with the other sessions' steps */
            cmol_step_t st = {s->slot, next, pos, host_logits ? s->logits : NULL, 0, 0, 0};
            drc = cmol_sched_step(&m->sched, &st);
            dev_next = st.next;
        } else {
            drc = cmolhip_decode(m->dev, s->slot, next, pos, host_logits ? s->logits : NULL, &dev_next);
        }
        if (drc != 0) {
            out = (cmol_err_t)drc;
            break;
        }
        pos++;
        s->n_tokens = pos;
    }
    if (m->sched_on) cmol_sched_leave(&m->sched);
    return out;
}

typedef struct {
    cmol_model_t *m;
    cmol_token_cb_t cb;
    void *ud;
} text_emit_t;

static int emit_text(void *ud, int32_t id, int is_eos)
{
    text_emit_t *t = (text_emit_t *)ud;
    if (!t->cb) return 0;
    const char *piece = cmol_tokenizer_decode_token(&t->m->tokenizer, id);
    return t->cb(piece ? piece : "", piece ? strlen(piece) : 0, is_eos, t->ud);
}

cmol_err_t cmol_generate(cmol_session_t *s, const char *prompt, const cmol_gen_params_t *params,
                         cmol_token_cb_t on_token, void *userdata)
{
    static const cmol_gen_params_t def = CMOL_DEFAULT_PARAMS;
    if (!s || !prompt) return CMOL_ERR_ARGS;
    if (!params) params = &def;
    cmol_model_t *m = s->model;
    if (s->n_tokens >= s->max_tokens) return CMOL_ERR_CTX_FULL;
    int n = cmol_tokenizer_encode(&m->tokenizer, prompt, s->token_buf, s->token_buf_cap,
                                  m->tokenizer.add_bos);
    if (n < 0) return (cmol_err_t)n;
    if (n == 0) return CMOL_OK;
    text_emit_t t = {m, on_token, userdata};
    return generate_core(s, n, params, emit_text, &t);
}

/* ---- internal entry points ------------------------------------------------- */

typedef struct {
    int32_t *out;
    int cap, n;
} id_emit_t;

static int emit_id(void *ud, int32_t id, int is_eos)
{
    (void)is_eos;
    id_emit_t *e = (id_emit_t *)ud;
    if (e->n < e->cap) e->out[e->n] = id;
    e->n++;
    return e->n >= e->cap;   /* stop when the caller's buffer is full */
}

int cmol__generate_ids(cmol_session_t *s, const int32_t *prompt, int n_prompt,
                       const cmol_gen_params_t *params, int32_t *out, int out_cap)
{
    static const cmol_gen_params_t def = CMOL_DEFAULT_PARAMS;
    if (!s || !prompt || n_prompt < 1 || !out || out_cap < 1) return CMOL_ERR_ARGS;
    if (!params) params = &def;
    if (s->n_tokens >= s->max_tokens) return CMOL_ERR_CTX_FULL;
    if (n_prompt > s->token_buf_cap) n_prompt = s->token_buf_cap;
    for (int i = 0; i < n_prompt; i++) {
        if (prompt[i] < 0 || prompt[i] >= s->model->hparams.vocab_size) return CMOL_ERR_ARGS;
        s->token_buf[i] = prompt[i];
    }
    id_emit_t e = {out, out_cap, 0};
    cmol_err_t rc = generate_core(s, n_prompt, params, emit_id, &e);
    return rc == CMOL_OK ? (e.n < out_cap ? e.n : out_cap) : rc;
}

int cmol__forward(cmol_session_t *s, int32_t token, int pos, float *logits_out)
{
    if (!s) return CMOL_ERR_ARGS;
    int32_t next = 0;
    int rc = cmolhip_decode(s->model->dev, s->slot, token, pos, logits_out, &next);
    return rc ? rc : next;
}

int cmol__prefill(cmol_session_t *s, const int32_t *tokens, int n, float *logits_out)
{
    if (!s || !tokens || n < 1) return CMOL_ERR_ARGS;
    if (s->n_tokens + n > s->max_tokens) return CMOL_ERR_CTX_FULL;
    int32_t next = 0;
    int rc = cmolhip_prefill(s->model->dev, s->slot, tokens, n, s->n_tokens, logits_out, &next);
    if (rc) return rc;
    s->n_tokens += n;
    return next;
}

int cmol__decode_batch(cmol_session_t *const *ss, const int32_t *tokens, int n, int32_t *next)
{
    if (!ss || !tokens || !next || n < 1 || n > CMOL_MAX_SESSIONS) return CMOL_ERR_ARGS;
    cmol_model_t *m = ss[0] ? ss[0]->model : NULL;
    if (!m) return CMOL_ERR_ARGS;
    int32_t slots[CMOL_MAX_SESSIONS], pos[CMOL_MAX_SESSIONS];
    for (int i = 0; i < n; i++) {
        if (!ss[i] || ss[i]->model != m) return CMOL_ERR_ARGS;
        if (ss[i]->n_tokens >= ss[i]->max_tokens) return CMOL_ERR_CTX_FULL;
        slots[i] = ss[i]->slot;
        pos[i] = ss[i]->n_tokens;
    }
    int rc = cmolhip_decode_batch(m->dev, n, slots, tokens, pos, NULL, next);
    if (rc) return rc;
    for (int i = 0; i < n; i++) ss[i]->n_tokens++;
    return CMOL_OK;
}

int cmol__session_fill_kv(cmol_session_t *s, int n_tokens, uint64_t seed)
{
    if (!s || n_tokens < 0 || n_tokens > s->max_tokens) return CMOL_ERR_ARGS;
    int rc = cmolhip_kv_fill_synthetic(s->model->dev, s->slot, n_tokens, seed);
    if (rc) return rc;
    s->n_tokens = n_tokens;
    return CMOL_OK;
}

int cmol__sched_stats(cmol_model_t *m, uint64_t out[3])
{
    if (!m || !out) return CMOL_ERR_ARGS;
    if (!m->sched_on) {
        out[0] = out[1] = out[2] = 0;
        return 0;
    }
    cmol_sched_stats(&m->sched, out);
    return 1;
}

int cmol__session_length(const cmol_session_t *s) { return s ? s->n_tokens : CMOL_ERR_ARGS; }
int cmol__session_slot(const cmol_session_t *s) { return s ? s->slot : CMOL_ERR_ARGS; }
cmolhip_model_t *cmol__device(cmol_model_t *m) { return m ? m->dev : NULL; }
