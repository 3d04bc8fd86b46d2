/*
 * ref_shim.c — flat entry points over the reference library built from its
 * own sources (see oracle/Makefile target `ref`).  Lets the tests and the
 * golden-vector script call the reference's internal hot-path functions
 * through ctypes.  TEST INFRASTRUCTURE ONLY; never linked into the product.
 *
 * Compiled against the reference headers in place (include/, src/); nothing
 * from the reference is copied into this repository.
 */
#include "cmol_internal.h"
#include "model.h"
#include "quant.h"
#include "sampler.h"

#include <string.h>

void shim_dequant_row(const void *src, float *dst, int n, int dtype)
{
    cmol_dequant_row(src, dst, n, (cmol_dtype_t)dtype);
}

/* kind 0 = scalar, 1 = avx512, 2 = avx2, 3 = the runtime-selected kernel */
int shim_matmul(int kind, float *out, const void *a, const float *b,
                int m, int k, int n, int dtype)
{
    switch (kind) {
    case 0: cmol_matmul_scalar(out, a, b, m, k, n, (cmol_dtype_t)dtype); return 0;
#if defined(__x86_64__)
    case 1: cmol_matmul_avx512(out, a, b, m, k, n, (cmol_dtype_t)dtype); return 0;
    case 2: cmol_matmul_avx2(out, a, b, m, k, n, (cmol_dtype_t)dtype); return 0;
#endif
    case 3: {
        cmol_kernels_t kn = cmol_kernels_select();
        kn.matmul(out, a, b, m, k, n, (cmol_dtype_t)dtype);
        return 0;
    }
    default: return -1;
    }
}

const char *shim_kernel_name(void) { return cmol_kernels_select().name; }

void shim_rms_norm(const float *x, const float *w, float *o, int n, float eps)
{ cmol_rms_norm(x, w, o, n, eps); }
void shim_softmax(float *x, int n) { cmol_softmax(x, n); }
void shim_swiglu(const float *g, const float *u, float *o, int n) { cmol_swiglu(g, u, o, n); }
void shim_rope(float *q, float *k, int pos, int nh, int nkv, int hd, float base)
{ cmol_rope_apply(q, k, pos, nh, nkv, hd, base); }

/* Load through the public API; returns the model handle or NULL. */
cmol_model_t *shim_load(const char *path, int max_ctx, int sessions, int *err)
{
    cmol_config_t cfg = CMOL_DEFAULT_CONFIG;
    cfg.max_ctx = max_ctx;
    cfg.max_sessions = sessions;
    cmol_err_t e = CMOL_OK;
    cmol_model_t *m = cmol_load(path, &cfg, &e);
    if (err) *err = (int)e;
    return m;
}

void shim_free(cmol_model_t *m) { cmol_free(m); }
cmol_session_t *shim_acquire(cmol_model_t *m) { return cmol_session_acquire(m); }
void shim_release(cmol_session_t *s) { cmol_session_release(s); }

/* One cmol_model_forward step; copies vocab logits out. Returns 0 or -1. */
int shim_forward(cmol_model_t *m, cmol_session_t *s, int token, int pos,
                 float *logits_out)
{
    float *lg = cmol_model_forward(m, s, token, pos);
    if (!lg) return -1;
    if (logits_out) memcpy(logits_out, lg, (size_t)m->hparams.vocab_size * sizeof(float));
    return 0;
}

int shim_vocab(cmol_model_t *m) { return m->hparams.vocab_size; }
int shim_max_ctx(cmol_model_t *m) { return m->cfg.max_ctx; }

/* Token-ID greedy generation following the reference's own generate loop
 * semantics (prefill token by token, argmax, repetition ring).  Uses the
 * reference's cmol_model_forward, cmol_apply_repeat_penalty, cmol_sample. */
int shim_generate_greedy(cmol_model_t *m, cmol_session_t *s,
                         const int32_t *prompt, int n_prompt, int pos0,
                         int n_new, float penalty, int last_n, int32_t *out)
{
    int V = m->hparams.vocab_size;
    float *lg = NULL;
    int pos = pos0;
    for (int i = 0; i < n_prompt; i++) lg = cmol_model_forward(m, s, prompt[i], pos++);
    if (!lg) return -1;
    cmol_gen_params_t p = CMOL_DEFAULT_PARAMS;
    p.temperature = 0.0f;
    p.repeat_penalty = penalty;
    p.repeat_last_n = last_n;
    int32_t ring[CMOL_REPEAT_BUF];
    if (last_n <= 0 || last_n > CMOL_REPEAT_BUF) last_n = CMOL_REPEAT_BUF;
    int seed_n = n_prompt < last_n ? n_prompt : last_n, head, fill;
    for (int i = 0; i < seed_n; i++) ring[i] = prompt[n_prompt - seed_n + i];
    head = seed_n % CMOL_REPEAT_BUF;
    fill = seed_n;
    int produced = 0;
    for (;;) {
        if (penalty > 1.0f && fill > 0) cmol_apply_repeat_penalty(lg, V, ring, fill, penalty);
        int32_t next = cmol_sample(lg, V, &p, NULL);
        out[produced++] = next;
        if (m->tokenizer.eos_id >= 0 && next == m->tokenizer.eos_id) break;
        ring[head] = next;
        head = (head + 1) % CMOL_REPEAT_BUF;
        if (fill < CMOL_REPEAT_BUF) fill++;
        if (produced >= n_new) break;
        if (pos >= s->kvcache.max_tokens) break;
        lg = cmol_model_forward(m, s, next, pos++);
        if (!lg) return -1;
    }
    return produced;
}

/* Full public cmol_generate with a counting callback (API-level check). */
typedef struct { int32_t *ids; int cap, n; cmol_model_t *m; } cb_state_t;
static int cb_collect(const char *piece, size_t len, int eos, void *ud)
{
    (void)len; (void)eos;
    cb_state_t *st = (cb_state_t *)ud;
    /* map the piece back to its id by pointer identity of decoded strings */
    for (int i = 0; i < st->m->tokenizer.vocab_size; i++)
        if (cmol_decode_token(st->m, i) == piece) {
            if (st->n < st->cap) st->ids[st->n] = i;
            st->n++;
            return 0;
        }
    if (st->n < st->cap) st->ids[st->n] = -1;
    st->n++;
    return 0;
}

int shim_generate_text(cmol_model_t *m, cmol_session_t *s, const char *prompt,
                       int max_new, float temperature, unsigned seed,
                       float penalty, int32_t *ids, int cap)
{
    cmol_gen_params_t p = CMOL_DEFAULT_PARAMS;
    p.temperature = temperature;
    p.max_new_tokens = max_new;
    p.seed = seed;
    p.repeat_penalty = penalty;
    cb_state_t st = {ids, cap, 0, m};
    cmol_err_t e = cmol_generate(s, prompt, &p, cb_collect, &st);
    return e == CMOL_OK ? st.n : (int)e;
}

int shim_encode(cmol_model_t *m, const char *text, int32_t *out, int cap)
{ return cmol_encode(m, text, out, cap); }

/* KV cache access: layout [layer][pos][n_kv][d_head] fp32. */
float *shim_kv(cmol_session_t *s, int which) { return which ? s->kvcache.v : s->kvcache.k; }
int shim_n_tokens(cmol_session_t *s) { return s->kvcache.n_tokens; }
