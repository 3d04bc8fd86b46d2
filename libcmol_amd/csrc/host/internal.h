/*
 * internal.h — host-side internal types of libcmol (MI355X build).
 *
 * Mirrors the reference's internal model (reference src/cmol_internal.h):
 * dtype tags, tensor descriptors, hparams, tokenizer tables, arena and the
 * opaque model/session structs.  The compute state lives on the device
 * (cmolhip_model_t); the host keeps the mapped GGUF, metadata, the session
 * pool and per-session logits/token buffers carved from one host arena.
 */
#ifndef CMOL_HOST_INTERNAL_H
#define CMOL_HOST_INTERNAL_H

#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

#include "../../../include/cmol.h"
#include "../../../include/cmol_hip.h"

/* GGUF dtype tags (reference src/cmol_internal.h:27-37). */
typedef enum {
    CMOL_DTYPE_F32 = 0,
    CMOL_DTYPE_F16 = 1,
    CMOL_DTYPE_Q4_0 = 2,
    CMOL_DTYPE_Q4_1 = 3,
    CMOL_DTYPE_Q5_0 = 6,
    CMOL_DTYPE_Q8_0 = 8,
    CMOL_DTYPE_Q4_K = 12,
    CMOL_DTYPE_Q6_K = 14,
    CMOL_DTYPE_COUNT
} cmol_dtype_t;

#define CMOL_MAX_DIMS 4
#define CMOL_MAX_TENSOR_NAME 96
#define CMOL_MAX_SESSIONS 32
#define CMOL_REPEAT_BUF 128

typedef struct {
    char name[CMOL_MAX_TENSOR_NAME];
    int n_dims;
    int64_t shape[CMOL_MAX_DIMS]; /* shape[0] innermost */
    cmol_dtype_t dtype;
    uint64_t file_offset;
    void *data;                   /* into the mapping */
    size_t n_bytes;
} cmol_tensor_t;

typedef struct {
    int n_layers, n_heads, n_kv_heads, d_model, d_head, d_ffn, vocab_size;
    int model_max_ctx;
    float rope_freq_base, rms_norm_eps;
    int32_t bos_token_id, eos_token_id;
    int tie_embeddings;
    int no_rope_layer_interval;
    int yarn_factor_x100;
    char arch[32];
} cmol_hparams_t;

#define CMOL_TOK_LLAMA 0
#define CMOL_TOK_GPT2 1

typedef struct {
    const char **vocab;
    float *scores;
    uint8_t *token_type;
    int vocab_size;
    int tok_model;
    int32_t *merge_left, *merge_right;
    int n_merges;
    int32_t bos_id, eos_id, unk_id;
    int add_bos;
    const char **decoded_vocab;
    int32_t *vocab_sort_idx;
    int32_t *merge_result;
    int32_t *msort_idx;
} cmol_tokenizer_t;

typedef struct {
    uint8_t *base;
    size_t size, used;
} cmol_arena_t;

typedef struct {
    void *data;
    size_t size;
} cmol_mmap_t;

/* One decode step posted to the cross-session scheduler (sched.c). */
typedef struct cmol_step {
    int slot;                 /* device session slot */
    int32_t token, pos;
    float *logits;            /* host logits wanted here, or NULL */
    int32_t next;             /* out: argmax of the logits */
    int rc;                   /* out: 0 or a cmol_err_t */
    int done;
} cmol_step_t;

/* Runs n posted steps (distinct slots) as one batch; sets next / rc. */
typedef int (*cmol_batch_fn)(void *ctx, cmol_step_t *const *steps, int n);

typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t cv;        /* CLOCK_MONOTONIC */
    int ready;
    int active;               /* callers inside their decode loop */
    int running;              /* a batch is in flight */
    int n_pending;
    cmol_step_t *pending[CMOL_MAX_SESSIONS];
    uint64_t wait_ns, idle_since_ns;
    uint64_t batches, steps, max_batch;
    cmol_batch_fn run;
    void *ctx;
} cmol_sched_t;

struct cmol_model {
    cmol_hparams_t hparams;
    cmol_mmap_t mmap;
    cmol_tensor_t *tensors;
    int n_tensors;
    cmol_tokenizer_t tokenizer;
    cmol_config_t cfg;
    uint8_t *arena_buf;
    cmol_arena_t arena;
    struct cmol_session *session_slots;
    pthread_mutex_t pool_lock;
    uint32_t pool_free;
    cmolhip_model_t *dev;     /* device weights, KV caches, decode graphs */
    int kv_f16;
    cmol_sched_t sched;       /* batches concurrent decode steps (max_sessions > 1) */
    int sched_on;
    int sampler_held;            /* this model holds a start of the sampler pool */
};

struct cmol_session {
    cmol_model_t *model;
    int n_tokens;             /* next write position */
    int max_tokens;           /* = cfg.max_ctx       */
    float *logits;            /* host copy of the last logits [vocab] */
    int32_t *token_buf;
    int token_buf_cap;
    int slot;
};

/* platform.c */
cmol_err_t cmol_mmap_open(const char *path, cmol_mmap_t *out);
void cmol_mmap_close(cmol_mmap_t *m);

/* arena.c */
void cmol_arena_init(cmol_arena_t *a, void *buf, size_t size);
void *cmol_arena_alloc(cmol_arena_t *a, size_t size, size_t align);
void *cmol_arena_alloc_n(cmol_arena_t *a, size_t count, size_t elem_size);

/* gguf.c */
cmol_err_t cmol_gguf_parse(const cmol_mmap_t *mmap, cmol_arena_t *arena, cmol_hparams_t *hp,
                           cmol_tensor_t **tensors, int *n_tensors, cmol_tokenizer_t *tok);
cmol_tensor_t *cmol_gguf_find_tensor(cmol_tensor_t *tensors, int n, const char *name);
cmol_err_t cmol_gguf_peek(const char *path, cmol_hparams_t *hp, size_t *n_tensors);
size_t cmol_tensor_nbytes(cmol_dtype_t dtype, int64_t n_elems);

/* tokenizer.c */
cmol_err_t cmol_tokenizer_build(cmol_tokenizer_t *tok, cmol_arena_t *arena);
int cmol_tokenizer_encode(const cmol_tokenizer_t *tok, const char *text, int32_t *out,
                          int out_cap, int add_bos);
const char *cmol_tokenizer_decode_token(const cmol_tokenizer_t *tok, int32_t id);
size_t cmol_tokenizer_arena_bytes(int vocab_size, int n_merges_hint);

/* sched.c */
int cmol_sched_init(cmol_sched_t *q, cmol_batch_fn run, void *ctx, long wait_us);
void cmol_sched_destroy(cmol_sched_t *q);
void cmol_sched_enter(cmol_sched_t *q);
void cmol_sched_leave(cmol_sched_t *q);
int cmol_sched_step(cmol_sched_t *q, cmol_step_t *st);
void cmol_sched_stats(cmol_sched_t *q, uint64_t out[3]);

/* sampler.c */
int32_t cmol_sample(float *logits, int vocab_size, const cmol_gen_params_t *params,
                    uint64_t *rng_state);
void cmol_rng_seed(uint64_t state[4], unsigned int seed);
uint64_t cmol_rng_next(uint64_t state[4]);
void cmol_apply_repeat_penalty(float *logits, int vocab_size, const int32_t *tokens,
                               int n_tokens, float penalty);
/* The softmax worker pool: started by every cmol_load, stopped by every
 * cmol_free; the first start creates the threads, the last stop joins them. */
void cmol_sampler_pool_start(void);
void cmol_sampler_pool_stop(void);

/* api.c */
void cmol_log(const cmol_model_t *m, int level, const char *fmt, ...);

#endif
