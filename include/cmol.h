/*
 * cmol.h — libcmol public C API (MI355X build).
 *
 * Drop-in for the reference interface include/cmol.h: every declaration,
 * struct layout, macro and enum value below is kept identical so that code
 * written against the reference compiles and links unchanged.
 *   error codes          reference include/cmol.h:63-73
 *   logging              reference include/cmol.h:82-89
 *   cmol_config_t        reference include/cmol.h:93-104
 *   cmol_gen_params_t    reference include/cmol.h:110-125
 *   token callback       reference include/cmol.h:144-145
 *   lifecycle/sessions   reference include/cmol.h:164-200
 *   generate             reference include/cmol.h:218-222
 *   tokenizer/utilities  reference include/cmol.h:236-262
 *   ChatML helpers       reference include/cmol.h:296-316
 *
 * Behaviour differences of this build (documented, not ABI-visible):
 *   - weights, KV caches and activations live in one device arena on the GPU,
 *     allocated inside cmol_load; nothing is allocated after cmol_load;
 *   - an unsupported tensor dtype on the decode path fails cmol_load with
 *     CMOL_ERR_UNSUPPORTED instead of computing silently wrong output.
 */
#ifndef CMOL_H
#define CMOL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CMOL_VERSION_MAJOR  0
#define CMOL_VERSION_MINOR  1
#define CMOL_VERSION_PATCH  0
#define CMOL_VERSION_STRING "0.1.0"

/* Negative values are errors, CMOL_OK == 0; int-returning calls use
 * non-negative values for counts. */
typedef enum {
    CMOL_OK              =  0,
    CMOL_ERR_OOM         = -1, /* host or device memory exhausted        */
    CMOL_ERR_IO          = -2, /* file open / mmap failed                */
    CMOL_ERR_INVALID     = -3, /* malformed GGUF or missing tensor       */
    CMOL_ERR_UNSUPPORTED = -4, /* dtype / architecture / no usable GPU   */
    CMOL_ERR_NO_SESSION  = -5, /* session pool exhausted                 */
    CMOL_ERR_ARGS        = -6, /* NULL or out-of-range argument          */
    CMOL_ERR_CTX_FULL    = -7, /* KV cache full                          */
    CMOL_ERR_TRUNC       = -8, /* output buffer too small                */
} cmol_err_t;

#define CMOL_LOG_ERROR  0
#define CMOL_LOG_WARN   1
#define CMOL_LOG_INFO   2
#define CMOL_LOG_DEBUG  3

typedef void (*cmol_log_fn_t)(int level, const char *msg, void *userdata);

typedef struct {
    int           max_ctx;       /* context window per session (tokens)   */
    int           max_sessions;  /* sessions pre-allocated at load (<=32) */
    int           prefill_chunk; /* prompt tokens per batched prefill pass */
    cmol_log_fn_t log_fn;        /* optional log callback; NULL = silent  */
    void         *log_ud;
} cmol_config_t;

#define CMOL_DEFAULT_CONFIG \
    { .max_ctx = 2048, .max_sessions = 4, .prefill_chunk = 512, \
      .log_fn = NULL, .log_ud = NULL }

typedef struct {
    float        temperature;    /* 0.0 = greedy                          */
    float        top_p;          /* nucleus cutoff; 1.0 = disabled        */
    int          top_k;          /* 0 = disabled                          */
    int          max_new_tokens; /* -1 = until EOS / context full         */
    unsigned int seed;           /* 0 = non-deterministic                 */
    float        repeat_penalty; /* > 1.0 penalises recent tokens         */
    int          repeat_last_n;  /* window, clamped to 128                */
} cmol_gen_params_t;

#define CMOL_DEFAULT_PARAMS \
    { .temperature = 0.8f, .top_p = 0.95f, .top_k = 40, \
      .max_new_tokens = 256, .seed = 0, \
      .repeat_penalty = 1.1f, .repeat_last_n = 64 }

typedef struct cmol_model   cmol_model_t;
typedef struct cmol_session cmol_session_t;

/* Called once per generated piece (not NUL-terminated, `len` bytes).
 * Return non-zero to stop; cmol_generate still returns CMOL_OK. */
typedef int (*cmol_token_cb_t)(const char *piece, size_t len,
                                int is_eos, void *userdata);

cmol_model_t *cmol_load(const char          *gguf_path,
                         const cmol_config_t *cfg,
                         cmol_err_t          *err);
void cmol_free(cmol_model_t *m);

cmol_session_t *cmol_session_acquire(cmol_model_t *m);
void cmol_session_release(cmol_session_t *s);
void cmol_session_reset(cmol_session_t *s);

cmol_err_t cmol_generate(cmol_session_t          *s,
                          const char              *prompt,
                          const cmol_gen_params_t *params,
                          cmol_token_cb_t          on_token,
                          void                    *userdata);

int cmol_encode(cmol_model_t *m, const char *text, int32_t *out, int out_cap);
const char *cmol_decode_token(cmol_model_t *m, int32_t token_id);

const char *cmol_strerror(cmol_err_t err);
const char *cmol_version(void);
size_t cmol_arena_estimate(const char *gguf_path, const cmol_config_t *cfg);

int cmol_format_chatml(const char *system, const char *user,
                        char *buf, size_t buf_cap);
int cmol_format_chatml_turn(const char *user, char *buf, size_t buf_cap);

#ifdef __cplusplus
}
#endif

#endif /* CMOL_H */
