/*
 * host_check.c — drives the C host of libcmol and the oracle under the
 * sanitizers (AddressSanitizer + UndefinedBehaviorSanitizer, and
 * ThreadSanitizer), without a device (tests/native/no_device.c answers the
 * device calls).  Test infrastructure only; tests/test_sanitizers.py builds
 * and runs it.
 *
 *   host_check <gguf with a tokenizer>
 *
 * Parts:
 *   1. the cross-session scheduler's self-test: 32 threads posting ragged
 *      numbers of steps with host jitter;
 *   2. the sampler: draws over a 128256-entry vocabulary from four threads
 *      at once while the worker pool is held (one caller owns the pool, the
 *      others run single-threaded), each compared with the same draw made
 *      alone without the pool; then the pool is released (threads joined);
 *   3. the GGUF parser and tokenizer: cmol__load_text, encode / decode of a
 *      few texts, cmol_arena_estimate, and cmol_load failing cleanly at the
 *      device stage;
 *   4. the oracle: model load, forward and greedy generation with the
 *      repetition penalty on the same GGUF, and matmul for every format.
 * Exit status 0 when every check holds; the sanitizers abort on a finding.
 */
#ifndef _DEFAULT_SOURCE
#define _DEFAULT_SOURCE
#endif
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/cmol.h"
#include "../../include/cmol_ext.h"
#include "../../oracle/oracle.h"

static int failures = 0;
#define CHECK(c, what)                                              \
    do {                                                            \
        if (!(c)) {                                                 \
            fprintf(stderr, "FAIL %s (%s:%d)\n", what, __FILE__, __LINE__); \
            failures++;                                             \
        }                                                           \
    } while (0)

static uint64_t lcg(uint64_t *s)
{
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return *s >> 11;
}

/* ---- 2. sampler ------------------------------------------------------------ */
#define V 128256
#define DRAWS 6

typedef struct {
    int id;
    int32_t got[DRAWS], want[DRAWS];
} samp_job_t;

static void fill_logits(float *x, int job, int d)
{
    uint64_t s = (uint64_t)(job * 131 + d + 1);
    for (int i = 0; i < V; i++) x[i] = (float)((double)(lcg(&s) % 20000) / 2500.0 - 4.0);
    x[(job * 7919 + d) % V] = 9.0f;   /* a clear favourite now and then */
}

static void params_for(int job, cmol_gen_params_t *p)
{
    cmol_gen_params_t d = CMOL_DEFAULT_PARAMS;
    *p = d;
    p->temperature = 0.6f + 0.1f * (float)job;
    p->top_k = job == 3 ? 0 : 40 * (job + 1);
    p->top_p = job == 2 ? 1.0f : 0.9f;
}

static void draw_all(samp_job_t *j, int32_t *out)
{
    float *x = (float *)malloc((size_t)V * 4);
    cmol_gen_params_t p;
    params_for(j->id, &p);
    uint64_t rng[4];
    cmol_rng_seed(rng, (unsigned)(100 + j->id));
    for (int d = 0; d < DRAWS; d++) {
        fill_logits(x, j->id, d);
        out[d] = cmol_sample(x, V, &p, rng);
    }
    free(x);
}

static void *samp_thread(void *arg)
{
    samp_job_t *j = (samp_job_t *)arg;
    draw_all(j, j->got);
    return NULL;
}

static void check_sampler(void)
{
    samp_job_t jobs[4];
    for (int i = 0; i < 4; i++) {
        jobs[i].id = i;
        draw_all(&jobs[i], jobs[i].want);   /* no pool held: single-threaded */
    }
    const int prev = cmol__sampler_config(3, 16384);
    CHECK(cmol__sampler_pool(1) == 3, "pool started with 3 workers");
    pthread_t th[4];
    for (int i = 0; i < 4; i++) pthread_create(&th[i], NULL, samp_thread, &jobs[i]);
    for (int i = 0; i < 4; i++) pthread_join(th[i], NULL);
    CHECK(cmol__sampler_pool(0) == 0, "pool joined");
    cmol__sampler_config(prev, 16384);
    for (int i = 0; i < 4; i++)
        for (int d = 0; d < DRAWS; d++) CHECK(jobs[i].got[d] == jobs[i].want[d], "pooled draw == single-threaded");
    uint64_t a[4], b[4];
    cmol_rng_seed(a, 0);
    cmol_rng_seed(b, 0);
    CHECK(cmol_rng_next(a) != cmol_rng_next(b), "seed 0 streams differ");
}

/* ---- 3. parser, tokenizer, load error path --------------------------------- */
static void check_text(const char *path)
{
    cmol_err_t err = CMOL_OK;
    cmol_model_t *m = cmol__load_text(path, &err);
    CHECK(m && err == CMOL_OK, "cmol__load_text");
    if (!m) return;
    static const char *texts[] = {"", "Hello world", "  spaces   and\ttabs\n", "caf\xc3\xa9 \xe2\x82\xac 12",
                                  "<|im_start|>user\nhi<|im_end|>"};
    int32_t ids[256];
    for (size_t t = 0; t < sizeof texts / sizeof *texts; t++) {
        int n = cmol_encode(m, texts[t], ids, 256);
        CHECK(n >= 0, "encode");
        for (int i = 0; i < n; i++) CHECK(cmol_decode_token(m, ids[i]) != NULL, "decode");
        if (n > 1) CHECK(cmol_encode(m, texts[t], ids, 1) == CMOL_ERR_TRUNC, "encode into a short buffer");
    }
    CHECK(cmol_decode_token(m, -1) == NULL, "decode of an invalid id");
    cmol_free(m);
    CHECK(cmol_arena_estimate(path, NULL) > 0, "arena estimate");
    cmol_config_t cfg = CMOL_DEFAULT_CONFIG;
    cfg.max_sessions = 3;
    m = cmol_load(path, &cfg, &err);
    CHECK(m == NULL && err == CMOL_ERR_UNSUPPORTED, "cmol_load without a device fails cleanly");
    CHECK(cmol_load("/nonexistent.gguf", NULL, &err) == NULL && err == CMOL_ERR_IO, "missing file");
}

/* ---- 4. oracle ------------------------------------------------------------- */
static void check_oracle(const char *path)
{
    o_model_t *om = o_model_load(path, O_ORDER_AVX512, 2);
    CHECK(om != NULL, "oracle load");
    if (!om) return;
    int32_t hp[11];
    float hf[2];
    o_model_hparams(om, hp, hf);
    o_sess_t *s = o_sess_new(om, 64);
    o_sess_kv_f16(s, 1);
    int32_t prompt[6] = {1, 5, 9, 2, 7, 3}, out[20];
    float margins[20];
    for (int i = 0; i < 6; i++) prompt[i] %= hp[6];
    int n = o_generate_greedy(om, s, prompt, 6, 0, 20, 1.3f, 8, out, margins);
    CHECK(n == 20, "oracle greedy with penalty");
    o_sess_free(s);
    o_model_free(om);
    const int dts[] = {O_Q4_0, O_Q5_0, O_Q8_0, O_Q4_K, O_Q6_K, O_F32, O_F16};
    uint64_t st = 9;
    for (size_t t = 0; t < sizeof dts / sizeof *dts; t++) {
        const int m = 24, k = 512, nv = 3;
        size_t rb = o_row_bytes(k, dts[t]);
        uint8_t *a = (uint8_t *)malloc(rb * m);
        for (size_t i = 0; i < rb * m; i++) a[i] = (uint8_t)lcg(&st);
        if (dts[t] == O_F32)
            for (size_t i = 0; i < (size_t)m * k; i++) ((float *)a)[i] = (float)(lcg(&st) % 1000) / 500.0f - 1.0f;
        float b[512 * 3], y[24 * 3];
        for (int i = 0; i < k * nv; i++) b[i] = (float)(lcg(&st) % 1000) / 500.0f - 1.0f;
        o_matmul(y, a, b, m, k, nv, dts[t], O_ORDER_AVX512);
        o_matmul(y, a, b, m, k, nv, dts[t], O_ORDER_SCALAR);
        free(a);
    }
}

int main(int argc, char **argv)
{
    if (argc < 2) {
        fprintf(stderr, "usage: %s <gguf with tokenizer>\n", argv[0]);
        return 2;
    }
    uint64_t stats[3];
    int bad = cmol__sched_selftest(32, 20, 300, 40, 60, stats);
    CHECK(bad == 0, "scheduler self-test");
    CHECK(stats[1] > 0 && stats[2] <= 32, "scheduler stats");
    printf("scheduler: %llu batches, %llu steps, largest %llu\n", (unsigned long long)stats[0],
           (unsigned long long)stats[1], (unsigned long long)stats[2]);
    check_sampler();
    check_text(argv[1]);
    check_oracle(argv[1]);
    printf("%s: %d failures\n", failures ? "FAILED" : "ok", failures);
    return failures ? 1 : 0;
}
