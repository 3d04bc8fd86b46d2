/*
 * sampler.c — token selection on the host (reference src/sampler.c).
 *
 * Greedy: first index of the maximum logit (src/sampler.c:199-204).
 * Otherwise: temperature scaling, softmax, optional top-k (min-heap of at most
 * 512) and top-p nucleus, then one draw from xoshiro256** seeded by
 * splitmix64 (src/sampler.c:37-75), so the same seed selects the same token as
 * the reference.  The repetition penalty divides positive / multiplies
 * non-positive logits, once per occurrence in the window (src/sampler.c:171-184).
 *
 * For large vocabularies the element-wise parts of the softmax (temperature
 * scale, chunk maxima, expf, the final scale) run on a small pool of worker
 * threads; the sum stays one sequential pass in index order, so every
 * probability is bit-identical to the single-threaded computation.
 */
#ifndef _DEFAULT_SOURCE
#define _DEFAULT_SOURCE
#endif
#ifndef _GNU_SOURCE
#define _GNU_SOURCE   /* sched_getaffinity, CPU_COUNT */
#endif
#include "internal.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* xoshiro256** step (Blackman & Vigna). */
uint64_t cmol_rng_next(uint64_t s[4])
{
    const uint64_t out = rotl(s[1] * 5u, 7) * 9u;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

/* splitmix64 (Steele, Lea, Flood) used to expand the 32-bit seed. */
static uint64_t splitmix(uint64_t *x)
{
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Seed 0 asks for a non-reproducible stream: 8 bytes from the kernel's
 * entropy source, or, where that is unavailable, the monotonic clock in
 * nanoseconds with a process-wide call counter; either way splitmix64 then
 * expands the value as it does a caller's seed. */
static uint64_t fresh_seed(void)
{
    uint64_t x = 0;
    if (getentropy(&x, sizeof x) == 0 && x) return x;
    static uint64_t calls = 0;
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    const uint64_t c = __atomic_add_fetch(&calls, 1, __ATOMIC_RELAXED);
    x = (uint64_t)t.tv_sec * 1000000000ull + (uint64_t)t.tv_nsec;
    return x + (c << 40) + c;
}

void cmol_rng_seed(uint64_t st[4], unsigned int seed)
{
    uint64_t x = seed ? (uint64_t)seed : fresh_seed();
    for (int i = 0; i < 4; i++) st[i] = splitmix(&x);
}

/* Uniform float in [0,1): 23 random mantissa bits under exponent 127. */
static float rng_unit(uint64_t st[4])
{
    uint32_t bits = 0x3F800000u | (uint32_t)(cmol_rng_next(st) >> 41);
    float f;
    memcpy(&f, &bits, 4);
    return f - 1.0f;
}

void cmol_apply_repeat_penalty(float *logits, int vocab, const int32_t *tokens, int n, float penalty)
{
    if (penalty <= 1.0f || !logits || !tokens || n <= 0) return;
    for (int i = 0; i < n; i++) {
        int32_t id = tokens[i];
        if (id < 0 || id >= vocab) continue;
        logits[id] = logits[id] > 0.0f ? logits[id] / penalty : logits[id] * penalty;
    }
}

static int32_t argmax_first(const float *x, int n)
{
    int32_t best = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return best;
}

static void softmax_inplace(float *x, int n)
{
    float mx = x[0], sum = 0.0f;
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    sum = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= sum;
}

/* ---- worker pool for the element-wise parts of a large softmax ---------- */

#define POOL_MAX 16
enum { PH_SCALE_MAX, PH_EXP, PH_SCALE };

/* The pool lives while a model is loaded: cmol_load starts it (the first
 * load creates the workers) and cmol_free stops it (the last free wakes the
 * workers with `stop` set and joins them), so no thread is created on a
 * decode path and none outlives the library's last model. */
static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    int refs;                 /* loaded models (and harness holds) */
    int created;              /* worker threads */
    int used;                 /* workers a softmax uses (<= created) */
    int min_vocab;            /* smaller vocabularies run single-threaded */
    int busy;                 /* a caller owns the pool */
    int stop;                 /* workers exit */
    unsigned gen;             /* job generation */
    unsigned gen0;            /* generation when the workers were created */
    int left;                 /* workers still on the current job */
    int phase, V, parts;
    float *x, a;
    float cmax[POOL_MAX + 1];
    pthread_t tid[POOL_MAX];
} pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER,
          0, 0, 0, 16384, 0, 0, 0, 0, 0, 0, 0, 0, NULL, 0.0f, {0}, {0}};
static pthread_mutex_t pool_life = PTHREAD_MUTEX_INITIALIZER;   /* start / stop */
static int pool_threads_wanted = -1;   /* cmol__sampler_config before the start */

/* Part j of the current job: elements [V j / parts, V (j+1) / parts). */
static void pool_part(int j)
{
    if (j >= pool.parts) return;
    const int lo = (int)((long)pool.V * j / pool.parts), hi = (int)((long)pool.V * (j + 1) / pool.parts);
    float *x = pool.x;
    const float a = pool.a;
    if (pool.phase == PH_SCALE_MAX) {
        float m = -INFINITY;   /* NaNs never replace it, as in the sequential scan */
        for (int i = lo; i < hi; i++) {
            x[i] *= a;
            if (x[i] > m) m = x[i];
        }
        pool.cmax[j] = m;
    } else if (pool.phase == PH_EXP) {
        for (int i = lo; i < hi; i++) x[i] = expf(x[i] - a);
    } else {
        for (int i = lo; i < hi; i++) x[i] *= a;
    }
}

/* Spin before sleeping: the three phases of one softmax follow each other
 * within a fraction of a millisecond, and a wake-up through the condition
 * variable costs tens of microseconds; between two draws (a decode step) the
 * workers sleep. */
#define POOL_SPIN_NS 300000ull

static uint64_t pool_now_ns(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (uint64_t)t.tv_sec * 1000000000ull + (uint64_t)t.tv_nsec;
}

static void *pool_worker(void *arg)
{
    const int j = (int)(intptr_t)arg;
    unsigned seen = pool.gen0;   /* jobs before this pool's start are not ours */
    for (;;) {
        const uint64_t t0 = pool_now_ns();
        while (__atomic_load_n(&pool.gen, __ATOMIC_ACQUIRE) == seen && pool_now_ns() - t0 < POOL_SPIN_NS)
            __builtin_ia32_pause();
        pthread_mutex_lock(&pool.mu);
        while (__atomic_load_n(&pool.gen, __ATOMIC_RELAXED) == seen && !pool.stop)
            pthread_cond_wait(&pool.go, &pool.mu);
        if (pool.stop) {
            pthread_mutex_unlock(&pool.mu);
            return NULL;
        }
        seen = __atomic_load_n(&pool.gen, __ATOMIC_RELAXED);
        pthread_mutex_unlock(&pool.mu);
        pool_part(j);
        /* the release publishes this part's results to a caller that sees
         * left reach 0 with its acquire load, spinning or after the wait */
        pthread_mutex_lock(&pool.mu);
        if (__atomic_sub_fetch(&pool.left, 1, __ATOMIC_ACQ_REL) == 0) pthread_cond_signal(&pool.done);
        pthread_mutex_unlock(&pool.mu);
    }
}

/* CPUs the process may use: the online CPUs, bounded by its affinity mask
 * and by its cgroup's CPU quota (cgroup v2 cpu.max). */
static long usable_cpus(void)
{
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof set, &set) == 0) {
        const long c = CPU_COUNT(&set);
        if (c > 0 && c < n) n = c;
    }
    FILE *f = fopen("/sys/fs/cgroup/cpu.max", "r");
    if (f) {
        char q[32];
        long per = 0;
        if (fscanf(f, "%31s %ld", q, &per) == 2 && strcmp(q, "max") != 0 && per > 0) {
            long c = atol(q) / per;
            if (c < 1) c = 1;
            if (c < n) n = c;
        }
        fclose(f);
    }
    return n < 1 ? 1 : n;
}

/* Worker count: cmol__sampler_config's, else CMOL_SAMPLER_THREADS, else half
 * the CPUs the process may use, at most 8. */
static int pool_size(void)
{
    if (pool_threads_wanted >= 0) return pool_threads_wanted;
    const char *e = getenv("CMOL_SAMPLER_THREADS");
    long n = e ? atol(e) : usable_cpus() / 2;
    if (!e && n > 8) n = 8;
    if (n < 0) n = 0;
    if (n > POOL_MAX) n = POOL_MAX;
    return (int)n;
}

void cmol_sampler_pool_start(void)
{
    pthread_mutex_lock(&pool_life);
    if (pool.refs++ == 0) {
        const int n = pool_size();
        int made = 0;
        pthread_mutex_lock(&pool.mu);
        pool.stop = 0;
        __atomic_store_n(&pool.left, 0, __ATOMIC_RELAXED);
        pool.gen0 = __atomic_load_n(&pool.gen, __ATOMIC_RELAXED);
        pthread_mutex_unlock(&pool.mu);
        for (int j = 1; j <= n; j++) {
            if (pthread_create(&pool.tid[made], NULL, pool_worker, (void *)(intptr_t)j) != 0) break;
            made++;
        }
        pthread_mutex_lock(&pool.mu);
        pool.created = made;
        pool.used = made;
        pthread_mutex_unlock(&pool.mu);
    }
    pthread_mutex_unlock(&pool_life);
}

void cmol_sampler_pool_stop(void)
{
    pthread_mutex_lock(&pool_life);
    if (pool.refs > 0 && --pool.refs == 0) {
        pthread_mutex_lock(&pool.mu);
        const int n = pool.created;
        pool.stop = 1;
        pool.created = 0;
        pool.used = 0;
        __atomic_store_n(&pool.gen, pool.gen + 1, __ATOMIC_RELEASE);
        pthread_cond_broadcast(&pool.go);
        pthread_mutex_unlock(&pool.mu);
        for (int j = 0; j < n; j++) pthread_join(pool.tid[j], NULL);
    }
    pthread_mutex_unlock(&pool_life);
}

int cmol__sampler_pool(int on)
{
    if (on) cmol_sampler_pool_start();
    else cmol_sampler_pool_stop();
    pthread_mutex_lock(&pool.mu);
    const int n = pool.created;
    pthread_mutex_unlock(&pool.mu);
    return n;
}

/* Runs one phase on the workers and the caller (part 0); pool.mu held.
 * Every created worker takes part (parts beyond pool.parts do nothing). */
static void pool_run(int phase, float a)
{
    pool.phase = phase;
    pool.a = a;
    __atomic_store_n(&pool.left, pool.created, __ATOMIC_RELAXED);
    __atomic_store_n(&pool.gen, pool.gen + 1, __ATOMIC_RELEASE);
    pthread_cond_broadcast(&pool.go);
    pthread_mutex_unlock(&pool.mu);
    pool_part(0);
    const uint64_t t0 = pool_now_ns();
    while (__atomic_load_n(&pool.left, __ATOMIC_ACQUIRE) > 0 && pool_now_ns() - t0 < POOL_SPIN_NS)
        __builtin_ia32_pause();
    pthread_mutex_lock(&pool.mu);
    while (__atomic_load_n(&pool.left, __ATOMIC_ACQUIRE) > 0) pthread_cond_wait(&pool.done, &pool.mu);
}

/* Temperature scale and softmax of x[0..V) on the pool, with the results of
 * the sequential loops; returns 0 (nothing done) when the pool is off, busy
 * or the vocabulary small. */
static int pool_softmax(float *x, int V, float inv_t)
{
    pthread_mutex_lock(&pool.mu);
    if (pool.busy || pool.used < 1 || V < pool.min_vocab) {
        pthread_mutex_unlock(&pool.mu);
        return 0;
    }
    pool.busy = 1;
    pool.x = x;
    pool.V = V;
    pool.parts = pool.used + 1;
    pool_run(PH_SCALE_MAX, inv_t);
    /* the sequential scan's maximum: x[0], replaced by any greater element */
    float mx = x[0];
    for (int j = 0; j < pool.parts; j++)
        if (pool.cmax[j] > mx) mx = pool.cmax[j];
    pool_run(PH_EXP, mx);
    pthread_mutex_unlock(&pool.mu);
    float sum = 0.0f;
    for (int i = 0; i < V; i++) sum += x[i];
    pthread_mutex_lock(&pool.mu);
    pool_run(PH_SCALE, 1.0f / sum);
    pool.busy = 0;
    pthread_mutex_unlock(&pool.mu);
    return 1;
}

int cmol__sampler_config(int threads, int min_vocab)
{
    pthread_mutex_lock(&pool_life);
    pthread_mutex_lock(&pool.mu);
    const int prev = pool.refs ? pool.used : pool_size();
    if (threads >= 0) {
        if (pool.refs) pool.used = threads < pool.created ? threads : pool.created;
        else pool_threads_wanted = threads > POOL_MAX ? POOL_MAX : threads;
    }
    if (min_vocab > 0) pool.min_vocab = min_vocab;
    pthread_mutex_unlock(&pool.mu);
    pthread_mutex_unlock(&pool_life);
    return prev;
}

typedef struct { float p; int32_t id; } cand_t;
#define TOPK_MAX 512

static void heap_down(cand_t *h, int i, int n)
{
    for (;;) {
        int m = i, l = 2 * i + 1, r = l + 1;
        if (l < n && h[l].p < h[m].p) m = l;
        if (r < n && h[r].p < h[m].p) m = r;
        if (m == i) return;
        cand_t t = h[i]; h[i] = h[m]; h[m] = t;
        i = m;
    }
}

static void heap_up(cand_t *h, int i)
{
    while (i > 0) {
        int p = (i - 1) / 2;
        if (h[p].p <= h[i].p) return;
        cand_t t = h[i]; h[i] = h[p]; h[p] = t;
        i = p;
    }
}

static int by_p_desc(const void *a, const void *b)
{
    float x = ((const cand_t *)a)->p, y = ((const cand_t *)b)->p;
    return x < y ? 1 : x > y ? -1 : 0;
}

int32_t cmol_sample(float *logits, int V, const cmol_gen_params_t *prm, uint64_t *rng)
{
    if (!logits || V <= 0) return 0;
    if (!prm || prm->temperature == 0.0f) return argmax_first(logits, V);
    const float inv_t = 1.0f / prm->temperature;
    if (!pool_softmax(logits, V, inv_t)) {
        for (int i = 0; i < V; i++) logits[i] *= inv_t;
        softmax_inplace(logits, V);
    }
    const int use_k = prm->top_k > 0 && prm->top_k < V;
    const int use_p = prm->top_p > 0.0f && prm->top_p < 1.0f;
    if (!use_k && !use_p) {
        if (!rng) return argmax_first(logits, V);
        float r = rng_unit(rng), acc = 0.0f;
        for (int i = 0; i < V - 1; i++) {
            acc += logits[i];
            if (r < acc) return i;
        }
        return V - 1;
    }
    cand_t heap[TOPK_MAX];
    int k = use_k ? prm->top_k : V;
    if (k > TOPK_MAX) k = TOPK_MAX;
    int n = 0, i = 0;
    for (; i < V && n < k; i++) {
        heap[n].p = logits[i];
        heap[n].id = i;
        heap_up(heap, n++);
    }
    /* The same in-order scan, but a run of 16 elements none of which beats
     * the heap's minimum (NaN never does) is passed over in one vector
     * compare: the minimum only changes on a hit, so the heap ends the same. */
    while (i < V) {
        if (i + 16 <= V) {
            const float h = heap[0].p;
            int any = 0;
            for (int j = 0; j < 16; j++) any |= logits[i + j] > h;
            if (!any) {
                i += 16;
                continue;
            }
        }
        if (logits[i] > heap[0].p) {
            heap[0].p = logits[i];
            heap[0].id = i;
            heap_down(heap, 0, k);
        }
        i++;
    }
    qsort(heap, (size_t)n, sizeof(cand_t), by_p_desc);
    int nuc = n;
    if (use_p) {
        float cum = 0.0f;
        for (int i = 0; i < n; i++) {
            cum += heap[i].p;
            if (cum >= prm->top_p) { nuc = i + 1; break; }
        }
    }
    float sum = 0.0f;
    for (int i = 0; i < nuc; i++) sum += heap[i].p;
    if (!rng || sum <= 0.0f) return heap[0].id;
    float r = rng_unit(rng) * sum, acc = 0.0f;
    for (int i = 0; i < nuc; i++) {
        acc += heap[i].p;
        if (r < acc) return heap[i].id;
    }
    return heap[nuc - 1].id;
}
