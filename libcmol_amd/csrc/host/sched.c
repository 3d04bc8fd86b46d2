/*
 * sched.c — cross-session batching of decode steps (rendezvous per step).
 *
 * The reference runs each session's cmol_generate on its caller's thread and
 * every decode step streams the whole model's weights for one token
 * (reference src/api.c:309-334 for the thread-per-session contract,
 * src/api.c:443-521 for the loop).  On the device a lock-step batch of n
 * sessions streams the weights once for all n, so concurrent callers are
 * worth batching.  The reference has no such scheduler; this one keeps its
 * contract: each caller still owns its session and sees the same results.
 *
 * Protocol.  A caller in its decode loop is "active" (cmol_sched_enter /
 * cmol_sched_leave).  For each token it posts a step and waits.  A waiter
 * becomes the leader when no batch is in flight and either every active
 * caller has posted or its wait window has passed; the window counts from
 * the later of its own arrival and the end of the previous batch, so the
 * callers a batch releases can rejoin the next one.  The leader takes every
 * posted step, runs them as one batch outside the lock, publishes each
 * result and wakes the others.  At most one batch runs at a time.
 */
#ifndef _DEFAULT_SOURCE
#define _DEFAULT_SOURCE
#endif
#include "internal.h"

#include <errno.h>
#include <string.h>
#include <time.h>

static uint64_t now_ns(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (uint64_t)t.tv_sec * 1000000000ull + (uint64_t)t.tv_nsec;
}

int cmol_sched_init(cmol_sched_t *q, cmol_batch_fn run, void *ctx, long wait_us)
{
    memset(q, 0, sizeof *q);
    pthread_condattr_t ca;
    if (pthread_condattr_init(&ca)) return CMOL_ERR_OOM;
    pthread_condattr_setclock(&ca, CLOCK_MONOTONIC);
    int rc = pthread_cond_init(&q->cv, &ca);
    pthread_condattr_destroy(&ca);
    if (rc) return CMOL_ERR_OOM;
    if (pthread_mutex_init(&q->mu, NULL)) {
        pthread_cond_destroy(&q->cv);
        return CMOL_ERR_OOM;
    }
    q->run = run;
    q->ctx = ctx;
    q->wait_ns = (uint64_t)(wait_us > 0 ? wait_us : 0) * 1000ull;
    q->idle_since_ns = now_ns();
    q->ready = 1;
    return CMOL_OK;
}

void cmol_sched_destroy(cmol_sched_t *q)
{
    if (!q->ready) return;
    pthread_mutex_destroy(&q->mu);
    pthread_cond_destroy(&q->cv);
    q->ready = 0;
}

void cmol_sched_enter(cmol_sched_t *q)
{
    pthread_mutex_lock(&q->mu);
    q->active++;
    pthread_mutex_unlock(&q->mu);
}

void cmol_sched_leave(cmol_sched_t *q)
{
    pthread_mutex_lock(&q->mu);
    q->active--;
    /* waiters may now all have posted */
    pthread_cond_broadcast(&q->cv);
    pthread_mutex_unlock(&q->mu);
}

int cmol_sched_step(cmol_sched_t *q, cmol_step_t *st)
{
    st->done = 0;
    st->rc = CMOL_OK;
    pthread_mutex_lock(&q->mu);
    if (q->n_pending >= CMOL_MAX_SESSIONS) {   /* more posters than sessions: misuse */
        pthread_mutex_unlock(&q->mu);
        return CMOL_ERR_ARGS;
    }
    const uint64_t arrived = now_ns();
    q->pending[q->n_pending++] = st;
    /* No wake-up here: the poster that completes the set finds it below
     * itself, a batch in flight wakes everyone when it ends, and a waiter
     * whose window passes wakes by its own timeout; waking every waiter on
     * every post cost 32 x 31 wake-ups per step at 32 sessions. */
    while (!st->done) {
        if (!q->running && q->n_pending > 0) {
            const uint64_t from = arrived > q->idle_since_ns ? arrived : q->idle_since_ns;
            const uint64_t t = now_ns();
            if (q->n_pending >= q->active || t >= from + q->wait_ns) {
                cmol_step_t *batch[CMOL_MAX_SESSIONS];
                const int n = q->n_pending;
                memcpy(batch, q->pending, (size_t)n * sizeof batch[0]);
                q->n_pending = 0;
                q->running = 1;
                pthread_mutex_unlock(&q->mu);
                q->run(q->ctx, batch, n);
                pthread_mutex_lock(&q->mu);
                for (int i = 0; i < n; i++) batch[i]->done = 1;
                q->running = 0;
                q->idle_since_ns = now_ns();
                q->batches++;
                q->steps += (uint64_t)n;
                if ((uint64_t)n > q->max_batch) q->max_batch = (uint64_t)n;
                pthread_cond_broadcast(&q->cv);
                continue;
            }
            const uint64_t until = from + q->wait_ns;
            struct timespec ts;
            ts.tv_sec = (time_t)(until / 1000000000ull);
            ts.tv_nsec = (long)(until % 1000000000ull);
            pthread_cond_timedwait(&q->cv, &q->mu, &ts);
        } else {
            pthread_cond_wait(&q->cv, &q->mu);
        }
    }
    pthread_mutex_unlock(&q->mu);
    return st->rc;
}

void cmol_sched_stats(cmol_sched_t *q, uint64_t out[3])
{
    pthread_mutex_lock(&q->mu);
    out[0] = q->batches;
    out[1] = q->steps;
    out[2] = q->max_batch;
    pthread_mutex_unlock(&q->mu);
}

/* ---- self-test of the rendezvous (no device) ------------------------------ */

typedef struct {
    cmol_sched_t *q;
    int id, steps;
    unsigned host_us;         /* host work between steps (0..host_us, varied) */
    int bad;
} selftest_thread_t;

typedef struct {
    long device_us;
    int bad;
} selftest_dev_t;

/* Stand-in for the device step: checks that no session appears twice in a
 * batch, "computes" next = token * 7 + pos, and takes device_us. */
static int selftest_run(void *ctx, cmol_step_t *const *st, int n)
{
    selftest_dev_t *d = (selftest_dev_t *)ctx;
    for (int i = 0; i < n; i++)
        for (int j = 0; j < i; j++)
            if (st[i]->slot == st[j]->slot) d->bad++;
    for (int i = 0; i < n; i++) {
        st[i]->next = st[i]->token * 7 + st[i]->pos;
        st[i]->rc = CMOL_OK;
    }
    struct timespec ts = {d->device_us / 1000000L, (d->device_us % 1000000L) * 1000L};
    nanosleep(&ts, NULL);
    return CMOL_OK;
}

static void *selftest_thread(void *arg)
{
    selftest_thread_t *t = (selftest_thread_t *)arg;
    cmol_sched_enter(t->q);
    uint32_t r = 0x9E3779B9u * (uint32_t)(t->id + 1);
    for (int k = 0; k < t->steps; k++) {
        cmol_step_t st;
        memset(&st, 0, sizeof st);
        st.slot = t->id;
        st.token = t->id;
        st.pos = k;
        if (cmol_sched_step(t->q, &st) != CMOL_OK || st.next != t->id * 7 + k) t->bad++;
        if (t->host_us) {
            r = r * 1664525u + 1013904223u;
            struct timespec ts = {0, (long)((r >> 8) % (t->host_us + 1)) * 1000L};
            nanosleep(&ts, NULL);
        }
    }
    cmol_sched_leave(t->q);
    return NULL;
}

/* Returns the count of wrong results (0: all right) or CMOL_ERR_ARGS / OOM. */
int cmol__sched_selftest(int threads, int steps, long wait_us, long device_us, unsigned host_us,
                         uint64_t stats[3])
{
    if (threads < 1 || threads > CMOL_MAX_SESSIONS || steps < 1 || !stats) return CMOL_ERR_ARGS;
    cmol_sched_t q;
    selftest_dev_t dev = {device_us, 0};
    if (cmol_sched_init(&q, selftest_run, &dev, wait_us)) return CMOL_ERR_OOM;
    pthread_t th[CMOL_MAX_SESSIONS];
    selftest_thread_t ts[CMOL_MAX_SESSIONS];
    int started = 0, bad = 0;
    for (int i = 0; i < threads; i++) {
        /* ragged: thread i leaves after steps + i steps */
        ts[i] = (selftest_thread_t){&q, i, steps + i, host_us, 0};
        if (pthread_create(&th[i], NULL, selftest_thread, &ts[i])) {
            bad++;
            break;
        }
        started++;
    }
    for (int i = 0; i < started; i++) {
        pthread_join(th[i], NULL);
        bad += ts[i].bad;
    }
    cmol_sched_stats(&q, stats);
    cmol_sched_destroy(&q);
    return bad + dev.bad;
}
