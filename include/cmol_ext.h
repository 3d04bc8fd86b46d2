/*
 * cmol_ext.h — internal entry points of libcmol (MI355X build) for test and
 * benchmark harnesses.  Not part of the public API (include/cmol.h).
 *
 * The reference exposes the same capabilities only inside its library:
 *   cmol__forward          reference src/model.c:176-276 (cmol_model_forward)
 *   cmol__generate_ids     reference src/api.c:412-524 with token ids instead
 *                          of text and the callback replaced by an id list
 *   cmol__prefill          reference src/api.c:443-452 (prompt prefill loop)
 *   cmol__decode_batch     no reference counterpart: lock-step decode of many
 *                          sessions (the reference runs one thread per session)
 *   cmol__session_fill_kv  no reference counterpart: synthetic KV contents of a
 *                          given length, for long-context benchmarks
 *   cmol__sched_stats,     no reference counterpart: counters and a device-free
 *   cmol__sched_selftest   self-test of the scheduler that batches concurrent
 *                          cmol_generate decode steps (the reference runs each
 *                          caller's steps alone, src/api.c:443-521)
 */
#ifndef CMOL_EXT_H
#define CMOL_EXT_H

#include "cmol.h"
#include "cmol_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One forward step of session s for `token` at position `pos`; copies the
 * logits (vocab floats) when logits_out != NULL and returns the argmax id
 * (>= 0) or a negative cmol_err_t.  Does not change the session's length. */
int cmol__forward(cmol_session_t *s, int32_t token, int pos, float *logits_out);

/* Prefill n prompt tokens at the session's current length, advancing it;
 * returns the argmax of the last logits or a negative cmol_err_t. */
int cmol__prefill(cmol_session_t *s, const int32_t *tokens, int n, float *logits_out);

/* cmol_generate on token ids: appends the prompt, then samples until EOS,
 * max_new_tokens or a full context; out receives the sampled ids (EOS
 * included).  Returns the number written or a negative cmol_err_t. */
int cmol__generate_ids(cmol_session_t *s, const int32_t *prompt, int n_prompt,
                       const cmol_gen_params_t *params, int32_t *out, int out_cap);

/* One lock-step decode step for n distinct sessions: session i consumes
 * tokens[i] at its current length (then advanced by one); next[i] receives
 * the argmax.  Returns CMOL_OK or a negative cmol_err_t. */
int cmol__decode_batch(cmol_session_t *const *ss, const int32_t *tokens, int n,
                       int32_t *next);

/* Fill positions [0, n_tokens) of every layer of the session's KV cache with
 * seeded synthetic values and set its length to n_tokens. */
int cmol__session_fill_kv(cmol_session_t *s, int n_tokens, uint64_t seed);

/* The host sampler, exported for parity checks; same signatures and
 * semantics as the reference's (src/sampler.h:20-34, src/sampler.c:171-268):
 * cmol_sample scales, softmaxes and may reorder `logits` in place;
 * rng_state is a 4-word xoshiro256** state seeded by cmol_rng_seed. */
int32_t cmol_sample(float *logits, int vocab_size, const cmol_gen_params_t *params,
                    uint64_t *rng_state);
void cmol_rng_seed(uint64_t state[4], unsigned int seed);
uint64_t cmol_rng_next(uint64_t state[4]);
void cmol_apply_repeat_penalty(float *logits, int vocab_size, const int32_t *tokens,
                               int n_tokens, float penalty);

/* No reference counterpart: the sampler's worker pool, which runs the
 * element-wise parts of the softmax of vocabularies of at least min_vocab
 * entries (default 16384) on worker threads with bit-identical results.
 * The pool exists while a model is loaded: cmol_load starts it and the last
 * cmol_free joins its threads.  cmol__sampler_config sets the workers a
 * softmax uses (at most the pool's; before the first start, the pool's size,
 * else CMOL_SAMPLER_THREADS or half the CPUs, at most 8) and min_vocab;
 * threads < 0 or min_vocab <= 0 keep the current value; returns the previous
 * worker count.  cmol__sampler_pool(1) holds the pool as a load does and
 * cmol__sampler_pool(0) releases that hold (sampler checks without a model);
 * it returns the pool's worker count after the call. */
int cmol__sampler_config(int threads, int min_vocab);
int cmol__sampler_pool(int on);

/* Parse a GGUF and build its tokenizer only, without a device or sessions:
 * cmol_encode, cmol_decode_token and cmol_free work on the result (text-path
 * parity checks on machines without a GPU).  Same errors as cmol_load's
 * parse stage. */
cmol_model_t *cmol__load_text(const char *path, cmol_err_t *err);

/* Counters of the cross-session scheduler: out[0] batches run, out[1] steps
 * in them, out[2] the largest batch.  Returns 1 when the model batches
 * concurrent decode steps (max_sessions > 1 and CMOL_BATCH is not 0), 0 when
 * it does not (counters 0), or a negative cmol_err_t. */
int cmol__sched_stats(cmol_model_t *m, uint64_t out[3]);

/* The scheduler's rendezvous without a device: `threads` posters (thread i
 * leaves after steps + i steps, with 0..host_us µs of host work between its
 * steps) against a stand-in batch that takes device_us µs; wait_us is the
 * straggler window.  stats as in cmol__sched_stats.  Returns the count of
 * wrong results (0 when every poster got its own answer and no batch held a
 * session twice) or a negative cmol_err_t. */
int cmol__sched_selftest(int threads, int steps, long wait_us, long device_us, unsigned host_us,
                         uint64_t stats[3]);

int cmol__session_length(const cmol_session_t *s);
int cmol__session_slot(const cmol_session_t *s);
cmolhip_model_t *cmol__device(cmol_model_t *m);

#ifdef __cplusplus
}
#endif
#endif
