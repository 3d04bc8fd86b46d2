/*
 * oracle.h — CPU restatement of libcmol's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This code is the checker for the MI355X
 * implementation: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never links it.
 *
 * Every function restates the reference arithmetic (same operation order,
 * same rounding points) and cites the reference file:line it follows.
 * Pinning (what checks each function against something independent):
 *   o_f16_to_f32        golden bit patterns from the built reference
 *                       (all 65536 halves) + IEEE special cases
 *   o_dequant_row       reference KATs tests/test_quant.c:97-127, golden
 *                       vectors from the built reference (Q8_0, Q5_0, F16,
 *                       F32); Q4_0 by lossless transcoding to Q8_0 and by
 *                       the closed form d*(nibble-8)
 *   o_matmul (both orders) reference KATs tests/test_quant.c:217-320 and
 *                       bit-exact golden outputs of cmol_matmul_scalar /
 *                       cmol_matmul_avx512 built from the reference
 *   o_rms_norm/softmax/swiglu/rope   KATs tests/test_model.c:45-166, closed
 *                       forms, bit-exact vs the built reference
 *   o_forward / o_generate  bit-exact logits and token IDs vs the built
 *                       reference's cmol_model_forward on synthetic GGUFs
 *                       (Q4_0 via transcoding), brute-force float64
 *                       attention on tiny shapes
 */
#ifndef CMOL_ORACLE_H
#define CMOL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF dtype tags used on the path (reference src/cmol_internal.h:27-37). */
enum { O_F32 = 0, O_F16 = 1, O_Q4_0 = 2, O_Q5_0 = 6, O_Q8_0 = 8, O_Q4_K = 12, O_Q6_K = 14 };

/* Matmul accumulation orders of the reference kernels. */
enum { O_ORDER_SCALAR = 0,   /* cmol_matmul_scalar  src/quant.c:334-376 */
       O_ORDER_AVX512 = 1 }; /* cmol_matmul_avx512  src/quant.c:488-566 */

float  o_f16_to_f32(uint16_t h);
uint16_t o_f32_to_f16(float f);
size_t o_row_bytes(int k, int dtype);
int    o_block_params(int dtype, size_t *bsz);
void   o_dequant_row(const void *src, float *dst, int n, int dtype);
void   o_matmul(float *out, const void *a, const float *b,
                int m, int k, int n, int dtype, int order);

void o_rms_norm(const float *x, const float *w, float *out, int n, float eps);
void o_softmax(float *x, int n);
void o_swiglu(const float *gate, const float *up, float *out, int n);
void o_rope_apply(float *q, float *k, int pos, int n_heads, int n_kv_heads,
                  int head_dim, float freq_base);
int  o_argmax(const float *logits, int n);
void o_apply_repeat_penalty(float *logits, int vocab, const int32_t *tokens,
                            int n_tokens, float penalty);

/* Attention for one token of one layer over an fp32 cache laid out
 * [pos][n_kv][d_head] (one layer slice); writes out[n_heads*d_head]. */
void o_attention(const float *q, const float *kc, const float *vc,
                 int seqlen, int n_heads, int n_kv, int d_head,
                 float *scores, float *out);

/* ---- whole model ------------------------------------------------------ */
typedef struct o_model o_model_t;
typedef struct o_sess  o_sess_t;

/* hparams, in this order: n_layers, n_heads, n_kv_heads, d_model, d_head,
 * d_ffn, vocab, model_max_ctx, no_rope_interval, tie, eos_id            */
o_model_t *o_model_load(const char *gguf_path, int order, int nthreads);
void       o_model_free(o_model_t *m);
void       o_model_hparams(const o_model_t *m, int32_t out[11],
                           float out_f[2]);
o_sess_t  *o_sess_new(o_model_t *m, int max_ctx);
/* on != 0: every K/V value is rounded to fp16 (o_f32_to_f16) as it is
 * written to the cache, as in an fp16 KV cache; the cache stays fp32
 * storage.  No reference counterpart (its cache is fp32). */
void       o_sess_kv_f16(o_sess_t *s, int on);
void       o_sess_free(o_sess_t *s);
/* One forward step (reference src/model.c:176-276); returns logits. */
const float *o_forward(o_model_t *m, o_sess_t *s, int32_t token, int pos);
/* Prefill `n_prompt` tokens from `pos0` then greedy-decode `n_new`; fills
 * out_tokens[n_new]; optional per-step top-2 margin in margins[n_new].
 * repeat_penalty <= 1 disables the penalty (reference src/api.c:412-524). */
int o_generate_greedy(o_model_t *m, o_sess_t *s, const int32_t *prompt,
                      int n_prompt, int pos0, int n_new, float repeat_penalty,
                      int repeat_last_n, int32_t *out_tokens, float *margins);
/* Raw access to the session KV cache, layout [layer][pos][n_kv][d_head]. */
float *o_sess_k(o_sess_t *s);
float *o_sess_v(o_sess_t *s);
/* Copy of the last logits (vocab floats). */
const float *o_sess_logits(o_sess_t *s);

#ifdef __cplusplus
}
#endif
#endif
