/*
 * cmol_hip.h — C ABI of the MI355X (gfx950) backend of libcmol.
 *
 * This is the platform backend that sits beside the reference's CPU
 * platform layer (reference src/platform.h:21-63) and replaces the CPU
 * kernel seam:
 *   cmol_matmul_fn_t / cmol_kernels_t   reference src/cmol_internal.h:175-187
 *   cmol_kernels_select                  reference src/quant.c:676-705
 *   cmol_dequant_row                     reference src/quant.c:241-289
 *   cmol_attn_forward                    reference src/attn.c:27-146
 *   cmol_model_forward                   reference src/model.c:176-276
 * Plain pointers and sizes only; every call returns a cmol_err_t value
 * (0 = CMOL_OK, negative = error).  Device memory comes from one arena that
 * is allocated once (cmolhip_ctx_create / cmolhip_model_create); no entry
 * point allocates device memory afterwards.
 */
#ifndef CMOL_HIP_H
#define CMOL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device context --------------------------------------------------- */
typedef struct cmolhip_ctx cmolhip_ctx_t;

/* Number of visible GPUs (0 when none or the runtime is unusable). */
int cmolhip_device_count(void);
/* Select `device`, create a stream and one device arena of `arena_bytes`. */
int cmolhip_ctx_create(int device, size_t arena_bytes, cmolhip_ctx_t **out);
void cmolhip_ctx_destroy(cmolhip_ctx_t *c);
/* Bump-allocate from the arena (never calls the device allocator). */
int cmolhip_alloc(cmolhip_ctx_t *c, size_t bytes, size_t align, void **dptr);
size_t cmolhip_arena_used(const cmolhip_ctx_t *c);
size_t cmolhip_arena_size(const cmolhip_ctx_t *c);
int cmolhip_memcpy_h2d(cmolhip_ctx_t *c, void *dst, const void *src, size_t n);
int cmolhip_memcpy_d2h(cmolhip_ctx_t *c, void *dst, const void *src, size_t n);
int cmolhip_memcpy_d2d(cmolhip_ctx_t *c, void *dst, const void *src, size_t n);
int cmolhip_synchronize(cmolhip_ctx_t *c);
/* The context's hipStream_t, for callers that time work with HIP events. */
void *cmolhip_stream(cmolhip_ctx_t *c);

/* ---- quantised weights in the device layout -----------------------------
 * GGUF block formats Q4_0 (2), Q5_0 (6) and Q8_0 (8) are repacked at upload
 * into tiles of 16 MFMA columns x 4 blocks matched to the gfx950 MFMA
 * operand layout (bit-preserving: codes and fp16 scales are moved, never
 * re-quantised).  With fold F (1, 2, 4 or 8) a tile holds 16/F rows and the
 * k range is cut into F parts that share the tile's 16 columns, so narrow
 * matrices still spread over every compute unit at batch 1. */
typedef struct {
    void   *qs;          /* packed codes                                  */
    void   *d;           /* fp16 scales                                   */
    void   *qh;          /* Q5_0 fifth bits, NULL for other formats       */
    int32_t dtype;       /* GGUF dtype id                                 */
    int32_t rows;        /* output features                               */
    int32_t cols;        /* input features (multiple of 32)               */
    int32_t row_tiles;   /* ceil(rows / (16 / fold))                      */
    int32_t block_quads; /* block quads per k part                        */
    int32_t fold;        /* k parts per tile: 1, 2, 4 or 8                */
} cmolhip_qtensor_t;

/* Device bytes a tensor needs (0 when dtype/shape/fold is unsupported). */
size_t cmolhip_qtensor_bytes(int dtype, int rows, int cols, int fold);

/* The fold cmolhip_model_create gives a rows x cols projection of a model
 * with max_sessions sessions (1 for models serving several sessions). */
int cmolhip_pick_fold(int rows, int cols, int max_sessions);

#define CMOLHIP_PARTS_CONCAT     0 /* parts stacked row-wise              */
#define CMOLHIP_PARTS_INTERLEAVE 1 /* two parts, rows alternate p0,p1,... */

/* Upload raw GGUF rows (host memory) of `n_parts` tensors sharing dtype and
 * cols into one device tensor.  `staging` is device scratch of at least
 * staging_bytes >= largest part's raw size. */
int cmolhip_qtensor_upload(cmolhip_ctx_t *c, int dtype, int cols, int fold, int n_parts,
                           const void *const *parts, const int32_t *part_rows,
                           int mode, void *staging, size_t staging_bytes,
                           cmolhip_qtensor_t *out);

/* fp32 dequantisation of the whole tensor to dout[rows][cols] (device),
 * bit-identical to the reference's cmol_dequant_row row by row. */
int cmolhip_dequant(cmolhip_ctx_t *c, const cmolhip_qtensor_t *t, float *dout);

/* dy[n][rows] = W . dx[n][cols] for n activation vectors (fp32 accumulate).
 * When norm_w != NULL each x is RMS-normalised first (weights norm_w[cols],
 * epsilon eps).  n in 1..65535: up to 32 vectors run the streaming matvec,
 * more the tiled MFMA GEMM (64 vectors x 128 rows per work-group).  Device
 * pointers; runs on the context stream. */
int cmolhip_gemm(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const float *dx,
                 float *dy, int n, const float *norm_w, float eps);

/* The same product in two steps, for callers that reuse one activation
 * operand: cmolhip_act_prepare converts dx[n][cols] (optionally keeping
 * per-32-input sums of squares for an RMSNorm with weights norm_w) into the
 * device operand `op` of cmolhip_act_bytes(cols, n) bytes for weights of
 * dtype `dtype`; cmolhip_gemm_prepared runs the matvec on it (ss as written
 * by the prepare step, or NULL without norm). */
size_t cmolhip_act_bytes(int cols, int n);
int cmolhip_act_prepare(cmolhip_ctx_t *c, const float *dx, int n, int cols, int dtype,
                        const float *norm_w, void *op, float *ss);
int cmolhip_gemm_prepared(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const void *op, int n,
                          const float *ss, float eps, float *dy);
/* cmolhip_gemm_prepared whose kernel records two hipEvent_t (start, stop)
 * at its own start and end, for kernel-only timing. */
int cmolhip_gemm_prepared_timed(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const void *op,
                                int n, const float *ss, float eps, float *dy, void *ev_start,
                                void *ev_stop);

/* No reference counterpart.  cmolhip_gemm for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * device allocation): the same product, computed by the same kernels, with
 * every piece of scratch (the activation operand, the RMSNorm partial sums,
 * the batched matvec's k-split partial sums and those of the split-K
 * prompt GEMM for narrow matrices) in one fixed device array
 * of cmolhip_noalloc_scratch_bytes() bytes (16 MiB) per GPU, held from the
 * first cmolhip_ctx_create on that GPU until the process ends.  It calls no
 * allocator, host or device, and does not touch the context's arena.  A call
 * whose scratch would exceed the array (operand act_bytes(cols, n), plus
 * n*cols/32 floats with norm_w, plus the k-split sums of 9..32 vectors or
 * of the prompt GEMM's 2-4 k ranges: ranges x n x rows floats)
 * returns CMOL_ERR_ARGS without launching anything.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other threads or
 * other streams) race, so callers serialise them; each call writes all the
 * scratch it reads, so nothing carries over from the previous call. */
int cmolhip_gemm_noalloc(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const float *dx,
                         float *dy, int n, const float *norm_w, float eps);
size_t cmolhip_noalloc_scratch_bytes(void);

/* Reference kernel seam replacement (cmol_matmul_fn_t semantics on host
 * memory, src/cmol_internal.h:175-187): out[m][n] = A[m][k] . B[k][n], A raw
 * GGUF rows.  Block formats need k a multiple of 32; F32 (dtype 0) and F16
 * (dtype 1) rows take any k and give the reference AVX-512 kernel's results
 * bit for bit (src/quant.c:506-530).  Uses the context arena for the
 * transient copies; fails with CMOL_ERR_OOM when the arena cannot hold
 * them. */
int cmolhip_matmul_host(cmolhip_ctx_t *c, float *out, const void *a,
                        const float *b, int m, int k, int n, int dtype);

/* Decode attention (reference src/attn.c:103-137) for `n` sessions whose
 * fp32 or fp16 caches are stacked as [n][n_kv][max_ctx][d_head]; q is
 * [n][n_heads*d_head] after RoPE, seqlen[n] (device int32) the number of
 * positions attended, out [n][n_heads*d_head].  Each work-group covers
 * `split` positions (a multiple of 64, or of 32 for d_head 64 / 128; 0
 * picks 64) and splits are merged with log-sum-exp rescaling.  Device
 * pointers. */
int cmolhip_attn_decode(cmolhip_ctx_t *c, int n, const float *q,
                        const void *kcache, const void *vcache,
                        const int32_t *seqlen, int n_heads, int n_kv,
                        int d_head, int max_ctx, int kv_f16, int split, float *out);

/* ---- whole-model decode path ------------------------------------------- */
typedef struct cmolhip_model cmolhip_model_t;

typedef struct {
    int32_t n_layers, n_heads, n_kv_heads, d_model, d_head, d_ffn, vocab;
    int32_t max_ctx, max_sessions, no_rope_interval, kv_f16;
    int32_t prefill_chunk;   /* prompt tokens per batched prefill pass (<= 0: 512) */
    float   rope_base, rms_eps;
} cmolhip_hparams_t;

typedef struct {
    const void *data;    /* host pointer into the mapped GGUF            */
    int32_t dtype;       /* GGUF dtype id                                 */
    int32_t rows, cols;  /* rows = GGUF shape[1] (out), cols = shape[0]  */
} cmolhip_host_tensor_t;

typedef struct {
    cmolhip_host_tensor_t attn_norm, q, k, v, o, q_norm, k_norm,
                          ffn_norm, gate, up, down;
} cmolhip_layer_tensors_t;

typedef struct {
    cmolhip_hparams_t hp;
    cmolhip_host_tensor_t embd, out_norm, lm_head;
    const cmolhip_layer_tensors_t *layers;   /* [n_layers] */
    const float *rope_table;                 /* [max_ctx][d_head/2][cos,sin] */
} cmolhip_model_desc_t;

/* Validate the description and report the device arena it needs. */
int cmolhip_model_plan(const cmolhip_model_desc_t *desc, size_t *device_bytes);
/* Launch planning, without a device.  The batched matvec (9..32 vectors)
 * may split k over work-groups and keep partial sums in a scratch buffer:
 * cmolhip_gemv_scratch_floats gives the floats one launch over a rows x
 * cols tensor (dtype, fold) of n vectors needs (0: no split, or a shape it
 * does not run); cmolhip_batch_scratch_floats the scratch a model reserves
 * for a batch of up to cap vectors (the largest need of any launch of a
 * decode step of 1..cap vectors; q, k and v launch once per run of parts
 * that share a format).  A launch whose need exceeds the scratch it is
 * given is refused with CMOL_ERR_ARGS.  These replace no reference
 * interface: the reference's n > 1 matvec (src/quant.c:546-553) needs no
 * scratch. */
size_t cmolhip_gemv_scratch_floats(int dtype, int rows, int cols, int fold, int n);
int cmolhip_batch_scratch_floats(const cmolhip_model_desc_t *desc, int cap, size_t *floats);
/* Allocate the arena once, upload every tensor, create per-session streams
 * and capture each session's decode graph.  Nothing is allocated later. */
int cmolhip_model_create(const cmolhip_model_desc_t *desc, int device,
                         cmolhip_model_t **out);
void cmolhip_model_destroy(cmolhip_model_t *m);
cmolhip_ctx_t *cmolhip_model_ctx(cmolhip_model_t *m);

/* One decode step of session `slot` (reference cmol_model_forward):
 * token at position pos.  logits_host (vocab floats) and argmax are
 * optional outputs; argmax is the first index of the maximum logit. */
int cmolhip_decode(cmolhip_model_t *m, int slot, int32_t token, int32_t pos,
                   float *logits_host, int32_t *argmax);
/* 1 when cmolhip_decode runs the model's single session with the persistent
 * kernel (one cooperative launch per token; no device-wide barrier: each
 * stage's readers poll the vectors they consume; opt-in with CMOL_PERSIST=1
 * at model creation), 0 when it replays the per-kernel decode graph. */
int cmolhip_model_persistent(cmolhip_model_t *m);
/* Profiling of the persistent kernel (model created with CMOL_PERSIST_TRACE=1
 * in the environment): device timestamps (100 MHz wall clock) of the last
 * decode step, out[0] when work-group 0 started and out[1] when it ended.
 * Returns the count written (0 when tracing is off). */
int cmolhip_persist_trace(cmolhip_model_t *m, uint64_t *out, int cap);
/* Per-work-group stage times of the last step (same profiling mode):
 * out[stage][work-group][8] for the stages embedding, then per layer QKV,
 * attention, merge, Wo, gate/up, down, then the LM head: [0] the io waves
 * start polling the stage's input, [1] the input is complete, [2] the
 * stage's outputs are issued, [3] the mac waves start the stage's products,
 * [4] their products are done, [5] their next weights are issued; [6] the
 * work-group ends (last stage only) (0 where a work-group had no part).
 * Returns the work-group count, CMOL_ERR_TRUNC when cap is too small. */
int cmolhip_persist_marks(cmolhip_model_t *m, uint64_t *out, size_t cap);
/* Lock-step decode of n sessions (distinct slots, each at its own pos).
 * logits_host: NULL or [n][vocab]. */
int cmolhip_decode_batch(cmolhip_model_t *m, int n, const int32_t *slots,
                         const int32_t *tokens, const int32_t *pos,
                         float *logits_host, int32_t *argmax);
/* As cmolhip_decode_batch, with each vector's logits copied to its own host
 * buffer: logits_each NULL, or n pointers each NULL (no copy) or [vocab]
 * (the cross-session scheduler hands each session its own logits). */
int cmolhip_decode_batch_each(cmolhip_model_t *m, int n, const int32_t *slots,
                              const int32_t *tokens, const int32_t *pos,
                              float *const *logits_each, int32_t *argmax);
/* Prompt of n tokens at positions pos0.. into session `slot`, in batched
 * passes of prefill_chunk tokens (prompt GEMMs on MFMA, causal attention
 * over the cache); outputs as in cmolhip_decode for the last prompt token. */
int cmolhip_prefill(cmolhip_model_t *m, int slot, const int32_t *tokens, int n,
                    int32_t pos0, float *logits_host, int32_t *argmax);

/* KV cache of one session and layer in the reference layout
 * [pos][n_kv][d_head] fp32 for positions [0, n). */
int cmolhip_kv_download(cmolhip_model_t *m, int slot, int layer, int n,
                        float *k_out, float *v_out);
int cmolhip_kv_upload(cmolhip_model_t *m, int slot, int layer, int n,
                      const float *k_in, const float *v_in);
/* Fill positions [0, n) of every layer with seeded synthetic values. */
int cmolhip_kv_fill_synthetic(cmolhip_model_t *m, int slot, int n, uint64_t seed);
/* Stream of a session slot (hipStream_t), for event timing. */
void *cmolhip_session_stream(cmolhip_model_t *m, int slot);

#ifdef __cplusplus
}
#endif
#endif
