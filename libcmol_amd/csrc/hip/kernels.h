// kernels.h — device-side tensor view and the host launchers each kernel
// translation unit exports to the C-ABI layer (cmol_hip.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Device view of a quad-tiled quantised tensor (see common.h).
struct QTensor {
    uint8_t *qs;
    uint16_t *d;
    uint32_t *qh;
    int dtype, rows, cols, row_tiles, block_quads;
};

// KV caches of one layer for a batch of activation vectors: vector n uses
// slot slot_ids[n], whose K cache starts at k_base + slot*slot_stride +
// layer_off elements (fp32 or fp16 per kv_f16).
struct KVRef {
    void *k_base, *v_base;
    size_t slot_stride, layer_off;
    const int32_t *slot_ids;
};

__device__ inline size_t kv_offset(const KVRef &r, int n)
{
    return (size_t)r.slot_ids[n] * r.slot_stride + r.layer_off;
}

// ---- qtensor.hip
// Repack `rows` raw GGUF rows into destination rows row0.. (concat) or
// 2*(row0+i)+part (interleave).
int launch_repack(const QTensor &t, const uint8_t *raw, int rows, int row0,
                  int mode, int part, hipStream_t s);
int launch_dequant(const QTensor &t, float *out, hipStream_t s);
int launch_embed(const QTensor &t, const int32_t *token, int token_stride, float *x,
                 int x_stride, unsigned long long *argmax, int n, hipStream_t s);

// ---- gemv.hip
// The LM-head argmax of one vector is spread over this many 64-bit slots
// (work-group t uses slot t % ARGMAX_SLOTS); the host reduces the slots.
#define ARGMAX_SLOTS 64

enum GemvEpilogue {
    EPI_STORE = 0,   // out[n][row] = y
    EPI_RESID = 1,   // out[n][row] += y
    EPI_SWIGLU = 2,  // rows interleaved gate/up: out[n][row/2] = silu(g)*u
    EPI_QKV = 3,     // q rows -> q_out (RoPE), k/v rows -> KV cache at pos
    EPI_LOGITS = 4,  // out[n][row] = y and argmax over rows
};

struct GemvArgs {
    QTensor w;
    const float *x;         // activations [n][x_stride]
    int x_stride;
    const float *norm_w;    // RMSNorm weights [cols] or nullptr
    float eps;
    float *out;             // epilogue output [n][out_stride]
    int out_stride;
    int n;                  // activation vectors (sessions)
    // EPI_QKV
    int nq, nkv, d_head, max_ctx, kv_f16, rope_on;
    const float *rope;      // [max_ctx][d_head/2][2]
    KVRef kv;               // caches of this layer (layout [n_kv][max_ctx][d_head])
    const int32_t *pos;     // per-vector position, pos[n * pos_stride]
    int pos_stride;
    // EPI_LOGITS
    unsigned long long *argmax;   // ARGMAX_SLOTS slots per vector
};

int launch_gemv(const GemvArgs &a, int epi, hipStream_t s);

// ---- attn.hip
struct AttnArgs {
    const float *q;         // [n][n_heads*d_head]
    int q_stride;
    KVRef kv;               // caches of this layer
    const int32_t *seqlen;  // per-vector attended length, seqlen[n * seqlen_stride]
    int seqlen_stride;
    int n, n_heads, n_kv, d_head, max_ctx, kv_f16;
    int split;              // positions per work-group
    int max_splits;
    float *pm, *pl, *po;    // partials [n][n_kv][max_splits][G]( [d_head])
    float *out;             // [n][out_stride]
    int out_stride;
};

int launch_attn(const AttnArgs &a, hipStream_t s);
int attn_max_splits(int max_ctx, int split);

// ---- misc.hip
int launch_fill_f32(float *p, size_t n, float v, hipStream_t s);
int launch_kv_synth(void *kc, void *vc, int n_kv, int max_ctx, int d_head,
                    int n_tokens, int kv_f16, uint64_t seed, hipStream_t s);
int launch_kv_convert(const void *src, float *dst, int n_kv, int max_ctx,
                      int d_head, int n, int kv_f16, int to_ref, hipStream_t s);
int launch_kv_import(const float *src, void *dst, int n_kv, int max_ctx,
                     int d_head, int n, int kv_f16, hipStream_t s);
