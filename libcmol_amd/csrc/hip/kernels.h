// kernels.h — device-side tensor views and the host launchers each kernel
// translation unit exports to the C-ABI layer (cmol_hip.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

// Device view of a quad-tiled quantised tensor (see common.h).
struct QTensor {
    uint8_t *qs;
    uint16_t *d;
    uint32_t *qh;
    int dtype, rows, cols, row_tiles, block_quads, fold;
};

// ---------------------------------------------------------------------------
// Per-format lane data of one (cell, lane) and the per-block contraction,
// shared by the matvec, batched matvec and GEMM kernels.
// ---------------------------------------------------------------------------
// Scales of a cell's column: 4 fp16 (32-value blocks) or the K-quant record.
template <int DT> struct QScale { typedef u32x2 T; };
template <> struct QScale<DT_Q4_K> { typedef u32x4 T; };
template <> struct QScale<DT_Q6_K> { typedef u32x4 T; };

// Load instructions per (cell, lane): codes (1, or 2 for Q8_0) + scales +
// Q5_0 fifth bits / Q6_K high bits.
template <int DT>
constexpr int q_loads()
{
    return (DT == DT_Q8_0 ? 2 : 1) + 1 + (DT == DT_Q5_0 || DT == DT_Q6_K ? 1 : 0);
}

// Codes of lane `lane` and scales of column `col` of cell `cell`: c1 holds
// the second half of the Q8_0 codes or the Q6_K high bits (.x blocks 0-1, .y
// blocks 2-3); h the Q5_0 fifth bits.
template <int DT>
__device__ __forceinline__ void q_load(const QTensor &w, size_t cell, int col, int lane, u32x4 &c0,
                                       u32x4 &c1, typename QScale<DT>::T &sv, uint32_t &h)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    const u32x4 *p = (const u32x4 *)(w.qs + (cell * 64 + lane) * LB);
    c0 = p[0];
    if constexpr (DT == DT_Q8_0) c1 = p[1];
    else if constexpr (DT == DT_Q6_K) {
        const u32x2 hb = *(const u32x2 *)(w.qh + (cell * 64 + lane) * 2);
        c1 = u32x4{hb[0], hb[1], 0u, 0u};
    } else c1 = u32x4{0, 0, 0, 0};
    if constexpr (is_kquant(DT)) sv = *(const u32x4 *)((const uint8_t *)w.d + (cell * 16 + col) * 16);
    else sv = *(const u32x2 *)(w.d + cell * 64 + col * 4);
    if constexpr (DT == DT_Q5_0) h = w.qh[cell * 64 + lane];
    else h = 0u;
}

// fp32 factors of block bi: s0 multiplies A . codes; Q4_K adds s1 times the
// operand's block sum (the min, plus 8 d sc for the codes' -8 bias); Q6_K
// scales the low (s0) and high (s1) 16 values of the block separately.
struct BlockScale {
    float s0, s1;
};

__device__ __forceinline__ float f16lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float f16hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

template <int DT>
__device__ __forceinline__ BlockScale block_scale(const typename QScale<DT>::T &sv, int bi)
{
#pragma clang fp contract(off)
    BlockScale r;
    if constexpr (DT == DT_Q4_K) {
        const uint32_t sm = (sv[1 + (bi >> 1)] >> (16 * (bi & 1))) & 0xFFFFu;
        const float db = f16lo(sv[0]) * (float)(sm & 0xFFu);
        r.s0 = db;
        r.s1 = 8.0f * db - f16hi(sv[0]) * (float)(sm >> 8);
    } else if constexpr (DT == DT_Q6_K) {
        const uint32_t ss = (sv[1 + (bi >> 1)] >> (16 * (bi & 1))) & 0xFFFFu;
        const float d = f16lo(sv[0]);
        r.s0 = d * (float)(int8_t)(ss & 0xFFu);
        r.s1 = d * (float)(int8_t)(ss >> 8);
    } else {
        const uint32_t dw = sv[bi >> 1];
        r.s0 = (bi & 1) ? f16hi(dw) : f16lo(dw);
        r.s1 = 0.0f;
    }
    return r;
}

// acc += the block's contribution for A rows xv against decoded codes wv.
template <int DT>
__device__ __forceinline__ void mfma_block(f32x4 &acc, const f16x8 &xv, const f16x8 &wv, const BlockScale &s)
{
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (DT == DT_Q4_K) {
        const f16x8 ones = {(_Float16)1, (_Float16)1, (_Float16)1, (_Float16)1,
                            (_Float16)1, (_Float16)1, (_Float16)1, (_Float16)1};
        const f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, z, 0, 0, 0);
        const f32x4 cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, ones, z, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s1, cs[i], fmaf(s.s0, cc[i], acc[i]));
    } else if constexpr (DT == DT_Q6_K) {
        const _Float16 o = (_Float16)0;
        const f16x8 wl = {wv[0], wv[1], wv[2], wv[3], o, o, o, o};
        const f16x8 wh = {o, o, o, o, wv[4], wv[5], wv[6], wv[7]};
        const f32x4 cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wl, z, 0, 0, 0);
        const f32x4 ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wh, z, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s1, ch[i], fmaf(s.s0, cl[i], acc[i]));
    } else {
        const f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, z, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s0, cc[i], acc[i]);
    }
}

// KV caches of one layer for a batch of activation vectors: vector n uses
// slot slot_ids[n], whose K cache starts at k_base + slot*slot_stride +
// layer_off elements (fp32 or fp16 per kv_f16); without slot_ids every
// vector uses k_base + layer_off.
struct KVRef {
    void *k_base, *v_base;
    size_t slot_stride, layer_off;
    const int32_t *slot_ids;
};

__device__ inline size_t kv_offset(const KVRef &r, int n)
{
    return (r.slot_ids ? (size_t)r.slot_ids[n] * r.slot_stride : 0) + r.layer_off;
}

// ---------------------------------------------------------------------------
// Activation operands.
//
// A matvec consumes its activation vectors already in MFMA A-operand form:
// for block b (32 inputs), k-group g (0..3) and operand row r the 8 halves
// q[((b*4 + g)*nrows + r)*8 + e] hold input 32b + kmap(dt, g, e), where
// operand row 2n is the f16 rounding hi of t = vector n times ACT_SCALE and
// row 2n+1 the f16 rounding of the remainder (t - hi) times LO_SCALE.  The
// two rows land in separate MFMA result rows, so the consumer forms
// (hi + lo / LO_SCALE) / ACT_SCALE with exact power-of-two factors: 22
// significant bits for |x| in [2^-6, 2^24), an absolute error below 2^-28
// under that, and exact products with the integer codes.  When the
// consumer starts with an RMSNorm the producer stores w (.) x instead of x
// and per-tile sums of x^2; the consumer applies 1/sqrt(mean + eps) in its
// epilogue (the matvec is linear).  Producers of these operands: the
// embedding gather, residual-add / SwiGLU epilogues, attention, and
// k_act_prep for standalone calls.
// ---------------------------------------------------------------------------
#define ACT_SCALE (1.0f / 256.0f)
#define ACT_INV_SCALE 256.0f
#define LO_SCALE 2048.0f
#define LO_INV_SCALE (1.0f / 2048.0f)

// ---------------------------------------------------------------------------
// Store policies.  Plain stores suffice when a kernel boundary separates a
// producer from its consumers.  Inside the persistent decode kernel a value
// written by one work-group is read by others after a device-wide barrier,
// possibly on another XCD, whose L2 is not coherent with the writer's: those
// stores are relaxed agent-scope atomic stores (sc1: written through to
// memory).  Every buffer that kernel hands over is written once per launch
// before any work-group reads it, so the loads stay plain.
// ---------------------------------------------------------------------------
struct StPlain {
    template <typename T> __device__ static void st(T *p, T v) { *p = v; }
};
struct StDev {
    __device__ static void st(float *p, float v)
    {
        __hip_atomic_store(gptr((uint32_t *)p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __device__ static void st(_Float16 *p, _Float16 v)
    {
        __hip_atomic_store(gptr((uint16_t *)p), __builtin_bit_cast(uint16_t, v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
};

struct ActOut {
    _Float16 *q;            // operand buffer of the consumer
    int dt;                 // consumer weight format (selects kmap)
    int nrows;              // 2 * vectors
    const float *norm_w;    // consumer RMSNorm weights, or nullptr
    float *ss;              // sum-of-squares partials [vector][ss_stride]
    int ss_stride;
};

struct ActIn {
    const _Float16 *q;      // operand buffer (layout above)
    int nrows;              // 2 * vectors
    const float *ss;        // partials [vector][ss_stride] or nullptr (no norm)
    int ss_count, ss_stride;
    float eps;
    // the struct's tail dword as a field: the kernels pin it with the other
    // arguments, so the wide argument load that fetches it beside ss_count,
    // ss_stride and eps keeps its register live, and the next argument load
    // cannot target that register while the wide load is still in flight
    // (which made the compiler wait for a second round trip)
    int tail;
};

// ---- qtensor.hip
// Repack `rows` raw GGUF rows into destination rows row0.. (concat, mode 0)
// or 2*(row0+i)+part (interleave, mode 1).
int launch_repack(const QTensor &t, const uint8_t *raw, int rows, int row0,
                  int mode, int part, hipStream_t s);
int launch_dequant(const QTensor &t, float *out, hipStream_t s);
// Embedding rows of n vectors -> x (fp32) and the first consumer's operand.
int launch_embed(const QTensor &t, const int32_t *token, int token_stride, float *x,
                 int x_stride, const ActOut &o, unsigned long long *argmax, int n,
                 hipStream_t s);

// ---- gemv.hip
// The LM-head argmax of one vector is spread over this many 64-bit slots
// (work-group t uses slot t % ARGMAX_SLOTS); the host reduces the slots.
#define ARGMAX_SLOTS 64

enum GemvEpilogue {
    EPI_STORE = 0,   // out[n][row] = y
    EPI_RESID = 1,   // out[n][row] += y, then the next consumer's operand
    EPI_SWIGLU = 2,  // rows interleaved gate/up: silu(g)*u -> operand (+ out)
    EPI_QKV = 3,     // q rows -> out (RoPE), k/v rows -> KV cache at pos
    EPI_LOGITS = 4,  // out[n][row] = y and argmax over rows
};

struct GemvArgs {
    QTensor w;
    ActIn in;
    float *out;             // epilogue output [n][out_stride]
    int out_stride;
    const float *res;       // EPI_RESID: residual input [n][out_stride] (nullptr: out itself)
    int n;                  // activation vectors
    ActOut next;            // EPI_RESID / EPI_SWIGLU: operand of the consumer
    // EPI_QKV (row_base: first output row of this launch in the q|k|v rows,
    // when the three are split over tensors of different formats)
    int nq, nkv, d_head, max_ctx, kv_f16, rope_on, row_base;
    const float *rope;      // [max_ctx][d_head/2][2]
    KVRef kv;
    const int32_t *pos;     // per-vector position, pos[n * pos_stride] (nullptr: pos0)
    int pos_stride, pos0;
    // EPI_LOGITS
    unsigned long long *argmax;   // ARGMAX_SLOTS slots per vector
    // when set, recorded at the kernel's own start and end (kernel timing)
    hipEvent_t ev_start, ev_stop;
    // batches of more than 8 vectors: k-split partial sums of part_cap
    // floats; a launch needing more (gemv_part_floats(w, n)) is refused
    float *part;
    size_t part_cap;
};

int launch_gemv(const GemvArgs &a, int epi, hipStream_t s);
// Scratch floats a batched (n > 8) matvec over w needs for its k-split
// partial sums (0 when it does not split k).
size_t gemv_part_floats(const QTensor &w, int n);
// Most k ranges a split-K prompt GEMM takes (its partial sums go to a.part).
#define GEMM_KS_MAX 4
// The same product for many vectors (prompt tokens): 64-vector x 128-row
// output tiles, epilogues EPI_STORE..EPI_QKV; any n >= 1.  With a.part,
// narrow matrices whose tiles would not fill the chip split k (fp32 partial
// sums, then the k-split finish).
int launch_gemm(const GemvArgs &a, int epi, hipStream_t s);
// Partial-sum floats the split-K prompt GEMM of n vectors over w takes when
// given room without limit (0 when it does not split).
size_t gemm_part_floats(const QTensor &w, int n);
// x [n][x_stride] fp32 -> operand (and sum-of-squares partials per 32 inputs).
int launch_act_prep(const float *x, int x_stride, int K, int n, const ActOut &o, hipStream_t s);
// Operand bytes for K inputs (padded to whole block quads) and n vectors.
size_t act_bytes(int K, int n);

// ---- attn.hip
#define ATT_MAX_G 8          // query heads per kv head
#define ATT_MAX_MERGE 1024   // splits one merge can combine

struct AttnArgs {
    const float *q;         // [n][n_heads*d_head]
    int q_stride;
    KVRef kv;               // caches of this layer
    const int32_t *seqlen;  // per-vector attended length, seqlen[n * seqlen_stride]
    int seqlen_stride;
    int n, n_heads, n_kv, d_head, max_ctx, kv_f16;
    int split;              // positions per work-group
    int max_splits;
    int bal;                // > 0 (fp16 cache, d_head 64..256): bal balanced ranges per
                            // kv head instead of one work-group per split; partials
                            // [n_kv][bal + n][G]( [d_head]), bal + n <= n * max_splits
    float *pm, *pl, *po;    // partials [n][n_kv][max_splits][G]( [d_head])
    float *out;             // [n][out_stride] fp32, or nullptr
    int out_stride;
    ActOut next;            // operand of the output projection (q == nullptr: none)
};

int launch_attn(const AttnArgs &a, hipStream_t s);
// Balanced ranges per kv head (AttnArgs::bal) for n vectors over a cache
// planned with max_splits splits, or 0 where they do not apply (one vector,
// fp32 cache, d_head outside 64..256).  The grid is bal + n work-groups per
// kv head; CMOL_ATTN_BAL=<total work-groups> sets it (0: off).  The
// default is one round of the four work-groups a CU holds.
#define ATT_BAL_WGS_PER_CU 4
int attn_bal_wgs(int n, int n_kv, int d_head, int kv_f16, int max_splits);
int launch_attn_bal(const AttnArgs &a, hipStream_t s);   // a.bal > 0 (launch_attn calls it)
// The split merge with one wave per (query head, vector), d_head 64 / 128:
// prompt passes (the split layout of launch_attn).
int launch_attn_merge_wave(const AttnArgs &a, hipStream_t s);
// Prompt-pass attention (flash style on MFMA) for vectors that are
// consecutive tokens of one session over an fp32 cache, d_head 64 / 128;
// returns -4 for shapes it does not take (the caller runs launch_attn).
// kv_hl: attn_prompt_kv_bytes of scratch for the high/low f16 copy of the
// session's cache positions 0 .. last-1 (last = the pass's largest seqlen).
int launch_attn_prompt(const AttnArgs &a, _Float16 *kv_hl, int last, hipStream_t s);
size_t attn_prompt_kv_bytes(int n_kv, int d_head, int max_ctx);

// QK-norm models (src/attn.c:62-101): the QKV matvec stores raw q|k|v rows;
// this stage normalises each q and k head (RMSNorm over d_head, weights
// shared by the heads), applies RoPE and writes q and the KV cache.
struct QkArgs {
    const float *raw;        // [n][raw_stride]: q rows, then k, then v
    int raw_stride;
    float *q;                // [n][q_stride]
    int q_stride;
    const float *qn_w, *kn_w;   // [d_head] or nullptr (no norm of that part)
    float eps;
    int n, n_heads, n_kv, d_head, max_ctx, kv_f16, rope_on;
    const float *rope;       // [max_ctx][d_head/2][2]
    const int32_t *pos;      // pos[v * pos_stride]
    int pos_stride;
    KVRef kv;
};
int launch_qk_rope(const QkArgs &a, hipStream_t s);
int attn_max_splits(int max_ctx, int split);

// ---- persist_q4/q5/q8.hip: the persistent single-session decode kernel
// One cooperative launch per token, one work-group of PK_THREADS per CU.
// Waves 0..PK_IO-1 ("io waves") poll the vectors a stage consumes, stage
// them into LDS, run attention's softmax bookkeeping and the split merge and
// store those results; waves PK_IO.. ("mac waves") hold the weight rings,
// prefetch weights and the KV tile ahead of need and run the matvecs.
// Stages hand over fp32 vectors through exchange buffers that start each
// launch filled with PK_POISON (a signalling-NaN pattern no arithmetic
// produces): a reader waits until every element it needs differs from it.
// The buffers are double-buffered by launch parity, and during a launch each
// work-group refills the elements it writes with PK_POISON in the other
// parity's (idle) buffers, ready for the next launch.
#define PK_THREADS 512
#define PK_WAVES (PK_THREADS / 64)
#define PK_IO 4                     // io waves
#define PK_MAC (PK_WAVES - PK_IO)   // mac waves
#define PK_SPIN_MAX (1 << 16)       // poll rounds of one wait before it gives up
#define PK_MAX_WGS 1024
#define PK_POISON 0x7FBADBADu
#define PK_KV_POS 64                // attention positions staged in LDS per chunk
#define PK_MSLICE 32                // output dimensions per merge item
#define PK_MAXI 8                   // (block, group) items per io thread: inputs <= 16384
#define PK_ZW_TILES 64              // tiles of one matrix per mac wave (tile scratch)
#define PK_MARKS 8                  // profiling marks per (stage, work-group)

// Exchange vectors of one layer and launch parity.
struct PkEx {
    float *q;          // roped queries [d]
    float *kn, *vn;    // this position's K and V rows [n_kv * d_head], as cached
    float *part;       // attention split partials [n_heads][max_splits][d_head + 4]: o, m, l
    float *att;        // attention output [d]
    float *xa;         // residual after the attention block [d]
    float *h;          // SwiGLU output [d_ffn]
    float *xo;         // layer output [d]
};

// Weights of one layer and its exchange buffers (device copy, read-only).
struct PkLayer {
    QTensor qkv, o, gu, down;
    const float *attn_norm, *ffn_norm;
    int rope_on;
    size_t kv_off;     // layer offset in the KV caches (elements)
    PkEx ex[2];
};

struct PkArgs {
    const PkLayer *layers;
    int n_layers;
    QTensor embd, lm;
    const float *out_norm, *rope;
    float *x0;                     // embedding rows [2][d], by parity
    float *logits;                 // [vocab]
    unsigned long long *argmax;    // [ARGMAX_SLOTS]
    void *k_base, *v_base;
    size_t slot_stride;
    const int32_t *slot_id;        // device [1]: the session's KV slot
    const int32_t *step;           // device {token, pos, seqlen}
    int d, n_heads, n_kv, d_head, d_ffn, max_ctx, kv_f16, max_splits;
    int op_bytes;                  // LDS operand area (largest matrix operand + zero slot)
    float eps;
    int par;                       // this launch's exchange-buffer set: launches since the last reset, mod 2
    int *err;                      // set when a wait gave up (the step's outputs are invalid)
    unsigned long long *trace;     // optional: work-group 0's stage times
    unsigned long long *marks;     // optional: [stage][work-group][PK_MARKS] phase times
};

// Positions per attention split for attended length L (at most max_splits
// splits, every work-group an item while there are positions for it).
__host__ __device__ inline int pk_split(int L, int max_splits)
{
    const int s = (L + max_splits - 1) / max_splits;
    return s < 1 ? 1 : s;
}

// Stages one launch passes: the embedding, 6 per layer (QKV, attention,
// merge, Wo, gate/up, down), the LM head.
__host__ __device__ inline int pk_stages(int n_layers) { return 2 + 6 * n_layers; }

// LDS layout of the kernel (byte offsets).
struct PkLds {
    int op, kv, xr1, xr2, q, sc, red, ss, zw, ml, mrg, total;
};
__host__ __device__ inline PkLds pk_lds(int op_bytes, int d, int d_head, int kv_f16, int G, int max_splits)
{
    PkLds L;
    int o = 0;
    auto take = [&](int bytes) { const int r = o; o += (bytes + 15) & ~15; return r; };
    L.op = take(op_bytes);                                   // matvec operand (+ zero slot)
    L.kv = take(2 * PK_KV_POS * d_head * (kv_f16 ? 2 : 4));   // K rows, then V rows
    L.xr1 = take(4 * d);                                     // residual of the Wo stage (fp32)
    L.xr2 = take(4 * d);                                     // residual of the down stage (fp32)
    L.q = take(4 * G * d_head);                              // the item's queries; merge rows
    L.sc = take(4 * G * PK_KV_POS);                          // scores / weights
    L.red = take(4 * G * d_head);                            // attention output accumulators
    L.ss = take(4 * 16);                                     // io waves' sums of squares, nrm
    L.zw = take(4 * 16 * PK_ZW_TILES * PK_MAC);              // mac waves' tile scratch
    L.ml = take(4 * 4 * 8);                                  // running max / sum / alpha per head
    L.mrg = take(4 * max_splits * (PK_MSLICE + 2));          // merge: the splits' rows
    L.total = o;
    return L;
}
// LDS the matvec operand of a matrix needs (all k parts, padding blocks, a
// zero slot).
__host__ __device__ inline int pk_op_bytes(int fold, int block_quads) { return 4 * fold * block_quads * 128 + 16; }

// Launch (cooperative, nwg work-groups, lds dynamic LDS bytes) for layer
// format q4/q5/q8; 0, -4 unsupported shape, -5 launch failure.
int launch_persist_q4(const PkArgs &a, int nwg, int lds, hipStream_t s);
int launch_persist_q5(const PkArgs &a, int nwg, int lds, hipStream_t s);
int launch_persist_q8(const PkArgs &a, int nwg, int lds, hipStream_t s);
// Work-groups such a launch keeps resident (0: it cannot run here).
int persist_capacity_q4(int d_head, int kv_f16, int lds);
int persist_capacity_q5(int d_head, int kv_f16, int lds);
int persist_capacity_q8(int d_head, int kv_f16, int lds);

// ---- misc.hip
// dst[cols][rows] = transpose of src[rows][cols] (fp32).
int launch_transpose(const float *src, float *dst, int rows, int cols, hipStream_t s);
// The kernel seam's F32 (dtype 0) and F16 (dtype 1) weight products:
// out[m][n] = A[m][k] . x[n][k]^T in the reference AVX-512 kernel's order.
int launch_matmul_dense(const void *a, int dtype, const float *x, float *out, int m, int k, int n, hipStream_t s);
// out[i] = i, i < n.
int launch_iota(int32_t *out, int n, hipStream_t s);
int launch_kv_synth(void *kc, void *vc, int n_kv, int max_ctx, int d_head,
                    int n_tokens, int kv_f16, uint64_t seed, hipStream_t s);
int launch_kv_convert(const void *src, float *dst, int n_kv, int max_ctx,
                      int d_head, int n, int kv_f16, int to_ref, hipStream_t s);
int launch_kv_import(const float *src, void *dst, int n_kv, int max_ctx,
                     int d_head, int n, int kv_f16, hipStream_t s);
// Vector v of an n-vector operand (K inputs) -> one-vector operand, and its
// sum-of-squares partials (ss_src may be null).
int launch_act_extract(const _Float16 *src, int K, int n, int v, _Float16 *dst, const float *ss_src,
                       int ss_stride, int ss_count, float *ss_dst, hipStream_t s);

// Writes value v of input k of vector n into an operand (see ActOut).
template <typename M = StPlain>
__device__ inline void act_put(const ActOut &o, int n, int k, float v)
{
#pragma clang fp contract(off)
    const float t = (o.norm_w ? o.norm_w[k] * v : v) * ACT_SCALE;
    const _Float16 hi = (_Float16)t;
    const _Float16 lo = (_Float16)((t - (float)hi) * LO_SCALE);
    const int b = k >> 5, kk = k & 31;
    int g, e;
    if (o.dt == 8) {
        g = kk >> 3;
        e = kk & 7;
    } else {
        const int hi16 = kk >> 4, r = kk & 15;   // kmap inverse for the nibble order
        g = r >> 2;
        const int j = r & 3;
        e = hi16 * 4 + (j == 1 ? 2 : j == 2 ? 1 : j);
    }
    const size_t base = (((size_t)b * 4 + g) * o.nrows + 2 * n) * 8 + e;
    M::st(o.q + base, hi);
    M::st(o.q + base + 8, lo);
}
