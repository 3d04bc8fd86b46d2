// persist_impl.h — the persistent single-session decode kernel: one launch
// per token runs the embedding gather, every layer (QKV + RoPE + KV write,
// split-K attention and its merge, Wo + residual, gate/up + SwiGLU, down +
// residual) and the LM head with argmax, with device-wide barriers between
// the stages instead of kernel boundaries.  Instantiated per layer weight
// format by persist_q4.hip / persist_q5.hip / persist_q8.hip.
//
// The launch is cooperative (every work-group resident, one per CU) and each
// work-group has PK_THREADS threads.  Stages:
//   * matvec (pk_gemv): tile t of the matrix belongs to wave t mod W of the
//     launch's W waves (wave w = wid * nwg + wg, so neighbouring tiles land on
//     different CUs); a wave streams the quads of its tiles through a ring of
//     U loads and finishes each tile on its own (one MFMA column set per
//     tile: R rows x F k parts), so no work-group-wide reduction is needed.
//     Each work-group first copies the whole operand (and the RMSNorm
//     partials) into LDS.
//   * attention: work-group w takes (kv head, split) items w, w + nwg, ...;
//     splits are sized so the items cover the work-groups; a merge stage
//     follows when there is more than one split.
// Data handed from one stage to the next is plain fp32 vectors in per-layer
// buffers, written once per launch with write-through stores (StDev) before
// the barrier that precedes their first read, so readers on other XCDs see
// the new values with plain loads.  A matvec stage converts the vector it
// consumes into its MFMA operand (high/low f16 parts, RMSNorm weights
// applied) while staging it into LDS, and forms the RMSNorm scale from the
// same values.
#pragma once
#include "attn_impl.h"
#include "gemv_impl.h"
#include "qtensor_impl.h"

// Profiling marks of this work-group's current stage (null: off): [0] left
// the previous barrier, [1] operand and first weights in LDS/registers,
// [2] work done (entering the barrier), [3] own stores drained.
__shared__ unsigned long long *pk_mark;

__device__ inline void pk_mark_at(int i)
{
    if (pk_mark && threadIdx.x == 0) pk_mark[i] = wall_clock64();
}

__device__ inline unsigned ld_dev(const unsigned *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_dev(unsigned *p, unsigned v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait for *p >= target: gives up (and flags the launch) after
// PK_SPIN_MAX polls, or early once another wait of the launch gave up, so
// every wave always reaches the end of the kernel.
__device__ inline void pk_spin(const unsigned *p, unsigned target, int *err)
{
    for (int i = 0; ld_dev(p) < target; i++) {
        if (i >= PK_SPIN_MAX || ((i & 255) == 255 && ld_dev((const unsigned *)err) != 0)) {
            atomicOr(err, 1);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Device-wide barrier in three parts.  pk_arrive: every wave drains its
// stores, then the work-group announces itself; work-group 0 collects every
// arrival word and raises one release word per group of work-groups (8
// groups, so at most nwg/8 pollers share a word).  pk_poll: thread 0 polls
// its group's release word.  pk_sync: the work-group's waves meet.  Loads
// that do not depend on other work-groups (the next stage's weights) are
// issued around the poll: by waves 1.. before it, by wave 0 after it, so
// they never delay the poll's own loads.
__device__ inline void pk_arrive(const PkArgs &a, unsigned target)
{
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x;
    pk_mark_at(2);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    pk_mark_at(3);
    if (tid == 0) st_dev(a.sync + 16 * wg, target);
    if (wg == 0) {
        for (int w = tid; w < nwg; w += PK_THREADS) pk_spin(a.sync + 16 * w, target, a.err);
        __syncthreads();
        if (tid < 8) st_dev(a.sync + 16 * PK_MAX_WGS + 32 * tid, target);
        if (a.trace && tid == 0) a.trace[target - a.epoch0] = wall_clock64();
    }
}

__device__ inline void pk_poll(const PkArgs &a, unsigned target)
{
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x;
    if (tid == 0) pk_spin(a.sync + 16 * PK_MAX_WGS + 32 * (wg & 7), target, a.err);
    if (a.marks && tid == 0) pk_mark = a.marks + ((size_t)(target - a.epoch0) * nwg + wg) * 4;
}

// Execution barrier of the work-group without a memory fence (a fence would
// make every wave wait for its outstanding loads, the prefetches included).
__device__ inline void pk_sync()
{
    __builtin_amdgcn_s_barrier();
    pk_mark_at(0);
}

// Weight ring of one wave: U in-flight quads (codes, scales, fifth bits).
template <int DT>
struct PkRing {
    static constexpr int U = (DT == DT_Q8_0) ? 6 : 8;
    u32x4 c0[U], c1[U];
    u32x2 dv[U];
    uint32_t hv[U];
};

// The calling wave's share of a matrix: tile t belongs to wave t mod W of
// the launch (wave w = wid * nwg + wg, so neighbouring tiles land on
// different CUs); its items are the quads of its tiles, len in all.
struct PkWork {
    int gw, W, len;
};

__device__ __forceinline__ PkWork pk_work(const QTensor &w)
{
    PkWork k;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    k.W = PK_WAVES * gridDim.x;
    k.gw = wid * gridDim.x + blockIdx.x;
    const int ntw = k.gw < w.row_tiles ? (w.row_tiles - 1 - k.gw) / k.W + 1 : 0;
    k.len = ntw * w.block_quads;
    return k;
}

// Loads item i (clamped to the wave's last item) into ring slot u.
template <int DT>
__device__ __forceinline__ void pk_load(PkRing<DT> &r, int u, const QTensor &w, const PkWork &k, int i)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    const int l = threadIdx.x & 63, BQ = w.block_quads;
    i = min(i, k.len - 1);
    const int kt = i / BQ, q = i - kt * BQ;
    const size_t cell = (size_t)(k.gw + kt * k.W) * BQ + q;
    const auto *p = gptr((const u32x4 *)(w.qs + (cell * 64 + l) * LB));
    r.c0[u] = p[0];
    if constexpr (LB == 32) r.c1[u] = p[1];
    else r.c1[u] = u32x4{0, 0, 0, 0};
    r.dv[u] = *gptr((const u32x2 *)(w.d + cell * 64 + (l & 15) * 4));
    if constexpr (DT == DT_Q5_0) r.hv[u] = *gptr(w.qh + cell * 64 + l);
    else r.hv[u] = 0u;
}

// Slot u holds nothing (keeps no earlier stage's registers alive).
template <int DT>
__device__ __forceinline__ void pk_clear(PkRing<DT> &r, int u)
{
    r.c0[u] = u32x4{0, 0, 0, 0};
    r.c1[u] = u32x4{0, 0, 0, 0};
    r.dv[u] = u32x2{0, 0};
    r.hv[u] = 0u;
}

// The wave's first min(U, len) items of matrix w.
template <int DT>
__device__ __forceinline__ void pk_prefetch(PkRing<DT> &r, const QTensor &w)
{
    const PkWork k = pk_work(w);
#pragma unroll
    for (int u = 0; u < PkRing<DT>::U; u++) {
        if (u < k.len) pk_load(r, u, w, k, u);
        else pk_clear(r, u);
    }
}

// MFMA operand of the fp32 vector x[K] (times norm_w when given) for weight
// format DT, written into LDS in the layout of kernels.h (n = 1: row 0 the
// high f16 part of x*ACT_SCALE, row 1 the scaled low part), one (block,
// k-group) per thread and step: two float4 loads, one 16-byte LDS store per
// row.  Returns this thread's share of sum(x^2).
template <int DT>
__device__ __forceinline__ float pk_stage_x(const float *x, const float *norm_w, int nblk, uint8_t *s_op)
{
#pragma clang fp contract(off)
    float ss = 0.0f;
    for (int it = threadIdx.x; it < nblk * 4; it += PK_THREADS) {
        const int b = it >> 2, g = it & 3;
        // kmap: Q8_0 k = 8g + e; Q4_0/Q5_0 k = (e>=4 ? 16 : 0) + 4g + {0,2,1,3}[e&3]
        const int k0 = 32 * b + (DT == DT_Q8_0 ? 8 * g : 4 * g);
        const int k1 = k0 + (DT == DT_Q8_0 ? 4 : 16);
        const float4 a = ldg((const float4 *)(x + k0)), c = ldg((const float4 *)(x + k1));
        float v[8];
        if constexpr (DT == DT_Q8_0) {
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
        } else {
            v[0] = a.x; v[1] = a.z; v[2] = a.y; v[3] = a.w;
            v[4] = c.x; v[5] = c.z; v[6] = c.y; v[7] = c.w;
        }
        float wn[8];
        if (norm_w) {
            const float4 wa = ldg((const float4 *)(norm_w + k0)), wc = ldg((const float4 *)(norm_w + k1));
            if constexpr (DT == DT_Q8_0) {
                wn[0] = wa.x; wn[1] = wa.y; wn[2] = wa.z; wn[3] = wa.w;
                wn[4] = wc.x; wn[5] = wc.y; wn[6] = wc.z; wn[7] = wc.w;
            } else {
                wn[0] = wa.x; wn[1] = wa.z; wn[2] = wa.y; wn[3] = wa.w;
                wn[4] = wc.x; wn[5] = wc.z; wn[6] = wc.y; wn[7] = wc.w;
            }
        }
        f16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            ss += v[e] * v[e];
            const float t = (norm_w ? wn[e] * v[e] : v[e]) * ACT_SCALE;
            hi[e] = (_Float16)t;
            lo[e] = (_Float16)((t - (float)hi[e]) * LO_SCALE);
        }
        *(f16x8 *)(s_op + (size_t)(it * 2) * 16) = hi;
        *(f16x8 *)(s_op + (size_t)(it * 2 + 1) * 16) = lo;
    }
    return ss;
}

// One matvec stage for the single activation vector (n = 1), consuming the
// fp32 vector xin (RMSNorm with weights norm_w when given).  With `pre` the
// wave's ring was filled before the stage (pk_prefetch).
// EPI_LOGITS keeps each wave's best (value, row) key and merges it into the
// argmax slots once at the end.
template <int DT, int EPI>
__device__ __forceinline__ void pk_gemv(const GemvArgs &a, const float *xin, const float *norm_w, float eps,
                                        uint8_t *smem, PkRing<DT> &r, bool pre)
{
#pragma clang fp contract(off)
    constexpr int U = PkRing<DT>::U;
    const int tid = threadIdx.x, l = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int BQ = a.w.block_quads, F = a.w.fold, R = 16 / F;
    const int nblk = a.w.cols >> 5;
    const int opb = 4 * F * BQ * 128;
    uint8_t *s_op = smem;                                 // operand + 16 zero bytes at opb
    float *s_zw = (float *)(smem + opb + 16) + 16 * wid;  // this wave's tile scratch
    float *s_ssw = (float *)(smem + opb + 16) + 16 * PK_WAVES;   // per-wave sums of squares
    const PkWork k = pk_work(a.w);
    if (!pre) pk_prefetch(r, a.w);

    // ---- 1. epilogue inputs of the wave's first tile (residual rows, RoPE
    // pairs), then the operand built in LDS ----
    const int row0 = k.gw * R + l;
    const bool pre_ok = k.len > 0 && l < R && row0 < a.w.rows;
    float pres = 0.0f;
    float2 pcs = make_float2(1.0f, 0.0f);
    if constexpr (EPI == EPI_RESID)
        if (pre_ok) pres = *gptr(a.res + row0);
    if constexpr (EPI == EPI_QKV)
        if (pre_ok) pcs = rope_cs(a, row0, a.pos0);
    float ss = pk_stage_x<DT>(xin, norm_w, nblk, s_op);
    lds_zero<PK_WAVES>(s_op + nblk * 128, opb + 16 - nblk * 128, tid);
    if (norm_w) {
        ss = wave_sum(ss);
        if (l == 0) s_ssw[wid] = ss;
    }
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
    __builtin_amdgcn_s_barrier();
    pk_mark_at(1);

    // ---- 2. RMSNorm scale (every wave, the waves' sums in a fixed order) ----
    float nrm = 1.0f;
    if (norm_w) {
        float s = 0.0f;
        for (int w = 0; w < PK_WAVES; w++) s += s_ssw[w];
        nrm = 1.0f / sqrtf(s / (float)a.w.cols + eps);
    }

    // A row fed by this lane: 2p + h = high (h = 0) or scaled low (h = 1) part
    // of k part p; rows past 2F read the zero slot
    const int g = l >> 4, ar = l & 15;
    const bool aok = ar < 2 * F;
    const int abase = aok ? (ar >> 1) * 4 * BQ * 128 + (g * 2 + (ar & 1)) * 16 : opb;
    const int astride = aok ? 128 : 0;

    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc = zero4;
    unsigned long long best = 0ull;

    // tile end: lane l (column c = part c/R x row c%R) keeps the high/low
    // pair of its own part; lanes 0..R-1 sum the F parts of row l in order
    auto finish_tile = [&](int kt) {
        const int t = k.gw + kt * k.W;
        const int c = l & 15, pc = c / R, rc = c % R;
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int pp = 2 * (l >> 4) + qq;
            if (pp < F && pp == pc) s_zw[rc * F + pp] = acc[2 * qq] + acc[2 * qq + 1] * LO_INV_SCALE;
        }
        float z = 0.0f;
        if (l < R)
            for (int p = 0; p < F; p++) z += s_zw[l * F + p];
        float y = z * ACT_INV_SCALE;
        if (norm_w) y *= nrm;
        const int row = t * R + l;
        const bool act = l < R && row < a.w.rows;
        if constexpr (EPI == EPI_LOGITS) {
            if (act) *gptr(a.out + row) = y;
            const unsigned long long key = act ? argmax_key(y, (uint32_t)row) : 0ull;
            best = key > best ? key : best;
        } else if constexpr (EPI == EPI_RESID) {
            const float x = act ? (kt == 0 ? pres : *gptr(a.res + row)) + y : 0.0f;
            resid_out<StDev>(a, t, l, R, 0, act, x);
        } else if constexpr (EPI == EPI_QKV) {
            const float partner = __shfl_xor(y, 1, 64);
            if (act) qkv_out<StDev>(a, 0, row, y, partner, kt == 0 ? pcs : rope_cs(a, row, a.pos0), a.pos0,
                                    kv_offset(a.kv, 0));
        } else {
            epilogue<EPI, StDev>(a, t, l, R, 0, l < R, y);
        }
        acc = zero4;
    };
    auto compute = [&](int u, int i) {
        const float dsc[4] = {
            (float)__builtin_bit_cast(_Float16, (uint16_t)(r.dv[u][0] & 0xFFFFu)),
            (float)__builtin_bit_cast(_Float16, (uint16_t)(r.dv[u][0] >> 16)),
            (float)__builtin_bit_cast(_Float16, (uint16_t)(r.dv[u][1] & 0xFFFFu)),
            (float)__builtin_bit_cast(_Float16, (uint16_t)(r.dv[u][1] >> 16))};
        const int kt = i / BQ, q = i - kt * BQ;
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            const f16x8 wv = deq_block<DT>(r.c0[u], r.c1[u], r.hv[u], bi);
            const f16x8 xv = *(const f16x8 *)(s_op + abase + (4 * q + bi) * astride);
            const f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, zero4, 0, 0, 0);
            acc[0] = fmaf(dsc[bi], cc[0], acc[0]);
            acc[1] = fmaf(dsc[bi], cc[1], acc[1]);
            acc[2] = fmaf(dsc[bi], cc[2], acc[2]);
            acc[3] = fmaf(dsc[bi], cc[3], acc[3]);
        }
        if (q == BQ - 1) finish_tile(kt);
    };
    // rounds of U: while another round follows, slot u is refilled right
    // after use (rolling prefetch); the last round issues no loads
    for (int i0 = 0; i0 < k.len; i0 += U) {
        if (i0 + U < k.len) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                compute(u, i0 + u);
                pk_load(r, u, a.w, k, i0 + u + U);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++)
                if (i0 + u < k.len) compute(u, i0 + u);
        }
    }
    if constexpr (EPI == EPI_LOGITS) {
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(best, o, 64);
            best = other > best ? other : best;
        }
        if (l == 0 && best)
            __hip_atomic_fetch_max(gptr(a.argmax + (k.gw & (ARGMAX_SLOTS - 1))), best, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();   // the LDS operand area is rewritten by the next stage
}

template <int EPI>
__device__ __forceinline__ void pk_gemv_any(const GemvArgs &g, const float *xin, const float *norm_w, float eps,
                                            uint8_t *smem)
{
    switch (g.w.dtype) {
    case DT_Q4_0: { PkRing<DT_Q4_0> r; pk_gemv<DT_Q4_0, EPI>(g, xin, norm_w, eps, smem, r, false); break; }
    case DT_Q5_0: { PkRing<DT_Q5_0> r; pk_gemv<DT_Q5_0, EPI>(g, xin, norm_w, eps, smem, r, false); break; }
    default: { PkRing<DT_Q8_0> r; pk_gemv<DT_Q8_0, EPI>(g, xin, norm_w, eps, smem, r, false); break; }
    }
}

template <int DL, int DH, typename KT>
__global__ __launch_bounds__(PK_THREADS) void k_persist(PkArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    unsigned ep = a.epoch0;
    if (a.trace && wg == 0 && tid == 0) a.trace[0] = wall_clock64();
    if (tid == 0) pk_mark = a.marks ? a.marks + (size_t)wg * 4 : nullptr;
    __syncthreads();
    pk_mark_at(0);
    const int L = min(a.step[2], a.max_ctx);
    const int pos = min(max(a.step[1], 0), a.max_ctx - 1);
    const size_t slot_off = (size_t)a.slot_id[0] * a.slot_stride;
    void *const k_base = a.k_base, *const v_base = a.v_base;
    const int split = pk_split(L, a.n_kv, nwg);
    const int nsplit = (L + split - 1) / split;
    const int kvd = a.n_kv * a.d_head;
    PkRing<DL> ring;
    // end of a stage: barrier at epoch ep + 1; the rings of the next matrix
    // (when there is one) are filled around the poll
    auto cross = [&](const QTensor *next) {
        pk_arrive(a, ++ep);
        if (next && wid != 0) pk_prefetch(ring, *next);
        pk_poll(a, ep);
        if (next && wid == 0) pk_prefetch(ring, *next);
        pk_sync();
    };

    // ---- embedding row -> x0; argmax slots cleared ----
    {
        ActOut o{};
        if (wg == 0 && tid < ARGMAX_SLOTS)
            __hip_atomic_store(a.argmax + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int tok = a.step[0];
        const int nthr = (a.d / 32) * 4;
        for (int g0 = wg * PK_THREADS; g0 < nthr; g0 += nwg * PK_THREADS) {
            switch (a.embd.dtype) {
            case DT_Q4_0: embed_group<DT_Q4_0, StDev>(a.embd, tok, g0 + tid, a.x0, o, 0); break;
            case DT_Q5_0: embed_group<DT_Q5_0, StDev>(a.embd, tok, g0 + tid, a.x0, o, 0); break;
            default: embed_group<DT_Q8_0, StDev>(a.embd, tok, g0 + tid, a.x0, o, 0); break;
            }
        }
    }
    {
        const QTensor w0 = a.layers[0].qkv;
        cross(&w0);
    }

    for (int li = 0; li < a.n_layers; li++) {
        const PkLayer &Yl = a.layers[li];
        const QTensor w_qkv = Yl.qkv, w_o = Yl.o, w_gu = Yl.gu, w_down = Yl.down;
        float *const q = Yl.q, *const att = Yl.att;
        float *const x_attn = Yl.x_attn, *const x_ffn = Yl.x_ffn, *const h = Yl.h;
        const float *const x_in = li == 0 ? a.x0 : a.layers[li - 1].x_ffn;
        KVRef kv;
        kv.k_base = k_base;
        kv.v_base = v_base;
        kv.slot_stride = a.slot_stride;
        kv.layer_off = slot_off + Yl.kv_off;
        kv.slot_ids = nullptr;

        // RMSNorm + QKV + RoPE + KV write
        {
            GemvArgs g{};
            g.w = w_qkv;
            g.out = q;
            g.out_stride = a.d;
            g.n = 1;
            g.nq = a.d;
            g.nkv = kvd;
            g.d_head = a.d_head;
            g.max_ctx = a.max_ctx;
            g.kv_f16 = a.kv_f16;
            g.rope_on = Yl.rope_on;
            g.rope = a.rope;
            g.kv = kv;
            g.pos = nullptr;
            g.pos0 = pos;
            pk_gemv<DL, EPI_QKV>(g, x_in, Yl.attn_norm, a.eps, smem, ring, true);
        }
        cross(nullptr);

        // attention over the cache (+ merge of the splits)
        {
            AttnArgs at{};
            at.q = q;
            at.q_stride = a.d;
            at.kv = kv;
            at.seqlen = a.step + 2;
            at.seqlen_stride = 3;
            at.n = 1;
            at.n_heads = a.n_heads;
            at.n_kv = a.n_kv;
            at.d_head = a.d_head;
            at.max_ctx = a.max_ctx;
            at.kv_f16 = a.kv_f16;
            at.split = split;
            at.max_splits = a.max_splits;
            at.pm = Yl.pm;
            at.pl = Yl.pl;
            at.po = Yl.po;
            at.out = att;
            at.out_stride = a.d;
            for (int it = wg; it < a.n_kv * nsplit; it += nwg)
                attn_split<DH, KT, PK_THREADS, StDev>(at, it % a.n_kv, it / a.n_kv, 0);
            if (nsplit > 1) {
                cross(nullptr);
                for (int hq = wg; hq < a.n_heads; hq += nwg) attn_merge_head<DH, PK_THREADS, StDev>(at, hq, 0);
            }
            cross(&w_o);
        }

        // Wo + residual
        {
            GemvArgs g{};
            g.w = w_o;
            g.out = x_attn;
            g.res = x_in;
            g.out_stride = a.d;
            g.n = 1;
            pk_gemv<DL, EPI_RESID>(g, att, nullptr, a.eps, smem, ring, true);
        }
        cross(&w_gu);

        // RMSNorm + gate/up + SwiGLU
        {
            GemvArgs g{};
            g.w = w_gu;
            g.out = h;
            g.out_stride = 0;
            g.n = 1;
            pk_gemv<DL, EPI_SWIGLU>(g, x_attn, Yl.ffn_norm, a.eps, smem, ring, true);
        }
        cross(&w_down);

        // down + residual
        {
            GemvArgs g{};
            g.w = w_down;
            g.out = x_ffn;
            g.res = x_attn;
            g.out_stride = a.d;
            g.n = 1;
            pk_gemv<DL, EPI_RESID>(g, h, nullptr, a.eps, smem, ring, true);
        }
        if (li + 1 < a.n_layers) {
            const QTensor wn = a.layers[li + 1].qkv;
            cross(&wn);
        } else {
            cross(nullptr);
        }
    }

    // RMSNorm + LM head: logits and argmax
    {
        GemvArgs g{};
        g.w = a.lm;
        g.out = a.logits;
        g.out_stride = a.lm.rows;
        g.n = 1;
        g.argmax = a.argmax;
        pk_gemv_any<EPI_LOGITS>(g, a.layers[a.n_layers - 1].x_ffn, a.out_norm, a.eps, smem);
    }
    if (a.trace && wg == 0 && tid == 0) a.trace[ep - a.epoch0 + 1] = wall_clock64();
}

// Launches k_persist for layer format DL (cooperative: all work-groups
// resident).  Returns 0, -4 for an unsupported shape, or -5 when the launch
// itself fails.
template <int DL>
int launch_persist_dl(const PkArgs &a, int nwg, int lds, hipStream_t s)
{
    void *args[] = {(void *)&a};
    const void *f = nullptr;
    if (a.d_head == 64) f = a.kv_f16 ? (const void *)k_persist<DL, 64, _Float16> : (const void *)k_persist<DL, 64, float>;
    else if (a.d_head == 128) f = a.kv_f16 ? (const void *)k_persist<DL, 128, _Float16> : (const void *)k_persist<DL, 128, float>;
    else return -4;
    if (hipLaunchCooperativeKernel(f, dim3(nwg), dim3(PK_THREADS), args, (unsigned)lds, s) != hipSuccess) return -5;
    return 0;
}

// Work-groups the launch can keep resident (0: cannot run).
template <int DL>
int persist_capacity_dl(int d_head, int kv_f16, int lds)
{
    const void *f = nullptr;
    if (d_head == 64) f = kv_f16 ? (const void *)k_persist<DL, 64, _Float16> : (const void *)k_persist<DL, 64, float>;
    else if (d_head == 128) f = kv_f16 ? (const void *)k_persist<DL, 128, _Float16> : (const void *)k_persist<DL, 128, float>;
    else return 0;
    int per_cu = 0, dev = 0, cus = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, PK_THREADS, (size_t)lds) != hipSuccess ||
        per_cu < 1)
        return 0;
    return cus < PK_MAX_WGS ? cus : PK_MAX_WGS;
}
