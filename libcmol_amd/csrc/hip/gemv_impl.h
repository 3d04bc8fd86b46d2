// gemv_impl.h — the quantised matvec kernel template (see gemv.hip) and its
// per-format launchers; instantiated once per weight format by
// gemv_q4.hip / gemv_q5.hip / gemv_q8.hip so the three compile in parallel.
#pragma once
#include "common.h"
#include "kernels.h"

#include <hip/hip_ext.h>

#include <atomic>
#include <cstdlib>

// k-split finish of the batched matvec (gemv.hip): sums the `splits`
// partial sums of every (vector, row) in a fixed order and runs the epilogue.
int launch_gemv_b_finish(const GemvArgs &a, int epi, int splits, int ss_count, hipStream_t s);

// Launch shape of one matvec (host-computed, see plan_gemv).
struct GemvShape {
    int epi;        // GemvEpilogue
    int qpc;        // quads per wave per operand chunk
    int op_bytes;   // LDS bytes of the operand area (staged blocks + zero slot)
    int zslot;      // LDS byte offset of the 16 zero bytes unused operand rows read
    int ss_bytes;   // LDS bytes of the sum-of-squares partials
    int groups = 1; // vector groups of 8 (grid.y): more than 8 vectors run as n = 8 per work-group
};

template <typename M = StPlain>
__device__ inline void store_kv(void *base, int kv_f16, size_t idx, float v)
{
    if (kv_f16) M::st((_Float16 *)base + idx, (_Float16)v);
    else M::st((float *)base + idx, v);
}

// Sum / max over aligned groups of R lanes (R = 2, 4, 8 or 16).
__device__ inline float group_sum(float v, int R)
{
    for (int o = R >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Copies `bytes` (a multiple of 16) from global memory into LDS with
// direct-to-LDS loads, 1 KiB per wave instruction; lanes past the end are
// masked off.
template <int NW>
__device__ inline void stage_dma(const void *src, uint8_t *dst, int bytes, int wid, int l)
{
    for (int k = wid; k * 1024 < bytes; k += NW) {
        const int off = k * 1024 + l * 16;
        if (off < bytes)
            __builtin_amdgcn_global_load_lds((const gvoid_t *)((const uint8_t *)src + off),
                                             (lvoid_t *)(dst + k * 1024), 16, 0, 0);
    }
}

// The operand rows of vectors v0 .. v0 + nv - 1 (nv <= 8) of an nb-vector
// operand, gathered into LDS in the 8-vector layout: block k takes 1 KiB,
// [4 k-groups][16 rows][16 B]; lane l copies row l % 16 of k-group l / 16
// (rows past the group re-read its last row: their products are discarded).
template <int NW>
__device__ inline void stage_dma_group(const void *src, uint8_t *dst, int nblk, int nb, int v0, int nv, int wid,
                                       int l)
{
    const int r = 2 * v0 + min(l & 15, 2 * nv - 1);
    for (int k = wid; k < nblk; k += NW) {
        const uint8_t *p = (const uint8_t *)src + (((size_t)k * 4 + (l >> 4)) * 2 * nb + r) * 16;
        __builtin_amdgcn_global_load_lds((const gvoid_t *)p, (lvoid_t *)(dst + (size_t)k * 1024), 16, 0, 0);
    }
}

// Sum-of-squares partials [rows][stride] (count per row) packed into LDS as
// [rows][count], 4-byte direct-to-LDS loads.
template <int NW>
__device__ inline void stage_ss_dma(const float *src, int stride, int count, int rows, float *dst,
                                    int wid, int l)
{
    const int total = rows * count;
    for (int k = wid; k * 64 < total; k += NW) {
        const int f = k * 64 + l;
        if (f < total) {
            const int r = f / count, i = f - r * count;
            __builtin_amdgcn_global_load_lds((const gvoid_t *)(src + (size_t)r * stride + i),
                                             (lvoid_t *)(dst + k * 64), 4, 0, 0);
        }
    }
}

// Register-path copy for the chunked loop (direct-to-LDS loads issued inside
// the k loop would make later LDS reads wait for the whole weight ring).
template <int NW>
__device__ inline void stage_vgpr(const uint8_t *src, uint8_t *dst, int bytes, int tid)
{
    constexpr int STEP = NW * 64 * 16;
    for (int off = tid * 16; off < bytes; off += 4 * STEP) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int o = min(off + k * STEP, bytes - 16);
            v[k] = *(const u32x4 *)(src + o);
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (off + k * STEP < bytes) *(u32x4 *)(dst + off + k * STEP) = v[k];
    }
}

template <int NW>
__device__ inline void lds_zero(uint8_t *dst, int bytes, int tid)
{
    for (int off = tid * 16; off < bytes; off += NW * 64 * 16) *(u32x4 *)(dst + off) = u32x4{0, 0, 0, 0};
}

// Residual tail for row R*t + rl of vector v, x = residual + y already
// formed: stores x, the next consumer's operand and the tile's sum of
// squares.  Every lane of the wave calls it (shuffles in groups of R).
template <typename M>
__device__ __forceinline__ void resid_out(const GemvArgs &a, int t, int rl, int R, int v, bool act, float x)
{
#pragma clang fp contract(off)
    const int row = t * R + rl;
    if (act) {
        M::st(a.out + (size_t)v * a.out_stride + row, x);
        if (a.next.q) act_put<M>(a.next, v, row, x);
    }
    const float ss = group_sum(act ? x * x : 0.0f, R);
    if (act && rl == 0 && a.next.ss) M::st(a.next.ss + (size_t)v * a.next.ss_stride + t, ss);
}

// Position of vector v for the QKV epilogue, clamped to the cache.
__device__ __forceinline__ int epi_pos(const GemvArgs &a, int v)
{
    const int p = a.pos ? a.pos[(size_t)v * a.pos_stride] : a.pos0;
    return min(max(p, 0), a.max_ctx - 1);
}

// RoPE (cos, sin) of QKV output row `row` at position pos (identity for
// v rows or layers without RoPE).
__device__ __forceinline__ float2 rope_cs(const GemvArgs &a, int row, int pos)
{
    if (!a.rope_on || row >= a.nq + a.nkv) return make_float2(1.0f, 0.0f);
    const int rr = row < a.nq ? row : row - a.nq;
    const auto *cs = gptr(a.rope + ((size_t)pos * (a.d_head / 2) + ((rr % a.d_head) >> 1)) * 2);
    return make_float2(cs[0], cs[1]);
}

// QKV tail for row `row` of vector v: q rows (roped with cs) -> out, k rows
// (roped) and v rows -> the KV cache at pos; `partner` is the pair's other
// row (row ^ 1).
template <typename M>
__device__ __forceinline__ void qkv_out(const GemvArgs &a, int v, int row, float y, float partner, float2 cs, int pos,
                                        size_t kvo)
{
#pragma clang fp contract(off)
    if (row < a.nq + a.nkv) {
        const int rr = row < a.nq ? row : row - a.nq;
        const int i = rr % a.d_head;
        float val = y;
        if (a.rope_on) {
            if (!(i & 1)) val = y * cs.x - partner * cs.y;
            else val = partner * cs.y + y * cs.x;
        }
        if (row < a.nq) {
            M::st(a.out + (size_t)v * a.out_stride + row, val);
        } else {
            const int h = rr / a.d_head;
            store_kv<M>(a.kv.k_base, a.kv_f16, kvo + ((size_t)h * a.max_ctx + pos) * a.d_head + i, val);
        }
    } else {
        const int rr = row - a.nq - a.nkv;
        const int h = rr / a.d_head, i = rr % a.d_head;
        store_kv<M>(a.kv.v_base, a.kv_f16, kvo + ((size_t)h * a.max_ctx + pos) * a.d_head + i, y);
    }
}

// Epilogue inputs a matvec loads at its start, while its weights stream in,
// so that the epilogue does not wait on memory: the residual (EPI_RESID);
// the position, cache offset and RoPE (cos, sin) of the row (EPI_QKV).
struct EpiPre {
    float x = 0.0f;
    int pos = 0, slot = 0;
    size_t kvo = 0;
    float2 cs = {1.0f, 0.0f};
};

// First part, for output (vector v, row): three unconditional loads (a
// load whose value the epilogue does not need reads the operand buffer
// instead), so that no branch and no use of a loaded value makes the
// kernel wait here; epi_pre_cs interprets them.
__device__ __forceinline__ void epi_pre_load(const GemvArgs &a, int epi, int v, int row, bool act, EpiPre &p)
{
    const float *dummy = (const float *)a.in.q;
    const bool resid = act && epi == EPI_RESID, qkv = act && epi == EPI_QKV;
    const float *xa = resid ? (a.res ? a.res : a.out) + ((size_t)v * a.out_stride + row) : dummy;
    const int *pa = qkv && a.pos ? a.pos + (size_t)v * a.pos_stride : (const int *)dummy;
    const int *sa = qkv && a.kv.slot_ids ? a.kv.slot_ids + v : (const int *)dummy;
    p.x = *gptr(xa);
    p.pos = *gptr(pa);
    p.slot = *gptr(sa);
}

// Second part, once the first part's loads have landed: the clamped
// position, the cache offset, and the RoPE pair of the row.
__device__ __forceinline__ void epi_pre_cs(const GemvArgs &a, int epi, int row, bool act, EpiPre &p)
{
    if (act && epi == EPI_QKV) {
        const int pos = a.pos ? p.pos : a.pos0;
        p.pos = min(max(pos, 0), a.max_ctx - 1);
        p.kvo = (a.kv.slot_ids ? (size_t)p.slot * a.kv.slot_stride : 0) + a.kv.layer_off;
        p.cs = rope_cs(a, row + a.row_base, p.pos);
    }
}

// Epilogue for vector v, weight row R*t + rl.  Every lane of the wave calls
// it (shuffles within aligned groups of R lanes, one group per (vector,
// tile)); `act` marks lanes whose (row, v) is real.  With `has_pre`, `pre`
// holds this output's inputs loaded by epi_pre_load / epi_pre_cs.
template <int EPI, typename M = StPlain>
__device__ __forceinline__ void epilogue(const GemvArgs &a, int t, int rl, int R, int v, bool act, float y,
                                         bool has_pre = false, EpiPre pre = EpiPre())
{
#pragma clang fp contract(off)
    const int row = t * R + rl;
    act = act && row < a.w.rows;
    if constexpr (EPI == EPI_STORE) {
        if (act) M::st(a.out + (size_t)v * a.out_stride + row, y);
    } else if constexpr (EPI == EPI_RESID) {
        float x = 0.0f;
        if (act) {
            const size_t i = (size_t)v * a.out_stride + row;
            x = (has_pre ? pre.x : a.res ? a.res[i] : a.out[i]) + y;
        }
        resid_out<M>(a, t, rl, R, v, act, x);
    } else if constexpr (EPI == EPI_SWIGLU) {
        const float u = __shfl_xor(y, 1, 64);
        if (act && !(row & 1)) {
            const float h = (y / (1.0f + expf(-y))) * u;
            if (a.out) M::st(a.out + (size_t)v * a.out_stride + (row >> 1), h);
            if (a.next.q) act_put<M>(a.next, v, row >> 1, h);
        }
    } else if constexpr (EPI == EPI_QKV) {
        const float partner = __shfl_xor(y, 1, 64);
        if (act) {
            const int grow = row + a.row_base;
            if (has_pre) {
                qkv_out<M>(a, v, grow, y, partner, pre.cs, pre.pos, pre.kvo);
            } else {
                const int pos = epi_pos(a, v);
                qkv_out<M>(a, v, grow, y, partner, rope_cs(a, grow, pos), pos, kv_offset(a.kv, v));
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        if (act) a.out[(size_t)v * a.out_stride + row] = y;
        unsigned long long key = act ? argmax_key(y, (uint32_t)row) : 0ull;
        for (int o = R >> 1; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, 64);
            key = other > key ? other : key;
        }
        if (act && rl == 0)
            atomicMax(a.argmax + (size_t)v * ARGMAX_SLOTS + (t & (ARGMAX_SLOTS - 1)), key);
    }
}

// One work-group per row tile (16 MFMA columns: R = 16/F rows x F k parts).
// The activation operand of the whole k range is copied into LDS with
// direct-to-LDS loads issued before the weights (in chunks only when it
// exceeds the LDS budget); the NW waves split every k part into runs of qpc
// quads, and each wave streams its weight quads through a ring of U
// in-flight loads (one coalesced 16/32-byte load per lane per quad).
// DIRECT (one group, fold 1): no operand copy; each ring slot also loads
// the quad's four operand pieces of the lane from global memory.
//
// MFMA A rows: row 2(vF + p) + h is the high (h = 0) or scaled low (h = 1)
// f16 part of vector v restricted to k part p; column c of the tile holds
// part c / R, so only the entries with matching parts are used.  Each wave
// combines its high/low pairs and leaves the useful entries in LDS, where one
// thread per (vector, row) sums them over waves and parts in a fixed order.
//
// EPI >= 0 fixes the epilogue at compile time (the decode kernels: one
// straight code path, so that a launch's cold instruction cache fetches
// little); EPI < 0 takes it from sh.epi.
//
// The four-wave Q4_0 decode instances with a four-deep ring fit 80 VGPRs
// without spilling and are held there (six waves per SIMD, six work-groups
// per CU): pick_nw gives them matrices with more tiles than eight-wave
// groups can keep resident at once.
template <int DT, int NW, int NG, bool CHUNKED, int U, int EPI, bool DIRECT = false, bool GRP = false>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(DT == DT_Q4_0 && NW == 4 && NG == 1 && U == 4 && EPI != EPI_QKV && !DIRECT ? 6 : 1)))
void k_gemv(GemvArgs a, GemvShape sh)
{
    static_assert(!DIRECT || (NG == 1 && !CHUNKED), "direct operand: one group, no chunks");
    static_assert(!GRP || (NG == 1 && !CHUNKED && !DIRECT), "vector groups: one operand group, staged whole");
    // launch arguments needed before the weight loads go out, fetched in
    // one round trip
    sgpr_pin(a.w.qs);
    sgpr_pin(a.w.d);
    if constexpr (DT == DT_Q5_0 || DT == DT_Q6_K) sgpr_pin(a.w.qh);
    sgpr_pin(a.w.rows);
    sgpr_pin(a.w.cols);
    sgpr_pin(a.w.block_quads);
    sgpr_pin(a.w.fold);
    sgpr_pin(a.n);
    sgpr_pin(a.in.q);
    sgpr_pin(a.in.ss);
    sgpr_pin(a.in.ss_count);
    sgpr_pin(a.in.ss_stride);
    sgpr_pin(a.in.eps);
    sgpr_pin(a.in.tail);
    sgpr_pin(sh.qpc);
    sgpr_pin(sh.zslot);
    sgpr_pin(a.out);
    sgpr_pin(a.out_stride);
    // the epilogue's own arguments only where it can use them (fewer loads
    // in the batch)
    if constexpr (EPI < 0) sgpr_pin(sh.epi);
    if constexpr (EPI < 0 || EPI == EPI_RESID) sgpr_pin(a.res);
    if constexpr (EPI < 0 || EPI == EPI_QKV) {
        sgpr_pin(a.pos);
        sgpr_pin(a.pos_stride);
        sgpr_pin(a.kv.slot_ids);
    }
    const int epi = EPI >= 0 ? EPI : sh.epi;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *s_op = smem;
    float *s_ss = (float *)(smem + sh.op_bytes);
    float *s_nrm = (float *)(smem + sh.op_bytes + sh.ss_bytes);
    // vector group (GRP: grid.y runs over groups of 8 of more than 8
    // vectors): the work-group serves vectors v0 .. v0 + n - 1 of the batch,
    // its operand rows gathered into the 8-vector LDS layout (nl vectors);
    // a compile-time switch, so the decode instances keep their code
    constexpr bool grouped = GRP;
    const int v0 = grouped ? (int)blockIdx.y * 8 : 0;
    const int nl = grouped ? 8 : a.n;
    float *s_z = s_nrm + ((nl + 3) & ~3);

    // fold F = 2^lf (1..8) parts of R = 16/F = 2^lr rows per tile
    const int BQ = a.w.block_quads, F = a.w.fold, lf = __builtin_ctz(F), lr = 4 - lf, R = 1 << lr;
    const int t = blockIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
    const int n = grouped ? min(8, a.n - v0) : a.n;   // this work-group's vectors
    const int vb = 128 * nl;             // operand bytes per block in LDS
    const int nblk = a.w.cols >> 5;
    const int qpc = sh.qpc, cq = NW * qpc;
    const int nchunks = CHUNKED ? (BQ + cq - 1) / cq : 1;
    const int len = nchunks * qpc;
    const size_t cell0 = (size_t)t * BQ;

    // ---- 0. the epilogue inputs, when every output of the tile has a
    // thread of its own (one pass of step 6) ----
    const bool pre_on = n * R <= NW * 64;
    const int pv = (int)threadIdx.x >> lr, prow = t * R + ((int)threadIdx.x & (R - 1));
    const bool pact = pre_on && (int)threadIdx.x < n * R && prow < a.w.rows;
    EpiPre pre;
    epi_pre_load(a, epi, v0 + pv, prow, pact, pre);

    // ---- 1. operand and norm partials into LDS (issued first) ----
    if constexpr (!CHUNKED && !DIRECT) {
        if constexpr (GRP) stage_dma_group<NW>(a.in.q, s_op, nblk, a.n, v0, n, wid, l);
        else stage_dma<NW>(a.in.q, s_op, nblk * vb, wid, l);
    }
    if (a.in.ss)
        stage_ss_dma<NW>(a.in.ss + (size_t)v0 * a.in.ss_stride, a.in.ss_stride, a.in.ss_count, n, s_ss, wid, l);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weight ring: slot u holds sequence element i with i % U == u;
    // elements past the wave's run re-read its last quad so every slot is
    // loaded unconditionally and the load counters stay exact ----
    u32x4 c0[U], c1[U];
    typename QScale<DT>::T dv[U];
    uint32_t hv[U];
    // direct operand (fold 1, one group): the slot also holds the quad's four
    // operand pieces of this lane, read from global memory (L2) in the
    // layout a staged copy would have; A rows past the batch re-read the
    // last vector's row (their outputs are discarded)
    f16x8 xo[DIRECT ? U : 1][4];
    // (global layout of the whole batch: a.n vectors; a group's rows start at 2 v0)
    const uint32_t vbg = 128u * (uint32_t)a.n;
    const uint32_t xoff = DIRECT ? (uint32_t)(((l >> 4) * 2 * a.n + 2 * v0 + min(l & 15, 2 * n - 1)) * 16) : 0u;
    auto quad_of = [&](int i) {
        i = min(i, len - 1);
        const int c = CHUNKED ? i / qpc : 0;
        return min(c * cq + wid * qpc + (i - c * qpc), BQ - 1);
    };
    auto load_slot = [&](int u, int i) {
        const int qd = quad_of(i);
        q_load<DT>(a.w, cell0 + qd, l & 15, l, c0[u], c1[u], dv[u], hv[u]);
        if constexpr (DIRECT) {
            // padding blocks of the last quad (k/32 not a multiple of 4) have
            // no operand rows: they re-read the last real block's, so the
            // product with their zero scale is 0, whatever stale bytes lie
            // past the operand
#pragma unroll
            for (int bi = 0; bi < 4; bi++)
                xo[u][bi] = ldg((const f16x8 *)((const uint8_t *)a.in.q +
                                                (uint32_t)min(4 * qd + bi, nblk - 1) * vbg + xoff));
        }
    };
#pragma unroll
    for (int u = 0; u < U; u++) load_slot(u, u);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. zero padding blocks and the zero slot, then wait for the copies
    // (loads retire in issue order: every load but the ring's) and meet ----
    if constexpr (DIRECT) {
    } else if constexpr (!CHUNKED) {
        lds_zero<NW>(s_op + nblk * vb, sh.zslot + 16 - nblk * vb, threadIdx.x);
    } else {
        lds_zero<NW>(s_op + sh.zslot, 16, threadIdx.x);
    }
    // load instructions per ring slot
    constexpr int LPS = q_loads<DT>() + (DIRECT ? 4 : 0);
    static_assert(LPS * U <= 63, "ring loads beyond the vector memory counter");
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(LPS * U));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    epi_pre_cs(a, epi, prow, pact, pre);

    // A-operand row fed by this lane per group: LDS address of block 0 and
    // per-block stride (rows beyond 2nF read the zero slot)
    const int g = l >> 4;
    int abase[NG], astride[NG];
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const int ar = 16 * gi + (l & 15);
        const int v = ar >> (lf + 1), p = (ar >> 1) & (F - 1), h = ar & 1;
        const bool ok = v < n;
        const int p0 = CHUNKED ? 0 : p * 4 * BQ;
        abase[gi] = ok ? p0 * vb + (g * 2 * nl + 2 * v + h) * 16 : sh.zslot;
        astride[gi] = ok ? vb : 0;
    }

    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc[NG];
#pragma unroll
    for (int gi = 0; gi < NG; gi++) acc[gi] = zero4;

    auto compute = [&](int u, int i) {
        const int c = CHUNKED ? i / qpc : 0, j = i - c * qpc;
        if (CHUNKED && j == 0) {   // next operand chunk (uniform over the work-group)
            if (c > 0) __syncthreads();
            const int b0 = 4 * c * cq;
            const int nb_c = min(4 * cq, nblk - b0);
            stage_vgpr<NW>((const uint8_t *)a.in.q + (size_t)b0 * vb, s_op, nb_c * vb, threadIdx.x);
            lds_zero<NW>(s_op + nb_c * vb, (4 * cq - nb_c) * vb, threadIdx.x);
            __syncthreads();
        }
        const int lq = wid * qpc + j;
        if (c * cq + lq >= BQ) return;
        // the quad's four operand reads go out together, ahead of the decode
        f16x8 xv[4][NG];
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                if constexpr (DIRECT) xv[bi][gi] = xo[u][bi];
                else xv[bi][gi] = *(const f16x8 *)(s_op + abase[gi] + (4 * lq + bi) * astride[gi]);
            }
        }
        // (four-wave instances with a deep ring keep the serial form: the
        // extra result registers would cost them a wave per SIMD, e.g. the
        // Q8_0 LM head 128 -> 140 VGPRs)
        if constexpr (is_kquant(DT) || NG > 1 || (NW == 4 && U > 4)) {
#pragma unroll
            for (int bi = 0; bi < 4; bi++) {
                const f16x8 wv = deq_block<DT>(c0[u], c1[u], hv[u], bi);
                const BlockScale bs = block_scale<DT>(dv[u], bi);
#pragma unroll
                for (int gi = 0; gi < NG; gi++) mfma_block<DT>(acc[gi], xv[bi][gi], wv, bs);
            }
        } else {
            // four independent products, then the scale FMAs in block order
            // (mfma_block's sums, without serialising the MFMAs on one
            // result register)
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            f32x4 cc[4];
#pragma unroll
            for (int bi = 0; bi < 4; bi++)
                cc[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[bi][0], deq_block<DT>(c0[u], c1[u], hv[u], bi), z,
                                                                0, 0, 0);
#pragma unroll
            for (int bi = 0; bi < 4; bi++) {
                const BlockScale bs = block_scale<DT>(dv[u], bi);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[0][e] = fmaf(bs.s0, cc[bi][e], acc[0][e]);
            }
        }
    };
    // rounds of U: while another round follows, slot u is refilled right
    // after use (rolling prefetch); the last round issues no loads
    for (int i0 = 0; i0 < len; i0 += U) {
        if (i0 + U < len) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                compute(u, i0 + u);
                load_slot(u, i0 + u + U);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++)
                if (i0 + u < len) compute(u, i0 + u);
        }
    }

    // ---- 4. RMSNorm scale per vector from the staged partials ----
    if (EPI != EPI_RESID && a.in.ss) {
        for (int v = wid; v < n; v += NW) {
            float s = 0.0f;
            for (int i = l; i < a.in.ss_count; i += 64) s += s_ss[v * a.in.ss_count + i];
            s = wave_sum(s);
            if (l == 0) s_nrm[v] = 1.0f / sqrtf(s / (float)a.w.cols + a.in.eps);
        }
    }
    // ---- 5. the waves' useful entries meet in LDS: lane l (column c = part
    // p x row rl) holds, per group and component pair, the high/low parts of
    // A row 2(vF + p') + h; the pairs with p' == p are combined and stored at
    // s_z[w][v][rl][p], an LDS area of its own (no wait for the other waves
    // to finish with the operand) ----
    {
        const int c = l & 15, pc = c >> lr, rc = c & (R - 1);
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const int ar = 16 * gi + 4 * (l >> 4) + 2 * q;
                const int v = ar >> (lf + 1), pp = (ar >> 1) & (F - 1);
                if (v < n && pp == pc)
                    s_z[((wid * n + v) * R + rc) * F + pp] = acc[gi][2 * q] + acc[gi][2 * q + 1] * LO_INV_SCALE;
            }
        }
    }
    __syncthreads();

    // ---- 6. one thread per (vector, row): sum over waves and parts in a
    // fixed order, scale, epilogue ----
    const int nout = n * R;
    for (int o0 = 0; o0 < nout; o0 += NW * 64) {
        const int o = o0 + (int)threadIdx.x;
        const bool act = o < nout;
        const int v = act ? o >> lr : 0, rl = o & (R - 1);
        float z = 0.0f;
        if (act) {
            const float *zp = s_z + ((size_t)v * R + rl) * F;
            const int wstride = n * R * F;
            if (F == 1) {
#pragma unroll
                for (int w = 0; w < NW; w++) z += zp[w * wstride];
            } else if (F == 2) {
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    const float2 e = *(const float2 *)(zp + w * wstride);
                    z += e.x;
                    z += e.y;
                }
            } else {
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    for (int p4 = 0; p4 < F; p4 += 4) {
                        const float4 e = *(const float4 *)(zp + w * wstride + p4);
                        z += e.x;
                        z += e.y;
                        z += e.z;
                        z += e.w;
                    }
                }
            }
        }
        float y = z * ACT_INV_SCALE;
        if (EPI != EPI_RESID && a.in.ss) y *= s_nrm[v];
        const int gv = v0 + v;   // the vector's index in the batch
        if constexpr (EPI >= 0) {
            epilogue<EPI >= 0 ? EPI : 0>(a, t, rl, R, gv, act, y, pre_on, pre);
        } else {
            switch (sh.epi) {
            case EPI_STORE: epilogue<EPI_STORE>(a, t, rl, R, gv, act, y); break;
            case EPI_RESID: epilogue<EPI_RESID>(a, t, rl, R, gv, act, y, pre_on, pre); break;
            case EPI_SWIGLU: epilogue<EPI_SWIGLU>(a, t, rl, R, gv, act, y); break;
            case EPI_QKV: epilogue<EPI_QKV>(a, t, rl, R, gv, act, y, pre_on, pre); break;
            default: epilogue<EPI_LOGITS>(a, t, rl, R, gv, act, y); break;
            }
        }
    }
}

// positive integer from the environment, else def
static inline int gb_env_int(const char *name, int def)
{
    const char *e = getenv(name);
    const int v = e ? atoi(e) : def;
    return v < 1 ? 1 : v;
}

// Compute units of the current device (cached: one device type per process).
static inline int gemv_cus()
{
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return n > 0 ? n : 256;
    }();
    return cus;
}

static inline int pick_nw(int tiles, int quads, bool four_held)
{
    static const int t16 = gb_env_int("CMOL_NW16_BELOW", 128), t8 = gb_env_int("CMOL_NW8_BELOW", 4096);   // measurements
    int nw = tiles < t16 ? 16 : tiles < t8 ? 8 : 4;
    // eight-wave groups keep 4 per CU resident (32 waves): a matrix with more
    // tiles runs a second round of work-groups, each as long as the first;
    // four-wave groups held to six per CU (four_held) finish it in one
    // (SmolLM3-3B gate/up, 1376 tiles: 10.3 us in two rounds)
    if (four_held && nw == 8 && tiles > 4 * gemv_cus() && tiles <= 6 * gemv_cus() && quads >= 13 && quads <= 16)
        nw = 4;
    if (const char *e = getenv("CMOL_GEMV_NW")) nw = atoi(e);
    static const int minq = [] {
        const char *e = getenv("CMOL_GEMV_MINQ");   // measurements
        const int v = e ? atoi(e) : 2;
        return v < 1 ? 1 : v;
    }();
    while (nw > 1 && quads < minq * nw) nw >>= 1;
    return nw;
}

static inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// LDS budget of one work-group: 80 KB keeps two resident per CU.  A grid of
// at most one work-group per CU may take most of the CU's LDS.  An operand
// beyond the budget is staged in chunks, each a barrier-separated round
// trip, or (one operand group, grid of at most one work-group per CU) read
// by the waves straight from L2.  CMOL_GEMV_LDS_KB overrides the budget for
// measurements.
static inline int gemv_lds_budget(int wgs)
{
    static const int kb = [] {
        const char *e = getenv("CMOL_GEMV_LDS_KB");
        return e ? atoi(e) : 0;
    }();
    if (kb > 0) return kb * 1024;
    return wgs <= gemv_cus() ? 156 * 1024 : 80 * 1024;
}

// Chooses quads per wave per chunk and the LDS areas; returns the dynamic
// LDS bytes or -1 when the operand cannot be staged (`chunked` is set when
// it takes more than one chunk, only possible with fold 1).
static inline int plan_gemv(const GemvArgs &a, int nw, GemvShape &sh, bool &chunked, int groups = 1)
{
    const int BQ = a.w.block_quads, F = a.w.fold;
    const int n = groups > 1 ? 8 : a.n;   // vectors per work-group
    sh.groups = groups;
    const int vb = 128 * n;
    sh.ss_bytes = a.in.ss ? round_up(n * a.in.ss_count * 4, 16) : 0;
    const int nrm = round_up(n * 4, 16);
    const int red = nw * n * 64;   // per-wave useful entries (16 columns x n floats)
    const int cap = gemv_lds_budget(a.w.row_tiles * groups) - sh.ss_bytes - nrm - red - 16;
    const long full = (long)F * 4 * BQ * vb;
    if (full <= cap) {
        chunked = false;
        sh.qpc = (BQ + nw - 1) / nw;
        sh.zslot = (int)full;
    } else {
        if (F != 1 || groups > 1) return -1;
        chunked = true;
        sh.qpc = cap / (4 * vb * nw);
        if (sh.qpc < 1) return -1;
        sh.zslot = 4 * sh.qpc * nw * vb;
    }
    sh.op_bytes = round_up(sh.zslot + 16, 16);
    return sh.op_bytes + sh.ss_bytes + nrm + red;
}

// Ring depths: the long ring, and the short one for a wave whose whole run
// fits it.
template <int DT>
struct GemvRing {
    static constexpr int L = DT == DT_Q8_0 ? 6 : 8, S = L / 2;
};

template <typename K>
static void gemv_go(K kern, const GemvArgs &a, const GemvShape &sh, int lds, int nw, hipStream_t s)
{
    const dim3 grid(a.w.row_tiles, sh.groups), block(nw * 64);
    // a refused attribute skips the launch; launch_gemv reports it
    // through hipGetLastError
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
        return;
    if (a.ev_start) hipExtLaunchKernelGGL(kern, grid, block, lds, s, a.ev_start, a.ev_stop, 0, a, sh);
    else hipLaunchKernelGGL(kern, grid, block, lds, s, a, sh);
}

// Launch of the one-group kernel with its epilogue fixed at compile time
// (instantiated per format in gemv_q*_epi.hip).
template <int DT, int NW>
int launch_gemv_epi(const GemvArgs &a, const GemvShape &sh, int lds, int len, hipStream_t s);

#ifdef GEMV_EPI_TU
template <int DT, int NW, int EPI>
static void launch_epi_u(const GemvArgs &a, const GemvShape &sh, int lds, int len, hipStream_t s)
{
    using RG = GemvRing<DT>;
    if (len <= 2) gemv_go(k_gemv<DT, NW, 1, false, 2, EPI>, a, sh, lds, NW, s);
    else if (len <= RG::S) gemv_go(k_gemv<DT, NW, 1, false, RG::S, EPI>, a, sh, lds, NW, s);
    else gemv_go(k_gemv<DT, NW, 1, false, RG::L, EPI>, a, sh, lds, NW, s);
}

template <int DT, int NW>
int launch_gemv_epi(const GemvArgs &a, const GemvShape &sh, int lds, int len, hipStream_t s)
{
    switch (sh.epi) {
    case EPI_STORE: launch_epi_u<DT, NW, EPI_STORE>(a, sh, lds, len, s); break;
    case EPI_RESID: launch_epi_u<DT, NW, EPI_RESID>(a, sh, lds, len, s); break;
    case EPI_SWIGLU: launch_epi_u<DT, NW, EPI_SWIGLU>(a, sh, lds, len, s); break;
    case EPI_QKV: launch_epi_u<DT, NW, EPI_QKV>(a, sh, lds, len, s); break;
    case EPI_LOGITS: launch_epi_u<DT, NW, EPI_LOGITS>(a, sh, lds, len, s); break;
    default: return -6;
    }
    return 0;
}
#endif

template <int DT, int NW, int NG>
static int launch_cfg(const GemvArgs &a, int epi, hipStream_t s, int groups = 1)
{
    if (epi < EPI_STORE || epi > EPI_LOGITS) return -6;
    GemvShape sh;
    sh.epi = epi;
    bool chunked = false;
    const int lds = plan_gemv(a, NW, sh, chunked, groups);
    if (lds < 0 || (groups > 1 && (NG != 1 || a.w.fold != 1 || chunked))) return -6;
    using RG = GemvRing<DT>;
    // an operand beyond the budget on a grid of at most one work-group per
    // CU: each wave reads its own quads' operand from L2 in its weight ring
    // (no chunk barriers; every work-group reads the whole operand once, as
    // the chunked copy does)
    if constexpr (NG == 1) {
        static const bool direct_on = [] {
            const char *e = getenv("CMOL_GEMV_DIRECT");   // measurements
            return !(e && e[0] == '0');
        }();
        if (chunked && direct_on && a.w.fold == 1 && a.w.row_tiles <= gemv_cus()) {
            sh.qpc = (a.w.block_quads + NW - 1) / NW;
            sh.zslot = 0;
            sh.op_bytes = 16;
            const int dl = sh.op_bytes + sh.ss_bytes + round_up(a.n * 4, 16) + NW * a.n * 64;
            // a four-deep ring (eight-deep measured slower: 2048x11008 at n=8
            // 12.5 vs 10.3 us); sixteen waves have 128 VGPRs a lane: two-deep
            gemv_go(k_gemv<DT, NW, 1, false, NW >= 16 ? 2 : RG::S, -1, true>, a, sh, dl, NW, s);
            return 0;
        }
    }
    const int len = chunked ? ((a.w.block_quads + sh.qpc * NW - 1) / (sh.qpc * NW)) * sh.qpc : sh.qpc;
    if constexpr (NG == 1) {
        // vector groups: the instance with the group gather, epilogue chosen
        // at run time
        if (groups > 1) {
            if (len <= RG::S) gemv_go(k_gemv<DT, NW, 1, false, RG::S, -1, false, true>, a, sh, lds, NW, s);
            else gemv_go(k_gemv<DT, NW, 1, false, RG::L, -1, false, true>, a, sh, lds, NW, s);
            return 0;
        }
        // the decode shape (one operand group, operand staged whole; residual
        // epilogues take no RMSNorm there) runs the epilogue-specialised kernel
        if (!chunked && !(epi == EPI_RESID && a.in.ss)) return launch_gemv_epi<DT, NW>(a, sh, lds, len, s);
    }
    if (chunked) {
        if (len <= RG::S) gemv_go(k_gemv<DT, NW, NG, true, RG::S, -1>, a, sh, lds, NW, s);
        else gemv_go(k_gemv<DT, NW, NG, true, RG::L, -1>, a, sh, lds, NW, s);
    } else {
        if (len <= RG::S) gemv_go(k_gemv<DT, NW, NG, false, RG::S, -1>, a, sh, lds, NW, s);
        else gemv_go(k_gemv<DT, NW, NG, false, RG::L, -1>, a, sh, lds, NW, s);
    }
    return 0;
}

// Widest wave count the launch heuristics allow whose LDS plan fits.
template <int DT, int NG>
static int launch_dt(const GemvArgs &a, int epi, hipStream_t s, int groups = 1)
{
    int nw = pick_nw(a.w.row_tiles * groups, a.w.block_quads, DT == DT_Q4_0 && NG == 1);
    for (;; nw >>= 1) {
        GemvShape sh;
        bool ch;
        if (nw <= 1 || plan_gemv(a, nw, sh, ch, groups) >= 0) break;
    }
    // 16 waves leave 128 VGPRs a lane: only the single-group Q4_0 kernel
    // fits without spilling
    if constexpr (NG == 1 && DT == DT_Q4_0) {
        if (nw >= 16) return launch_cfg<DT, 16, NG>(a, epi, s, groups);
    }
    if (nw >= 8) return launch_cfg<DT, 8, NG>(a, epi, s, groups);
    if (nw >= 4) return launch_cfg<DT, 4, NG>(a, epi, s, groups);
    if (nw >= 2) return launch_cfg<DT, 2, NG>(a, epi, s, groups);
    return launch_cfg<DT, 1, NG>(a, epi, s, groups);
}

// ---------------------------------------------------------------------------
// Batched matvec for more than 8 vectors (lock-step multi-session decode).
//
// The vectors are cut into groups of GB_VG = 8 (16 MFMA A rows: the high and
// low f16 parts of each), the rows into blocks of GB_NW * tpw 16-row tiles
// and k into `splits` ranges of sq block quads.  One work-group per (vector
// group, row block, k range) copies that operand slice into LDS once and its
// waves stream the weight quads of tpw contiguous tiles each, so the
// operand is read from L2 once per work-group rather than once per tile.
// Work-groups b, b+8, b+16, ... (one XCD) take the same row block for the
// successive vector groups, so the weights they share stay in that XCD's L2.
// With one k range the epilogue runs in place; otherwise the partial sums go
// to a scratch buffer and k_gemv_b_finish adds them in a fixed order and runs
// the epilogue.
// ---------------------------------------------------------------------------
#define GB_NW 8
#define GB_VG 8
#define GB_OP_BUDGET (64 * 1024)   // LDS bytes of one operand slice
// Work-groups a batched matvec aims for: fewer tiles per wave until the
// grid reaches GB_TARGET_WGS, then k splits while it is below GB_SPLIT_WGS
// (CMOL_GB_TARGET / CMOL_GB_SPLIT override them for measurements).
#define GB_TARGET_WGS gb_target_wgs()
#define GB_SPLIT_WGS gb_split_wgs()
static inline int gb_target_wgs()
{
    static const int v = gb_env_int("CMOL_GB_TARGET", 512);
    return v;
}
static inline int gb_split_wgs()
{
    static const int v = gb_env_int("CMOL_GB_SPLIT", 256);
    return v;
}

// Whether a matvec of n vectors over w runs the batched kernel rather than
// k_gemv.  CMOL_GEMV_B=1 in the environment sends every unfolded matrix there.
static inline bool gemv_batched(const QTensor &w, int n)
{
    static const bool forced = [] {
        const char *e = getenv("CMOL_GEMV_B");
        return e && e[0] == '1';
    }();
    return w.fold == 1 && (n > GB_VG || forced);
}

struct GbShape {
    int epi;
    int groups, tpw, rblocks, splits, sq;
    int ss_count;   // RMSNorm partials per vector (0: none)
};

static inline int gb_plan(const QTensor &w, int n, GbShape &sh)
{
    const int T = w.row_tiles, BQ = w.block_quads;
    sh.groups = (n + GB_VG - 1) / GB_VG;
    sh.splits = (BQ * 4 * 1024 + GB_OP_BUDGET - 1) / GB_OP_BUDGET;
    sh.sq = (BQ + sh.splits - 1) / sh.splits;
    sh.splits = (BQ + sh.sq - 1) / sh.sq;
    for (sh.tpw = 4; sh.tpw > 1; sh.tpw >>= 1) {
        sh.rblocks = (T + GB_NW * sh.tpw - 1) / (GB_NW * sh.tpw);
        if (sh.groups * sh.rblocks * sh.splits >= GB_TARGET_WGS) break;
    }
    sh.rblocks = (T + GB_NW * sh.tpw - 1) / (GB_NW * sh.tpw);
    // still too few work-groups: split k further
    while (sh.groups * sh.rblocks * sh.splits < GB_SPLIT_WGS && sh.sq > 1) {
        sh.sq = (sh.sq + 1) / 2;
        sh.splits = (BQ + sh.sq - 1) / sh.sq;
    }
    return sh.groups * sh.rblocks * sh.splits;
}

template <int DT, int U, int EPI>
__global__ __launch_bounds__(GB_NW * 64) void k_gemv_b(GemvArgs a, GbShape sh)
{
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int BQ = a.w.block_quads, nblk = a.w.cols >> 5, T = a.w.row_tiles;
    const int b = blockIdx.x;
    const int vg = (b >> 3) % sh.groups;
    const int rest = (b / (8 * sh.groups)) * 8 + (b & 7);
    if (rest >= sh.rblocks * sh.splits) return;
    const int rb = rest % sh.rblocks, ks = rest / sh.rblocks;
    const int n = a.n, nrows = 2 * n;
    const int v0 = vg * GB_VG, nv = min(GB_VG, n - v0);
    const int q0 = ks * sh.sq, nq = min(sh.sq, BQ - q0);
    const int tid = threadIdx.x, l = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t *s_op = smem;                                   // [4 sq blocks][4 groups][16 rows][16 B]
    float *s_ss = (float *)(smem + (size_t)4 * sh.sq * 1024);   // [GB_VG][ss_count]
    float *s_nrm = s_ss + ((GB_VG * sh.ss_count + 3) & ~3);

    // ---- 1. operand slice and RMSNorm partials into LDS: lane l copies row
    // 2*v0 + l%16 of k-group l/16 of a block (rows past the batch and blocks
    // past the matrix re-read valid data: their products are discarded or
    // meet zero weights) ----
    for (int k = wid; k < 4 * nq; k += GB_NW) {
        const int blk = min(4 * q0 + k, nblk - 1);
        const int r = min(2 * v0 + (l & 15), nrows - 1);
        const uint8_t *src = (const uint8_t *)a.in.q + ((((size_t)blk * 4 + (l >> 4)) * nrows) + r) * 16;
        __builtin_amdgcn_global_load_lds((const gvoid_t *)src, (lvoid_t *)(s_op + (size_t)k * 1024), 16, 0, 0);
    }
    if (sh.ss_count)
        stage_ss_dma<GB_NW>(a.in.ss + (size_t)v0 * a.in.ss_stride, a.in.ss_stride, sh.ss_count, nv, s_ss, wid, l);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weight ring over this wave's items: quad q0+q of tile t0+j ----
    const int t0 = (rb * GB_NW + wid) * sh.tpw;
    const int ntw = max(0, min(sh.tpw, T - t0));
    const int len = ntw * nq;
    u32x4 c0[U], c1[U];
    typename QScale<DT>::T dv[U];
    uint32_t hv[U];
    auto load_slot = [&](int u, int i) {
        i = min(i, len - 1);
        const int j = i / nq, q = i - j * nq;
        q_load<DT>(a.w, (size_t)(t0 + j) * BQ + q0 + q, l & 15, l, c0[u], c1[u], dv[u], hv[u]);
    };
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (u < len) load_slot(u, u);
    }
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
    __syncthreads();
    // RMSNorm scale per vector of the group (wave w: vectors w, w + GB_NW)
    if (sh.ss_count && sh.splits == 1) {
        for (int v = wid; v < nv; v += GB_NW) {
            float s = 0.0f;
            for (int i = l; i < sh.ss_count; i += 64) s += s_ss[v * sh.ss_count + i];
            s = wave_sum(s);
            if (l == 0) s_nrm[v] = 1.0f / sqrtf(s / (float)a.w.cols + a.in.eps);
        }
        __syncthreads();
    }

    const int g = l >> 4, ar = l & 15;
    const uint8_t *abase = s_op + (g * 16 + ar) * 16;
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc = zero4;
    // lane l holds rows 16t + l%16 of vectors v0 + 2(l/16) + {0, 1}
    auto finish_tile = [&](int j) {
        const int t = t0 + j, row = t * 16 + (l & 15);
#pragma unroll
        for (int pr = 0; pr < 2; pr++) {
            const int vl = 2 * (l >> 4) + pr;
            const bool act = vl < nv && row < a.w.rows;
            float y = (acc[2 * pr] + acc[2 * pr + 1] * LO_INV_SCALE) * ACT_INV_SCALE;
            if (sh.splits > 1) {
                if (act) a.part[((size_t)ks * n + v0 + vl) * a.w.rows + row] = y;
                continue;
            }
            if (sh.ss_count) y *= s_nrm[vl < nv ? vl : 0];
            const int vv = act ? v0 + vl : 0;
            epilogue<EPI>(a, t, l & 15, 16, vv, act, y);
        }
        acc = zero4;
    };
    auto compute = [&](int u, int i) {
        const int j = i / nq, q = i - j * nq;
        if constexpr (DT != DT_Q4_0 || EPI == EPI_RESID || EPI == EPI_LOGITS) {
#pragma unroll
            for (int bi = 0; bi < 4; bi++) {
                const f16x8 wv = deq_block<DT>(c0[u], c1[u], hv[u], bi);
                const f16x8 xv = *(const f16x8 *)(abase + (size_t)(4 * q + bi) * 1024);
                mfma_block<DT>(acc, xv, wv, block_scale<DT>(dv[u], bi));
            }
        } else {
            // Q4_0 instances whose epilogue leaves room (elsewhere the extra
            // registers push the kernel past 128 VGPRs, one work-group per CU
            // instead of two): the quad's four operand reads go out together,
            // then four independent products, then the scale FMAs in block
            // order (the same sums as mfma_block's, without serialising the
            // MFMAs on one result register)
            f16x8 xv[4];
#pragma unroll
            for (int bi = 0; bi < 4; bi++) xv[bi] = *(const f16x8 *)(abase + (size_t)(4 * q + bi) * 1024);
            f32x4 cc[4];
#pragma unroll
            for (int bi = 0; bi < 4; bi++)
                cc[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[bi], deq_block<DT>(c0[u], c1[u], hv[u], bi), zero4,
                                                                0, 0, 0);
#pragma unroll
            for (int bi = 0; bi < 4; bi++) {
                const BlockScale bs = block_scale<DT>(dv[u], bi);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = fmaf(bs.s0, cc[bi][e], acc[e]);
            }
        }
        if (q == nq - 1) finish_tile(j);
    };
    for (int i0 = 0; i0 < len; i0 += U) {
        if (i0 + U < len) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                compute(u, i0 + u);
                load_slot(u, i0 + u + U);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++)
                if (i0 + u < len) compute(u, i0 + u);
        }
    }
}

// Batched matvec over one round of sixteen-wave work-groups for 17-32
// vectors of an unsplit k range (the gate/up shape at 32 sessions), where
// the kernel above would need a second round of work-groups.  A work-group
// holds the operand of 16 vectors over the whole k range in LDS ([block]
// [k-group][16 high rows, 16 low rows][16 B]); each wave streams one 16-row
// tile.  Per block the low part's product joins the high part's MFMA sum
// (codes times 2^-11 against the low part times 2^11, exact), so one decode
// and one scale FMA per output serve 16 vectors.  Lane (c, g) ends with
// row 16t + c of vectors 4g .. 4g+3.
#define GB16_NW 16
template <int DT, int U, int EPI, int NWB = GB16_NW>
__global__ __launch_bounds__(NWB * 64) void k_gemv_b16(GemvArgs a, int groups, int rblocks, int sq, int splits)
{
#pragma clang fp contract(off)
    // launch arguments needed before the operand and weight loads go out,
    // fetched in one round trip
    sgpr_pin(a.w.qs);
    sgpr_pin(a.w.d);
    if constexpr (DT == DT_Q5_0 || DT == DT_Q6_K) sgpr_pin(a.w.qh);
    sgpr_pin(a.w.block_quads);
    sgpr_pin(a.w.cols);
    sgpr_pin(a.w.row_tiles);
    sgpr_pin(a.n);
    sgpr_pin(a.in.q);
    sgpr_pin(a.in.ss);
    sgpr_pin(a.in.ss_count);
    sgpr_pin(a.in.ss_stride);
    sgpr_pin(a.in.eps);
    sgpr_pin(a.in.tail);
    sgpr_pin(groups);
    sgpr_pin(rblocks);
    sgpr_pin(sq);
    sgpr_pin(splits);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int BQ = a.w.block_quads, nblk = a.w.cols >> 5, T = a.w.row_tiles;
    const int b = blockIdx.x;
    const int vg = (b >> 3) % groups;
    const int rest = (b / (8 * groups)) * 8 + (b & 7);
    if (rest >= rblocks * splits) return;
    const int rb = rest % rblocks, ks = rest / rblocks;
    const int q0 = ks * sq, nq = min(sq, BQ - q0);
    const int n = a.n, nrows = 2 * n, v0 = vg * 16;
    const int tid = threadIdx.x, l = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    // every block of every quad is staged (blocks past the matrix re-read
    // the last one: they meet zero weights)
    float *s_nrm = (float *)(smem + (size_t)sq * 4 * 2048);
    for (int pc = wid; pc < 8 * nq; pc += NWB) {
        const int blk = min(4 * q0 + (pc >> 1), nblk - 1), kg = 2 * (pc & 1) + (l >> 5), r = l & 31;
        const int row = min(2 * (v0 + (r & 15)) + (r >> 4), nrows - 1);
        const uint8_t *src = (const uint8_t *)a.in.q + (((size_t)blk * 4 + kg) * nrows + row) * 16;
        __builtin_amdgcn_global_load_lds((const gvoid_t *)src, (lvoid_t *)(smem + (size_t)pc * 1024), 16, 0, 0);
    }
    const int t = rb * NWB + wid;
    const int tt = t < T ? t : T - 1;
    u32x4 c0[U], c1[U];
    typename QScale<DT>::T dv[U];
    uint32_t hv[U];
    auto load_slot = [&](int u, int q) {
        q = min(q, nq - 1);
        q_load<DT>(a.w, (size_t)tt * BQ + q0 + q, l & 15, l, c0[u], c1[u], dv[u], hv[u]);
    };
#pragma unroll
    for (int u = 0; u < U; u++) load_slot(u, u);
    // RMSNorm scale of vector v0 + j from its producer's partials (wave
    // j mod NWB), summed in the order k_gemv_b sums them
    if (a.in.ss && splits == 1) {
        for (int j = wid; j < 16; j += NWB) {
            const int v = min(v0 + j, n - 1);
            float sum = 0.0f;
            for (int i = l; i < a.in.ss_count; i += 64) sum += a.in.ss[(size_t)v * a.in.ss_stride + i];
            sum = wave_sum(sum);
            if (l == 0) s_nrm[j] = 1.0f / sqrtf(sum / (float)a.w.cols + a.in.eps);
        }
    }
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
    __syncthreads();
    const int g = l >> 4, cl = l & 15;
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc = z;
    auto compute = [&](int u, int q) {
        f16x8 xh[4], xl[4];
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            const uint8_t *p = smem + (size_t)(4 * q + bi) * 2048 + (g * 32 + cl) * 16;
            xh[bi] = *(const f16x8 *)p;
            xl[bi] = *(const f16x8 *)(p + 256);
        }
        f32x4 cc[4];
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            const f16x8 wv = deq_block<DT>(c0[u], c1[u], hv[u], bi);
            const f16x8 wl = wv * (_Float16)LO_INV_SCALE;
            cc[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[bi], wv, z, 0, 0, 0);
            cc[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[bi], wl, cc[bi], 0, 0, 0);
        }
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            const BlockScale bs = block_scale<DT>(dv[u], bi);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(bs.s0, cc[bi][e], acc[e]);
        }
    };
    // the loop is uniform over the wave (every wave runs all BQ quads, a
    // wave past the last tile on a valid tile's data) so every wait count
    // is the same
    for (int i0 = 0; i0 < nq; i0 += U) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (i0 + u < nq) compute(u, i0 + u);
            load_slot(u, i0 + u + U);
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int vl = 4 * g + e, v = v0 + vl;
        const bool act = v < n && t < T && t * 16 + cl < a.w.rows;
        float y = acc[e] * ACT_INV_SCALE;
        if (splits > 1) {
            // k-split partial sums: k_gemv_b_finish adds them and runs the
            // epilogue, as for k_gemv_b
            if (act) a.part[((size_t)ks * n + v) * a.w.rows + t * 16 + cl] = y;
            continue;
        }
        if (a.in.ss) y *= s_nrm[vl];
        epilogue<EPI>(a, t, cl, 16, act ? v : 0, act, y);
    }
}

// The plan of k_gemv_b16: 17-32 vectors of a 32-value block format in two
// groups of 16; sixteen-wave work-groups, one per CU resident.  Taken where
// k_gemv_b's own plan
//   * needs more than one round of work-groups without a k split (gate/up
//     at 32 sessions: 688 work-groups for 512 resident), or
//   * splits a long k range into slices of 8 quads or more (down at 32
//     sessions: 6 slices of 15 quads); k_gemv_b16 then splits it so that its
//     work-groups fill the CUs once (15 slices of 6 quads) and
//     k_gemv_b_finish adds the slices as for k_gemv_b.
// CMOL_B16_SPLITS=<s> forces it with s slices (measurements).
struct Gb16Shape {
    int groups, rblocks, sq, splits;
    int nw;   // waves per work-group (12 or 16)
};

static inline bool gb16_plan(const QTensor &w, int n, Gb16Shape &p)
{
    if (is_kquant(w.dtype) || n <= 16 || n > 32 || w.fold != 1) return false;
    static const int forced = [] {
        const char *e = getenv("CMOL_B16_SPLITS");
        return e ? atoi(e) : 0;
    }();
    static const int nw_env = [] {
        const char *e = getenv("CMOL_B16_WAVES");   // measurements: 12 or 16
        return e ? atoi(e) : 0;
    }();
    const int BQ = w.block_quads;
    p.groups = (n + 15) / 16;
    int s = 1;
    if (forced > 0) {
        s = forced;
    } else {
        GbShape sh;
        const int wgs = gb_plan(w, n, sh);
        if (sh.splits == 1) {
            if (wgs <= 2 * gemv_cus()) return false;
        } else {
            if (sh.sq < 8) return false;
            s = max(1, gemv_cus() / (p.groups * ((w.row_tiles + GB16_NW - 1) / GB16_NW)));
        }
    }
    p.sq = (BQ + min(s, BQ) - 1) / min(s, BQ);
    p.splits = (BQ + p.sq - 1) / p.sq;
    // twelve-wave work-groups where the unsplit grid then still runs in one
    // round (SmolLM3-3B gate/up at n=32: 230 work-groups instead of 172 on
    // 256 CUs, 16.9 vs 20.1 us); the k-split shapes keep sixteen (down:
    // 15.7 vs 17.0 us)
    const int r12 = (w.row_tiles + 11) / 12;
    p.nw = nw_env == 12 || nw_env == 16 ? nw_env
           : (p.splits == 1 && p.groups * r12 <= gemv_cus()) ? 12 : GB16_NW;
    p.rblocks = (w.row_tiles + p.nw - 1) / p.nw;
    return (size_t)p.sq * 4 * 2048 + 64 <= 160 * 1024;
}

template <int DT, int EPI, int NWB>
static int launch_gemv_b16_nw(const GemvArgs &a, const Gb16Shape &p, hipStream_t s)
{
    constexpr int U = (DT == DT_Q8_0) ? 6 : 8;
    const size_t lds = (size_t)p.sq * 4 * 2048 + 64;
    // set once; a refusal (e.g. inside a stream capture) is retried on the
    // next launch rather than remembered (decode threads of several sessions
    // may get here at once: the flag is atomic, the attribute call idempotent)
    static std::atomic<bool> lds_ok{false};
    if (!lds_ok.load(std::memory_order_relaxed)) {
        if (hipFuncSetAttribute((const void *)k_gemv_b16<DT, U, EPI, NWB>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return -6;
        lds_ok.store(true, std::memory_order_relaxed);
    }
    const long blocks = (long)((p.rblocks * p.splits + 7) / 8) * 8 * p.groups;
    const bool split = p.splits > 1;
    if (a.ev_start)
        hipExtLaunchKernelGGL((k_gemv_b16<DT, U, EPI, NWB>), dim3((unsigned)blocks), dim3(NWB * 64), lds, s,
                              a.ev_start, split ? nullptr : a.ev_stop, 0, a, p.groups, p.rblocks, p.sq, p.splits);
    else
        hipLaunchKernelGGL((k_gemv_b16<DT, U, EPI, NWB>), dim3((unsigned)blocks), dim3(NWB * 64), lds, s, a,
                           p.groups, p.rblocks, p.sq, p.splits);
    return 0;
}

template <int DT, int EPI>
static int launch_gemv_b16(const GemvArgs &a, const Gb16Shape &p, hipStream_t s)
{
    return p.nw == 12 ? launch_gemv_b16_nw<DT, EPI, 12>(a, p, s) : launch_gemv_b16_nw<DT, EPI, GB16_NW>(a, p, s);
}

template <int DT>
static int launch_gemv_b(const GemvArgs &a, int epi, hipStream_t s)
{
    if (epi < EPI_STORE || epi > EPI_LOGITS || a.w.fold != 1) return -6;
    GbShape sh;
    sh.epi = epi;
    sh.ss_count = a.in.ss ? a.in.ss_count : 0;
    const int wgs = gb_plan(a.w, a.n, sh);
    if constexpr (!is_kquant(DT)) {
        Gb16Shape p;
        if (gb16_plan(a.w, a.n, p)) {
            if (p.splits > 1) {
                if (!a.part || (size_t)p.splits * a.n * a.w.rows > a.part_cap) return -6;
                const int rc = launch_gemv_b16<DT, EPI_STORE>(a, p, s);
                return rc ? rc : launch_gemv_b_finish(a, epi, p.splits, sh.ss_count, s);
            }
            switch (epi) {
            case EPI_STORE: return launch_gemv_b16<DT, EPI_STORE>(a, p, s);
            case EPI_RESID: return launch_gemv_b16<DT, EPI_RESID>(a, p, s);
            case EPI_SWIGLU: return launch_gemv_b16<DT, EPI_SWIGLU>(a, p, s);
            case EPI_QKV: return launch_gemv_b16<DT, EPI_QKV>(a, p, s);
            default: return launch_gemv_b16<DT, EPI_LOGITS>(a, p, s);
            }
        }
    }
    if (sh.splits > 1 && (!a.part || (size_t)sh.splits * a.n * a.w.rows > a.part_cap)) return -6;
    const long blocks = (long)((sh.rblocks * sh.splits + 7) / 8) * 8 * sh.groups;
    const size_t lds = (size_t)4 * sh.sq * 1024 + ((GB_VG * sh.ss_count + 3) & ~3) * 4 + GB_VG * 4;
    (void)wgs;
    constexpr int U = (DT == DT_Q8_0) ? 6 : 8;
    // the epilogue is fixed at compile time (one straight code path: a
    // launch's cold instruction cache fetches little); with a k split the
    // finish kernel runs it and this kernel only stores partial sums
    auto go = [&](auto kern) {
        // kernel timing: the start event on the first kernel, the stop event
        // on the last (the finish kernel when k is split)
        if (a.ev_start)
            hipExtLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(GB_NW * 64), lds, s, a.ev_start,
                                  sh.splits == 1 ? a.ev_stop : nullptr, 0, a, sh);
        else
            hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(GB_NW * 64), lds, s, a, sh);
    };
    switch (sh.splits > 1 ? EPI_STORE : epi) {
    case EPI_STORE: go(k_gemv_b<DT, U, EPI_STORE>); break;
    case EPI_RESID: go(k_gemv_b<DT, U, EPI_RESID>); break;
    case EPI_SWIGLU: go(k_gemv_b<DT, U, EPI_SWIGLU>); break;
    case EPI_QKV: go(k_gemv_b<DT, U, EPI_QKV>); break;
    default: go(k_gemv_b<DT, U, EPI_LOGITS>); break;
    }
    if (sh.splits > 1) return launch_gemv_b_finish(a, epi, sh.splits, sh.ss_count, s);
    return 0;
}

// 9..32 vectors as groups of 8 on grid.y of the one-group matvec (waves
// split k inside the work-group, the epilogue runs in place): taken where the
// batched kernel would split k across work-groups (a finish kernel after it)
// and the 8-vector operand fits LDS whole.  CMOL_GEMV_GROUPS=0 turns it off
// (measurements).
template <int DT>
static bool gemv_grouped(const GemvArgs &a)
{
    static const bool on = [] {
        const char *e = getenv("CMOL_GEMV_GROUPS");
        return !(e && e[0] == '0');
    }();
    if (!on || is_kquant(DT) || a.w.fold != 1 || a.n <= GB_VG || a.n > 32) return false;
    GbShape sh;
    gb_plan(a.w, a.n, sh);
    Gb16Shape p;
    const int splits = gb16_plan(a.w, a.n, p) ? p.splits : sh.splits;
    if (splits <= 1) return false;
    const int groups = (a.n + GB_VG - 1) / GB_VG;
    GemvShape gs;
    bool ch = false;
    for (int nw = 16; nw >= 2; nw >>= 1)
        if (plan_gemv(a, nw, gs, ch, groups) >= 0 && !ch) return true;
    return false;
}

template <int DT>
int launch_ng(const GemvArgs &a, int epi, hipStream_t s)
{
    if (gemv_grouped<DT>(a)) return launch_dt<DT, 1>(a, epi, s, (a.n + GB_VG - 1) / GB_VG);
    if (gemv_batched(a.w, a.n)) return launch_gemv_b<DT>(a, epi, s);
    const int rows = 2 * a.n * a.w.fold;   // MFMA A rows
    if (rows <= 16) return launch_dt<DT, 1>(a, epi, s);
    if (rows <= 32) return launch_dt<DT, 2>(a, epi, s);
    if (rows <= 64) return launch_dt<DT, 4>(a, epi, s);
    return -6;
}
