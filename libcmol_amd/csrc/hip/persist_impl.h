// persist_impl.h — the persistent single-session decode kernel: one launch
// per token runs the embedding gather, every layer (QKV + RoPE + KV write,
// split-K attention and its merge, Wo + residual, gate/up + SwiGLU, down +
// residual) and the LM head with argmax.  Instantiated per layer weight
// format by persist_q4.hip / persist_q5.hip / persist_q8.hip.
//
// No device-wide barrier separates the stages.  A stage's reader waits for
// the data itself: every exchange vector starts the launch filled with
// PK_POISON, writers store their elements with write-through stores, and a
// reader polls the elements it needs until none is poisoned (first with
// plain loads, then re-reading only poisoned 16-byte pieces with coherent
// 64-bit loads).  Each element is written once per launch, so a value other
// than PK_POISON is final.  Exchange buffers alternate between two sets by
// launch parity; during a launch each work-group refills the elements it
// writes in the other (idle) set with PK_POISON, layer by layer.
//
// Roles inside a work-group (vector memory operations of one wave complete
// in issue order, so a wave that waits on a poll must not have weight
// prefetches outstanding):
//   * io waves (0..PK_IO-1) poll the stage inputs, convert them into the
//     MFMA operand in LDS (RMSNorm partial sums included), keep the fp32
//     residuals in LDS, stage queries and the new K/V row for attention,
//     store attention partials and run the split merge;
//   * mac waves hold per-matrix weight rings in registers, issued one or more
//     stages before use (gate/up right after the QKV stage, Wo too, down and
//     the next layer's QKV after gate/up), prefetch their attention item's
//     K/V tile into LDS with direct-to-LDS loads during the QKV stage, and
//     run the matvecs and their epilogues.  Their waits use fixed load
//     counts (every ring load is issued unconditionally).
// Matvec work: tile t belongs to mac wave t mod W (wave gw = mw * nwg + wg,
// W = PK_MAC * nwg), so work-group wg writes the rows of tiles t = wg mod
// nwg.  A mac wave finishes each tile's columns into LDS scratch in its
// ring loop and runs the epilogues afterwards in a compact loop.
#pragma once
#include "gemv_impl.h"
#include "qtensor_impl.h"

// ---- exchange memory ---------------------------------------------------------
// Write-through store of a value (never the poison pattern itself).
__device__ __forceinline__ void pk_st(float *p, float v)
{
    uint32_t b = __float_as_uint(v);
    b = b == PK_POISON ? 0x7FC00000u : b;
    __hip_atomic_store(gptr((uint32_t *)p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void pk_poison(float *p)
{
    __hip_atomic_store(gptr((uint32_t *)p), PK_POISON, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool pk_bad(float v) { return __float_as_uint(v) == PK_POISON; }
__device__ __forceinline__ bool pk_bad4(const float4 &v)
{
    return (int)pk_bad(v.x) | (int)pk_bad(v.y) | (int)pk_bad(v.z) | (int)pk_bad(v.w);
}

// 16 bytes read past this CU's L2 (two coherent 64-bit loads).
__device__ __forceinline__ float4 pk_reload4(const float *p)
{
    const unsigned long long a =
        __hip_atomic_load(gptr((const unsigned long long *)p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long b =
        __hip_atomic_load(gptr((const unsigned long long *)p + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}

// Poll round `round` of a wait: gives up (flagging the launch) after
// PK_SPIN_MAX rounds, or early once another wait of the launch gave up, so
// every wave always reaches the end of the kernel.
__device__ __forceinline__ bool pk_give_up(int round, int *err)
{
    if (round >= PK_SPIN_MAX) {
        atomicOr(err, 1);
        return true;
    }
    return (round & 127) == 127 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Waits until the N float4 pieces at p[i] (enabled ones) hold no poison.
template <int N>
__device__ __forceinline__ void pk_wait4(float4 (&v)[N], const float *const (&p)[N], const bool (&on)[N], int *err)
{
#pragma unroll
    for (int j = 0; j < N; j++)
        if (on[j]) v[j] = ldg((const float4 *)p[j]);
    for (int round = 0;; round++) {
        bool any = false;
#pragma unroll
        for (int j = 0; j < N; j++) {
            if (on[j] && pk_bad4(v[j])) {
                any = true;
                v[j] = pk_reload4(p[j]);
            }
        }
        if (!any || pk_give_up(round, err)) break;
    }
}

// Profiling marks (null: off).
__device__ __forceinline__ void pk_mark(const PkArgs &a, int stage, int k)
{
    if (a.marks && (threadIdx.x & 63) == 0)
        a.marks[((size_t)stage * gridDim.x + blockIdx.x) * PK_MARKS + k] = wall_clock64();
}

// Work-group execution barrier that waits for LDS traffic only (a fence
// would make the waves wait for their outstanding prefetches).
__device__ __forceinline__ void pk_bar()
{
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(63));
    __builtin_amdgcn_s_barrier();
}

// A copy of *p read through the constant address space: the layer table is
// read-only for the whole launch, so uniform reads of it become scalar loads
// (plain global reads could be clobbered by the launch's stores, for the
// compiler).
template <typename T>
__device__ __forceinline__ T pk_cload(const T *p)
{
    static_assert(sizeof(T) % 4 == 0, "word copy");
    const auto *q = (const __attribute__((address_space(4))) uint32_t *)p;
    struct W {
        uint32_t w[sizeof(T) / 4];
    } v;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 4); i++) v.w[i] = q[i];
    return __builtin_bit_cast(T, v);
}

// Layer li's table entry (li made uniform).
__device__ __forceinline__ const PkLayer *pk_layer(const PkArgs &a, int li)
{
    return a.layers + __builtin_amdgcn_readfirstlane(li);
}

// ---- operand staging (io waves) ---------------------------------------------
// The thread index, opaque to the optimiser: per-thread offsets computed from
// it stay inside the layer loop instead of being hoisted out of it (and held
// in registers across the whole loop).
__device__ __forceinline__ int pk_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Inputs of (block b, k-group g) item `it` in the operand layout of kernels.h:
// two float4 pieces starting at k0 and k1.
template <int DT>
__device__ __forceinline__ void pk_koff(int it, int &k0, int &k1)
{
    const int b = it >> 2, g = it & 3;
    k0 = 32 * b + (DT == DT_Q8_0 ? 8 * g : 4 * g);
    k1 = k0 + (DT == DT_Q8_0 ? 4 : 16);
}

// The io thread's share of vector x[K] (items it = t + j * 64 PK_IO), polled.
template <int DT>
__device__ __forceinline__ void pk_poll_x(const float *x, int K, float4 (&v)[2 * PK_MAXI], int *err)
{
    const int t = pk_tid(), nit = K / 8;
    const float *p[2 * PK_MAXI];
    bool on[2 * PK_MAXI];
#pragma unroll
    for (int j = 0; j < PK_MAXI; j++) {
        const int it = t + j * 64 * PK_IO;
        int k0 = 0, k1 = 0;
        if (it < nit) pk_koff<DT>(it, k0, k1);
        p[2 * j] = x + k0;
        p[2 * j + 1] = x + k1;
        on[2 * j] = on[2 * j + 1] = it < nit;
    }
    pk_wait4<2 * PK_MAXI>(v, p, on, err);
}

// Polled values -> the MFMA operand in LDS (norm_w applied when given; the
// zero padding after the last block is written by the caller), optionally
// the fp32 vector itself into xr; returns the thread's sum of squares.
template <int DT>
__device__ __forceinline__ float pk_put_x(const float4 (&v)[2 * PK_MAXI], int K, const float *norm_w, uint8_t *s_op,
                                          float *xr)
{
#pragma clang fp contract(off)
    const int t = pk_tid(), nit = K / 8;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PK_MAXI; j++) {
        const int it = t + j * 64 * PK_IO;
        if (it >= nit) continue;
        int k0, k1;
        pk_koff<DT>(it, k0, k1);
        const float4 a = v[2 * j], c = v[2 * j + 1];
        if (xr) {
            *(float4 *)(xr + k0) = a;
            *(float4 *)(xr + k1) = c;
        }
        float x[8];
        // operand element order: Q8_0 k = 8g + e; Q4_0/Q5_0 k = (e>=4 ? 16 : 0) + 4g + {0,2,1,3}[e&3]
        if constexpr (DT == DT_Q8_0) {
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
        } else {
            x[0] = a.x; x[1] = a.z; x[2] = a.y; x[3] = a.w;
            x[4] = c.x; x[5] = c.z; x[6] = c.y; x[7] = c.w;
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
            ss += x[e] * x[e];
            const float tt = (norm_w ? wn[e] * x[e] : x[e]) * ACT_SCALE;
            hi[e] = (_Float16)tt;
            lo[e] = (_Float16)((tt - (float)hi[e]) * LO_SCALE);
        }
        *(f16x8 *)(s_op + (size_t)(it * 2) * 16) = hi;
        *(f16x8 *)(s_op + (size_t)(it * 2 + 1) * 16) = lo;
    }
    return ss;
}

// io waves: poll x, build the operand (+ padding zeros), keep xr, publish the
// sum of squares in s_ss[0..PK_IO) — the caller separates this from the
// previous stage's operand readers with pk_bar() and from the readers with
// another.
template <int DT>
__device__ __forceinline__ void pk_io_stage(const float4 (&v)[2 * PK_MAXI], const QTensor &w, const float *norm_w,
                                            uint8_t *s_op, float *xr, float *s_ss)
{
    const int t = pk_tid(), l = t & 63, wid = t >> 6;
    const int nblk = w.cols >> 5, opb = 4 * w.fold * w.block_quads * 128;
    float ss = pk_put_x<DT>(v, w.cols, norm_w, s_op, xr);
    for (int off = nblk * 128 + t * 16; off < opb + 16; off += 64 * PK_IO * 16)
        *(u32x4 *)(s_op + off) = u32x4{0, 0, 0, 0};
    ss = wave_sum(ss);
    if (l == 0) s_ss[wid] = ss;
}

// ---- weight rings (mac waves) -------------------------------------------------
template <int DT, int CAP>
struct PkRing {
    u32x4 c0[CAP];
    u32x4 c1[DT == DT_Q8_0 ? CAP : 1];
    u32x2 dv[CAP];
    uint32_t hv[DT == DT_Q5_0 ? CAP : 1];
};

// A mac wave's share of a matrix: its tiles gw, gw + W, ...; len items
// (quads of its tiles in order).
struct PkWork {
    int gw, W, ntw, len;
};

__device__ __forceinline__ PkWork pk_work(const QTensor &w, int gw, int W)
{
    PkWork k;
    k.gw = gw;
    k.W = W;
    k.ntw = gw < w.row_tiles ? (w.row_tiles - 1 - gw) / W + 1 : 0;
    k.len = k.ntw * w.block_quads;
    return k;
}

// Cursor over a wave's items (uniform): the first cell of the current tile
// and the quad within it.  Items past the wave's last one map to the wave's
// first cell (cell 0 for a wave without items): loaded, never used.
struct PkCur {
    size_t tile, step, first;
    int q, bq, left;
};

__device__ __forceinline__ PkCur pk_cur(const QTensor &w, const PkWork &k)
{
    PkCur c;
    c.bq = w.block_quads;
    c.first = k.len ? (size_t)k.gw * c.bq : 0;
    c.tile = c.first;
    c.step = (size_t)k.W * c.bq;
    c.q = 0;
    c.left = k.len;
    return c;
}

__device__ __forceinline__ size_t pk_cell(const PkCur &c) { return c.left > 0 ? c.tile + c.q : c.first; }

__device__ __forceinline__ void pk_next(PkCur &c)
{
    c.left--;
    if (++c.q == c.bq) {
        c.q = 0;
        c.tile += c.step;
    }
}

// Loads the cursor's item into slot u and moves the cursor on.
template <int DT, int CAP>
__device__ __forceinline__ void pk_load(PkRing<DT, CAP> &r, int u, const QTensor &w, PkCur &c)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    const int l = pk_tid() & 63;
    const size_t cell = pk_cell(c);
    const auto *p = gptr((const u32x4 *)((w.qs + cell * 64 * LB) + l * LB));
    r.c0[u] = p[0];
    if constexpr (DT == DT_Q8_0) r.c1[u] = p[1];
    r.dv[u] = *gptr((const u32x2 *)((w.d + cell * 64) + (l & 15) * 4));
    if constexpr (DT == DT_Q5_0) r.hv[u] = *gptr((w.qh + cell * 64) + l);
    pk_next(c);
}

// Issues the wave's first CAP items of w.
template <int DT, int CAP>
__device__ __forceinline__ void pk_fill(PkRing<DT, CAP> &r, const QTensor &w, const PkWork &k)
{
    PkCur c = pk_cur(w, k);
#pragma unroll
    for (int u = 0; u < CAP; u++) pk_load<DT, CAP>(r, u, w, c);
}

// One item: the quad's four blocks against the operand in LDS (ap: this
// lane's A row of the quad's first block, astride: bytes per block).  The
// four products are issued back to back and scaled into acc afterwards, in
// block order.
template <int DT>
__device__ __forceinline__ void pk_item(f32x4 &acc, const u32x4 &c0, const u32x4 &c1, const u32x2 &dv, uint32_t hv,
                                        const uint8_t *ap, int astride)
{
#pragma clang fp contract(off)
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f16x8 xv[4];
#pragma unroll
    for (int bi = 0; bi < 4; bi++) xv[bi] = *(const f16x8 *)(ap + bi * astride);
    f32x4 cc[4];
#pragma unroll
    for (int bi = 0; bi < 4; bi++) cc[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[bi], deq_block<DT>(c0, c1, hv, bi), zero4, 0, 0, 0);
    const float dsc[4] = {f16lo(dv[0]), f16hi(dv[0]), f16lo(dv[1]), f16hi(dv[1])};
#pragma unroll
    for (int bi = 0; bi < 4; bi++) {
        acc[0] = fmaf(dsc[bi], cc[bi][0], acc[0]);
        acc[1] = fmaf(dsc[bi], cc[bi][1], acc[1]);
        acc[2] = fmaf(dsc[bi], cc[bi][2], acc[2]);
        acc[3] = fmaf(dsc[bi], cc[bi][3], acc[3]);
    }
}

// Per-lane constants of a matrix's products: A rows fed by this lane (2p + h
// = high (h = 0) or scaled low (h = 1) part of k part p; rows past 2F read
// the zero slot at opb) and the tile-result slot it finishes.
struct PkA {
    const uint8_t *ap;   // quad 0's first block
    int astride;         // bytes per block (0: the zero slot)
    int qstride;         // bytes per quad
    int sel;             // accumulator pair this lane finishes (-1: none)
    int off;             // its slot in a tile's 16 results
};
__device__ __forceinline__ PkA pk_arows(const QTensor &w, const uint8_t *s_op)
{
    const int l = pk_tid() & 63, F = w.fold, BQ = w.block_quads;
    const int lgR = 4 - __builtin_ctz((unsigned)F);
    const int g = l >> 4, ar = l & 15;
    const bool ok = ar < 2 * F;
    PkA A;
    A.ap = s_op + (ok ? (ar >> 1) * 4 * BQ * 128 + (g * 2 + (ar & 1)) * 16 : 4 * F * BQ * 128);
    A.astride = ok ? 128 : 0;
    A.qstride = 4 * A.astride;
    // column c = part pc x row rc: lane group pc / 2 holds it, entry pair pc % 2
    const int c = l & 15, pc = c >> lgR, rc = c & ((1 << lgR) - 1);
    A.sel = (pc >> 1) == g && pc < F ? (pc & 1) : -1;
    A.off = rc * F + pc;
    return A;
}

// End of tile kt: the lane keeps the high/low pair of its own part in the
// wave's scratch zw[kt][16].
__device__ __forceinline__ void pk_tile_out(f32x4 &acc, float *zw, int kt, const PkA &A)
{
#pragma clang fp contract(off)
    const float v = A.sel ? acc[2] + acc[3] * LO_INV_SCALE : acc[0] + acc[1] * LO_INV_SCALE;
    if (A.sel >= 0) zw[kt * 16 + A.off] = v;
    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}

// The wave's products of matrix w: items from ring r (first CAP prefetched),
// any further items streamed through two more slots; tile results go to
// zw[kt][16] (LDS).  The operand is in s_op.
template <int DT, int CAP>
__device__ __forceinline__ void pk_mac(PkRing<DT, CAP> &r, const QTensor &w, const PkWork &k, const uint8_t *s_op,
                                       float *zw)
{
    const int BQ = w.block_quads;
    const PkA A = pk_arows(w, s_op);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    int q = 0, kt = 0;   // the item's tile and quad
    // the prefetched items: no load is issued here, so every wait is for
    // one slot's own loads
#pragma unroll
    for (int u = 0; u < CAP; u++) {
        if (u < k.len) {
            pk_item<DT>(acc, r.c0[u], DT == DT_Q8_0 ? r.c1[u] : u32x4{0, 0, 0, 0}, r.dv[u],
                        DT == DT_Q5_0 ? r.hv[u] : 0u, A.ap + q * A.qstride, A.astride);
            q = __builtin_amdgcn_readfirstlane(q + 1);   // uniform: keeps the branch scalar
            if (q == BQ) {
                pk_tile_out(acc, zw, kt, A);
                q = 0;
                kt++;
            }
        }
    }
    // items past the ring (larger models): two in flight at a time
    if (k.len > CAP) {
        PkCur c = pk_cur(w, k);
        c.tile += (size_t)kt * c.step;
        c.q = q;
        c.left -= CAP;
        PkRing<DT, 2> s2;
        pk_load<DT, 2>(s2, 0, w, c);
        pk_load<DT, 2>(s2, 1, w, c);
        for (int i = CAP; i < k.len; i += 2) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                if (i + u < k.len) {
                    pk_item<DT>(acc, s2.c0[u], DT == DT_Q8_0 ? s2.c1[u] : u32x4{0, 0, 0, 0}, s2.dv[u],
                                DT == DT_Q5_0 ? s2.hv[u] : 0u, A.ap + q * A.qstride, A.astride);
                    q = __builtin_amdgcn_readfirstlane(q + 1);   // uniform: keeps the branch scalar
                    if (q == BQ) {
                        pk_tile_out(acc, zw, kt, A);
                        q = 0;
                        kt++;
                    }
                }
                pk_load<DT, 2>(s2, u, w, c);
            }
        }
    }
}

// The wave's output rows (ntw tiles x R rows), 64 at a time, one per lane:
// f(ok, e, row, y) with e the row's index among the wave's rows and y the sum
// of its F parts (in order) times ACT_INV_SCALE.  Every lane calls f (ok
// false past the last row), so f may shuffle; lanes e and e ^ 1 hold rows
// 2i and 2i + 1 of one tile.
template <typename Fn>
__device__ __forceinline__ void pk_rows(const QTensor &w, const PkWork &k, const float *zw, Fn &&f)
{
#pragma clang fp contract(off)
    const int l = pk_tid() & 63, F = w.fold, lgR = 4 - __builtin_ctz((unsigned)F);
    const int n = k.ntw << lgR;
    for (int e0 = 0; e0 < n; e0 += 64) {
        const int e = e0 + l, kt = e >> lgR, rr = e & ((1 << lgR) - 1);
        const bool ok = e < n;
        float v[8];
        const float *p = zw + (ok ? kt * 16 + rr * F : 0);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = j < F ? p[j] : 0.0f;
        float z = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j < F) z += v[j];
        f(ok, e, ((k.gw + kt * k.W) << lgR) + rr, z * ACT_INV_SCALE);
    }
}

// ---- LM head (all waves, streamed) -------------------------------------------------
template <int DT>
__device__ __forceinline__ void pk_head(const PkArgs &a, const QTensor &w, const uint8_t *s_op, float nrm)
{
#pragma clang fp contract(off)
    constexpr int U = 8;
    const int l = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int BQ = w.block_quads, F = w.fold, R = 16 >> __builtin_ctz((unsigned)F);
    const PkWork k = pk_work(w, wid * gridDim.x + blockIdx.x, PK_WAVES * gridDim.x);
    PkCur c = pk_cur(w, k);
    PkRing<DT, U> r;
#pragma unroll
    for (int u = 0; u < U; u++) pk_load<DT, U>(r, u, w, c);
    const PkA A = pk_arows(w, s_op);
    // the part-p column of row rc sits in lane group p/2 at column p*R + rc,
    // entry pair p%2: this lane's value of that column
    const int cc = l & 15, pc = cc / R;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    unsigned long long best = 0ull;
    int q = 0, kt = 0;
    for (int i0 = 0; i0 < k.len; i0 += U) {
        const bool more = i0 + U < k.len;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u;
            if (i < k.len) {
                pk_item<DT>(acc, r.c0[u], DT == DT_Q8_0 ? r.c1[u] : u32x4{0, 0, 0, 0}, r.dv[u],
                            DT == DT_Q5_0 ? r.hv[u] : 0u, A.ap + q * A.qstride, A.astride);
                q = __builtin_amdgcn_readfirstlane(q + 1);   // uniform: keeps the branch scalar
                if (q == BQ) {
                    float own = 0.0f;
#pragma unroll
                    for (int qq = 0; qq < 2; qq++) {
                        const int pp = 2 * (l >> 4) + qq;
                        if (pp < F && pp == pc) own = acc[2 * qq] + acc[2 * qq + 1] * LO_INV_SCALE;
                    }
                    float z = 0.0f;
                    for (int p = 0; p < F; p++) {
                        const int src = 16 * (p >> 1) + p * R + (l % R);
                        z += __shfl(own, src, 64);
                    }
                    const int t = k.gw + kt * k.W, row = t * R + l;
                    const bool act = l < R && row < w.rows;
                    const float y = z * ACT_INV_SCALE * nrm;
                    if (act) a.logits[row] = y;
                    const unsigned long long key = act ? argmax_key(y, (uint32_t)row) : 0ull;
                    best = key > best ? key : best;
                    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    q = 0;
                    kt++;
                }
            }
            if (more) pk_load<DT, U>(r, u, w, c);
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    if (l == 0 && best)
        __hip_atomic_fetch_max(gptr(a.argmax + (k.gw & (ARGMAX_SLOTS - 1))), best, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// ---- ownership of exchange elements ---------------------------------------------
// Work-group wg writes (and re-poisons) the rows of the tiles t = wg mod nwg
// of each matrix, attention item it = wg (split it / n_kv of kv head
// it % n_kv: the partial slots of its query heads), merge item wg (query head
// wg / (d_head / PK_MSLICE), dimension slice wg % (d_head / PK_MSLICE)) and
// embedding block b = wg mod nwg.  The other parity's buffers are idle for
// the whole launch (the previous launch has ended, the next one has not
// begun), so the io waves re-poison them layer by layer while they wait.

// Element e of this work-group's rows of a matrix with row_tiles tiles of R
// = 1 << lgR rows: -1 past its rows.
__device__ __forceinline__ int pk_own_row(int e, int row_tiles, int lgR)
{
    const int t = blockIdx.x + (e >> lgR) * gridDim.x;
    return t < row_tiles ? (t << lgR) + (e & ((1 << lgR) - 1)) : -1;
}

// Rows of this work-group of a matrix (upper bound of pk_own_row's e).
__device__ __forceinline__ int pk_own_rows(int row_tiles, int lgR)
{
    const int wg = blockIdx.x, nwg = gridDim.x;
    return wg < row_tiles ? ((row_tiles - 1 - wg) / nwg + 1) << lgR : 0;
}

// Re-poisons this work-group's elements of layer li, parity par (io threads
// t of nt).
__device__ __forceinline__ void pk_repoison_layer(const PkArgs &a, int par, int li, int t, int nt)
{
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int d = a.d, kvd = a.n_kv * a.d_head, G = a.n_heads / a.n_kv, slot = a.d_head + 4;
    const PkLayer *Yp = pk_layer(a, li);
    const PkEx E = pk_cload(&Yp->ex[par]);
    const QTensor Yqkv = pk_cload(&Yp->qkv), Yo = pk_cload(&Yp->o), Ydown = pk_cload(&Yp->down),
                  Ygu = pk_cload(&Yp->gu);
    {   // QKV rows
        const int lgR = 4 - __builtin_ctz((unsigned)Yqkv.fold);
        const int n = pk_own_rows(Yqkv.row_tiles, lgR);
        for (int e = t; e < n; e += nt) {
            const int row = pk_own_row(e, Yqkv.row_tiles, lgR);
            if (row < 0) continue;
            if (row < d) pk_poison(E.q + row);
            else if (row < d + kvd) pk_poison(E.kn + row - d);
            else if (row < d + 2 * kvd) pk_poison(E.vn + row - d - kvd);
        }
    }
    {   // Wo and down rows
        const int lgR = 4 - __builtin_ctz((unsigned)Yo.fold);
        const int n = pk_own_rows(Yo.row_tiles, lgR);
        for (int e = t; e < n; e += nt) {
            const int row = pk_own_row(e, Yo.row_tiles, lgR);
            if (row >= 0 && row < d) pk_poison(E.xa + row);
        }
        const int lgRd = 4 - __builtin_ctz((unsigned)Ydown.fold);
        const int nd = pk_own_rows(Ydown.row_tiles, lgRd);
        for (int e = t; e < nd; e += nt) {
            const int row = pk_own_row(e, Ydown.row_tiles, lgRd);
            if (row >= 0 && row < d) pk_poison(E.xo + row);
        }
    }
    {   // SwiGLU outputs: h[i] from gate/up rows 2i, 2i + 1
        const int lgR = 4 - __builtin_ctz((unsigned)Ygu.fold);
        const int n = pk_own_rows(Ygu.row_tiles, lgR);
        for (int e = t; e < n; e += nt) {
            const int row = pk_own_row(e, Ygu.row_tiles, lgR);
            if (row >= 0 && !(row & 1) && row < 2 * a.d_ffn) pk_poison(E.h + (row >> 1));
        }
    }
    for (int it = wg; it < a.n_kv * a.max_splits; it += nwg) {   // attention partials
        const int kvh = it % a.n_kv, sp = it / a.n_kv;
        for (int i = t; i < G * slot; i += nt) {
            const int h = kvh * G + i / slot;
            pk_poison(E.part + ((size_t)h * a.max_splits + sp) * slot + i % slot);
        }
    }
    const int nsl = a.d_head / PK_MSLICE;
    for (int it = wg; it < a.n_heads * nsl; it += nwg)   // merged attention output
        for (int i = t; i < PK_MSLICE; i += nt)
            pk_poison(E.att + (it / nsl) * a.d_head + (it % nsl) * PK_MSLICE + i);
}

// The embedding rows of this work-group, parity par.
__device__ __forceinline__ void pk_repoison_x0(const PkArgs &a, int par, int t, int nt)
{
    const int wg = blockIdx.x, nwg = gridDim.x;
    for (int b = wg; b < a.d / 32; b += nwg)
        for (int i = t; i < 32; i += nt) pk_poison((a.x0 + (size_t)par * a.d) + 32 * b + i);
}

// Shared per-launch state of the two roles.
struct PkSt {
    int par, tok, pos, L, split, nsplit;
    size_t slot_off;
    int akvh, asp, at0, at1;   // this work-group's attention item
    bool has_att;
};

// LDS areas.
template <typename KT>
struct PkSm {
    uint8_t *op;
    KT *k, *v;
    float *xr1, *xr2, *q, *sc, *red, *ss, *ml, *mrg, *zw;
};

// Barriers the attention stage passes (the mac waves pass the same number):
// two before the chunks, two per chunk, two more per later chunk, one after.
__device__ __forceinline__ int pk_att_bars(int cnt_all)
{
    const int nch = (cnt_all + PK_KV_POS - 1) / PK_KV_POS;
    return 3 + 2 * nch + 2 * (nch > 0 ? nch - 1 : 0);
}

// ---- io waves: every stage's inputs, attention, merge ----------------------------
template <int DL, int DH, typename KT>
__device__ __forceinline__ void pk_io_loop(const PkArgs &a, const PkSt &S, const PkSm<KT> &M)
{
#pragma clang fp contract(off)
    const int wg = blockIdx.x;
    constexpr int NT = 64 * PK_IO;   // io threads
    const int G = a.n_heads / a.n_kv, d = a.d;
    const int slot_f = DH + 4;   // floats per partial slot
    const float qk_scale = 1.0f / sqrtf((float)DH);
    const int nsl = DH / PK_MSLICE;
    float4 xv[2 * PK_MAXI];
    for (int li = 0; li < a.n_layers; li++) {
        // the layer's table entry (scalar loads)
        const int lu = __builtin_amdgcn_readfirstlane(li);
        const PkLayer *Yp = pk_layer(a, lu);
        const PkEx E = pk_cload(&Yp->ex[S.par]);
        const QTensor w_qkv = pk_cload(&Yp->qkv), w_o = pk_cload(&Yp->o), w_gu = pk_cload(&Yp->gu),
                      w_dn = pk_cload(&Yp->down);
        const float *const attn_norm = pk_cload(&Yp->attn_norm), *const ffn_norm = pk_cload(&Yp->ffn_norm);
        const size_t kvo = S.slot_off + pk_cload(&Yp->kv_off);
        const float *x_in = lu == 0 ? (a.x0 + (size_t)S.par * a.d) : pk_cload(&pk_layer(a, lu - 1)->ex[S.par].xo);
        const int st = 1 + 6 * li;
        const int tid = pk_tid(), l = tid & 63, wid = tid >> 6;

        // S1: the QKV operand (attn_norm) and the Wo residual
        pk_mark(a, st, 0);
        pk_poll_x<DL>(x_in, d, xv, a.err);
        pk_mark(a, st, 1);
        pk_bar();
        pk_io_stage<DL>(xv, w_qkv, attn_norm, M.op, M.xr1, M.ss);
        pk_bar();
        pk_repoison_layer(a, S.par ^ 1, lu, tid, NT);

        // S2: attention of this work-group's item
        {
            const bool newrow = S.has_att && S.pos >= S.at0 && S.pos < S.at0 + PK_KV_POS;
            if (S.has_att) {
                pk_mark(a, st + 1, 0);
                constexpr int QP = ATT_MAX_G * DH / 4 / NT + 1;
                float4 qv[QP];
                const float *qp[QP];
                bool qon[QP];
#pragma unroll
                for (int j = 0; j < QP; j++) {
                    const int ci = tid + j * NT;
                    qon[j] = ci < G * DH / 4;
                    qp[j] = E.q + (size_t)S.akvh * G * DH + 4 * (qon[j] ? ci : 0);
                }
                pk_wait4<QP>(qv, qp, qon, a.err);
#pragma unroll
                for (int j = 0; j < QP; j++)
                    if (qon[j]) *(float4 *)(M.q + 4 * (tid + j * NT)) = qv[j];
                pk_mark(a, st + 1, 1);
            }
            float4 nk[1] = {make_float4(0.f, 0.f, 0.f, 0.f)};
            if (newrow) {   // this position's K (threads 0..DH/4) and V rows
                const int ci = tid % (DH / 4);
                const bool isv = tid >= DH / 4;
                const float *pp[1] = {(isv ? E.vn : E.kn) + (size_t)S.akvh * DH + 4 * ci};
                const bool on[1] = {tid < DH / 2};
                pk_wait4<1>(nk, pp, on, a.err);
            }
            pk_bar();   // the mac waves' K/V tile has landed
            if (newrow && tid < DH / 2) {
                const int ci = tid % (DH / 4);
                KT *dst = (tid >= DH / 4 ? M.v : M.k) + (size_t)(S.pos - S.at0) * DH + 4 * ci;
                dst[0] = (KT)nk[0].x;
                dst[1] = (KT)nk[0].y;
                dst[2] = (KT)nk[0].z;
                dst[3] = (KT)nk[0].w;
            }
            if (tid < ATT_MAX_G) {
                M.ml[tid] = -INFINITY;   // running max
                M.ml[8 + tid] = 0.0f;    // running sum
            }
            for (int i = tid; i < G * DH; i += NT) M.red[i] = 0.0f;
            pk_bar();
            const int cnt_all = S.has_att ? S.at1 - S.at0 : 0;
            for (int c0 = 0; c0 < cnt_all; c0 += PK_KV_POS) {
                const int cnt = min(PK_KV_POS, cnt_all - c0);
                if (c0 > 0) {   // a later chunk of a long split, loaded here
                    pk_bar();
                    const KT *kb = (const KT *)a.k_base + kvo + (size_t)S.akvh * a.max_ctx * DH;
                    const KT *vb = (const KT *)a.v_base + kvo + (size_t)S.akvh * a.max_ctx * DH;
                    constexpr int EPL = 16 / (int)sizeof(KT);
                    for (int e = tid; e < 2 * cnt * DH / EPL; e += NT) {
                        const int row = e / (DH / EPL), col = (e % (DH / EPL)) * EPL;
                        const bool isv = row >= cnt;
                        const int r = isv ? row - cnt : row;
                        const int p = S.at0 + c0 + r;
                        if (p == S.pos) continue;   // from the exchange row below
                        const u32x4 v = *gptr((const u32x4 *)((isv ? vb : kb) + (size_t)p * DH + col));
                        *(u32x4 *)((isv ? M.v : M.k) + (size_t)r * DH + col) = v;
                    }
                    if (S.pos >= S.at0 + c0 && S.pos < S.at0 + c0 + cnt) {   // this position's row, polled
                        const int ci = tid % (DH / 4);
                        const bool isv = tid >= DH / 4;
                        float4 v[1];
                        const float *pp[1] = {(isv ? E.vn : E.kn) + (size_t)S.akvh * DH + 4 * ci};
                        const bool on[1] = {tid < DH / 2};
                        pk_wait4<1>(v, pp, on, a.err);
                        if (tid < DH / 2) {
                            KT *dst = (isv ? M.v : M.k) + (size_t)(S.pos - S.at0 - c0) * DH + 4 * ci;
                            dst[0] = (KT)v[0].x;
                            dst[1] = (KT)v[0].y;
                            dst[2] = (KT)v[0].z;
                            dst[3] = (KT)v[0].w;
                        }
                    }
                    pk_bar();
                }
                // scores: (head h, position p) by 4 threads, a quarter of DH each
                for (int e = tid; e < G * PK_KV_POS * 4; e += NT) {
                    const int j = e & 3, hp = e >> 2, h = hp / PK_KV_POS, p = hp % PK_KV_POS;
                    float dot = 0.0f;
                    if (p < cnt) {
                        const float *qq = M.q + h * DH;
                        const KT *kk = M.k + (size_t)p * DH;
#pragma unroll
                        for (int i = j * 4; i < DH; i += 16) {
                            dot = fmaf(qq[i], (float)kk[i], dot);
                            dot = fmaf(qq[i + 1], (float)kk[i + 1], dot);
                            dot = fmaf(qq[i + 2], (float)kk[i + 2], dot);
                            dot = fmaf(qq[i + 3], (float)kk[i + 3], dot);
                        }
                    }
                    dot += __shfl_xor(dot, 1, 64);
                    dot += __shfl_xor(dot, 2, 64);
                    if (j == 0) M.sc[h * PK_KV_POS + p] = p < cnt ? dot * qk_scale : -INFINITY;
                }
                pk_bar();
                // online softmax: io wave w takes heads w, w + PK_IO, ...
                for (int h = wid; h < G; h += PK_IO) {
                    const float sv = M.sc[h * PK_KV_POS + l];
                    const float mc = wave_max(sv);
                    const float mo = M.ml[h], mn = fmaxf(mo, mc);
                    const float e = expf(sv - mn);
                    M.sc[h * PK_KV_POS + l] = e;
                    const float ls = wave_sum(e);
                    if (l == 0) {
                        const float al = expf(mo - mn);
                        M.ml[16 + h] = al;
                        M.ml[h] = mn;
                        M.ml[8 + h] = M.ml[8 + h] * al + ls;
                    }
                }
                pk_bar();
                // weighted sum of V: thread (h, dim)
                for (int e = tid; e < G * DH; e += NT) {
                    const int h = e / DH, i = e % DH;
                    float o = M.red[e] * M.ml[16 + h];
                    for (int p = 0; p < cnt; p++) o = fmaf(M.sc[h * PK_KV_POS + p], (float)M.v[(size_t)p * DH + i], o);
                    M.red[e] = o;
                }
            }
            pk_bar();
            if (S.has_att) {   // partial slots of the item's query heads: o, then (m, l)
                for (int e = tid; e < G * DH; e += NT) {
                    const int h = e / DH, i = e % DH;
                    pk_st(E.part + ((size_t)(S.akvh * G + h) * a.max_splits + S.asp) * slot_f + i, M.red[e]);
                }
                if (tid < G) {
                    float *sl = E.part + ((size_t)(S.akvh * G + tid) * a.max_splits + S.asp) * slot_f + DH;
                    pk_st(sl, M.ml[tid]);
                    pk_st(sl + 1, M.ml[8 + tid]);
                }
                pk_mark(a, st + 1, 2);
            }
        }

        // S3: merge of the splits of (query head, dimension slice) item wg
        const bool has_mrg = wg < a.n_heads * nsl;
        if (has_mrg) {
            const int qh = wg / nsl, ds = wg % nsl;
            pk_mark(a, st + 2, 0);
            // 9 pieces per split: 8 of the slice's outputs, then (m, l, -, -)
            constexpr int MP = 12;
            float4 pv[MP];
            const float *pp[MP];
            bool pon[MP], ml_piece[MP];
#pragma unroll
            for (int j = 0; j < MP; j++) {
                const int ci = tid + j * NT;
                const int sp = ci / 9, c = ci % 9;
                pon[j] = sp < S.nsplit;
                ml_piece[j] = c == 8;
                const float *slot = E.part + ((size_t)qh * a.max_splits + (pon[j] ? sp : 0)) * slot_f;
                pp[j] = c < 8 ? slot + ds * PK_MSLICE + 4 * c : slot + DH;
            }
#pragma unroll
            for (int j = 0; j < MP; j++)
                if (pon[j]) pv[j] = ldg((const float4 *)pp[j]);
            for (int round = 0;; round++) {   // the (m, l) piece's last two floats are padding
                bool any = false;
#pragma unroll
                for (int j = 0; j < MP; j++) {
                    const bool bad =
                        pon[j] && (ml_piece[j] ? ((int)pk_bad(pv[j].x) | (int)pk_bad(pv[j].y)) : pk_bad4(pv[j]));
                    if (bad) {
                        any = true;
                        pv[j] = pk_reload4(pp[j]);
                    }
                }
                if (!any || pk_give_up(round, a.err)) break;
            }
#pragma unroll
            for (int j = 0; j < MP; j++) {
                const int ci = tid + j * NT;
                const int sp = ci / 9, c = ci % 9;
                if (!pon[j]) continue;
                float *rw = M.mrg + sp * (PK_MSLICE + 2);
                if (c < 8) {
                    rw[4 * c] = pv[j].x;
                    rw[4 * c + 1] = pv[j].y;
                    rw[4 * c + 2] = pv[j].z;
                    rw[4 * c + 3] = pv[j].w;
                } else {
                    rw[PK_MSLICE] = pv[j].x;
                    rw[PK_MSLICE + 1] = pv[j].y;
                }
            }
        }
        pk_bar();
        if (has_mrg && tid < PK_MSLICE) {
            // out = sum_s o_s e^(m_s - mx) / sum_s l_s e^(m_s - mx)
            const int qh = wg / nsl, ds = wg % nsl;
            float mx = -INFINITY;
            for (int sp = 0; sp < S.nsplit; sp++) mx = fmaxf(mx, M.mrg[sp * (PK_MSLICE + 2) + PK_MSLICE]);
            float lsum = 0.0f, o = 0.0f;
            for (int sp = 0; sp < S.nsplit; sp++) {
                const float w = expf(M.mrg[sp * (PK_MSLICE + 2) + PK_MSLICE] - mx);
                lsum = fmaf(M.mrg[sp * (PK_MSLICE + 2) + PK_MSLICE + 1], w, lsum);
                o = fmaf(M.mrg[sp * (PK_MSLICE + 2) + tid], w, o);
            }
            pk_st(E.att + qh * DH + ds * PK_MSLICE + tid, o / lsum);
            pk_mark(a, st + 2, 2);
        }

        // S4: the Wo operand
        pk_mark(a, st + 3, 0);
        pk_poll_x<DL>(E.att, d, xv, a.err);
        pk_mark(a, st + 3, 1);
        pk_bar();
        pk_io_stage<DL>(xv, w_o, nullptr, M.op, nullptr, M.ss);
        pk_bar();

        // S5: the gate/up operand (ffn_norm) and the down residual
        pk_mark(a, st + 4, 0);
        pk_poll_x<DL>(E.xa, d, xv, a.err);
        pk_mark(a, st + 4, 1);
        pk_bar();
        pk_io_stage<DL>(xv, w_gu, ffn_norm, M.op, M.xr2, M.ss);
        pk_bar();

        // S6: the down operand
        pk_mark(a, st + 5, 0);
        pk_poll_x<DL>(E.h, a.d_ffn, xv, a.err);
        pk_mark(a, st + 5, 1);
        pk_bar();
        pk_io_stage<DL>(xv, w_dn, nullptr, M.op, nullptr, M.ss);
        pk_bar();
    }

    // the LM head operand (out_norm)
    const int sl = pk_stages(a.n_layers) - 1;
    const float *xl = pk_cload(&pk_layer(a, a.n_layers - 1)->ex[S.par].xo);
    pk_mark(a, sl, 0);
    switch (a.lm.dtype) {
    case DT_Q4_0: pk_poll_x<DT_Q4_0>(xl, d, xv, a.err); break;
    case DT_Q5_0: pk_poll_x<DT_Q5_0>(xl, d, xv, a.err); break;
    default: pk_poll_x<DT_Q8_0>(xl, d, xv, a.err); break;
    }
    pk_mark(a, sl, 1);
    pk_bar();
    switch (a.lm.dtype) {
    case DT_Q4_0: pk_io_stage<DT_Q4_0>(xv, a.lm, a.out_norm, M.op, nullptr, M.ss); break;
    case DT_Q5_0: pk_io_stage<DT_Q5_0>(xv, a.lm, a.out_norm, M.op, nullptr, M.ss); break;
    default: pk_io_stage<DT_Q8_0>(xv, a.lm, a.out_norm, M.op, nullptr, M.ss); break;
    }
    pk_bar();
}

// RMSNorm scale from the io waves' sums of squares (fixed order).
__device__ __forceinline__ float pk_nrm(const float *ss, int n, float eps)
{
    float s = 0.0f;
    for (int w = 0; w < PK_IO; w++) s += ss[w];
    return 1.0f / sqrtf(s / (float)n + eps);
}

// ---- mac waves: weight rings, the K/V tile, matvecs --------------------------------
// Ring capacities (items per mac wave): the gate/up ring is filled right
// after the QKV stage and held through attention, merge and Wo, next to the
// Wo ring; every ring load counts against the 63 outstanding vector memory
// operations a wave can track.
template <int DL> struct PkCap;
template <> struct PkCap<DT_Q4_0> { static constexpr int Q = 4, O = 4, G = 24, D = 12; };
template <> struct PkCap<DT_Q5_0> { static constexpr int Q = 4, O = 4, G = 14, D = 12; };
template <> struct PkCap<DT_Q8_0> { static constexpr int Q = 4, O = 4, G = 12, D = 10; };

template <int DL, int DH, typename KT>
__device__ __forceinline__ void pk_mac_loop(const PkArgs &a, const PkSt &S, const PkSm<KT> &M)
{
#pragma clang fp contract(off)
    typedef PkCap<DL> C;
    constexpr int LPI = q_loads<DL>();
    constexpr int KV_LOADS = 2 * PK_KV_POS * DH * (int)sizeof(KT) / (16 * 64 * PK_MAC);   // per mac wave
    static_assert((C::G + C::O) * LPI <= 63 && (C::D + C::Q) * LPI <= 63, "ring loads exceed vmcnt");
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int mw = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) - PK_IO);
    const int gw = mw * nwg + wg, W = PK_MAC * nwg;
    const int d = a.d, kvd = a.n_kv * DH;
    float *const zw = M.zw + (size_t)mw * 16 * PK_ZW_TILES;   // this wave's tile scratch
    PkRing<DL, C::Q> rq;
    PkRing<DL, C::O> ro;
    PkRing<DL, C::G> rg;
    PkRing<DL, C::D> rd;
    {
        const QTensor w0 = pk_cload(&pk_layer(a, 0)->qkv);
        pk_fill<DL, C::Q>(rq, w0, pk_work(w0, gw, W));
    }
    for (int li = 0; li < a.n_layers; li++) {
        // the layer's table entry (scalar loads)
        const int lu = __builtin_amdgcn_readfirstlane(li);
        const PkLayer *Yp = pk_layer(a, lu);
        const PkEx E = pk_cload(&Yp->ex[S.par]);
        const QTensor w_qkv = pk_cload(&Yp->qkv), w_o = pk_cload(&Yp->o), w_gu = pk_cload(&Yp->gu),
                      w_dn = pk_cload(&Yp->down);
        const int rope_on = pk_cload(&Yp->rope_on);
        const size_t kvo = S.slot_off + pk_cload(&Yp->kv_off);
        const int st = 1 + 6 * li;
        const int l = pk_tid() & 63;

        // S1: RoPE pairs of the wave's first 64 QKV rows (one per lane, as
        // the epilogue maps them), then the attention item's K/V tile
        // (direct-to-LDS, fixed count) ...
        const PkWork kq = pk_work(w_qkv, gw, W);
        const int lgRq = 4 - __builtin_ctz((unsigned)w_qkv.fold);
        auto rope_of = [&](int row) {
            row = min(max(row, 0), d + 2 * kvd - 1);
            const int rr = row < d ? row : row - d;
            return ldg((const float2 *)(a.rope + ((size_t)S.pos * (DH / 2) + ((rr % DH) >> 1)) * 2));
        };
        const float2 cs0 = rope_of(((kq.gw + (l >> lgRq) * kq.W) << lgRq) + (l & ((1 << lgRq) - 1)));
        {
            const KT *kb = (const KT *)a.k_base + kvo + (size_t)S.akvh * a.max_ctx * DH;
            const KT *vb = (const KT *)a.v_base + kvo + (size_t)S.akvh * a.max_ctx * DH;
            constexpr int EPL = 16 / (int)sizeof(KT);   // elements per 16-byte piece
            constexpr int ROWL = DH / EPL;              // pieces per row
#pragma unroll
            for (int c = 0; c < KV_LOADS; c++) {
                const int e0 = (c * PK_MAC + mw) * 64 + l;   // K rows first, then V rows
                const int row = e0 / ROWL, col = (e0 % ROWL) * EPL;
                const bool isv = row >= PK_KV_POS;
                const int r = isv ? row - PK_KV_POS : row;
                const int p = max(min(S.at0 + r, S.pos - 1), 0);
                const KT *src = (isv ? vb : kb) + (size_t)p * DH + col;
                __builtin_amdgcn_global_load_lds((const gvoid_t *)src,
                                                 (lvoid_t *)((uint8_t *)M.k + (size_t)((c * PK_MAC + mw) * 64) * 16), 16,
                                                 0, 0);
            }
        }
        // ... and the QKV matvec once the operand is staged
        pk_bar();
        pk_bar();
        {
            pk_mark(a, st, 3);
            const float nrm = pk_nrm(M.ss, d, a.eps);
            pk_mac<DL, C::Q>(rq, w_qkv, kq, M.op, zw);
            pk_mark(a, st, 4);
            pk_rows(w_qkv, kq, zw, [&](bool ok, int e, int row, float y) {
                y *= nrm;
                const float partner = __shfl_xor(y, 1, 64);
                if (ok && row < d + 2 * kvd) {
                    float val = y;
                    if (row < d + kvd && rope_on) {
                        const float2 c2 = e < 64 ? cs0 : rope_of(row);
                        if (!(row & 1)) val = y * c2.x - partner * c2.y;
                        else val = partner * c2.y + y * c2.x;
                    }
                    if (row < d) {
                        pk_st(E.q + row, val);
                    } else {
                        const bool isk = row < d + kvd;
                        const int rr = isk ? row - d : row - d - kvd;
                        const int h = rr / DH, i = rr % DH;
                        const KT kv = (KT)val;
                        KT *base = (KT *)(isk ? a.k_base : a.v_base);
                        base[kvo + ((size_t)h * a.max_ctx + S.pos) * DH + i] = kv;
                        pk_st((isk ? E.kn : E.vn) + rr, (float)kv);
                    }
                }
            });
            pk_mark(a, st, 2);
            // the Wo and gate/up weights stream from here on
            pk_fill<DL, C::O>(ro, w_o, pk_work(w_o, gw, W));
            pk_fill<DL, C::G>(rg, w_gu, pk_work(w_gu, gw, W));
            pk_mark(a, st, 5);
        }

        // S2 and S3 belong to the io waves: the K/V tile must have landed
        // (everything older than the two rings' loads), then the barriers
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0((C::O + C::G) * LPI));
        const int nbar = pk_att_bars(S.has_att ? S.at1 - S.at0 : 0) + 1;
        for (int i = 0; i < nbar; i++) pk_bar();

        // S4: Wo + residual
        pk_bar();
        pk_bar();
        {
            pk_mark(a, st + 3, 3);
            const PkWork k = pk_work(w_o, gw, W);
            pk_mac<DL, C::O>(ro, w_o, k, M.op, zw);
            pk_mark(a, st + 3, 4);
            pk_rows(w_o, k, zw, [&](bool ok, int, int row, float y) {
                if (ok && row < d) pk_st(E.xa + row, M.xr1[row] + y);
            });
            pk_mark(a, st + 3, 2);
        }

        // S5: gate/up + SwiGLU
        pk_bar();
        pk_bar();
        {
            pk_mark(a, st + 4, 3);
            const float nrm = pk_nrm(M.ss, d, a.eps);
            const PkWork k = pk_work(w_gu, gw, W);
            pk_mac<DL, C::G>(rg, w_gu, k, M.op, zw);
            pk_mark(a, st + 4, 4);
            pk_rows(w_gu, k, zw, [&](bool ok, int, int row, float y) {
                y *= nrm;
                const float u = __shfl_xor(y, 1, 64);
                if (ok && !(row & 1) && row < 2 * a.d_ffn) pk_st(E.h + (row >> 1), (y / (1.0f + expf(-y))) * u);
            });
            pk_mark(a, st + 4, 2);
            // the down weights and the next layer's QKV weights stream from here on
            pk_fill<DL, C::D>(rd, w_dn, pk_work(w_dn, gw, W));
            if (li + 1 < a.n_layers) {
                const QTensor wn = pk_cload(&pk_layer(a, lu + 1)->qkv);
                pk_fill<DL, C::Q>(rq, wn, pk_work(wn, gw, W));
            }
            pk_mark(a, st + 4, 5);
        }

        // S6: down + residual
        pk_bar();
        pk_bar();
        {
            pk_mark(a, st + 5, 3);
            const PkWork k = pk_work(w_dn, gw, W);
            pk_mac<DL, C::D>(rd, w_dn, k, M.op, zw);
            pk_mark(a, st + 5, 4);
            pk_rows(w_dn, k, zw, [&](bool ok, int, int row, float y) {
                if (ok && row < d) pk_st(E.xo + row, M.xr2[row] + y);
            });
            pk_mark(a, st + 5, 2);
        }
    }
    // the LM head operand is staged by the io waves
    pk_bar();
    pk_bar();
}

template <int DL, int DH, typename KT>
__global__ __launch_bounds__(PK_THREADS) void k_persist(PkArgs a)
{
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.n_heads / a.n_kv, d = a.d;
    const PkLds Ld = pk_lds(a.op_bytes, d, DH, a.kv_f16, G, a.max_splits);
    PkSm<KT> M;
    M.op = smem + Ld.op;
    M.k = (KT *)(smem + Ld.kv);
    M.v = M.k + PK_KV_POS * DH;
    M.xr1 = (float *)(smem + Ld.xr1);
    M.xr2 = (float *)(smem + Ld.xr2);
    M.q = (float *)(smem + Ld.q);
    M.sc = (float *)(smem + Ld.sc);
    M.red = (float *)(smem + Ld.red);
    M.ss = (float *)(smem + Ld.ss);
    M.ml = (float *)(smem + Ld.ml);
    M.mrg = (float *)(smem + Ld.mrg);
    M.zw = (float *)(smem + Ld.zw);

    // per-launch values, uniform across the work-group (scalar registers:
    // the addresses built from them stay scalar)
    PkSt S;
    S.par = a.par & 1;
    S.tok = __builtin_amdgcn_readfirstlane(a.step[0]);
    S.pos = min(max(__builtin_amdgcn_readfirstlane(a.step[1]), 0), a.max_ctx - 1);
    S.L = min(max(__builtin_amdgcn_readfirstlane(a.step[2]), 1), a.max_ctx);
    S.slot_off = (size_t)__builtin_amdgcn_readfirstlane(a.slot_id[0]) * a.slot_stride;
    S.split = pk_split(S.L, a.max_splits);
    S.nsplit = (S.L + S.split - 1) / S.split;
    S.akvh = wg % a.n_kv;
    S.asp = wg / a.n_kv;
    S.has_att = S.asp < S.nsplit;
    S.at0 = S.asp * S.split;
    S.at1 = min(S.L, S.at0 + S.split);
    if (a.trace && wg == 0 && tid == 0) a.trace[0] = wall_clock64();

    // start: argmax slots cleared (work-group 0) and the embedding row (io
    // waves); the mac waves fill their first ring in their loop
    if (wid < PK_IO) {
        if (wg == 0 && tid < ARGMAX_SLOTS)
            __hip_atomic_store(a.argmax + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));   // cleared before any of this launch's outputs
        const int nb = d / 32, tok = (S.tok < 0 || S.tok >= a.embd.rows) ? 0 : S.tok;
        for (int b0 = wg; b0 < nb; b0 += nwg * (64 * PK_IO / 4)) {
            const int b = b0 + (tid >> 2) * nwg, g = tid & 3;
            if (b < nb) {
                float val[8];
                switch (a.embd.dtype) {
                case DT_Q4_0: block_vals8<DT_Q4_0>(a.embd, tok, b, g, val); break;
                case DT_Q5_0: block_vals8<DT_Q5_0>(a.embd, tok, b, g, val); break;
                default: block_vals8<DT_Q8_0>(a.embd, tok, b, g, val); break;
                }
                for (int e = 0; e < 8; e++) pk_st((a.x0 + (size_t)S.par * a.d) + 32 * b + kmap(a.embd.dtype, g, e), val[e]);
            }
        }
        pk_mark(a, 0, 0);
        pk_repoison_x0(a, S.par ^ 1, tid, 64 * PK_IO);
        pk_io_loop<DL, DH, KT>(a, S, M);
    } else {
        pk_mac_loop<DL, DH, KT>(a, S, M);
    }

    // RMSNorm + LM head (every wave): logits and argmax
    {
        const float nrm = pk_nrm(M.ss, d, a.eps);
        switch (a.lm.dtype) {
        case DT_Q4_0: pk_head<DT_Q4_0>(a, a.lm, M.op, nrm); break;
        case DT_Q5_0: pk_head<DT_Q5_0>(a, a.lm, M.op, nrm); break;
        default: pk_head<DT_Q8_0>(a, a.lm, M.op, nrm); break;
        }
        pk_mark(a, pk_stages(a.n_layers) - 1, 2);
    }

    pk_mark(a, pk_stages(a.n_layers) - 1, 6);
    if (a.trace && wg == 0 && tid == 0) a.trace[1] = wall_clock64();
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
    if (lds > 160 * 1024) return 0;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, PK_THREADS, (size_t)lds) != hipSuccess ||
        per_cu < 1)
        return 0;
    return cus < PK_MAX_WGS ? cus : PK_MAX_WGS;
}
