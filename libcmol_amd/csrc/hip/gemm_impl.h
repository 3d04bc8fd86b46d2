// gemm_impl.h — the prompt (prefill) GEMM: Y[n][rows] = X[n][K] . W^T for
// many activation vectors (n = prompt tokens), instantiated per weight
// format by gemm_q4.hip / gemm_q5.hip / gemm_q8.hip / gemm_q4k.hip /
// gemm_q6k.hip.
//
// One work-group computes a 64-vector x 128-row output tile (32 x 128 with
// four waves where 64-vector tiles would leave half the CUs idle).  Its
// eight waves form a 2 x 4 grid: wave (wm, wn) owns vectors 32wm..32wm+31
// (two groups of 16, each with a 16-row high and a 16-row low operand block
// in LDS) and output rows 32wn..32wn+31 (two 16-row "virtual tiles").  The
// k loop walks block quads through a two-stage pipeline: the activation
// operand of quad kk+1 is copied into LDS with direct-to-LDS loads and each
// wave loads the weight codes of its two virtual tiles for it into
// registers while quad kk is contracted.  Two stages (64 KiB of LDS) keep two work-groups on a CU,
// which hides more latency than a third stage in flight with one.
// Weights of any fold are read in place: virtual tile V of part p gathers,
// for column c', the codes of row 16V + c' from tile (16V + c') / R,
// column p*R + c' % R.
//
// Arithmetic follows the decode matvec's (gemv_impl.h): codes decoded to
// exact f16 integers, v_mfma_f32_16x16x32_f16 against the exact hi/lo
// operand, fp32 per-block scaling, and the same fused epilogues.  Unlike the
// matvec, each block's low-part products join the high-part MFMA sum (codes
// times 2^-11 against the low part times 2^11), so one scale FMA per output
// and block serves both.
#pragma once
#include "gemv_impl.h"

#define GEMM_BN 128   // output rows per work-group (8 virtual tiles)
#define GEMM_STAGES 2 // quads in flight

struct GemmShape {
    int epi;
    int mt;          // vector tiles (GEMM_BM vectors each)
    int nt;          // 128-row tiles
    int vt;          // 16-row virtual tiles (ceil(rows / 16))
    int ga;          // XCD slices along the vector tiles (1, 2, 4, 8)
    int mts, nts;    // vector / row tiles per slice
    int ks, kq;      // k ranges (grid.y) of kq block quads each; ks > 1: fp32 partial sums to a.part
};

// acc += the block's contribution for 16 vectors: xh holds their high
// operand parts, xl their low parts (scaled by LO_SCALE), wv the decoded
// codes and wl the codes times LO_INV_SCALE (exact: a power of two).  The
// low products go into the same fp32 sum as the high ones, so one scale FMA
// per output and block applies the block's factor to both.
template <int DT>
__device__ __forceinline__ void mfma_block_hl(f32x4 &acc, const f16x8 &xh, const f16x8 &xl, const f16x8 &wv,
                                              const f16x8 &wl, const BlockScale &s)
{
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (DT == DT_Q4_K) {
        const _Float16 o = (_Float16)1, ol = (_Float16)LO_INV_SCALE;
        const f16x8 ones = {o, o, o, o, o, o, o, o};
        const f16x8 onesl = {ol, ol, ol, ol, ol, ol, ol, ol};
        f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wv, z, 0, 0, 0);
        cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wl, cc, 0, 0, 0);
        f32x4 cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, ones, z, 0, 0, 0);
        cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, onesl, cs, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s1, cs[i], fmaf(s.s0, cc[i], acc[i]));
    } else if constexpr (DT == DT_Q6_K) {
        const _Float16 o = (_Float16)0;
        const f16x8 w0 = {wv[0], wv[1], wv[2], wv[3], o, o, o, o};
        const f16x8 w1 = {o, o, o, o, wv[4], wv[5], wv[6], wv[7]};
        const f16x8 l0 = {wl[0], wl[1], wl[2], wl[3], o, o, o, o};
        const f16x8 l1 = {o, o, o, o, wl[4], wl[5], wl[6], wl[7]};
        f32x4 c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, w0, z, 0, 0, 0);
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, l0, c0, 0, 0, 0);
        f32x4 c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, w1, z, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, l1, c1, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s1, c1[i], fmaf(s.s0, c0[i], acc[i]));
    } else {
        f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wv, z, 0, 0, 0);
        cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wl, cc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(s.s0, cc[i], acc[i]);
    }
}

// q_load with precomputed element offsets: e = cell * 64 + lane (codes,
// Q5_0 fifth bits, Q6_K high bits) and ds = the scale record's index
// (cell * 64 + col * 4 halves, or cell * 16 + col K-quant records).
template <int DT>
__device__ __forceinline__ void gemm_wload(const QTensor &w, uint32_t e, uint32_t ds, u32x4 &c0, u32x4 &c1,
                                           typename QScale<DT>::T &sv, uint32_t &h)
{
    constexpr uint32_t LB = QFmt<DT>::LANE_BYTES;
    const u32x4 *p = (const u32x4 *)(w.qs + e * LB);
    c0 = p[0];
    if constexpr (DT == DT_Q8_0) c1 = p[1];
    else if constexpr (DT == DT_Q6_K) {
        const u32x2 hb = *(const u32x2 *)((const uint8_t *)w.qh + e * 8u);
        c1 = u32x4{hb[0], hb[1], 0u, 0u};
    } else c1 = u32x4{0, 0, 0, 0};
    if constexpr (is_kquant(DT)) sv = *(const u32x4 *)((const uint8_t *)w.d + ds * 16u);
    else sv = *(const u32x2 *)((const uint8_t *)w.d + ds * 2u);
    if constexpr (DT == DT_Q5_0) h = *(const uint32_t *)((const uint8_t *)w.qh + e * 4u);
    else h = 0u;
}

// WM wave rows of HG groups of 16 vectors each (GEMM_BM = 16 HG WM vectors
// per work-group), four wave columns of 32 output rows: 4 WM waves
template <int DT, int WM, int HG>
__global__ __launch_bounds__(4 * WM * 64) void k_gemm(GemvArgs a, GemmShape sh)
{
    constexpr int GEMM_BM = 16 * HG * WM, GEMM_WAVES = 4 * WM;
    constexpr int SEGS = GEMM_BM / 32;            // 64-row operand segments per (block, group)
    constexpr int PW = 16 * SEGS / GEMM_WAVES;    // operand copies per wave and stage
    constexpr int ASTAGE = 4 * 4 * 2 * GEMM_BM * 16;   // [block][k-group][2 GEMM_BM rows][16 B]
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *s_a = smem;                                 // GEMM_STAGES x ASTAGE

    // XCD-aware tile order: work-groups b, b+8, b+16, ... share an XCD.  The
    // (vector tile, row tile) grid is cut into ga x (8 / ga) slices, one per
    // XCD; an XCD walks its slice vector tile fastest, so the operand tiles
    // of its slice stay in its L2 while the weights stream past
    const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
    const int mt_ = (xcd % sh.ga) * sh.mts + i % sh.mts;
    const int nt_ = (xcd / sh.ga) * sh.nts + i / sh.mts;
    if (mt_ >= sh.mt || nt_ >= sh.nt) return;
    const int m0 = mt_ * GEMM_BM;

    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, cl = l & 15;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid % WM, wn = wid / WM;
    const int n = a.n, nrows = 2 * n;
    const int BQ = a.w.block_quads, F = a.w.fold, R = 16 / F;
    const int nblk = a.w.cols >> 5;
    const int KQ = F * BQ;
    // this work-group's k range (split-K over grid.y): quads kb .. ke - 1
    const int kb = (int)blockIdx.y * sh.kq, ke = min(KQ, kb + sh.kq);

    // RMSNorm scales of the tile's vectors from the producer's partials,
    // passed through the last stage's LDS (untouched until the k loop's
    // first copy into it, which follows a wait and a barrier) to the lanes
    // that apply them: lane l's vectors 16 HG wm + 16h + 4(l>>4) + e
    float nrm[HG][4] = {};
    if (a.in.ss) {
        float *s_nrm = (float *)(smem + (GEMM_STAGES - 1) * ASTAGE);
        for (int vi = wid; vi < GEMM_BM; vi += GEMM_WAVES) {
            const int v = min(m0 + vi, n - 1);
            float s = 0.0f;
            for (int i = l; i < a.in.ss_count; i += 64) s += a.in.ss[(size_t)v * a.in.ss_stride + i];
            s = wave_sum(s);
            if (l == 0) s_nrm[vi] = 1.0f / sqrtf(s / (float)a.w.cols + a.in.eps);
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < HG; h++)
#pragma unroll
            for (int e = 0; e < 4; e++) nrm[h][e] = s_nrm[16 * HG * wm + 16 * h + 4 * (l >> 4) + e];
    }

    // weight gather for this lane: virtual tile V -> (tile, column).  The
    // lane's element offsets within the tensor (32-bit: the host checks the
    // size) are fixed here; each quad adds a uniform part
    uint32_t wq[2], wd[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int V = nt_ * 8 + wn * 2 + j;
        const int row = V * 16 + cl;
        const uint32_t wt = (uint32_t)min(row / R, a.w.row_tiles - 1), wc = (uint32_t)(row % R);
        wq[j] = wt * (uint32_t)BQ * 64u + wc + 16u * (uint32_t)g;   // cell * 64 + lane
        wd[j] = is_kquant(DT) ? wt * (uint32_t)BQ * 16u + wc : wt * (uint32_t)BQ * 64u + 4u * wc;
    }
    // operand rows of this lane's two 64-row halves (LDS rows of each 32-row
    // group: the 16 high parts, then the 16 low parts of its 16 vectors,
    // operand rows 2v and 2v+1)
    uint32_t arow[SEGS];
#pragma unroll
    for (int half = 0; half < SEGS; half++) {
        const int l5 = l & 31;
        arow[half] = 16u * (uint32_t)min(2 * m0 + 64 * half + (l & 32) + 2 * (l5 & 15) + (l5 >> 4), nrows - 1);
    }

    u32x4 c0[GEMM_STAGES][2], c1[GEMM_STAGES][2];
    typename QScale<DT>::T dv[GEMM_STAGES][2];
    uint32_t hv[GEMM_STAGES][2];
    // loads of quad kk into stage st: 4 operand copies (of the tile's 32
    // 1 KiB pieces) and the codes/scales of the wave's two virtual tiles;
    // every load is issued unconditionally (padding blocks re-read a valid
    // block) so the per-stage load count is fixed
    auto load_stage = [&](int st, int kk) {
        kk = min(kk, ke - 1);
        const int p = kk / BQ, q = kk - p * BQ;
        const int b0 = p * 4 * BQ + 4 * q;
#pragma unroll
        for (int i = 0; i < PW; i++) {
            const int s = wid * PW + i;           // 16 (block, group) pairs x SEGS segments
            const int seg = s / SEGS, half = i % SEGS;   // wid * PW % SEGS == 0
            const int bi = seg >> 2, gg = seg & 3;
            const int blk = min(b0 + bi, nblk - 1);
            const uint8_t *src = (const uint8_t *)a.in.q + ((size_t)blk * 4 + gg) * nrows * 16 + arow[half];
            uint8_t *dst = s_a + st * ASTAGE + ((bi * 4 + gg) * 2 * GEMM_BM + 64 * half) * 16;
            __builtin_amdgcn_global_load_lds((const gvoid_t *)src, (lvoid_t *)dst, 16, 0, 0);
        }
        const uint32_t uq = (uint32_t)(q * 64 + p * R);
        const uint32_t ud = is_kquant(DT) ? (uint32_t)(q * 16 + p * R) : (uint32_t)(q * 64 + 4 * p * R);
#pragma unroll
        for (int j = 0; j < 2; j++) gemm_wload<DT>(a.w, wq[j] + uq, wd[j] + ud, c0[st][j], c1[st][j], dv[st][j], hv[st][j]);
    };

    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc[HG][2];
#pragma unroll
    for (int h = 0; h < HG; h++) {
        acc[h][0] = zero4;
        acc[h][1] = zero4;
    }

    auto compute = [&](int st, int kk) {
        const int p = kk / BQ, q = kk - p * BQ;
        // blocks of this quad: padding blocks of the last part and the steps
        // past the end of the k range contribute nothing
        const int nb = kk < ke ? min(4, nblk - (p * 4 * BQ + 4 * q)) : 0;
        const uint8_t *sa = s_a + st * ASTAGE;
        auto block = [&](int bi) {
            f16x8 wv[2], wl[2];
            BlockScale bs[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                wv[j] = deq_block<DT>(c0[st][j], c1[st][j], hv[st][j], bi);
                wl[j] = wv[j] * (_Float16)LO_INV_SCALE;
                bs[j] = block_scale<DT>(dv[st][j], bi);
            }
#pragma unroll
            for (int h = 0; h < HG; h++) {
                const uint8_t *row = &sa[((bi * 4 + g) * 2 * GEMM_BM + 32 * HG * wm + 32 * h + cl) * 16];
                const f16x8 xh = *(const f16x8 *)row;
                const f16x8 xl = *(const f16x8 *)(row + 16 * 16);
#pragma unroll
                for (int j = 0; j < 2; j++) mfma_block_hl<DT>(acc[h][j], xh, xl, wv[j], wl[j], bs[j]);
            }
        };
        // a whole quad is one straight run (the four blocks' loads, MFMA
        // chains and scale FMAs interleave); the uniform test keeps branches
        // between blocks to the rare partial quads
        if (nb == 4) {
#pragma unroll
            for (int bi = 0; bi < 4; bi++) block(bi);
        } else {
#pragma unroll
            for (int bi = 0; bi < 4; bi++) {
                if (bi >= nb) break;
                block(bi);
            }
        }
    };

    // two-stage k loop: at the top of step kk only the loads of kk are
    // outstanding; the wait and the barrier publish every wave's copy of kk
    // (and every wave is done with kk-1), then kk+1 is issued into the stage
    // kk-1 freed
    load_stage(0, kb);
    __builtin_amdgcn_sched_barrier(0);
    // the body is unconditional (steps past the end compute nothing and
    // re-read the last quad) so every wait count is the same on each pass
    for (int k0 = kb; k0 < ke; k0 += GEMM_STAGES) {
#pragma unroll
        for (int u = 0; u < GEMM_STAGES; u++) {
            const int kk = k0 + u;
            __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            load_stage((u + 1) % GEMM_STAGES, kk + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(u, kk);
        }
    }
    // drain the trailing re-reads before the LDS can be released
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
    __syncthreads();

    // lane l holds, per vector group h and tile j, output row 16V + cl for
    // vectors m0 + 16 HG wm + 16h + 4(l>>4) + {0, 1, 2, 3}
#pragma unroll
    for (int h = 0; h < HG; h++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int V = nt_ * 8 + wn * 2 + j;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int vi = 16 * HG * wm + 16 * h + 4 * (l >> 4) + e;
                const int v = m0 + vi;
                const bool act = v < n;
                float y = acc[h][j][e] * ACT_INV_SCALE;
                if (sh.ks > 1) {
                    // this k range's partial sum (the finish kernel adds the
                    // ranges in order, then scales and runs the epilogue)
                    const int row = V * 16 + cl;
                    if (act && row < a.w.rows) a.part[((size_t)blockIdx.y * n + v) * a.w.rows + row] = y;
                    continue;
                }
                if (a.in.ss) y *= nrm[h][e];
                const int vv = act ? v : 0;
                switch (sh.epi) {
                case EPI_STORE: epilogue<EPI_STORE>(a, V, cl, 16, vv, act, y); break;
                case EPI_RESID: epilogue<EPI_RESID>(a, V, cl, 16, vv, act, y); break;
                case EPI_SWIGLU: epilogue<EPI_SWIGLU>(a, V, cl, 16, vv, act, y); break;
                default: epilogue<EPI_QKV>(a, V, cl, 16, vv, act, y); break;
                }
            }
        }
    }
}

template <int DT, int WM, int HG>
int launch_gemm_wm(const GemvArgs &a, int epi, hipStream_t s, int ks = 1)
{
    constexpr int BM = 16 * HG * WM;
    GemmShape sh;
    sh.epi = epi;
    const int KQ = a.w.fold * a.w.block_quads;
    sh.ks = ks;
    sh.kq = (KQ + ks - 1) / ks;
    if (ks > 1 && (!a.part || (size_t)ks * a.n * a.w.rows > a.part_cap)) return -6;
    sh.mt = (a.n + BM - 1) / BM;
    sh.vt = (a.w.rows + 15) / 16;
    sh.nt = (sh.vt + 7) / 8;
    // one slice of vector tiles per XCD (at M = 2048: 512 KiB of operand
    // per 64-vector tile, four per XCD) unless there are fewer vector tiles
    sh.ga = 8;
    while (sh.ga > 1 && sh.ga > sh.mt) sh.ga >>= 1;
    sh.mts = (sh.mt + sh.ga - 1) / sh.ga;
    sh.nts = (sh.nt + 8 / sh.ga - 1) / (8 / sh.ga);
    const long wgs = 8L * sh.mts * sh.nts;
    if (wgs > 0x7fffffffL) return -6;
    const size_t lds = (size_t)GEMM_STAGES * 4 * 4 * 2 * BM * 16;
    const dim3 grid((unsigned)wgs, (unsigned)ks);
    if (a.ev_start)
        hipExtLaunchKernelGGL((k_gemm<DT, WM, HG>), grid, dim3(4 * WM * 64), lds, s, a.ev_start,
                              ks > 1 ? nullptr : a.ev_stop, 0, a, sh);
    else
        hipLaunchKernelGGL((k_gemm<DT, WM, HG>), grid, dim3(4 * WM * 64), lds, s, a, sh);
    if (ks > 1) return launch_gemv_b_finish(a, epi, ks, a.in.ss ? a.in.ss_count : 0, s);
    return 0;
}

// k ranges of the split-K prompt GEMM: the fewest (a power of two, at most
// GEMM_KS_MAX) that give the 64-vector tiles two work-groups per CU, each
// range at least 8 block quads, within the partial-sum buffer; 1 when the
// tiles already fill the chip or no buffer is given.  CMOL_GEMM_KSPLIT=0
// turns it off (measurements).
static inline int gemm_ks(const QTensor &w, int n, size_t part_cap)
{
    static const bool on = [] {
        const char *e = getenv("CMOL_GEMM_KSPLIT");
        return !(e && e[0] == '0');
    }();
    const long tiles64 = (long)((n + 63) / 64) * (((w.rows + 15) / 16 + 7) / 8);
    const int KQ = w.fold * w.block_quads;
    int ks = 1;
    if (!on) return 1;
    while (ks < GEMM_KS_MAX && tiles64 * ks < 2L * gemv_cus() && KQ / (2 * ks) >= 8 &&
           (size_t)(2 * ks) * n * w.rows <= part_cap)
        ks *= 2;
    return ks;
}

static inline int gemm_ksplit(const GemvArgs &a, long)
{
    return a.part ? gemm_ks(a.w, a.n, a.part_cap) : 1;
}

// 64-vector work-groups (two per CU) unless their tiles cover at most half
// the CUs (2048 output rows at 512 tokens: 128 tiles); then 32-vector ones
// (five per CU), twice as many.  Four-wave 64-vector work-groups (four
// vector groups per wave: fewer decode and address instructions per
// product, 140 VGPRs, two waves per SIMD) ran 10-15 % slower at 2048 tokens:
// the kernel needs the waves to hide latency more than it needs fewer
// instructions.
template <int DT>
int launch_gemm_dt(const GemvArgs &a, int epi, hipStream_t s)
{
    if (epi < EPI_STORE || epi > EPI_QKV) return -6;
    // the kernel's per-lane weight offsets are 32-bit
    if ((size_t)a.w.row_tiles * a.w.block_quads * 64 * QFmt<DT>::LANE_BYTES > 0xffffffffUL) return -6;
    const long tiles64 = (long)((a.n + 63) / 64) * (((a.w.rows + 15) / 16 + 7) / 8);
    const int ks = gemm_ksplit(a, tiles64);
    if (ks > 1) return launch_gemm_wm<DT, 2, 2>(a, epi, s, ks);
    if (tiles64 <= gemv_cus() / 2) return launch_gemm_wm<DT, 1, 2>(a, epi, s);
    return launch_gemm_wm<DT, 2, 2>(a, epi, s);
}
