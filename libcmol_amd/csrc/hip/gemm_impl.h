// gemm_impl.h — the prompt (prefill) GEMM: Y[n][rows] = X[n][K] . W^T for
// many activation vectors (n = prompt tokens), instantiated per weight
// format by gemm_q4.hip / gemm_q5.hip / gemm_q8.hip.
//
// One work-group computes a 64-vector x 64-row output tile.  Its four waves
// form a 2 x 2 grid: wave (wm, wn) owns vectors 32wm..32wm+31 (A rows
// 64wm.. of the hi/lo operand, four 16-row MFMA groups) and output rows
// 32wn..32wn+31 (two 16-row "virtual tiles").  The k loop walks block quads:
// the activation operand of the next quad is copied into the other half of
// a double-buffered LDS tile with direct-to-LDS loads while the current quad
// is contracted, and each wave loads the weight codes of its two virtual
// tiles for the next quad into registers.  Weights of any fold are read in
// place: virtual tile V of part p gathers, for column c', the codes of row
// 16V + c' from tile (16V + c') / R, column p*R + c' % R.
//
// Arithmetic is the decode matvec's (gemv_impl.h): codes decoded to exact
// f16 integers, v_mfma_f32_16x16x32_f16 against the exact hi/lo operand,
// fp32 per-block scaling, and the same fused epilogues.
#pragma once
#include "gemv_impl.h"

#define GEMM_BM 64   // vectors per work-group
#define GEMM_BN 64   // output rows per work-group

struct GemmShape {
    int epi;
    int mt;          // 64-vector tiles
    int nt;          // 64-row tiles
    int vt;          // 16-row virtual tiles (ceil(rows / 16))
};

template <int DT>
__global__ __launch_bounds__(256) void k_gemm(GemvArgs a, GemmShape sh)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    // A tile per quad: [block 0..3][k-group 0..3][128 operand rows][16 B]
    __shared__ __attribute__((aligned(16))) uint8_t s_a[2][4 * 4 * 2 * GEMM_BM * 16];
    __shared__ float s_nrm[GEMM_BM];

    // XCD-aware tile order: work-groups b, b+8, b+16, ... share an XCD; give
    // them the same row tile so its weights are fetched into one L2
    const int b = blockIdx.x;
    const int grp = b / (8 * sh.mt);
    const int nt_ = grp * 8 + (b & 7), mt_ = (b >> 3) % sh.mt;
    if (nt_ >= sh.nt) return;
    const int m0 = mt_ * GEMM_BM;

    const int tid = threadIdx.x, wid = tid >> 6, l = tid & 63, g = l >> 4, cl = l & 15;
    const int wm = wid & 1, wn = wid >> 1;
    const int n = a.n, nrows = 2 * n;
    const int BQ = a.w.block_quads, F = a.w.fold, R = 16 / F;
    const int nblk = a.w.cols >> 5;
    const int KQ = F * BQ;

    // RMSNorm scales of the tile's vectors from the producer's partials
    if (a.in.ss) {
        for (int vi = wid; vi < GEMM_BM; vi += 4) {
            const int v = min(m0 + vi, n - 1);
            float s = 0.0f;
            for (int i = l; i < a.in.ss_count; i += 64) s += a.in.ss[(size_t)v * a.in.ss_stride + i];
            s = wave_sum(s);
            if (l == 0) s_nrm[vi] = 1.0f / sqrtf(s / (float)a.w.cols + a.in.eps);
        }
    }

    // weight gather for this lane: virtual tile V -> (tile, column)
    int wt[2], wc[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int V = nt_ * 4 + wn * 2 + j;
        const int row = V * 16 + cl;
        wt[j] = min(row / R, a.w.row_tiles - 1);
        wc[j] = row % R;   // + part * R
    }

    u32x4 c0[2][2], c1[2][2];
    u32x2 dv[2][2];
    uint32_t hv[2][2];
    auto load_b = [&](int buf, int kk) {
        const int p = kk / BQ, q = kk - p * BQ;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const size_t cell = (size_t)wt[j] * BQ + q;
            const int col = p * R + wc[j];
            const u32x4 *src = (const u32x4 *)(a.w.qs + (cell * 64 + col + 16 * g) * LB);
            c0[buf][j] = src[0];
            if constexpr (LB == 32) c1[buf][j] = src[1];
            else c1[buf][j] = u32x4{0, 0, 0, 0};
            dv[buf][j] = *(const u32x2 *)(a.w.d + cell * 64 + col * 4);
            if constexpr (DT == DT_Q5_0) hv[buf][j] = a.w.qh[cell * 64 + col + 16 * g];
            else hv[buf][j] = 0u;
        }
    };
    // operand rows 2*m0 .. 2*m0+127 of each (block, k-group) of quad kk;
    // rows past 2n re-read the last row (their outputs are discarded)
    auto load_a = [&](int buf, int kk) {
        const int p = kk / BQ, q = kk - p * BQ;
        const int b0 = p * 4 * BQ + 4 * q;
        for (int s = wid; s < 32; s += 4) {   // 16 (block, group) segments x 2 halves
            const int seg = s >> 1, half = s & 1;
            const int bi = seg >> 2, gg = seg & 3;
            if (b0 + bi >= nblk) continue;
            const int r = min(2 * m0 + 64 * half + l, nrows - 1);
            const uint8_t *src = (const uint8_t *)a.in.q + ((((size_t)(b0 + bi) * 4 + gg) * nrows) + r) * 16;
            uint8_t *dst = &s_a[buf][((bi * 4 + gg) * 2 * GEMM_BM + 64 * half) * 16];
            __builtin_amdgcn_global_load_lds((const gvoid_t *)src, (lvoid_t *)dst, 16, 0, 0);
        }
    };

    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc[4][2];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        acc[gi][0] = zero4;
        acc[gi][1] = zero4;
    }

    auto compute = [&](int buf, int kk) {
        const int p = kk / BQ, q = kk - p * BQ;
        const int b0 = p * 4 * BQ + 4 * q;
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
            if (b0 + bi >= nblk) break;   // padding blocks of the last part
            f16x8 wv[2];
            float dsc[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                wv[j] = deq_block<DT>(c0[buf][j], c1[buf][j], hv[buf][j], bi);
                const uint32_t dw = dv[buf][j][bi >> 1];
                dsc[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)((bi & 1) ? (dw >> 16) : (dw & 0xFFFFu)));
            }
#pragma unroll
            for (int gi = 0; gi < 4; gi++) {
                const f16x8 xv = *(const f16x8 *)&s_a[buf][((bi * 4 + g) * 2 * GEMM_BM + 64 * wm + 16 * gi + cl) * 16];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv[j], zero4, 0, 0, 0);
                    acc[gi][j][0] = fmaf(dsc[j], cc[0], acc[gi][j][0]);
                    acc[gi][j][1] = fmaf(dsc[j], cc[1], acc[gi][j][1]);
                    acc[gi][j][2] = fmaf(dsc[j], cc[2], acc[gi][j][2]);
                    acc[gi][j][3] = fmaf(dsc[j], cc[3], acc[gi][j][3]);
                }
            }
        }
    };

    // double-buffered k loop: at the top of step kk only its own copies are
    // outstanding, so the barrier's full wait is exactly what is needed
    load_a(0, 0);
    load_b(0, 0);
    for (int kk = 0; kk < KQ; kk += 2) {
        __syncthreads();
        if (kk + 1 < KQ) {
            load_a(1, kk + 1);
            load_b(1, kk + 1);
        }
        compute(0, kk);
        if (kk + 1 >= KQ) break;
        __syncthreads();
        if (kk + 2 < KQ) {
            load_a(0, kk + 2);
            load_b(0, kk + 2);
        }
        compute(1, kk + 1);
    }
    __syncthreads();   // s_nrm visible (written before the loop)

    // lane l holds, per group gi and tile j, output row 16V + cl for vectors
    // m0 + 32wm + 8gi + 2(l>>4) + {0, 1} (component pairs hi/lo)
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int V = nt_ * 4 + wn * 2 + j;
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                const int vi = 32 * wm + 8 * gi + 2 * (l >> 4) + pr;
                const int v = m0 + vi;
                const bool act = v < n;
                float y = (acc[gi][j][2 * pr] + acc[gi][j][2 * pr + 1] * LO_INV_SCALE) * ACT_INV_SCALE;
                if (a.in.ss) y *= s_nrm[vi];
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

template <int DT>
int launch_gemm_dt(const GemvArgs &a, int epi, hipStream_t s)
{
    if (epi < EPI_STORE || epi > EPI_QKV) return -6;
    GemmShape sh;
    sh.epi = epi;
    sh.mt = (a.n + GEMM_BM - 1) / GEMM_BM;
    sh.vt = (a.w.rows + 15) / 16;
    sh.nt = (sh.vt + 3) / 4;
    const long groups = (sh.nt + 7) / 8;
    const long wgs = groups * 8 * sh.mt;
    if (wgs > 0x7fffffffL) return -6;
    hipLaunchKernelGGL(k_gemm<DT>, dim3((unsigned)wgs), dim3(256), 0, s, a, sh);
    return 0;
}
