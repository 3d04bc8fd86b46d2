// attn_impl.h — split-K grouped-query decode attention over ragged KV
// lengths, as work-group device functions shared by the attention kernels
// (attn.hip) and the persistent decode kernel (persist_impl.h).
//
// Follows the arithmetic of reference src/attn.c:103-137: per query head h
// (kv head h*n_kv/n_heads), scores s_t = (q_h . K_t) / sqrtf(d_head) over
// t < seqlen, softmax, out_h = sum_t p_t V_t.  The positions of one session
// and kv head are cut into splits of `split` positions; one work-group per
// (kv head, split, vector) loads K/V for its split once and serves all G
// query heads of the group.  Each split keeps (max, sum of exp, unnormalised
// output); attn_merge_head combines the splits with the usual log-sum-exp
// rescaling.  A session whose length fits one split is finished directly by
// attn_split.
#pragma once
#include "common.h"
#include "kernels.h"

template <typename KT> struct KVec;   // 4 cache elements
template <> struct KVec<float> { typedef float4 T; };
template <> struct KVec<_Float16> { typedef f16x4 T; };

template <typename KT>
__device__ inline float4 to_f4(const typename KVec<KT>::T &v)
{
    if constexpr (sizeof(KT) == 4) return v;
    else return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

// Split `sp` of `split` positions of one (kv head, vector), computed by a
// work-group of NT threads: online softmax over chunks of CH = NT/4
// positions.  The K and V of the next chunk are loaded while the current one
// is reduced (K right after the scores, V right after the weighted sum).
// Score phase, fp32 cache: 4 threads per position, each a quarter of d_head
// (interleaved 16-byte pieces, so a position's row is read contiguously).
// Score phase, fp16 cache (256 threads): on MFMA.  Wave w scores positions
// 16w..16w+15 of the chunk with v_mfma_f32_16x16x32_f16: A rows 2h, 2h+1 are
// the high and low f16 parts of query head h (q = hi + lo/2048, exact to
// about 22 bits, split once per split), B columns are the cached K rows as
// stored (16-byte loads, 8 dimensions per lane), so every product is exact
// and the sums are fp32.
// Weighted-sum phase: thread (pg, dg) owns dims 4dg..4dg+3 and positions
// p = pg (mod PG) of the chunk, for all G query heads.  Results leave
// through the store policy M.
template <int DH, typename KT, int NT, typename M>
__device__ __forceinline__ void attn_split(const AttnArgs &a, int kvh, int sp, int n)
{
#pragma clang fp contract(off)
    typedef typename KVec<KT>::T KV4;
    constexpr int CH = NT / 4;                    // positions per chunk
    constexpr int KQ = DH / 16;                   // 4-element pieces per thread (scores)
    constexpr int DG = DH / 4, PG = NT / DG;
    constexpr int VP = CH / PG;                   // positions per thread (weighted sum)
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int G = a.n_heads / a.n_kv;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int t0 = sp * a.split;
    if (t0 >= L) return;
    const int cnt = min(L, t0 + a.split) - t0;
    const int nch = (cnt + CH - 1) / CH;
    const int nact = (L + a.split - 1) / a.split;

    __shared__ __attribute__((aligned(16))) float qsh[ATT_MAX_G][DH];
    __shared__ float esh[ATT_MAX_G][CH];
    __shared__ float alpha_sh[ATT_MAX_G], m_sh[ATT_MAX_G], l_sh[ATT_MAX_G];
    __shared__ __attribute__((aligned(16))) float red[PG * ATT_MAX_G * DH];

    const size_t off = kv_offset(a.kv, n) + (size_t)kvh * a.max_ctx * DH + (size_t)t0 * DH;
    const KT *kb = (const KT *)a.kv.k_base + off;
    const KT *vb = (const KT *)a.kv.v_base + off;

    // MFMA scores: fp16 cache, four waves of 16 positions per chunk
    constexpr bool MF = sizeof(KT) == 2 && NT == 256 && CH == 64 && DH % 32 == 0;
    constexpr int KS = MF ? DH / 32 : 1;          // MFMA k-steps per position
    const int sp_p = tid >> 2, sj = tid & 3;      // score phase
    const int dg = tid % DG, pg = tid / DG;       // weighted-sum phase
    KV4 kr[MF ? 1 : KQ], vr[VP];
    f16x8 km[KS];
    auto load_k = [&](int c) {
        if constexpr (MF) {
            const int p = min(c * CH + wid * 16 + (lane & 15), cnt - 1);
#pragma unroll
            for (int s = 0; s < KS; s++)
                km[s] = ldg((const f16x8 *)(kb + (size_t)p * DH + 32 * s + 8 * (lane >> 4)));
        } else {
            const int p = min(c * CH + sp_p, cnt - 1);
#pragma unroll
            for (int i = 0; i < KQ; i++) kr[i] = ldg((const KV4 *)(kb + (size_t)p * DH + 4 * (sj + 4 * i)));
        }
    };
    auto load_v = [&](int c) {
#pragma unroll
        for (int i = 0; i < VP; i++) {
            const int p = min(c * CH + pg + PG * i, cnt - 1);
            vr[i] = ldg((const KV4 *)(vb + (size_t)p * DH + 4 * dg));
        }
    };
    load_k(0);
    load_v(0);
    const float *qn = a.q + (size_t)n * a.q_stride + (size_t)kvh * G * DH;
    for (int i = tid; i < G * DH; i += NT) qsh[i / DH][i % DH] = *gptr(qn + i);
    if (tid < ATT_MAX_G) {
        m_sh[tid] = -INFINITY;
        l_sh[tid] = 0.0f;
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)DH);
    // MFMA A operand: lane l feeds row l%16 (query head (l%16)/2, high or
    // low part) with dimensions 32s + 8(l/16) .. +7 of k-step s
    f16x8 qa[KS];
    if constexpr (MF) {
        const int r = lane & 15, h = r >> 1;
#pragma unroll
        for (int s = 0; s < KS; s++) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = h < G ? qsh[h < G ? h : 0][32 * s + 8 * (lane >> 4) + e] : 0.0f;
                const _Float16 hi = (_Float16)x;
                qa[s][e] = (r & 1) ? (_Float16)((x - (float)hi) * 2048.0f) : hi;
            }
        }
    }
    float4 o[ATT_MAX_G];
#pragma unroll
    for (int h = 0; h < ATT_MAX_G; h++) o[h] = make_float4(0.f, 0.f, 0.f, 0.f);

    for (int c = 0; c < nch; c++) {
        const int ccnt = min(CH, cnt - c * CH);
        // scores of this chunk
        if constexpr (MF) {
            f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < KS; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], km[s], sc, 0, 0, 0);
            if (c + 1 < nch) load_k(c + 1);
            // lane l holds position 16w + l%16 for rows 4(l/16) .. +3:
            // heads 2(l/16) and 2(l/16) + 1, high and low parts
            const int pp = wid * 16 + (lane & 15), h0 = 2 * (lane >> 4);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int h = h0 + k;
                if (h < G) esh[h][pp] = pp < ccnt ? (sc[2 * k] + sc[2 * k + 1] * (1.0f / 2048.0f)) * scale : -INFINITY;
            }
        } else {
            float dot[ATT_MAX_G];
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++) dot[h] = 0.0f;
#pragma unroll
            for (int i = 0; i < KQ; i++) {
                const float4 kv = to_f4<KT>(kr[i]);
                const int d0 = 4 * (sj + 4 * i);
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++) {
                    if (h < G) {
                        const float4 qv = *(const float4 *)&qsh[h][d0];
                        dot[h] = fmaf(qv.x, kv.x, dot[h]);
                        dot[h] = fmaf(qv.y, kv.y, dot[h]);
                        dot[h] = fmaf(qv.z, kv.z, dot[h]);
                        dot[h] = fmaf(qv.w, kv.w, dot[h]);
                    }
                }
            }
            if (c + 1 < nch) load_k(c + 1);
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++) {
                dot[h] += __shfl_xor(dot[h], 1, 64);
                dot[h] += __shfl_xor(dot[h], 2, 64);
            }
            if (sj == 0) {
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++)
                    if (h < G) esh[h][sp_p] = sp_p < ccnt ? dot[h] * scale : -INFINITY;
            }
        }
        __syncthreads();
        // online softmax: wave w owns heads w, w + NT/64, ...; lane j holds
        // positions j, j + 64, ... of the chunk
        for (int h = wid; h < G; h += NT / 64) {
            float sv[CH / 64];
            float mc = -INFINITY;
#pragma unroll
            for (int j = 0; j < CH / 64; j++) {
                sv[j] = esh[h][lane + 64 * j];
                mc = fmaxf(mc, sv[j]);
            }
            mc = wave_max(mc);
            const float mo = m_sh[h];
            const float mn = fmaxf(mo, mc);
            float ls = 0.0f;
#pragma unroll
            for (int j = 0; j < CH / 64; j++) {
                const float e = expf(sv[j] - mn);
                esh[h][lane + 64 * j] = e;
                ls += e;
            }
            ls = wave_sum(ls);
            if (lane == 0) {
                const float al = expf(mo - mn);
                alpha_sh[h] = al;
                m_sh[h] = mn;
                l_sh[h] = l_sh[h] * al + ls;
            }
        }
        __syncthreads();
        // weighted sum of V
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) {
            if (h < G) {
                const float al = alpha_sh[h];
                o[h].x *= al;
                o[h].y *= al;
                o[h].z *= al;
                o[h].w *= al;
            }
        }
#pragma unroll
        for (int i = 0; i < VP; i++) {
            const int p = pg + PG * i;
            const float4 v = to_f4<KT>(vr[i]);
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++) {
                if (h < G) {
                    const float e = esh[h][p];   // 0 past the chunk's end
                    o[h].x = fmaf(e, v.x, o[h].x);
                    o[h].y = fmaf(e, v.y, o[h].y);
                    o[h].z = fmaf(e, v.z, o[h].z);
                    o[h].w = fmaf(e, v.w, o[h].w);
                }
            }
        }
        if (c + 1 < nch) load_v(c + 1);
        __syncthreads();   // esh / alpha are rewritten by the next chunk
    }

#pragma unroll
    for (int h = 0; h < ATT_MAX_G; h++)
        if (h < G) *(float4 *)&red[((size_t)pg * G + h) * DH + 4 * dg] = o[h];
    __syncthreads();
    const bool single = nact == 1;
    const size_t sbase = (((size_t)n * a.n_kv + kvh) * a.max_splits + sp) * G;
    for (int i = tid; i < G * DH; i += NT) {
        const int h = i / DH, d = i % DH;
        float sum = 0.0f;
        for (int q = 0; q < PG; q++) sum += red[((size_t)q * G + h) * DH + d];
        if (single) {
            const float ov = sum / l_sh[h];
            const int k = (kvh * G + h) * DH + d;
            if (a.out) M::st(a.out + (size_t)n * a.out_stride + k, ov);
            if (a.next.q) act_put<M>(a.next, n, k, ov);
        } else {
            M::st(a.po + (sbase + h) * DH + d, sum);
        }
    }
    if (!single && tid < G) {
        M::st(a.pm + sbase + tid, m_sh[tid]);
        M::st(a.pl + sbase + tid, l_sh[tid]);
    }
    __syncthreads();   // the LDS areas may be reused by the caller
}

// The same split over an fp16 cache, on MFMA (a work-group of 256 threads,
// d_head 64..256), in chunks of 64 positions:
//   * scores: wave w takes positions 16w..16w+15 of the chunk; A rows 2h,
//     2h+1 are the high and low f16 parts of query head h (q = hi + lo/2048),
//     B columns the cached K rows as stored (16-byte loads), 16x16x32 f16
//     MFMAs over d_head;
//   * online softmax: one wave per query head; the weights e are written to
//     LDS as exact f16 pairs (e = hi + lo/2048), the MFMA A rows of the next
//     step;
//   * weighted sum: wave w owns dimensions w*d_head/4 .. +d_head/4 of every
//     head; the chunk's V rows are staged in LDS row-major (rows padded by
//     four halves) and each B column (one dimension, eight positions) comes
//     from two transposing LDS reads (ds_read_b64_tr_b16) instead of eight
//     16-bit reads.
// Every product is exact and every sum fp32.  V goes through one LDS buffer:
// the chunk's V rows, loaded into registers during the previous chunk, are
// written after the first barrier (every wave is then done with the previous
// weighted sum), so a chunk needs two barriers and 21 KB of LDS (d_head
// 128).  Same partial format as attn_split.
template <int DH, typename M>
__device__ __forceinline__ void attn_piece_mf(const AttnArgs &a, int kvh, int n, int t0, int cnt, bool single,
                                              size_t sbase)
{
#pragma clang fp contract(off)
    constexpr int NT = 256, CH = 64;
    constexpr int KS = DH / 32;            // score k-steps
    constexpr int PPP = DH / 8;            // 16-byte pieces per cached row
    constexpr int VPT = CH * PPP / NT;     // V pieces per thread per chunk
    constexpr int DW = DH / 4;             // dimensions per wave
    constexpr int DTW = DW / 16;           // 16-dimension MFMA tiles per wave
    constexpr int RS = DH + 4;             // LDS row stride of the staged V (halves; rows 8-byte aligned)
    static_assert(DH >= 64 && DH % 64 == 0 && VPT >= 1, "shape");
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int G = a.n_heads / a.n_kv;
    const int nch = (cnt + CH - 1) / CH;

    __shared__ float esh[ATT_MAX_G][CH];
    __shared__ __attribute__((aligned(16))) _Float16 ph[2][ATT_MAX_G][CH];
    __shared__ __attribute__((aligned(16))) _Float16 vs[CH * RS];
    // the query is read once, into the MFMA operand, before chunk 0 is
    // staged: it lives in the V buffer
    static_assert(ATT_MAX_G * DH * 4 <= CH * RS * 2, "query area");
    float *qsh = (float *)vs;
    __shared__ float alpha_sh[ATT_MAX_G], m_sh[ATT_MAX_G], l_sh[ATT_MAX_G];

    const size_t off = kv_offset(a.kv, n) + (size_t)kvh * a.max_ctx * DH + (size_t)t0 * DH;
    const _Float16 *kb = (const _Float16 *)a.kv.k_base + off;
    const _Float16 *vb = (const _Float16 *)a.kv.v_base + off;

    f16x8 km[KS], vm[VPT];
    auto load_k = [&](int c) {
        const int p = min(c * CH + wid * 16 + (lane & 15), cnt - 1);
#pragma unroll
        for (int s = 0; s < KS; s++) km[s] = ldg((const f16x8 *)(kb + (size_t)p * DH + 32 * s + 8 * (lane >> 4)));
    };
    // piece q = tid + NT*i: position q / PPP, dimensions 8 (q % PPP) .. +7
    auto load_v = [&](int c) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int q = tid + NT * i;
            const int p = min(c * CH + q / PPP, cnt - 1);
            vm[i] = ldg((const f16x8 *)(vb + (size_t)p * DH + 8 * (q % PPP)));
        }
    };
    auto stage_v = [&](_Float16 *dst) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int q = tid + NT * i;
            uint32_t *w = (uint32_t *)(dst + (q / PPP) * RS + 8 * (q % PPP));
            const u32x4 u = __builtin_bit_cast(u32x4, vm[i]);
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = u[e];
        }
    };
    load_k(0);
    load_v(0);
    const float *qn = a.q + (size_t)n * a.q_stride + (size_t)kvh * G * DH;
    for (int i = tid; i < G * DH; i += NT) qsh[i] = *gptr(qn + i);
    if (tid < ATT_MAX_G) {
        m_sh[tid] = -INFINITY;
        l_sh[tid] = 0.0f;
        alpha_sh[tid] = 1.0f;
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)DH);
    // score A operand: lane l feeds row l%16 (query head (l%16)/2, high or
    // low part) with dimensions 32s + 8(l/16) .. +7 of k-step s
    const int r = lane & 15, rh = r >> 1, g = lane >> 4;
    f16x8 qa[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float x = rh < G ? qsh[(rh < G ? rh : 0) * DH + 32 * s + 8 * g + e] : 0.0f;
            const _Float16 hi = (_Float16)x;
            qa[s][e] = (r & 1) ? (_Float16)((x - (float)hi) * 2048.0f) : hi;
        }
    }
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 oc[DTW];
#pragma unroll
    for (int t = 0; t < DTW; t++) oc[t] = zero4;
    const int d0 = wid * DW + (lane & 15);   // this lane's output dimension in tile 0

    for (int c = 0; c < nch; c++) {
        const int ccnt = min(CH, cnt - c * CH);
        _Float16 *vcur = vs;
        // scores of positions 16w .. 16w+15: lane l holds position 16w + l%16
        // for rows 4(l/16) .. +3 (heads 2(l/16), 2(l/16)+1, high and low)
        f32x4 sc = zero4;
#pragma unroll
        for (int s = 0; s < KS; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], km[s], sc, 0, 0, 0);
        if (c + 1 < nch) load_k(c + 1);
        {
            const int pp = wid * 16 + (lane & 15);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int h = 2 * g + k;
                if (h < G) esh[h][pp] = pp < ccnt ? (sc[2 * k] + sc[2 * k + 1] * (1.0f / 2048.0f)) * scale : -INFINITY;
            }
        }
        __syncthreads();   // scores in LDS; every wave done with the last chunk's V
        stage_v(vcur);
        if (c + 1 < nch) load_v(c + 1);
        // online softmax: wave w owns heads w, w + 4; lane j holds position j
        for (int h = wid; h < G; h += NT / 64) {
            const float sv = esh[h][lane];
            const float mc = wave_max(sv);
            const float mo = m_sh[h];
            const float mn = fmaxf(mo, mc);
            const float e = expf(sv - mn);
            const _Float16 ehi = (_Float16)e;
            ph[0][h][lane] = ehi;
            ph[1][h][lane] = (_Float16)((e - (float)ehi) * 2048.0f);
            const float ls = wave_sum(e);
            if (lane == 0) {
                const float al = expf(mo - mn);
                alpha_sh[h] = al;
                m_sh[h] = mn;
                l_sh[h] = l_sh[h] * al + ls;
            }
        }
        __syncthreads();
        // weighted sum: rescale, then o += P . V over the chunk's 64 positions
        {
            const float a0 = alpha_sh[2 * g], a1 = alpha_sh[2 * g + 1];
#pragma unroll
            for (int t = 0; t < DTW; t++) {
                oc[t][0] *= a0;
                oc[t][1] *= a0;
                oc[t][2] *= a1;
                oc[t][3] *= a1;
            }
        }
#pragma unroll
        for (int ks = 0; ks < CH / 32; ks++) {
            const int pb = 32 * ks + 8 * g;   // this lane's eight positions
            f16x8 pa = *(const f16x8 *)&ph[r & 1][rh < G ? rh : 0][pb];
            if (rh >= G) pa = f16x8{};
#pragma unroll
            for (int t = 0; t < DTW; t++) {
                // B columns: lane (col, g) takes dimension d0 + 16t of
                // positions pb .. pb+7, gathered by two transposing LDS reads:
                // within each 16-lane group, lane s reads the four dimensions
                // 4(s%4) .. +3 of the tile at position pb + s/4 (+4), and the
                // read hands lane 4r+c element c of the lanes 4e+r
                const int s16 = lane & 15;
                const _Float16 *src = vcur + (pb + (s16 >> 2)) * RS + wid * DW + 16 * t + 4 * (s16 & 3);
                typedef short s16x4 __attribute__((ext_vector_type(4)));
                const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)src);
                const s16x4 hi4 =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(src + 4 * RS));
                const f16x8 bv = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                oc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, oc[t], 0, 0, 0);
            }
        }
    }

    // outputs: lane l holds dimension d0 + 16t of heads 2(l/16) (rows 0, 1)
    // and 2(l/16) + 1 (rows 2, 3)
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int h = 2 * g + k;
        if (h >= G) continue;
#pragma unroll
        for (int t = 0; t < DTW; t++) {
            const int d = d0 + 16 * t;
            const float ov = oc[t][2 * k] + oc[t][2 * k + 1] * (1.0f / 2048.0f);
            if (single) {
                const float fv = ov / l_sh[h];
                const int kk = (kvh * G + h) * DH + d;
                if (a.out) M::st(a.out + (size_t)n * a.out_stride + kk, fv);
                if (a.next.q) act_put<M>(a.next, n, kk, fv);
            } else {
                M::st(a.po + (sbase + h) * DH + d, ov);
            }
        }
    }
    if (!single && tid < G) {
        M::st(a.pm + sbase + tid, m_sh[tid]);
        M::st(a.pl + sbase + tid, l_sh[tid]);
    }
    __syncthreads();   // the LDS areas may be reused by the caller
}

// The same piece with the four waves independent: wave w takes positions
// 64j + 16w .. +15 of step j and keeps its own online softmax, so no
// barrier stands between a wave's loads of one step and the next; the
// waves meet once, at the end of the piece.
//   * scores transposed, S^T = K . Q^T (16x16x32 f16): the cached K rows
//     as stored are the A operand (row = position), the query's exact f16
//     halves the B operand (column 2h / 2h+1 = high / low part of head h);
//     lane l then holds positions 4(l/16) .. +3 of column l%16, the two
//     parts of a head sit in neighbouring lanes, and the layout is already
//     the A operand of the weighted sum (row = column, k = position);
//   * lazy online softmax: a head's reference maximum m moves only when a
//     score exceeds it by more than ATT_LAZY_T (a wave vote), so the common
//     step needs no cross-lane reduction; weights e = exp(s - m) <= e^T stay
//     exact f16 pairs (hi + lo/2048) and each lane sums its own e; scores
//     and m stay raw dot products t (m leaves the piece scaled), and e is
//     2^(t c - m c), c = log2(e)/sqrt(d_head), on the hardware exponential
//     (one FMA and v_exp_f32, whose exp2(-inf) = 0 also clears masked
//     positions), the product m c taken once per move of m;
//   * weighted sum P . V on 16x16x16 MFMAs: the wave's 16 V rows are staged
//     in its own LDS rows (padded by four halves) and each B column (one
//     dimension, four positions) is one transposing LDS read.
// Same partial format as attn_split_mf; products exact, sums fp32.
#define ATT_LAZY_T 8.0f
template <int DH, typename M>
__device__ __forceinline__ void attn_piece_mfw(const AttnArgs &a, int kvh, int n, int t0, int cnt, bool single,
                                               size_t sbase, size_t kvo)
{
#pragma clang fp contract(off)
    constexpr int NT = 256, NW = NT / 64;
    constexpr int KS = DH / 32;           // score k-steps
    constexpr int PPR = DH / 8;           // 16-byte pieces per cached row
    constexpr int VPL = 16 * PPR / 64;    // V pieces per lane per step (16 rows)
    constexpr int DT = DH / 16;           // 16-dimension output tiles
    constexpr int RS = DH + 4;            // LDS row stride of the staged V (halves)
    static_assert(DH >= 64 && DH % 64 == 0 && VPL >= 1, "shape");
    const int tid = threadIdx.x, wid = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int col = lane & 15, grp = lane >> 4, part = col & 1;
    const int G = a.n_heads / a.n_kv;
    cnt = __builtin_amdgcn_readfirstlane(cnt);   // the same in every lane
    t0 = __builtin_amdgcn_readfirstlane(t0);
    const int nst = (cnt + 63) / 64;

    __shared__ __attribute__((aligned(16))) _Float16 vsw[NW][16 * RS];
    // the end of the piece: each wave's (m, l, o) per head, over vsw
    static_assert(NW * ATT_MAX_G * DH * 4 <= NW * 16 * RS * 2, "combine area");
    __shared__ float xm[NW][ATT_MAX_G], xl[NW][ATT_MAX_G];
    float *xo = (float *)vsw;

    const size_t off = kvo + (size_t)kvh * a.max_ctx * DH + (size_t)t0 * DH;   // kvo: the vector's cache base
    const _Float16 *kb = uniform_ptr((const _Float16 *)a.kv.k_base + off);
    const _Float16 *vb = uniform_ptr((const _Float16 *)a.kv.v_base + off);
    f16x8 km[KS], vm[VPL];
    // 32-bit byte offsets from the piece's (uniform) base: the loads take
    // the base from scalar registers and need no 64-bit address arithmetic
    const char *kbc = (const char *)kb, *vbc = (const char *)vb;
    auto load_k = [&](int j) {
        const unsigned p = (unsigned)min(64 * j + 16 * wid + col, cnt - 1);
#pragma unroll
        for (int s = 0; s < KS; s++) km[s] = ldg((const f16x8 *)(kbc + 2u * (p * DH + 32 * s + 8 * grp)));
    };
    // piece q = lane + 64i: row q / PPR of the step, dimensions 8 (q % PPR) .. +7
    auto load_v = [&](int j) {
#pragma unroll
        for (int i = 0; i < VPL; i++) {
            const int q = lane + 64 * i;
            const unsigned p = (unsigned)min(64 * j + 16 * wid + q / PPR, cnt - 1);
            vm[i] = ldg((const f16x8 *)(vbc + 2u * (p * DH + 8 * (q % PPR))));
        }
    };
    // B operand of the scores: lane l feeds column l%16 (head (l%16)/2, high
    // or low part) with dimensions 32s + 8(l/16) .. +7 of k-step s, read
    // straight from the query rows before the first K and V loads are
    // issued (so waiting for them leaves those in flight)
    const int rh = col >> 1;
    const float *qh = a.q + (size_t)n * a.q_stride + (size_t)(kvh * G + (rh < G ? rh : 0)) * DH + 8 * grp;
    float4 qv[KS][2];
#pragma unroll
    for (int s = 0; s < KS; s++) {
        qv[s][0] = ldg((const float4 *)(qh + 32 * s));
        qv[s][1] = ldg((const float4 *)(qh + 32 * s + 4));
    }
    load_k(0);
    load_v(0);
    const float scale = 1.0f / sqrtf((float)DH);
    f16x8 qb[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) {
        const float xs[8] = {qv[s][0].x, qv[s][0].y, qv[s][0].z, qv[s][0].w,
                             qv[s][1].x, qv[s][1].y, qv[s][1].z, qv[s][1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float x = rh < G ? xs[e] : 0.0f;
            const _Float16 hi = (_Float16)x;
            qb[s][e] = part ? (_Float16)((x - (float)hi) * 2048.0f) : hi;
        }
    }
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 oc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) oc[t] = zero4;
    // scores stay as raw dot products t (the scale folds into the
    // exponent): e = 2^(t c - m c) with c = scale log2(e), m in raw units
    constexpr float L2E = 1.44269504088896341f;   // log2(e)
    const float c2 = scale * L2E, lazy = ATT_LAZY_T / scale;
    float m = -INFINITY, lsum = 0.0f;   // head rh of this lane's column
    float mk = INFINITY;                // -m c
    _Float16 *vme = vsw[wid];

    for (int j = 0; j < nst; j++) {
        const int pb = 64 * j + 16 * wid;   // the wave's first position of the step
        f32x4 sc = zero4;
#pragma unroll
        for (int s = 0; s < KS; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(km[s], qb[s], sc, 0, 0, 0);
        if (j + 1 < nst) load_k(j + 1);
        // the wave's 16 V rows into its LDS rows (8-byte writes)
#pragma unroll
        for (int i = 0; i < VPL; i++) {
            const int q = lane + 64 * i;
            uint64_t *w = (uint64_t *)(vme + (q / PPR) * RS + 8 * (q % PPR));
            const u32x4 u = __builtin_bit_cast(u32x4, vm[i]);
            w[0] = (uint64_t)u[0] | ((uint64_t)u[1] << 32);
            w[1] = (uint64_t)u[2] | ((uint64_t)u[3] << 32);
        }
        if (j + 1 < nst) load_v(j + 1);
        if (pb >= cnt) continue;   // every row of the wave past the piece (uniform)
        // raw scores of positions pb + 4 grp + i: the high and low parts
        // meet across the lane pair (l, l ^ 1); hi + lo / 2048 in one FMA
        // (the product is exact)
        float sv[4];
        bool up = false;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float other = __int_as_float(
                __builtin_amdgcn_mov_dpp(__float_as_int(sc[i]), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
            const float hi = part ? other : sc[i], lo = part ? sc[i] : other;
            sv[i] = pb + 4 * grp + i < cnt ? fmaf(lo, 1.0f / 2048.0f, hi) : -INFINITY;
            up |= sv[i] > m + lazy;
        }
        if (__ballot(up)) {
            // new reference maxima: the column's maximum over the 16 positions
            float cm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
            cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
            const float mn = fmaxf(m, cm);
            const float mkn = -mn * c2;
            const float al = mn == m ? 1.0f : __builtin_amdgcn_exp2f(mkn - mk);
            m = mn;
            mk = mkn;
            lsum *= al;
            // the output rows of this lane: heads 2 grp and 2 grp + 1, whose
            // factors sit in the lanes of columns 4 grp and 4 grp + 2
            const float a0 = __shfl(al, 4 * grp, 64), a1 = __shfl(al, 4 * grp + 2, 64);
#pragma unroll
            for (int t = 0; t < DT; t++) {
                oc[t][0] *= a0;
                oc[t][1] *= a0;
                oc[t][2] *= a1;
                oc[t][3] *= a1;
            }
        }
        f16x4 pa;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float e = __builtin_amdgcn_exp2f(fmaf(sv[i], c2, mk));
            lsum += e;
            const _Float16 ehi = (_Float16)e;
            pa[i] = part ? (_Float16)((e - (float)ehi) * 2048.0f) : ehi;
        }
        if (rh >= G) pa = f16x4{};
#pragma unroll
        for (int t = 0; t < DT; t++) {
            // B column: dimension 16t + col of positions 4 grp .. +3: within
            // each 16-lane group, lane c reads dimensions 4(c%4) .. +3 of row
            // 4 grp + c/4, and the read hands lane 4r+c element c of lanes 4e+r
            const _Float16 *src = vme + (4 * grp + (col >> 2)) * RS + 16 * t + 4 * (col & 3);
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const s16x4 v4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)src);
            oc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, v4), oc[t], 0, 0, 0);
        }
    }

    // the waves meet: lane sums over the four row groups, then per head
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    __syncthreads();   // every wave done with its V rows: the area takes the outputs
    if (grp == 0 && !part && rh < G) {
        xm[wid][rh] = m * scale;   // natural units, as the partials carry it
        xl[wid][rh] = lsum;
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int h = 2 * grp + k;
        if (h >= G) continue;
#pragma unroll
        for (int t = 0; t < DT; t++)
            xo[((size_t)wid * ATT_MAX_G + h) * DH + 16 * t + col] = oc[t][2 * k] + oc[t][2 * k + 1] * (1.0f / 2048.0f);
    }
    __syncthreads();
    for (int i = tid; i < G * DH; i += NT) {
        const int h = i / DH, d = i % DH;
        float mx = xm[0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) mx = fmaxf(mx, xm[w][h]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = xm[w][h] > -INFINITY ? expf(xm[w][h] - mx) : 0.0f;
            lt += xl[w][h] * f;
            ot += xo[((size_t)w * ATT_MAX_G + h) * DH + d] * f;
        }
        if (single) {
            const float fv = ot / lt;
            const int kk = (kvh * G + h) * DH + d;
            if (a.out) M::st(a.out + (size_t)n * a.out_stride + kk, fv);
            if (a.next.q) act_put<M>(a.next, n, kk, fv);
        } else {
            M::st(a.po + (sbase + h) * DH + d, ot);
            if (d == 0) {
                M::st(a.pm + sbase + h, mx);
                M::st(a.pl + sbase + h, lt);
            }
        }
    }
    __syncthreads();   // the LDS areas may be reused by the caller
}

// One split of attn_split's grid: positions sp*split .. of vector n; a
// session that fits one split is finished here.
template <int DH, typename M>
__device__ __forceinline__ void attn_split_mf(const AttnArgs &a, int kvh, int sp, int n)
{
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int t0 = sp * a.split;
    if (t0 >= L) return;
    const int G = a.n_heads / a.n_kv;
    attn_piece_mf<DH, M>(a, kvh, n, t0, min(L, t0 + a.split) - t0, L <= a.split,
                         (((size_t)n * a.n_kv + kvh) * a.max_splits + sp) * G);
}

// Balanced split (a.bal = B ranges per kv head).  The vectors' contexts are
// laid end to end on one line, each preceded by ATT_BAL_PAD positions that
// stand for the fixed cost of starting a piece (query load, pipeline fill);
// range w of a kv head is the line's [wR, wR + R) with
// R = max(split, ceil(line / B)), so the ranges hold about the same number
// of cached rows whatever the mix of lengths.  The cut of vector n's
// positions that falls in range w is a piece; pieces are in line order, so
// slot w + n is unique to it, and vector n's pieces are the consecutive
// slots w0 + n .. w1 + n.  Work-group k of a kv head (k < B + n_vectors)
// runs the piece of slot k, if any, with attn_piece_mfw: the whole context
// is finished here, a cut one written as the partial [kvh][k][G] that
// k_attn_merge combines.
// Unlike the split grid, no work-group starts only to find its split past
// the context, and a long context leaves no tail of its own splits.
#define ATT_BAL_PAD 64
__device__ inline int wave_sum_i(int v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline int wave_scan_i(int v)   // inclusive prefix sum over the lanes
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}
__device__ __forceinline__ int attn_len(const AttnArgs &a, int i)
{
    return i < a.n ? min(a.seqlen[i * a.seqlen_stride], a.max_ctx) : 0;
}
// Line length and range length of the balanced walk; every wave computes
// them (no barrier), the attention and merge kernels alike.  l0: this
// lane's context in the first 64 vectors.
__device__ __forceinline__ int attn_bal_range(const AttnArgs &a, int l0)
{
    const int lane = threadIdx.x & 63;
    int t = lane < a.n ? l0 + ATT_BAL_PAD : 0;
    for (int b = 64; b < a.n; b += 64) t += b + lane < a.n ? attn_len(a, b + lane) + ATT_BAL_PAD : 0;
    const int line = wave_sum_i(t);
    return max(a.split, (line + a.bal - 1) / a.bal);
}

template <int DH, typename M>
__device__ __forceinline__ void attn_bal_mf(const AttnArgs &a, int kvh, int k)
{
    const int lane = threadIdx.x & 63;
    const int G = a.n_heads / a.n_kv;
    const int l0 = attn_len(a, lane);
    const int R = attn_bal_range(a, l0);
    // the piece (w, s) with w + s = k: vector s's pieces are w0 .. w1
    // (wave scans over blocks of 64 vectors; at most one lane matches).
    // Each lane also loads its vector's cache slot beside its length, so
    // the piece's K/V addresses wait for no further load.
    int base = 0, s = -1, pj = 0, lj = 0, sj = 0;
    for (int b = 0; b < a.n; b += 64) {
        const int L = b == 0 ? l0 : attn_len(a, b + lane);
        const int slot = a.kv.slot_ids && b + lane < a.n ? a.kv.slot_ids[b + lane] : 0;
        const int v = b + lane < a.n ? L + ATT_BAL_PAD : 0;
        const int inc = wave_scan_i(v);
        const int p0 = base + inc - v + ATT_BAL_PAD;   // line offset of the vector's position 0
        const int w = k - (b + lane);
        const uint64_t m = __ballot(b + lane < a.n && L > 0 && w >= p0 / R && w <= (p0 + L - 1) / R);
        if (m) {
            const int j = __builtin_ctzll(m);
            s = b + j;
            pj = __builtin_amdgcn_readlane(p0, j);
            lj = __builtin_amdgcn_readlane(L, j);
            sj = __builtin_amdgcn_readlane(slot, j);
            break;
        }
        base += __builtin_amdgcn_readlane(inc, 63);
    }
    if (s < 0) return;   // no piece in this slot
    const int w = k - s;
    const int r0 = max(w * R - pj, 0), r1 = min((w + 1) * R - pj, lj);
    const size_t kvo = (a.kv.slot_ids ? (size_t)sj * a.kv.slot_stride : 0) + a.kv.layer_off;
    attn_piece_mfw<DH, M>(a, kvh, s, r0, r1 - r0, r0 == 0 && r1 == lj, ((size_t)kvh * (a.bal + a.n) + k) * G, kvo);
}

// Merge of the splits of one (query head, vector) by NT threads:
// mx = max_s m_s, L = sum_s l_s e^(m_s - mx), out = sum_s o_s e^(m_s - mx) / L.
// Thread (d, sg) sums the splits s = sg (mod SG) for dim d; the SG partial
// sums meet in LDS in a fixed order.  Every load of the first NT splits'
// (m, l) and of the thread's first MP o values is issued at once (one round
// trip); longer merges read the rest in loops.  Sessions whose length fits
// one split were finished by attn_split.
// The merge proper, for nact > 1 partials at hb + s * G.
template <int DH, int NT, typename M>
__device__ __forceinline__ void attn_merge_run(const AttnArgs &a, int hq, int n, int nact, size_t hb)
{
    constexpr int SG = NT / DH;
    constexpr int MP = 24;   // o values per thread loaded with the (m, l) (48 splits at d_head 128)
    const int tid = threadIdx.x;
    const int G = a.n_heads / a.n_kv;
    __shared__ float wsh[ATT_MAX_MERGE];
    __shared__ float rsh[NT / 64];
    __shared__ float part[SG][DH];
    const int w = tid >> 6, lane = tid & 63;
    const int d = tid % DH, sg = tid / DH;
    const float m0 = tid < nact ? a.pm[hb + (size_t)tid * G] : -INFINITY;
    const float l0 = tid < nact ? a.pl[hb + (size_t)tid * G] : 0.0f;
    float ov[MP];
#pragma unroll
    for (int i = 0; i < MP; i++) {
        const int s = sg + i * SG;
        ov[i] = s < nact ? a.po[(hb + (size_t)s * G) * DH + d] : 0.0f;
    }
    float mx = m0;
    for (int s = tid + NT; s < nact; s += NT) mx = fmaxf(mx, a.pm[hb + (size_t)s * G]);
    mx = wave_max(mx);
    if (lane == 0) rsh[w] = mx;
    __syncthreads();
    mx = rsh[0];
    for (int i = 1; i < NT / 64; i++) mx = fmaxf(mx, rsh[i]);
    float Ls = 0.0f;
    if (tid < nact) {
        const float e = expf(m0 - mx);
        wsh[tid] = e;
        Ls += l0 * e;
    }
    for (int s = tid + NT; s < nact; s += NT) {
        const float e = expf(a.pm[hb + (size_t)s * G] - mx);
        wsh[s] = e;
        Ls += a.pl[hb + (size_t)s * G] * e;
    }
    Ls = wave_sum(Ls);
    __syncthreads();   // everyone has read rsh (max)
    if (lane == 0) rsh[w] = Ls;
    __syncthreads();
    float Lt = 0.0f;
    for (int i = 0; i < NT / 64; i++) Lt += rsh[i];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < MP; i++)
        if (sg + i * SG < nact) acc += ov[i] * wsh[sg + i * SG];
#pragma unroll 8
    for (int s = sg + MP * SG; s < nact; s += SG) acc += a.po[(hb + (size_t)s * G) * DH + d] * wsh[s];
    part[sg][d] = acc;
    __syncthreads();
    if (tid < DH) {
        float o = 0.0f;
        for (int g = 0; g < SG; g++) o += part[g][tid];
        o /= Lt;
        const int k = hq * DH + tid;
        if (a.out) M::st(a.out + (size_t)n * a.out_stride + k, o);
        if (a.next.q) act_put<M>(a.next, n, k, o);
    }
    __syncthreads();   // the LDS areas may be reused by the caller
}

template <int DH, int NT, typename M>
__device__ __forceinline__ void attn_merge_head(const AttnArgs &a, int hq, int n)
{
    // the launch arguments the partial loads need, in the same batch as
    // the length's (not in a second round trip after it)
    sgpr_pin(a.seqlen);
    sgpr_pin(a.seqlen_stride);
    sgpr_pin(a.max_ctx);
    sgpr_pin(a.split);
    sgpr_pin(a.n_heads);
    sgpr_pin(a.n_kv);
    sgpr_pin(a.max_splits);
    sgpr_pin(a.pm);
    sgpr_pin(a.pl);
    sgpr_pin(a.po);
    const int G = a.n_heads / a.n_kv, kvh = hq / G, h = hq % G;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int nact = (L + a.split - 1) / a.split;
    if (nact <= 1) return;
    attn_merge_run<DH, NT, M>(a, hq, n, nact, (((size_t)n * a.n_kv + kvh) * a.max_splits) * G + h);
}

// The pieces w0 .. w1 of vector n in the balanced split, at slots
// w0 + n .. w1 + n of its kv head.
template <int DH, int NT, typename M>
__device__ __forceinline__ void attn_merge_bal(const AttnArgs &a, int hq, int n)
{
    const int G = a.n_heads / a.n_kv, kvh = hq / G, h = hq % G;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int lane = threadIdx.x & 63;
    const int l0 = attn_len(a, lane);
    const int R = attn_bal_range(a, l0);
    int pre = 0;   // line offset of vector n
    for (int b = 0; b < n; b += 64) {
        const int i = b + lane;
        pre += i < n ? (b == 0 ? l0 : attn_len(a, i)) + ATT_BAL_PAD : 0;
    }
    const int p0 = wave_sum_i(pre) + ATT_BAL_PAD;
    const int w0 = p0 / R;
    const int nact = L > 0 ? (p0 + L - 1) / R - w0 + 1 : 0;
    if (nact <= 1) return;
    attn_merge_run<DH, NT, M>(a, hq, n, nact, ((size_t)kvh * (a.bal + a.n) + w0 + n) * G + h);
}

