// attn.hip — the decode attention kernels over the work-group functions of
// attn_impl.h: one work-group of ATT_THREADS per (kv head, split, vector),
// then one per (query head, vector) to merge the splits.
#include "attn_impl.h"

#define ATT_THREADS 256
// Positions per chunk of a 256-thread work-group (a split is a multiple).
#define ATT_CHUNK (ATT_THREADS / 4)

template <int DH, typename KT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a)
{
    if constexpr (sizeof(KT) == 2 && DH >= 64 && ATT_THREADS == 256)
        attn_split_mf<DH, StPlain>(a, blockIdx.x, blockIdx.y, blockIdx.z);
    else
        attn_split<DH, KT, ATT_THREADS, StPlain>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_merge(AttnArgs a)
{
    attn_merge_head<DH, ATT_THREADS, StPlain>(a, blockIdx.x, blockIdx.y);
}

// Head-per-wave decode attention for d_head 64 and 128: one work-group of
// four waves per (kv head, split, vector); wave w serves query heads w and
// w + 4 of the group.  The split is walked in chunks of CH (32 or 64) positions whose
// K and V rows are staged in LDS by all 256 threads (coalesced 16-byte
// loads of the next chunk are in flight while the current one is used):
//   * scores: four lanes per position, each holding a quarter of the head's
//     query in registers (interleaved 16-byte pieces) against the same pieces
//     of the K row; K rows are padded to an odd multiple of 64 bytes so the
//     four rows a 16-lane pass reads fall in alternate LDS bank halves;
//   * online softmax over the 64 scores with wave reductions;
//   * weighted sum with lanes over the dimensions: each position's weight is
//     broadcast with readlane and its V row read once per wave.
// With NWV = 8 waves and at most four query heads per kv head, two waves
// serve each head, each on one half of every chunk's positions (their
// online softmaxes meet at the end of the split), so each wave's dependent
// chains are half as long and two waves share a SIMD; with more heads wave
// w serves head w alone.
// Same partial format as attn_split, merged by k_attn_merge.
#define ATH_CH 64
template <int DH, typename KT, int CH, int NWV>
__global__ __launch_bounds__(NWV * 64) void k_attn_h(AttnArgs a)
{
#pragma clang fp contract(off)
    constexpr int RB = DH * (int)sizeof(KT);        // row bytes
    constexpr int KS = RB + 64;                      // padded K row stride (bytes)
    constexpr int PE = 16 / (int)sizeof(KT);         // elements per 16-byte piece
    constexpr int NPL = RB / 16 / 4;                 // pieces per lane (a quarter of the row)
    constexpr int DL = DH / 64;                      // output dims per lane
    constexpr int NT = NWV * 64;
    constexpr int UNITS = CH * RB / 16;              // 16-byte units of a chunk's K (and of V)
    constexpr int UPT = UNITS / NT;                  // per thread
    constexpr int PS = CH / 16;                      // 16-position passes per chunk
    static_assert(UNITS % NT == 0 && CH % 16 == 0, "chunk size");
    static_assert(NWV == 4 || (NWV == 8 && PS % 2 == 0), "waves");
    __shared__ __attribute__((aligned(16))) uint8_t ks[2][CH * KS];
    __shared__ __attribute__((aligned(16))) uint8_t vs[2][CH * RB];
    __shared__ float xm[4], xl[4], xo[4][DH];        // NWV = 8: the second halves' results

    const int kvh = blockIdx.x, sp = blockIdx.y, n = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the prologue's launch arguments in one batch of loads, then the
    // vector's length and cache slot together (the slot read from a valid
    // address either way): two round trips before the K/V loads, not four
    sgpr_pin(a.seqlen);
    sgpr_pin(a.seqlen_stride);
    sgpr_pin(a.max_ctx);
    sgpr_pin(a.split);
    sgpr_pin(a.kv.k_base);
    sgpr_pin(a.kv.v_base);
    sgpr_pin(a.kv.slot_ids);
    sgpr_pin(a.kv.slot_stride);
    sgpr_pin(a.kv.layer_off);
    sgpr_pin(a.q);
    sgpr_pin(a.q_stride);
    const int32_t *lenp = a.seqlen + (size_t)n * a.seqlen_stride;
    const int32_t *slotp = a.kv.slot_ids ? a.kv.slot_ids + n : lenp;
    const int len = *lenp, slot = *slotp;
    sgpr_pin(len);
    sgpr_pin(slot);
    const int G = a.n_heads / a.n_kv;
    const int L = min(len, a.max_ctx);
    const int t0 = sp * a.split;
    if (t0 >= L) return;
    const int cnt = min(L, t0 + a.split) - t0;
    const int nch = (cnt + CH - 1) / CH;
    const int nact = (L + a.split - 1) / a.split;
    const size_t kvo = (a.kv.slot_ids ? (size_t)slot * a.kv.slot_stride : 0) + a.kv.layer_off;
    const size_t off = kvo + (size_t)kvh * a.max_ctx * DH + (size_t)t0 * DH;
    const uint8_t *kb = (const uint8_t *)((const KT *)a.kv.k_base + off);
    const uint8_t *vb = (const uint8_t *)((const KT *)a.kv.v_base + off);

    // staging: thread tid moves units tid + NT u of K and V (rows past the
    // split re-read its last row; their weights are zero)
    u32x4 kr[UPT], vr[UPT];
    auto fetch = [&](int c) {
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const int unit = tid + NT * u, row = unit / (RB / 16), col = unit % (RB / 16);
            const size_t src = (size_t)min(c * CH + row, cnt - 1) * RB + col * 16;
            kr[u] = ldg((const u32x4 *)(kb + src));
            vr[u] = ldg((const u32x4 *)(vb + src));
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const int unit = tid + NT * u, row = unit / (RB / 16), col = unit % (RB / 16);
            *(u32x4 *)&ks[buf][row * KS + col * 16] = kr[u];
            *(u32x4 *)&vs[buf][row * RB + col * 16] = vr[u];
        }
    };

    // queries of this wave's heads: lane quarter j holds pieces j, j+4, ...
    // (NWV = 8: head hw, passes ps0 .. ps0 + PSW - 1 of each chunk)
    const int j = lane & 3;
    constexpr bool PAIRS = NWV == 8;
    constexpr int PSW = PAIRS ? PS / 2 : PS;
    const int hw = PAIRS ? (wid & 3) : wid, half = PAIRS ? (wid >> 2) : 0;
    const int ps0 = half * PSW;
    const int nh = PAIRS ? (hw < G ? 1 : 0) : (wid < G ? (wid + 4 < G ? 2 : 1) : 0);
    float q[2][NPL * PE];
    float m[2], l[2], o[2][DL];
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < DL; d++) o[hh][d] = 0.0f;
        const int g = min(PAIRS ? hw : wid + 4 * hh, G - 1);
        const float *qh = a.q + (size_t)n * a.q_stride + (size_t)(kvh * G + g) * DH;
#pragma unroll
        for (int i = 0; i < NPL; i++)
#pragma unroll
            for (int e = 0; e < PE; e++) q[hh][i * PE + e] = ldg(qh + (j + 4 * i) * PE + e);
    }
    // scores and m stay raw dot products; a weight is 2^((t - m) c) with
    // c = log2(e)/sqrt(d_head) on the hardware exponential (exp2(-inf) = 0)
    const float scale = 1.0f / sqrtf((float)DH), c2 = scale * 1.44269504088896341f;

    fetch(0);
    put(0);
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        if (c + 1 < nch) fetch(c + 1);
        const int np = min(CH, cnt - c * CH);
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            if (hh >= nh) break;
            // scores: pass ps covers positions 16 ps + lane/4
            float sc[PSW];
#pragma unroll
            for (int pw = 0; pw < PSW; pw++) {
                const int ps = ps0 + pw;
                const uint8_t *kr0 = &ks[buf][(16 * ps + (lane >> 2)) * KS];
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < NPL; i++) {
                    const u32x4 w = *(const u32x4 *)(kr0 + (j + 4 * i) * 16);
                    float kv[PE];
                    if constexpr (sizeof(KT) == 4) {
                        const f32x4 wf = __builtin_bit_cast(f32x4, w);
#pragma unroll
                        for (int e = 0; e < 4; e++) kv[e] = wf[e];
                    } else {
                        const f16x8 h8 = __builtin_bit_cast(f16x8, w);
#pragma unroll
                        for (int e = 0; e < 8; e++) kv[e] = (float)h8[e];
                    }
#pragma unroll
                    for (int e = 0; e < PE; e++) dot = fmaf(q[hh][i * PE + e], kv[e], dot);
                }
                dot += __shfl_xor(dot, 1, 64);
                dot += __shfl_xor(dot, 2, 64);
                sc[pw] = (16 * ps + (lane >> 2)) < np ? dot : -INFINITY;   // raw score
            }
            float mc = sc[0];
#pragma unroll
            for (int pw = 1; pw < PSW; pw++) mc = fmaxf(mc, sc[pw]);
            mc = wave_max(mc);
            const float mn = fmaxf(m[hh], mc);
            // a half-chunk wave may not have met a valid position yet
            // (uniform over the wave)
            if (PAIRS && mn == -INFINITY) continue;
            float ev[PSW], ls = 0.0f;
#pragma unroll
            for (int pw = 0; pw < PSW; pw++) {
                ev[pw] = __builtin_amdgcn_exp2f((sc[pw] - mn) * c2);
                if (j == 0) ls += ev[pw];
            }
            ls = wave_sum(ls);
            const float al = __builtin_amdgcn_exp2f((m[hh] - mn) * c2);
            l[hh] = l[hh] * al + ls;
            m[hh] = mn;
#pragma unroll
            for (int d = 0; d < DL; d++) o[hh][d] *= al;
            // weighted sum: lane covers dims DL*lane ..
#pragma unroll
            for (int pw = 0; pw < PSW; pw++) {
                const int ps = ps0 + pw;
#pragma unroll 4
                for (int r = 0; r < 16; r++) {
                    const float ep = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev[pw]), 4 * r));
                    const uint8_t *vrow = &vs[buf][(16 * ps + r) * RB];
                    if constexpr (sizeof(KT) == 4) {
                        if constexpr (DL == 2) {
                            const float2 v = *(const float2 *)(vrow + lane * 8);
                            o[hh][0] = fmaf(ep, v.x, o[hh][0]);
                            o[hh][1] = fmaf(ep, v.y, o[hh][1]);
                        } else {
                            o[hh][0] = fmaf(ep, *(const float *)(vrow + lane * 4), o[hh][0]);
                        }
                    } else {
                        if constexpr (DL == 2) {
                            const f16x2 v = *(const f16x2 *)(vrow + lane * 4);
                            o[hh][0] = fmaf(ep, (float)v[0], o[hh][0]);
                            o[hh][1] = fmaf(ep, (float)v[1], o[hh][1]);
                        } else {
                            o[hh][0] = fmaf(ep, (float)*(const _Float16 *)(vrow + lane * 2), o[hh][0]);
                        }
                    }
                }
            }
        }
        if (c + 1 < nch) {
            __syncthreads();   // every wave is done with the other buffer
            put(buf ^ 1);
            __syncthreads();
        }
    }

    // NWV = 8: the second halves hand their (m, l, o) to the first, which
    // combine them with the log-sum-exp rule
    if constexpr (PAIRS) {
        if (half == 1 && nh) {
#pragma unroll
            for (int d = 0; d < DL; d++) xo[hw][DL * lane + d] = o[0][d];
            if (lane == 0) {
                xm[hw] = m[0];
                xl[hw] = l[0];
            }
        }
        __syncthreads();
        if (half == 1) return;
        if (nh) {
            const float m1 = xm[hw], M = fmaxf(m[0], m1);
            const float a0 = m[0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m[0] - M) * c2);
            const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m1 - M) * c2);
            l[0] = l[0] * a0 + xl[hw] * a1;
            m[0] = M;
#pragma unroll
            for (int d = 0; d < DL; d++) o[0][d] = o[0][d] * a0 + xo[hw][DL * lane + d] * a1;
        }
    }
    // partials (or the finished output when the session fits one split)
    const bool single = nact == 1;
    const size_t sbase = (((size_t)n * a.n_kv + kvh) * a.max_splits + sp) * G;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        if (hh >= nh) break;
        const int g = PAIRS ? hw : wid + 4 * hh;
#pragma unroll
        for (int d = 0; d < DL; d++) {
            const int dim = DL * lane + d;
            if (single) {
                const float ov = o[hh][d] / l[hh];
                const int k = (kvh * G + g) * DH + dim;
                if (a.out) a.out[(size_t)n * a.out_stride + k] = ov;
                if (a.next.q) act_put(a.next, n, k, ov);
            } else {
                a.po[(sbase + g) * DH + dim] = o[hh][d];
            }
        }
        if (!single && lane == 0) {
            a.pm[sbase + g] = m[hh] * scale;   // natural units, as the merge reads them
            a.pl[sbase + g] = l[hh];
        }
    }
}

// One wave per (head of q|k|v, vector): lane l holds dims DL*l .. DL*l+DL-1
// (DL = d_head/64; d_head 16/32 use the first d_head lanes).  q and k heads:
// RMSNorm s = 1/sqrtf(sum x^2 / d_head + eps), y = w * (x * s) (the
// reference's cmol_rms_norm order, wave-order sum), then RoPE on the pairs
// (2i, 2i+1) with the QKV epilogue's arithmetic; then q -> a.q, k and v ->
// the cache at the vector's position.
template <int DL>
__global__ __launch_bounds__(64) void k_qk_rope(QkArgs a)
{
#pragma clang fp contract(off)
    const int hh = blockIdx.x, v = blockIdx.y, lane = threadIdx.x;
    const int dh = a.d_head;
    const bool isq = hh < a.n_heads, isk = !isq && hh < a.n_heads + a.n_kv;
    const int row0 = hh * dh;   // q rows, then k rows, then v rows
    const bool act = lane * DL < dh;
    const float *src = a.raw + (size_t)v * a.raw_stride + row0;
    float x[DL];
#pragma unroll
    for (int j = 0; j < DL; j++) x[j] = act ? src[lane * DL + j] : 0.0f;
    const float *w = isq ? a.qn_w : isk ? a.kn_w : nullptr;
    if (w) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < DL; j++) ss += x[j] * x[j];
        ss = wave_sum(ss);
        const float sc = 1.0f / sqrtf(ss / (float)dh + a.eps);
#pragma unroll
        for (int j = 0; j < DL; j++) x[j] = act ? w[lane * DL + j] * (x[j] * sc) : 0.0f;
    }
    const int pos = min(max(a.pos[(size_t)v * a.pos_stride], 0), a.max_ctx - 1);
    if ((isq || isk) && a.rope_on) {
        float partner[DL];
        if constexpr (DL >= 2) {
#pragma unroll
            for (int j = 0; j < DL; j++) partner[j] = x[j ^ 1];
        } else {
            partner[0] = __shfl_xor(x[0], 1, 64);
        }
        float y[DL];
#pragma unroll
        for (int j = 0; j < DL; j++) {
            const int i = lane * DL + j;
            const float *cs = a.rope + ((size_t)pos * (dh / 2) + (i >> 1)) * 2;
            const float c = act ? cs[0] : 1.0f, sn = act ? cs[1] : 0.0f;
            y[j] = !(i & 1) ? x[j] * c - partner[j] * sn : partner[j] * sn + x[j] * c;
        }
#pragma unroll
        for (int j = 0; j < DL; j++) x[j] = y[j];
    }
    if (!act) return;
    if (isq) {
#pragma unroll
        for (int j = 0; j < DL; j++) a.q[(size_t)v * a.q_stride + row0 + lane * DL + j] = x[j];
        return;
    }
    const int kvh = isk ? hh - a.n_heads : hh - a.n_heads - a.n_kv;
    const size_t o = kv_offset(a.kv, v) + ((size_t)kvh * a.max_ctx + pos) * dh + lane * DL;
    void *base = isk ? a.kv.k_base : a.kv.v_base;
#pragma unroll
    for (int j = 0; j < DL; j++) {
        if (a.kv_f16) ((_Float16 *)base)[o + j] = (_Float16)x[j];
        else ((float *)base)[o + j] = x[j];
    }
}

int launch_qk_rope(const QkArgs &a, hipStream_t s)
{
    if (a.n < 1 || a.d_head < 16 || a.d_head > 256 || (a.d_head & (a.d_head - 1))) return -4;
    const dim3 grid(a.n_heads + 2 * a.n_kv, a.n), block(64);
    switch (a.d_head) {
    case 256: hipLaunchKernelGGL(k_qk_rope<4>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(k_qk_rope<2>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(k_qk_rope<1>, grid, block, 0, s, a); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Prompt-pass attention over an fp32 cache, flash style on MFMA.
//
// k_kv_hilo first rewrites positions 0 .. last-1 of the session's layer cache
// as exact f16 high and low parts (x = hi + lo / 2048) in the order the MFMA
// operands are read: per (kv head, 32-position tile) one block of KVT_HALVES
// halves,
//   K: for column tile c (positions 16c..16c+15) and k-step s (dimensions
//      32s..32s+31), a high and a low 1 KiB piece whose lane (col, g) holds
//      dimensions 32s + 8g .. +7 of position 16c + col;
//   V: for dimension tile t, a high and a low piece whose lane (col, g) holds
//      dimension 16t + col of positions 4g .. 4g+3 and 16+4g .. 16+4g+3 (the
//      positions whose scores that lane holds after the score products).
// Positions past `last` repeat position last-1, so every value is finite.
// Each prompt pass converts its cache prefix once per layer; before, every
// work-group converted each tile it read (the prefix once per 64 query rows).
//
// k_attn_prompt: the n vectors are consecutive prompt tokens of one session
// (vector v at position seqlen[v] - 1).  One work-group of four waves per (kv
// head, block of QT = 64 / G tokens, split of `split` positions): its QT x G
// query rows (row r = token r / G, head r % G) share every K/V tile.  The
// work-group walks its split's positions (up to its last token's) in tiles of
// 32, each copied whole into LDS with direct-to-LDS loads while the previous
// tile is used.  Wave w owns query rows 16w .. 16w+15, lane (col, g) row
// 16w + col:
//   * transposed scores S^T = K Q^T from three 16x16x32 f16 MFMA products per
//     step (hi.hi, lo.hi, hi.lo; the dropped lo.lo term is below 2^-22 of
//     each product), scaled by 1/sqrt(d_head), positions past a row's token
//     masked (causal): lane (col, g) holds positions 16c + 4g + i of its row;
//   * online softmax per row over the row's four lanes (two butterfly steps);
//   * the weights, split into f16 high / low parts in registers, are the B
//     operand of O^T = V^T P^T (same three products), whose k order is the
//     V pieces' position order: no weight goes through LDS.
// A token whose positions fit one split is finished here (out / next);
// otherwise each split leaves (max, sum of exp, unnormalised output) in the
// partial format of attn_split and k_attn_merge combines them.  Every
// product is exact in fp32 and every sum fp32; the error against fp32
// arithmetic is the dropped low-low term.
constexpr int KVT_POS = 32;   // positions per tile

template <int DH>
constexpr int kvt_halves() { return KVT_POS * DH * 4; }   // K and V, high and low

template <int DH>
__global__ __launch_bounds__(256) void k_kv_hilo(AttnArgs a, int last, _Float16 *hl, int tiles)
{
#pragma clang fp contract(off)
    constexpr int KS = DH / 32, DT = DH / 16, TH = kvt_halves<DH>(), KH = TH / 2;
    const int kvh = blockIdx.x, tile = blockIdx.y, tid = threadIdx.x;
    const int p0 = tile * KVT_POS;
    const size_t off = kv_offset(a.kv, 0) + (size_t)kvh * a.max_ctx * DH;
    const float *kb = (const float *)a.kv.k_base + off;
    const float *vb = (const float *)a.kv.v_base + off;
    _Float16 *dst = hl + ((size_t)kvh * tiles + tile) * TH;
    for (int it = tid; it < 2 * KS * 64; it += 256) {
        const int lane = it & 63, cs = it >> 6, c = cs / KS, s = cs - c * KS;
        const int p = min(p0 + 16 * c + (lane & 15), last - 1);
        const float4 *src = (const float4 *)(kb + (size_t)p * DH + 32 * s + 8 * (lane >> 4));
        const float4 x0 = src[0], x1 = src[1];
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        f16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            hi[e] = (_Float16)x[e];
            lo[e] = (_Float16)((x[e] - (float)hi[e]) * 2048.0f);
        }
        *(f16x8 *)&dst[(cs * 2) * 512 + lane * 8] = hi;
        *(f16x8 *)&dst[(cs * 2 + 1) * 512 + lane * 8] = lo;
    }
    for (int it = tid; it < DT * 64; it += 256) {
        const int lane = it & 63, t = it >> 6, g = lane >> 4, col = lane & 15;
        f16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int p = min(p0 + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4), last - 1);
            const float x = vb[(size_t)p * DH + 16 * t + col];
            hi[e] = (_Float16)x;
            lo[e] = (_Float16)((x - (float)hi[e]) * 2048.0f);
        }
        *(f16x8 *)&dst[KH + (t * 2) * 512 + lane * 8] = hi;
        *(f16x8 *)&dst[KH + (t * 2 + 1) * 512 + lane * 8] = lo;
    }
}

template <int DH>
constexpr int attn_prompt_lds() { return 2 * kvt_halves<DH>() * 2; }

template <int DH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_prompt(AttnArgs a, const _Float16 *hl,
                                                                                             int tiles)
{
#pragma clang fp contract(off)
    constexpr int TP = KVT_POS;         // positions per tile
    constexpr int KS = DH / 32;         // MFMA k-steps over the head dimensions
    constexpr int DT = DH / 16;         // 16-dimension output tiles
    constexpr int TH = kvt_halves<DH>(), KH = TH / 2;
    constexpr int PIECES = TH * 2 / 1024 / 4;   // 1 KiB copies per wave and tile
    extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];
    _Float16 *stg = lds_h;                      // 2 x TH

    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, col = lane & 15;
    const int G = a.n_heads / a.n_kv, QT = 64 / G;
    const int kvh = blockIdx.x, vb = blockIdx.y * QT, sp = blockIdx.z;
    const int nt = min(QT, a.n - vb);
    if (nt <= 0) return;
    const int last = min(a.seqlen[(size_t)(vb + nt - 1) * a.seqlen_stride], a.max_ctx);   // positions 0 .. last-1
    const int pa = sp * a.split, pb = min(pa + a.split, last);   // this split's positions
    if (pa >= last) return;
    // scores and m stay raw dot products; a weight is 2^(t c - m c) with
    // c = log2(e)/sqrt(d_head) on the hardware exponential (exp2(-inf) = 0)
    const float scale = 1.0f / sqrtf((float)DH), c2 = scale * 1.44269504088896341f;
    const uint8_t *tsrc = (const uint8_t *)(hl + ((size_t)kvh * tiles + pa / TP) * TH);
    // tile j of the split into stage st: 4 x PIECES pieces of 1 KiB
    auto issue = [&](int st, int j) {
        const uint8_t *src = tsrc + (size_t)j * TH * 2;
        uint8_t *dst = (uint8_t *)(stg + st * TH);
#pragma unroll
        for (int i = 0; i < PIECES; i++) {
            const int pc = wid * PIECES + i;
            __builtin_amdgcn_global_load_lds((const gvoid_t *)(src + pc * 1024 + lane * 16),
                                             (lvoid_t *)(dst + pc * 1024), 16, 0, 0);
        }
    };
    const int ntiles = (pb - pa + TP - 1) / TP;
    issue(0, 0);

    // this lane's query row 16w + col = (token at, head ah); its B operand of
    // the scores: dimensions 32s + 8g .. +7 of k-step s, high and low parts
    const int ar = 16 * wid + col, at = ar / G, ah = ar - at * G;
    const bool arow = at < nt;
    f16x8 qh[KS], ql[KS];
    {
        const float *qp = a.q + (size_t)(vb + (arow ? at : 0)) * a.q_stride + (size_t)(kvh * G + ah) * DH;
#pragma unroll
        for (int s = 0; s < KS; s++) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = arow ? qp[32 * s + 8 * g + e] : 0.0f;
                const _Float16 hi = (_Float16)x;
                qh[s][e] = hi;
                ql[s][e] = (_Float16)((x - (float)hi) * 2048.0f);
            }
        }
    }
    const int L = arow ? min(a.seqlen[(size_t)(vb + at) * a.seqlen_stride], a.max_ctx) : 0;
    const int nact = (L + a.split - 1) / a.split;
    const int lim = min(L, pb);   // visible positions of this split: pa .. lim-1
    float m = -INFINITY, lsum = 0.0f;
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 o1[DT], o2[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) {
        o1[t] = zero4;
        o2[t] = zero4;
    }

    for (int j = 0; j < ntiles; j++) {
        const int p0 = pa + j * TP;
        // tile j is in stage j & 1 once this wave's copies have landed and
        // every wave has passed the barrier (which also means every wave is
        // done with tile j - 1, whose stage the copy of tile j + 1 reuses)
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
        __syncthreads();
        if (j + 1 < ntiles) issue((j + 1) & 1, j + 1);
        const _Float16 *ks_ = stg + (j & 1) * TH, *vs_ = ks_ + KH;
        // ---- transposed scores: sc[c][i] = position 16c + 4g + i ----
        float sc[2][4];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            f32x4 s1 = zero4, s2 = zero4;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const f16x8 kh = *(const f16x8 *)&ks_[((c * KS + s) * 2) * 512 + lane * 8];
                const f16x8 kl = *(const f16x8 *)&ks_[((c * KS + s) * 2 + 1) * 512 + lane * 8];
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[s], s1, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[s], s2, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[s], s2, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int pos = p0 + 16 * c + 4 * g + i;
                sc[c][i] = pos < lim ? fmaf(s2[i], 1.0f / 2048.0f, s1[i]) : -INFINITY;   // raw score
            }
        }
        // ---- online softmax of the row: its 32 scores are in lanes col,
        // col + 16, col + 32, col + 48 ----
        float mx = sc[0][0];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) mx = fmaxf(mx, sc[c][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(m, mx);
        // a row with no visible position yet keeps m = -inf: weights 0
        const float mref = mn == -INFINITY ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f((m - mref) * c2);
        const float mk = -mref * c2;
        float ps = 0.0f;
        f16x8 ph, pl;
#pragma unroll
        for (int c = 0; c < 2; c++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = __builtin_amdgcn_exp2f(fmaf(sc[c][i], c2, mk));
                ps += e;
                const _Float16 eh = (_Float16)e;
                ph[4 * c + i] = eh;
                pl[4 * c + i] = (_Float16)((e - (float)eh) * 2048.0f);
            }
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        lsum = lsum * alpha + ps;
        m = mn;
        // ---- O^T = alpha O^T + V^T P^T ----
#pragma unroll
        for (int t = 0; t < DT; t++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                o1[t][i] *= alpha;
                o2[t][i] *= alpha;
            }
        }
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const f16x8 vh = *(const f16x8 *)&vs_[(t * 2) * 512 + lane * 8];
            const f16x8 vl = *(const f16x8 *)&vs_[(t * 2 + 1) * 512 + lane * 8];
            o1[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, o1[t], 0, 0, 0);
            o2[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, o2[t], 0, 0, 0);
            o2[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, o2[t], 0, 0, 0);
        }
    }

    // ---- outputs: lane (col, g) holds dimensions 16t + 4g + i of its row ----
    if (!arow || sp >= nact) return;   // no positions of this token here
    const int v = vb + at;
    if (nact == 1) {
        const float inv = 1.0f / lsum;
#pragma unroll
        for (int t = 0; t < DT; t++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ov = (o1[t][i] + o2[t][i] * (1.0f / 2048.0f)) * inv;
                const int k = (kvh * G + ah) * DH + 16 * t + 4 * g + i;
                if (a.out) a.out[(size_t)v * a.out_stride + k] = ov;
                if (a.next.q) act_put(a.next, v, k, ov);
            }
        }
    } else {
        const size_t sb = (((size_t)v * a.n_kv + kvh) * a.max_splits + sp) * G + ah;
#pragma unroll
        for (int t = 0; t < DT; t++) {
            float4 ov;
            ov.x = o1[t][0] + o2[t][0] * (1.0f / 2048.0f);
            ov.y = o1[t][1] + o2[t][1] * (1.0f / 2048.0f);
            ov.z = o1[t][2] + o2[t][2] * (1.0f / 2048.0f);
            ov.w = o1[t][3] + o2[t][3] * (1.0f / 2048.0f);
            *(float4 *)&a.po[sb * DH + 16 * t + 4 * g] = ov;
        }
        if (g == 0) {
            a.pm[sb] = m * scale;   // natural units, as the merge reads them
            a.pl[sb] = lsum;
        }
    }
}

size_t attn_prompt_kv_bytes(int n_kv, int d_head, int max_ctx)
{
    const size_t tiles = (size_t)(max_ctx + KVT_POS - 1) / KVT_POS;
    return (size_t)n_kv * tiles * KVT_POS * d_head * 4 * sizeof(_Float16);
}

static int attn_cus()
{
    static const int c = [] {
        int d = 0, n = 0;
        if (hipGetDevice(&d) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess ||
            n < 1) {
            (void)hipGetLastError();
            n = 256;
        }
        return n;
    }();
    return c;
}

template <int DH>
int launch_attn_prompt_dh(const AttnArgs &a, _Float16 *kv_hl, int last, hipStream_t s)
{
    static const bool lds_ok =
        hipFuncSetAttribute((const void *)k_attn_prompt<DH>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            attn_prompt_lds<DH>()) == hipSuccess;
    if (!lds_ok) return -4;
    const int G = a.n_heads / a.n_kv, QT = 64 / G;
    const int tiles = (a.max_ctx + KVT_POS - 1) / KVT_POS;
    hipLaunchKernelGGL(k_kv_hilo<DH>, dim3(a.n_kv, (last + KVT_POS - 1) / KVT_POS), dim3(256), 0, s, a, last,
                       kv_hl, tiles);
    const dim3 grid(a.n_kv, (a.n + QT - 1) / QT, a.max_splits), block(256), mgrid(a.n_heads, a.n);
    hipLaunchKernelGGL(k_attn_prompt<DH>, grid, block, attn_prompt_lds<DH>(), s, a, kv_hl, tiles);
    if (a.max_splits > 1) {
        static const bool wave = [] {   // CMOL_PROMPT_MERGE=1: the work-group merge (measurements)
            const char *e = getenv("CMOL_PROMPT_MERGE");
            return !(e && e[0] == '1');
        }();
        if (wave) return launch_attn_merge_wave(a, s);
        hipLaunchKernelGGL((k_attn_merge<DH>), mgrid, block, 0, s, a);
    }
    return 0;
}

int launch_attn_prompt(const AttnArgs &a, _Float16 *kv_hl, int last, hipStream_t s)
{
    const int G = a.n_heads / a.n_kv;
    if (a.kv_f16 || G < 1 || G > 8 || a.n_heads % a.n_kv || a.n < 1 || (a.d_head != 64 && a.d_head != 128))
        return -4;
    if (a.split < 64 || a.split % KVT_POS || a.max_splits > ATT_MAX_MERGE) return -4;
    if (!kv_hl || last < 1 || last > a.max_ctx) return -4;
    // the pass's split: the longest multiple of the planned one that still
    // gives every CU two work-groups (a 2048-token pass: one split, no
    // merge; 512-token passes: 256-512 positions).  Fewer splits than
    // planned always fit the partial buffers.
    AttnArgs b = a;
    const long blocks = (long)a.n_kv * ((a.n + 64 / G - 1) / (64 / G));
    while (b.split * 2 <= a.max_ctx && blocks * ((last + 2 * b.split - 1) / (2 * b.split)) >= 2L * attn_cus())
        b.split *= 2;
    b.max_splits = (last + b.split - 1) / b.split;
    const int rc = a.d_head == 128 ? launch_attn_prompt_dh<128>(b, kv_hl, last, s)
                                   : launch_attn_prompt_dh<64>(b, kv_hl, last, s);
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int attn_max_splits(int max_ctx, int split) { return (max_ctx + split - 1) / split; }

int launch_attn(const AttnArgs &a, hipStream_t s)
{
    const int G = a.n_heads / a.n_kv;
    // splits of whole 64-position chunks, or (head-per-wave kernel, d_head
    // 64 / 128) of whole 32-position chunks
    const bool half_chunks = a.split % ATT_CHUNK != 0;
    if (G < 1 || G > ATT_MAX_G || a.n_heads % a.n_kv || a.split < 1 || a.split % (ATT_CHUNK / 2) ||
        (half_chunks && a.d_head != 64 && a.d_head != 128))
        return -4;
    if (a.max_splits > ATT_MAX_MERGE) return -4;
    dim3 grid(a.n_kv, a.max_splits, a.n), block(ATT_THREADS), mgrid(a.n_heads, a.n);
    if (a.bal > 0) return launch_attn_bal(a, s);
#define ATT(DHV)                                                                          \
    if (a.kv_f16) hipLaunchKernelGGL((k_attn<DHV, _Float16>), grid, block, 0, s, a);      \
    else hipLaunchKernelGGL((k_attn<DHV, float>), grid, block, 0, s, a);
#define ATH(DHV)                                                                                      \
    if (half_chunks) {                                                                                \
        if (a.kv_f16) hipLaunchKernelGGL((k_attn_h<DHV, _Float16, 32, 4>), grid, block, 0, s, a);     \
        else hipLaunchKernelGGL((k_attn_h<DHV, float, 32, 4>), grid, block, 0, s, a);                \
    } else if (h8) {                                                                                  \
        if (a.kv_f16) hipLaunchKernelGGL((k_attn_h<DHV, _Float16, ATH_CH, 8>), grid, block8, 0, s, a); \
        else hipLaunchKernelGGL((k_attn_h<DHV, float, ATH_CH, 8>), grid, block8, 0, s, a);           \
    } else {                                                                                          \
        if (a.kv_f16) hipLaunchKernelGGL((k_attn_h<DHV, _Float16, ATH_CH, 4>), grid, block, 0, s, a); \
        else hipLaunchKernelGGL((k_attn_h<DHV, float, ATH_CH, 4>), grid, block, 0, s, a);            \
    }
    // head-per-wave kernel for short splits (one or two chunks); the
    // thread-per-dimension kernel streams long splits better
    const char *e = getenv("CMOL_ATTN_H");
    const bool head_waves = half_chunks || (e ? e[0] == '1' : a.split <= 2 * ATH_CH);
    // eight waves (two per query head) when the kv head has at most four
    // query heads (CMOL_ATTN_H8=0: four waves, measurements)
    static const bool h8_on = [] {
        const char *v = getenv("CMOL_ATTN_H8");
        return !(v && v[0] == '0');
    }();
    const bool h8 = h8_on && G <= 4;
    const dim3 block8(512);
    switch (a.d_head) {
    case 16: ATT(16); break;
    case 32: ATT(32); break;
    case 64: if (head_waves) { ATH(64); } else { ATT(64); } break;
    case 128: if (head_waves) { ATH(128); } else { ATT(128); } break;
    case 256: ATT(256); break;
    default: return -4;
    }
    if (a.max_splits > 1) {
        switch (a.d_head) {
        case 16: hipLaunchKernelGGL((k_attn_merge<16>), mgrid, block, 0, s, a); break;
        case 32: hipLaunchKernelGGL((k_attn_merge<32>), mgrid, block, 0, s, a); break;
        case 64: hipLaunchKernelGGL((k_attn_merge<64>), mgrid, block, 0, s, a); break;
        case 128: hipLaunchKernelGGL((k_attn_merge<128>), mgrid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_attn_merge<256>), mgrid, block, 0, s, a); break;
        }
    }
#undef ATT
#undef ATH
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
