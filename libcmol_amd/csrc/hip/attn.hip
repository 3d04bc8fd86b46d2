// attn.hip — split-K grouped-query decode attention over ragged KV lengths.
//
// Follows the arithmetic of reference src/attn.c:103-137: per query head h
// (kv head h*n_kv/n_heads), scores s_t = (q_h . K_t) / sqrtf(d_head) over
// t < seqlen, softmax, out_h = sum_t p_t V_t.  The positions of one session
// and kv head are cut into splits of `split` positions; one work-group per
// (kv head, split, vector) loads K/V for its split once and serves all G
// query heads of the group.  Each split keeps (max, sum of exp, unnormalised
// output); a second kernel (k_attn_merge) combines the splits with the usual
// log-sum-exp rescaling.  A session whose length fits one split is finished
// directly by k_attn.
#include "common.h"
#include "kernels.h"

#define ATT_THREADS 256
#define ATT_MAX_G 8
#define ATT_MAX_SPLIT 256
#define ATT_MAX_MERGE 1024

template <typename KT> struct KLoad;
template <> struct KLoad<float> {
    static __device__ inline float4 ld4(const float *p) { return *(const float4 *)p; }
};
template <> struct KLoad<_Float16> {
    static __device__ inline float4 ld4(const _Float16 *p)
    {
        f16x4 h = *(const f16x4 *)p;
        return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    }
};

template <int DH, typename KT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a)
{
#pragma clang fp contract(off)
    const int kvh = blockIdx.x, sp = blockIdx.y, n = blockIdx.z;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int G = a.n_heads / a.n_kv;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int C = a.split;
    const int t0 = sp * C;
    if (t0 >= L) return;
    const int cnt = min(L, t0 + C) - t0;
    const int nact = (L + C - 1) / C;

    __shared__ float qsh[ATT_MAX_G][DH];
    __shared__ float sc[ATT_MAX_G][ATT_MAX_SPLIT];
    __shared__ float hm[ATT_MAX_G], hl[ATT_MAX_G];
    __shared__ __attribute__((aligned(16))) float red[ATT_MAX_G * ATT_THREADS * 4];

    const size_t off = kv_offset(a.kv, n) + (size_t)kvh * a.max_ctx * DH;
    const KT *kb = (const KT *)a.kv.k_base + off;
    const KT *vb = (const KT *)a.kv.v_base + off;
    const float *qn = a.q + (size_t)n * a.q_stride + (size_t)kvh * G * DH;
    for (int i = tid; i < G * DH; i += ATT_THREADS) qsh[i / DH][i % DH] = qn[i];
    __syncthreads();

    // scores: 4 lanes per position, lane j takes 4-element chunks j, j+4, ...
    const float scale = 1.0f / sqrtf((float)DH);
    for (int base = 0; base < cnt; base += ATT_THREADS / 4) {
        const int p = base + (tid >> 2), j = tid & 3;
        float dot[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) dot[h] = 0.0f;
        if (p < cnt) {
            const KT *kp = kb + (size_t)(t0 + p) * DH;
#pragma unroll 4
            for (int c = j; c < DH / 4; c += 4) {
                float4 kv = KLoad<KT>::ld4(kp + 4 * c);
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++) {
                    if (h < G) {
                        dot[h] = fmaf(qsh[h][4 * c + 0], kv.x, dot[h]);
                        dot[h] = fmaf(qsh[h][4 * c + 1], kv.y, dot[h]);
                        dot[h] = fmaf(qsh[h][4 * c + 2], kv.z, dot[h]);
                        dot[h] = fmaf(qsh[h][4 * c + 3], kv.w, dot[h]);
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) {
            dot[h] += __shfl_xor(dot[h], 1, 64);
            dot[h] += __shfl_xor(dot[h], 2, 64);
        }
        if (j == 0 && p < cnt)
            for (int h = 0; h < G; h++) sc[h][p] = dot[h] * scale;
    }
    __syncthreads();

    // per-head max and sum of exp over this split
    for (int h = wid; h < G; h += ATT_THREADS / 64) {
        float m = -INFINITY;
        for (int i = lane; i < cnt; i += 64) m = fmaxf(m, sc[h][i]);
        m = wave_max(m);
        float s = 0.0f;
        for (int i = lane; i < cnt; i += 64) {
            float e = expf(sc[h][i] - m);
            sc[h][i] = e;
            s += e;
        }
        s = wave_sum(s);
        if (lane == 0) { hm[h] = m; hl[h] = s; }
    }
    __syncthreads();

    // o[h][d] = sum_p e_p V_p for all G heads at once: DG dim groups of 4 x
    // PG position groups; V of each position is loaded once.
    constexpr int DG = DH / 4, PG = ATT_THREADS / DG;
    const int dg = tid % DG, pg = tid / DG;
    const size_t sbase = (((size_t)n * a.n_kv + kvh) * a.max_splits + sp) * G;
    float4 o[ATT_MAX_G];
#pragma unroll
    for (int h = 0; h < ATT_MAX_G; h++) o[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int p = pg; p < cnt; p += PG) {
        const float4 v = KLoad<KT>::ld4(vb + (size_t)(t0 + p) * DH + 4 * dg);
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) {
            if (h < G) {
                const float e = sc[h][p];
                o[h].x = fmaf(e, v.x, o[h].x);
                o[h].y = fmaf(e, v.y, o[h].y);
                o[h].z = fmaf(e, v.z, o[h].z);
                o[h].w = fmaf(e, v.w, o[h].w);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < ATT_MAX_G; h++) {
        if (h < G) *(float4 *)&red[((size_t)pg * G + h) * DH + 4 * dg] = o[h];
    }
    __syncthreads();
    const bool single = nact == 1;
    for (int i = tid; i < G * DH; i += ATT_THREADS) {
        const int h = i / DH, d = i % DH;
        float s = 0.0f;
        for (int q = 0; q < PG; q++) s += red[((size_t)q * G + h) * DH + d];
        if (single) {
            const float o = s / hl[h];
            const int k = (kvh * G + h) * DH + d;
            if (a.out) a.out[(size_t)n * a.out_stride + k] = o;
            if (a.next.q) act_put(a.next, n, k, o);
        } else {
            a.po[(sbase + h) * DH + d] = s;
        }
    }
    if (single) return;
    if (tid < G) {
        a.pm[sbase + tid] = hm[tid];
        a.pl[sbase + tid] = hl[tid];
    }
}

// Merge of the splits of one (kv head, vector): M = max_s m_s,
// L = sum_s l_s e^(m_s - M), out = sum_s o_s e^(m_s - M) / L.  Sessions whose
// length fits one split were finished by k_attn.
template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_merge(AttnArgs a)
{
    const int kvh = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
    const int G = a.n_heads / a.n_kv;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int nact = (L + a.split - 1) / a.split;
    if (nact <= 1) return;
    __shared__ float wsh[ATT_MAX_G][ATT_MAX_MERGE];
    __shared__ float inv_l[ATT_MAX_G];
    const size_t hb = (((size_t)n * a.n_kv + kvh) * a.max_splits) * G;
    const int w = tid >> 6, lane = tid & 63;
    for (int h = w; h < G; h += ATT_THREADS / 64) {
        float M = -INFINITY;
        for (int s = lane; s < nact; s += 64) M = fmaxf(M, a.pm[hb + (size_t)s * G + h]);
        M = wave_max(M);
        float Ls = 0.0f;
        for (int s = lane; s < nact; s += 64) {
            const float e = expf(a.pm[hb + (size_t)s * G + h] - M);
            wsh[h][s] = e;
            Ls += a.pl[hb + (size_t)s * G + h] * e;
        }
        Ls = wave_sum(Ls);
        if (lane == 0) inv_l[h] = 1.0f / Ls;
    }
    __syncthreads();
    for (int i = tid; i < G * DH; i += ATT_THREADS) {
        const int h = i / DH, d = i % DH;
        float o = 0.0f;
        for (int s = 0; s < nact; s++) o += a.po[(hb + (size_t)s * G + h) * DH + d] * wsh[h][s];
        const int k = (kvh * G + h) * DH + d;
        if (a.out) a.out[(size_t)n * a.out_stride + k] = o * inv_l[h];
        if (a.next.q) act_put(a.next, n, k, o * inv_l[h]);
    }
}

int attn_max_splits(int max_ctx, int split) { return (max_ctx + split - 1) / split; }

int launch_attn(const AttnArgs &a, hipStream_t s)
{
    const int G = a.n_heads / a.n_kv;
    if (G < 1 || G > ATT_MAX_G || a.n_heads % a.n_kv || a.split < 1 || a.split > ATT_MAX_SPLIT)
        return -4;
    if (a.max_splits > ATT_MAX_MERGE) return -4;
    dim3 grid(a.n_kv, a.max_splits, a.n), block(ATT_THREADS), mgrid(a.n_kv, a.n);
#define ATT(DHV)                                                                          \
    if (a.kv_f16) hipLaunchKernelGGL((k_attn<DHV, _Float16>), grid, block, 0, s, a);      \
    else hipLaunchKernelGGL((k_attn<DHV, float>), grid, block, 0, s, a);                  \
    if (a.max_splits > 1) hipLaunchKernelGGL((k_attn_merge<DHV>), mgrid, block, 0, s, a);
    switch (a.d_head) {
    case 16: ATT(16); break;
    case 32: ATT(32); break;
    case 64: ATT(64); break;
    case 128: ATT(128); break;
    case 256: ATT(256); break;
    default: return -4;
    }
#undef ATT
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
