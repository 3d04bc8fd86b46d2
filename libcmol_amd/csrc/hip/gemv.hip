// gemv.hip — quantised decode matvec for gfx950 (one activation vector).
//
// y = W . x for a Q4_0/Q5_0/Q8_0 weight in the quad-tile layout.  One
// work-group owns one 16-row tile; its NW wavefronts split the k range.  Each
// wave streams its quads with one coalesced 16/32-byte load per lane, decodes
// the codes to exact small integers in f16 (common.h), and contracts them
// with v_mfma_f32_16x16x32_f16 against the activation split into an f16 high
// part and an f16 residual (two MFMA rows), so the products are exact and the
// sum is carried in fp32.  The per-block fp16 scale multiplies each block's
// 16x16 result tile.  Partial sums of the waves meet in LDS in a fixed order.
//
// Fused around the product:
//   prologue  RMSNorm of x (reference src/model.c:90-97) and the f16 hi/lo
//             split with a power-of-two range scale, staged once per
//             work-group in LDS in the weight format's k order;
//   epilogues plain store, residual add (src/model.c:232,259), SwiGLU over
//             interleaved gate/up rows (src/model.c:117-123), RoPE on q/k rows
//             and the KV-cache write at pos (src/attn.c:83-101), logits with
//             a first-index argmax (src/sampler.c:199-204).
#include "common.h"
#include "kernels.h"

// The 8 activation values a lane group g needs for block b, in the weight
// format's k order; zero beyond K.
template <int DT>
__device__ inline void load_group(const float *__restrict__ src, int K, int gi, float v[8])
{
    int b = gi >> 2, g = gi & 3;
    if (32 * b >= K) {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = 0.0f;
        return;
    }
    if constexpr (DT == DT_Q8_0) {
        const float4 *p = (const float4 *)(src + 32 * b + 8 * g);
        float4 a = p[0], c = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
        float4 a = *(const float4 *)(src + 32 * b + 4 * g);
        float4 c = *(const float4 *)(src + 32 * b + 16 + 4 * g);
        v[0] = a.x; v[1] = a.z; v[2] = a.y; v[3] = a.w;
        v[4] = c.x; v[5] = c.z; v[6] = c.y; v[7] = c.w;
    }
}

// Block-wide (sum, max, max) of three per-thread values with one exchange.
template <int NW>
__device__ inline void block_reduce3(float &sum, float &mx0, float &mx1, float *stat)
{
    sum = wave_sum(sum);
    mx0 = wave_max(mx0);
    mx1 = wave_max(mx1);
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        stat[wid] = sum;
        stat[NW + wid] = mx0;
        stat[2 * NW + wid] = mx1;
    }
    __syncthreads();
    sum = 0.0f;
    mx0 = 0.0f;
    mx1 = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        sum += stat[w];
        mx0 = fmaxf(mx0, stat[NW + w]);
        mx1 = fmaxf(mx1, stat[2 * NW + w]);
    }
}

// Stage x (optionally RMS-normalised) as f16 hi/lo into LDS:
// xs[(b*4+g)*2 + {0:hi,1:lo}] = 8 halves.  Returns 1/scale.  Pass 1 gathers
// the statistics, pass 2 re-reads x (cache-resident) to keep registers free
// for the weight prefetch that is in flight meanwhile.
template <int DT, int NW>
__device__ float stage_single(const GemvArgs &a, const float *__restrict__ x,
                              uint8_t *xs, float *stat)
{
#pragma clang fp contract(off)
    const int K = a.w.cols;
    const int G = a.w.block_quads * 16;
    const bool norm = a.norm_w != nullptr;
    float ss = 0.0f, mx = 0.0f, wm = 0.0f;
    for (int gi = threadIdx.x; gi < G; gi += NW * 64) {
        float v[8];
        load_group<DT>(x, K, gi, v);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            ss += v[e] * v[e];
            mx = fmaxf(mx, fabsf(v[e]));
        }
        if (norm) {
            float w[8];
            load_group<DT>(a.norm_w, K, gi, w);
#pragma unroll
            for (int e = 0; e < 8; e++) wm = fmaxf(wm, fabsf(w[e]));
        }
    }
    block_reduce3<NW>(ss, mx, wm, stat);
    const float s = norm ? 1.0f / sqrtf(ss / (float)K + a.eps) : 1.0f;
    const float bound = norm ? mx * s * wm : mx;
    float scale = 1.0f, inv = 1.0f;
    if (bound > 0.0f && bound < 3.0e38f) {
        int E;
        frexpf(bound, &E);
        scale = ldexpf(1.0f, 14 - E);
        inv = ldexpf(1.0f, E - 14);
    }
    for (int gi = threadIdx.x; gi < G; gi += NW * 64) {
        float v[8], w[8];
        load_group<DT>(x, K, gi, v);
        if (norm) load_group<DT>(a.norm_w, K, gi, w);
        f16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float xn = norm ? w[e] * (v[e] * s) : v[e];
            const float t = xn * scale;
            const _Float16 h = (_Float16)t;
            hi[e] = h;
            lo[e] = (_Float16)(t - (float)h);
        }
        *(f16x8 *)(xs + ((size_t)gi * 2 + 0) * 16) = hi;
        *(f16x8 *)(xs + ((size_t)gi * 2 + 1) * 16) = lo;
    }
    __syncthreads();
    return inv;
}

__device__ inline void store_kv(void *base, int kv_f16, size_t idx, float v)
{
    if (kv_f16) ((_Float16 *)base)[idx] = (_Float16)v;
    else ((float *)base)[idx] = v;
}

// Runs on wave 0; lane l < 16 holds the final value of row 16t + l.
template <int EPI>
__device__ void epilogue(const GemvArgs &a, int t, int l, float y)
{
#pragma clang fp contract(off)
    const int row = t * 16 + (l & 15);
    const bool act = l < 16 && row < a.w.rows;
    if constexpr (EPI == EPI_STORE) {
        if (act) a.out[row] = y;
    } else if constexpr (EPI == EPI_RESID) {
        if (act) a.out[row] = a.out[row] + y;
    } else if constexpr (EPI == EPI_SWIGLU) {
        float u = __shfl_xor(y, 1, 64);
        if (act && !(row & 1)) a.out[row >> 1] = (y / (1.0f + expf(-y))) * u;
    } else if constexpr (EPI == EPI_QKV) {
        const int pos = min(max(a.pos[0], 0), a.max_ctx - 1);
        float partner = __shfl_xor(y, 1, 64);
        if (act) {
            if (row < a.nq + a.nkv) {
                int rr = row < a.nq ? row : row - a.nq;
                int i = rr % a.d_head;
                float v = y;
                if (a.rope_on) {
                    const float *cs = a.rope + ((size_t)pos * (a.d_head / 2) + (i >> 1)) * 2;
                    float c = cs[0], sn = cs[1];
                    if (!(i & 1)) v = y * c - partner * sn;
                    else v = partner * sn + y * c;
                }
                if (row < a.nq) {
                    a.out[row] = v;
                } else {
                    int h = rr / a.d_head;
                    store_kv(a.kv.k_base, a.kv_f16,
                             kv_offset(a.kv, 0) + ((size_t)h * a.max_ctx + pos) * a.d_head + i, v);
                }
            } else {
                int rr = row - a.nq - a.nkv;
                int h = rr / a.d_head, i = rr % a.d_head;
                store_kv(a.kv.v_base, a.kv_f16,
                         kv_offset(a.kv, 0) + ((size_t)h * a.max_ctx + pos) * a.d_head + i, y);
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        if (act) a.out[row] = y;
        unsigned long long key = act ? argmax_key(y, (uint32_t)row) : 0ull;
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            unsigned long long other = __shfl_xor(key, o, 64);
            key = other > key ? other : key;
        }
        if (l == 0) atomicMax(a.argmax + (t & (ARGMAX_SLOTS - 1)), key);
    }
}

template <int DT, int NW, int EPI>
__global__ __launch_bounds__(NW * 64) void k_gemv1(GemvArgs a)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    constexpr int U = 8;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int BQ = a.w.block_quads;
    const int t = blockIdx.x;
    const int wid = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int qpw = (BQ + NW - 1) / NW;
    const int q0 = min(BQ, wid * qpw), q1 = min(BQ, q0 + qpw);

    uint8_t *xs = smem;
    float *red = (float *)(smem + (size_t)BQ * 512);
    float *stat = red + NW * 32;

    const size_t cell0 = (size_t)t * BQ;
    u32x4 c0[U], c1[U];
    u32x2 dv[U];
    uint32_t hv[U];
    // Weights do not depend on x: issue the first batch before the prologue
    // so its HBM latency overlaps the RMSNorm/staging work.
    auto load_batch = [&](int qb) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t cell = cell0 + (qb + u < q1 ? qb + u : qb);
            const u32x4 *p = (const u32x4 *)(a.w.qs + (cell * 64 + l) * LB);
            c0[u] = p[0];
            if constexpr (LB == 32) c1[u] = p[1];
            else c1[u] = u32x4{0, 0, 0, 0};
            dv[u] = *(const u32x2 *)(a.w.d + cell * 64 + (l & 15) * 4);
            if constexpr (DT == DT_Q5_0) hv[u] = a.w.qh[cell * 64 + l];
            else hv[u] = 0u;
        }
    };
    if (q0 < q1) load_batch(q0);

    const float inv_scale = stage_single<DT, NW>(a, a.x, xs, stat);

    const bool holds_x = (l & 15) < 2;
    const f16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int qb = q0; qb < q1; qb += U) {
        if (qb != q0) load_batch(qb);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (qb + u < q1) {
#pragma unroll
                for (int bi = 0; bi < 4; bi++) {
                    const int b = (qb + u) * 4 + bi;
                    f16x8 wv = deq_block<DT>(c0[u], c1[u], hv[u], bi);
                    f16x8 xv = zero8;
                    if (holds_x) xv = *(const f16x8 *)(xs + (((size_t)b * 4 + (l >> 4)) * 2 + (l & 15)) * 16);
                    f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, zero4, 0, 0, 0);
                    uint32_t dw = dv[u][bi >> 1];
                    uint16_t dh = (uint16_t)((bi & 1) ? (dw >> 16) : (dw & 0xFFFFu));
                    float d = (float)__builtin_bit_cast(_Float16, dh);
                    acc0 = fmaf(d, c[0], acc0);
                    acc1 = fmaf(d, c[1], acc1);
                }
            }
        }
    }
    if (l < 16) {
        red[(wid * 16 + l) * 2 + 0] = acc0;
        red[(wid * 16 + l) * 2 + 1] = acc1;
    }
    __syncthreads();
    if (wid == 0) {
        float hi = 0.0f, lo = 0.0f;
        if (l < 16) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                hi += red[(w * 16 + l) * 2 + 0];
                lo += red[(w * 16 + l) * 2 + 1];
            }
        }
        epilogue<EPI>(a, t, l, (hi + lo) * inv_scale);
    }
}

static int pick_nw(int tiles, int quads)
{
    int nw = tiles < 1024 ? 8 : 4;
    while (nw > 4 && nw > quads) nw >>= 1;
    return nw;
}

template <int DT, int NW>
static void launch_dt_nw(const GemvArgs &a, int epi, size_t lds, hipStream_t s)
{
    dim3 grid(a.w.row_tiles), block(NW * 64);
    switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((k_gemv1<DT, NW, EPI_STORE>), grid, block, lds, s, a); break;
    case EPI_RESID: hipLaunchKernelGGL((k_gemv1<DT, NW, EPI_RESID>), grid, block, lds, s, a); break;
    case EPI_SWIGLU: hipLaunchKernelGGL((k_gemv1<DT, NW, EPI_SWIGLU>), grid, block, lds, s, a); break;
    case EPI_QKV: hipLaunchKernelGGL((k_gemv1<DT, NW, EPI_QKV>), grid, block, lds, s, a); break;
    case EPI_LOGITS: hipLaunchKernelGGL((k_gemv1<DT, NW, EPI_LOGITS>), grid, block, lds, s, a); break;
    }
}

template <int DT>
static void launch_dt(const GemvArgs &a, int epi, hipStream_t s)
{
    const int nw = pick_nw(a.w.row_tiles, a.w.block_quads);
    const size_t lds = (size_t)a.w.block_quads * 512 + (size_t)nw * 32 * 4 + 64 * 4;
    if (nw == 8) launch_dt_nw<DT, 8>(a, epi, lds, s);
    else launch_dt_nw<DT, 4>(a, epi, lds, s);
}

size_t gemv_lds_bytes(int block_quads) { return (size_t)block_quads * 512 + 8 * 32 * 4 + 64 * 4; }

int launch_gemv(const GemvArgs &a, int epi, hipStream_t s)
{
    if (a.n != 1) return -4;
    if (gemv_lds_bytes(a.w.block_quads) > 65536) return -4;
    switch (a.w.dtype) {
    case DT_Q4_0: launch_dt<DT_Q4_0>(a, epi, s); break;
    case DT_Q5_0: launch_dt<DT_Q5_0>(a, epi, s); break;
    case DT_Q8_0: launch_dt<DT_Q8_0>(a, epi, s); break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
