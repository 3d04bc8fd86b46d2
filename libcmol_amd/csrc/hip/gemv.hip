// gemv.hip — quantised matvec / small-batch GEMM for gfx950.
//
// y[n] = W . x[n] for a Q4_0/Q5_0/Q8_0/Q4_K/Q6_K weight in the quad-tile layout and up
// to 32 activation vectors (kernel template in gemv_impl.h).  One work-group
// owns one 16-row tile and its NW wavefronts split the k range.  The
// activation operand of the whole k range is copied into LDS once with
// direct-to-LDS loads (in chunks only when it exceeds the LDS budget); each
// wave streams its weight quads through a ring of U in-flight loads (one
// coalesced 16/32-byte load per lane per quad), decodes the codes to exact
// small integers in f16 (common.h) and contracts them with
// v_mfma_f32_16x16x32_f16 against the operand (kernels.h: f16 high part and
// scaled f16 remainder in two MFMA rows per vector, eight vectors per MFMA),
// so every product is exact and the sum is carried in fp32.  The per-block
// fp16 scale multiplies each block's 16x16 result tile.  Partial sums of the
// waves meet in LDS in a fixed order.
//
// Fused around the product (reference arithmetic in brackets):
//   RMSNorm: 1/sqrt(mean(x^2)+eps) from the producer's sum-of-squares
//            partials, applied to the result [src/model.c:90-97];
//   epilogues: store; residual add + next operand [src/model.c:232,259];
//            SwiGLU over interleaved gate/up rows [src/model.c:117-123];
//            RoPE on q/k rows + KV-cache write at pos [src/attn.c:83-101];
//            logits + first-index argmax [src/sampler.c:199-204].
#include "gemm_impl.h"

int launch_gemv_q4(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemv_q5(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemv_q8(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemm_q4(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemm_q5(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemm_q8(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemv_q4k(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemv_q6k(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemm_q4k(const GemvArgs &a, int epi, hipStream_t s);
int launch_gemm_q6k(const GemvArgs &a, int epi, hipStream_t s);

size_t act_bytes(int K, int n)
{
    const size_t blocks = (size_t)((K / 32 + 3) / 4) * 4;
    return blocks * 4 * (size_t)(2 * n) * 8 * sizeof(_Float16);
}


int launch_gemv(const GemvArgs &a, int epi, hipStream_t s)
{
    if (a.n < 1 || a.n > 32 || a.in.nrows != 2 * a.n || !a.in.q) return -6;
    int rc;
    switch (a.w.dtype) {
    case DT_Q4_0: rc = launch_gemv_q4(a, epi, s); break;
    case DT_Q5_0: rc = launch_gemv_q5(a, epi, s); break;
    case DT_Q8_0: rc = launch_gemv_q8(a, epi, s); break;
    case DT_Q4_K: rc = launch_gemv_q4k(a, epi, s); break;
    case DT_Q6_K: rc = launch_gemv_q6k(a, epi, s); break;
    default: return -4;
    }
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_gemm(const GemvArgs &a, int epi, hipStream_t s)
{
    if (a.n < 1 || a.in.nrows != 2 * a.n || !a.in.q) return -6;
    int rc;
    switch (a.w.dtype) {
    case DT_Q4_0: rc = launch_gemm_q4(a, epi, s); break;
    case DT_Q5_0: rc = launch_gemm_q5(a, epi, s); break;
    case DT_Q8_0: rc = launch_gemm_q8(a, epi, s); break;
    case DT_Q4_K: rc = launch_gemm_q4k(a, epi, s); break;
    case DT_Q6_K: rc = launch_gemm_q6k(a, epi, s); break;
    default: return -4;
    }
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

size_t gemm_part_floats(const QTensor &w, int n)
{
    const int ks = gemm_ks(w, n, (size_t)-1);
    return ks > 1 ? (size_t)ks * n * w.rows : 0;
}

size_t gemv_part_floats(const QTensor &w, int n)
{
    if (!gemv_batched(w, n)) return 0;
    GbShape sh;
    gb_plan(w, n, sh);
    size_t f = sh.splits > 1 ? (size_t)sh.splits * n * w.rows : 0;
    Gb16Shape p;
    if (gb16_plan(w, n, p) && p.splits > 1) f = std::max(f, (size_t)p.splits * n * w.rows);
    return f;
}

// k-split finish: each wave takes RPT runs of 64 rows of one vector; lane
// l takes row l of each run, so the lanes of a 16-row tile are a 16-lane
// group, as the epilogues need.  The epilogue's own inputs and the first
// FS slices' partial sums of every run are loaded together,
// unconditionally (rows past the matrix re-read the last one), so the
// kernel waits for one round trip before the epilogues.  Four runs per
// wave (FS = 4: the prompt GEMM's k ranges) serve the large finishes of
// prompt passes with a quarter of the work-groups.
template <int EPI, int RPT, int FS>
__global__ __launch_bounds__(256) void k_gemv_b_finish(GemvArgs a, int splits, int ss_count)
{
#pragma clang fp contract(off)
    // the arguments of the partial-sum and epilogue-input loads, fetched in
    // one round trip
    sgpr_pin(a.w.rows);
    sgpr_pin(a.n);
    sgpr_pin(a.part);
    sgpr_pin(splits);
    sgpr_pin(ss_count);
    sgpr_pin(a.in.ss);
    sgpr_pin(a.in.ss_stride);
    sgpr_pin(a.in.q);
    sgpr_pin(a.in.tail);
    sgpr_pin(a.out);
    sgpr_pin(a.out_stride);
    if constexpr (EPI == EPI_RESID) sgpr_pin(a.res);
    if constexpr (EPI == EPI_QKV) {
        sgpr_pin(a.kv.layer_off);
        sgpr_pin(a.kv.slot_ids);
        sgpr_pin(a.pos);
        sgpr_pin(a.pos_stride);
        sgpr_pin(a.pos0);
    }
    const int v = blockIdx.y, l = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 64 * RPT;   // the wave's first row
    if (r0 >= a.w.rows) return;   // whole waves past the matrix
    const size_t kstride = (size_t)a.n * a.w.rows;
    EpiPre pre[RPT];
    float pv[RPT][FS];
#pragma unroll
    for (int p = 0; p < RPT; p++) {
        const int row = r0 + 64 * p + l;
        epi_pre_load(a, EPI, v, row, row < a.w.rows, pre[p]);
        const float *pp = a.part + (size_t)v * a.w.rows + min(row, a.w.rows - 1);
#pragma unroll
        for (int k = 0; k < FS; k++) pv[p][k] = pp[(size_t)min(k, splits - 1) * kstride];
    }
    float nrm = 1.0f;
    if (ss_count) {
        float s = 0.0f;
        for (int i = l; i < ss_count; i += 64) s += a.in.ss[(size_t)v * a.in.ss_stride + i];
        s = wave_sum(s);
        nrm = 1.0f / sqrtf(s / (float)a.w.cols + a.in.eps);
    }
#pragma unroll
    for (int p = 0; p < RPT; p++) {
        const int row = r0 + 64 * p + l;
        if (r0 + 64 * p >= a.w.rows) break;   // uniform
        const bool act = row < a.w.rows;
        epi_pre_cs(a, EPI, row, act, pre[p]);
        // slices added in ascending order
        float y = 0.0f;
#pragma unroll
        for (int k = 0; k < FS; k++)
            if (k < splits) y += pv[p][k];
        const float *pp = a.part + (size_t)v * a.w.rows + min(row, a.w.rows - 1);
        for (int k = FS; k < splits; k++) y += pp[(size_t)k * kstride];
        y *= nrm;
        epilogue<EPI>(a, row >> 4, row & 15, 16, v, act, y, true, pre[p]);
    }
}

template <int RPT, int FS>
static void launch_finish(const GemvArgs &a, int epi, int splits, int ss_count, hipStream_t s)
{
    const dim3 grid((a.w.rows + 256 * RPT - 1) / (256 * RPT), a.n), block(256);
    auto go = [&](auto kern) {
        if (a.ev_stop) hipExtLaunchKernelGGL(kern, grid, block, 0, s, nullptr, a.ev_stop, 0, a, splits, ss_count);
        else hipLaunchKernelGGL(kern, grid, block, 0, s, a, splits, ss_count);
    };
    switch (epi) {
    case EPI_STORE: go(k_gemv_b_finish<EPI_STORE, RPT, FS>); break;
    case EPI_RESID: go(k_gemv_b_finish<EPI_RESID, RPT, FS>); break;
    case EPI_SWIGLU: go(k_gemv_b_finish<EPI_SWIGLU, RPT, FS>); break;
    case EPI_QKV: go(k_gemv_b_finish<EPI_QKV, RPT, FS>); break;
    default: go(k_gemv_b_finish<EPI_LOGITS, RPT, FS>); break;
    }
}

int launch_gemv_b_finish(const GemvArgs &a, int epi, int splits, int ss_count, hipStream_t s)
{
    // four runs per wave where the one-run grid would take several rounds
    // of the CUs (prompt passes: 512 vectors x 2048 rows, 4096 work-groups)
    static const bool wide = [] {
        const char *e = getenv("CMOL_FINISH_RUNS");   // measurements: 1 turns it off
        return !(e && e[0] == '1');
    }();
    const long wgs = (long)((a.w.rows + 255) / 256) * a.n;
    if (wide && splits <= 4 && wgs >= 8L * gemv_cus()) launch_finish<4, 4>(a, epi, splits, ss_count, s);
    else launch_finish<1, 16>(a, epi, splits, ss_count, s);
    return 0;
}

// Standalone operand preparation: one thread per (vector, block of 32).
__global__ void k_act_prep(const float *__restrict__ x, int x_stride, int K, int n, ActOut o)
{
#pragma clang fp contract(off)
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    const int v = blockIdx.y;
    if (v >= n || b >= K / 32) return;
    float ss = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float xv = x[(size_t)v * x_stride + 32 * b + i];
        ss += xv * xv;
        act_put(o, v, 32 * b + i, xv);
    }
    if (o.ss) o.ss[(size_t)v * o.ss_stride + b] = ss;
}

int launch_act_prep(const float *x, int x_stride, int K, int n, const ActOut &o, hipStream_t s)
{
    const int nb = K / 32;
    hipLaunchKernelGGL(k_act_prep, dim3((nb + 63) / 64, n), dim3(64), 0, s, x, x_stride, K, n, o);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
