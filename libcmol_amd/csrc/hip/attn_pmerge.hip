// attn_pmerge.hip — the split merge of prompt passes: one wave per (query
// head, token) instead of a 256-thread work-group, so the 512 x 16 merges
// of a 512-token pass fill the CUs in one round of 2048 work-groups rather
// than four of 8192.  A translation unit of its own, beside the decode
// attention kernels' code object.
#include "attn_impl.h"

// mx = max_s m_s, L = sum_s l_s e^(m_s - mx), out = sum_s o_s e^(m_s - mx) / L
// over the nact splits in ascending order; lane l holds dimensions
// l, l + 64, ... of the head.
template <int DH>
__global__ __launch_bounds__(256) void k_attn_merge_wave(AttnArgs a)
{
#pragma clang fp contract(off)
    constexpr int DL = DH / 64;
    const int lane = threadIdx.x & 63;
    const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int hq = idx % a.n_heads, n = idx / a.n_heads;
    if (n >= a.n) return;
    const int G = a.n_heads / a.n_kv, kvh = hq / G, h = hq % G;
    const int L = min(a.seqlen[n * a.seqlen_stride], a.max_ctx);
    const int nact = (L + a.split - 1) / a.split;
    if (nact <= 1) return;   // finished by the attention kernel
    const size_t hb = (((size_t)n * a.n_kv + kvh) * a.max_splits) * G + h;   // + s * G
    float mx = -INFINITY;
    for (int s = lane; s < nact; s += 64) mx = fmaxf(mx, a.pm[hb + (size_t)s * G]);
    mx = wave_max(mx);
    float Ls = 0.0f, acc[DL];
#pragma unroll
    for (int i = 0; i < DL; i++) acc[i] = 0.0f;
#pragma unroll 4
    for (int s = 0; s < nact; s++) {
        const size_t o = hb + (size_t)s * G;
        const float e = expf(a.pm[o] - mx);
        Ls += a.pl[o] * e;
#pragma unroll
        for (int i = 0; i < DL; i++) acc[i] += a.po[o * DH + 64 * i + lane] * e;
    }
#pragma unroll
    for (int i = 0; i < DL; i++) {
        const float v = acc[i] / Ls;
        const int k = hq * DH + 64 * i + lane;
        if (a.out) a.out[(size_t)n * a.out_stride + k] = v;
        if (a.next.q) act_put<StPlain>(a.next, n, k, v);
    }
}

int launch_attn_merge_wave(const AttnArgs &a, hipStream_t s)
{
    if (a.d_head != 64 && a.d_head != 128) return -4;
    const long waves = (long)a.n_heads * a.n;
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    if (a.d_head == 128) hipLaunchKernelGGL((k_attn_merge_wave<128>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attn_merge_wave<64>), grid, block, 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
