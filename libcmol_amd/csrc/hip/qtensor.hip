// qtensor.hip — upload-time repack of GGUF blocks into the quad-tile layout,
// bit-exact dequantisation from that layout, and the embedding-row gather.
#include "qtensor_impl.h"

// The lane's share of one GGUF block: codes (LB/4 bytes) and, for Q5_0, the
// byte of fifth bits in the pair order deq_q5 expects (bit p = fifth bit of
// pair p's low element, bit 4+p = of its high element).
template <int DT>
__device__ inline void lane_block(const uint8_t *src, int g, uint8_t *out, uint32_t *hb)
{
    if constexpr (DT == DT_Q8_0) {
        for (int j = 0; j < 8; j++) out[j] = src[2 + 8 * g + j];
        *hb = 0;
    } else if constexpr (DT == DT_Q4_0) {
        for (int j = 0; j < 4; j++) out[j] = src[2 + 4 * g + j];
        *hb = 0;
    } else {
        for (int j = 0; j < 4; j++) out[j] = src[6 + 4 * g + j];
        const uint32_t qhw = (uint32_t)src[2] | ((uint32_t)src[3] << 8) |
                             ((uint32_t)src[4] << 16) | ((uint32_t)src[5] << 24);
        const int base = 4 * g;
        uint32_t h = 0;
        h |= ((qhw >> (base + 0)) & 1u) << 0;        // p0 lo: lo(b0)
        h |= ((qhw >> (base + 2)) & 1u) << 4;        // p0 hi: lo(b2)
        h |= ((qhw >> (base + 1)) & 1u) << 1;        // p1 lo: lo(b1)
        h |= ((qhw >> (base + 3)) & 1u) << 5;        // p1 hi: lo(b3)
        h |= ((qhw >> (16 + base + 0)) & 1u) << 2;   // p2 lo: hi(b0)
        h |= ((qhw >> (16 + base + 2)) & 1u) << 6;   // p2 hi: hi(b2)
        h |= ((qhw >> (16 + base + 1)) & 1u) << 3;   // p3 lo: hi(b1)
        h |= ((qhw >> (16 + base + 3)) & 1u) << 7;   // p3 hi: hi(b3)
        *hb = h;
    }
}

// One thread per (tile, quad, lane) of the destination tiles a chunk of
// source rows lands in.  Source row i of the chunk is destination row
// row0 + i (concat) or 2*(row0 + i) + part (interleave).  Lanes whose row
// belongs to another chunk are left alone (the tensor is zero-filled first,
// which also covers padding rows and blocks).
template <int DT>
__global__ void k_repack(const uint8_t *__restrict__ raw, int rows, int row0, int mode,
                         int part, QTensor t, int tile0, int tiles)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES, BB = QFmt<DT>::BLOCK_BYTES;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int BQ = t.block_quads, R = 16 / t.fold, nb = t.cols / 32;
    if (gid >= (long)tiles * BQ * 64) return;
    const int lane = (int)(gid & 63);
    const long cell = (gid >> 6) + (long)tile0 * BQ;
    const int q = (int)(cell % BQ), tt = (int)(cell / BQ);
    const int c = lane & 15, g = lane >> 4;
    const int drow = tt * R + c % R;
    const int kpart = c / R;
    int srow;
    if (mode == 0) {
        srow = drow - row0;
    } else {
        if ((drow & 1) != part) return;
        srow = (drow >> 1) - row0;
    }
    if (srow < 0 || srow >= rows) return;
    uint8_t out[LB];
    uint32_t hword = 0;
    uint16_t dv[4];
    for (int bi = 0; bi < 4; bi++) {
        const int b = kpart * 4 * BQ + q * 4 + bi;
        if (b < nb) {
            const uint8_t *src = raw + ((size_t)srow * nb + b) * BB;
            uint32_t hb;
            lane_block<DT>(src, g, out + bi * (LB / 4), &hb);
            hword |= hb << (8 * bi);
            dv[bi] = (uint16_t)(src[0] | (src[1] << 8));
        } else {
            for (int j = 0; j < LB / 4; j++) out[bi * (LB / 4) + j] = 0;
            dv[bi] = 0;
        }
    }
    uint8_t *dst = t.qs + ((size_t)cell * 64 + lane) * LB;
    for (int j = 0; j < LB; j += 4)
        *(uint32_t *)(dst + j) = (uint32_t)out[j] | ((uint32_t)out[j + 1] << 8) |
                                 ((uint32_t)out[j + 2] << 16) | ((uint32_t)out[j + 3] << 24);
    if constexpr (DT == DT_Q5_0) t.qh[(size_t)cell * 64 + lane] = hword;
    if (g == 0) {
        uint16_t *dd = t.d + (size_t)cell * 64 + c * 4;
        for (int bi = 0; bi < 4; bi++) dd[bi] = dv[bi];
    }
}

// Code k (0..31) of sub-block j (0..7) of a K-quant super-block, and for
// Q6_K its two high bits separately (src/quant.c:172-231).
__device__ inline int q4k_code(const uint8_t *sb, int j, int k)
{
    return (sb[16 + 32 * (j >> 1) + k] >> ((j & 1) ? 4 : 0)) & 0xF;
}
__device__ inline int q6k_lo(const uint8_t *sb, int j, int k)
{
    return (sb[(j < 4 ? 0 : 64) + (j & 1) * 32 + k] >> ((j & 2) ? 4 : 0)) & 0xF;
}
__device__ inline int q6k_hi(const uint8_t *sb, int j, int k)
{
    return (sb[128 + (j < 4 ? 0 : 32) + k] >> ((j & 3) * 2)) & 0x3;
}

// Six-bit scale / min of sub-block j of a Q4_K super-block (12 packed
// bytes at offset 4; src/quant.c:113-132).
__device__ inline void q4k_scale_min(const uint8_t *sb, int j, int *sc, int *mn)
{
    const uint8_t *s = sb + 4;
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *mn = s[j + 4] & 0x3F;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// K-quant repack, one thread per (tile, quad, lane) as k_repack: the lane's
// codes of the cell's four sub-blocks in the Q4_0 byte layout (byte i: code
// 4g+i low, code 16+4g+i high), Q6_K's high bits in pair order, and (lanes
// of group 0) the column's scale record.
template <int DT>
__global__ void k_repack_k(const uint8_t *__restrict__ raw, int rows, int row0, int mode,
                           int part, QTensor t, int tile0, int tiles)
{
    constexpr int BB = QFmt<DT>::BLOCK_BYTES;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int BQ = t.block_quads, R = 16 / t.fold, nb = t.cols / 32, nsb = t.cols / 256;
    if (gid >= (long)tiles * BQ * 64) return;
    const int lane = (int)(gid & 63);
    const long cell = (gid >> 6) + (long)tile0 * BQ;
    const int q = (int)(cell % BQ), tt = (int)(cell / BQ);
    const int c = lane & 15, g = lane >> 4;
    const int drow = tt * R + c % R;
    const int kpart = c / R;
    int srow;
    if (mode == 0) {
        srow = drow - row0;
    } else {
        if ((drow & 1) != part) return;
        srow = (drow >> 1) - row0;
    }
    if (srow < 0 || srow >= rows) return;
    const int b0 = kpart * 4 * BQ + q * 4;   // first sub-block: a quad lies in one super-block
    if (b0 >= nb) return;                    // padding quad: stays zero
    const uint8_t *sb = raw + ((size_t)srow * nsb + b0 / 8) * BB;
    uint32_t words[4], hbits[2] = {0u, 0u};
    for (int bi = 0; bi < 4; bi++) {
        const int j = (b0 + bi) & 7;
        uint32_t w = 0, hq = 0;
        for (int i = 0; i < 4; i++) {
            const int klo = 4 * g + i, khi = 16 + 4 * g + i;
            int lo, hi;
            if constexpr (DT == DT_Q4_K) {
                lo = q4k_code(sb, j, klo);
                hi = q4k_code(sb, j, khi);
            } else {
                lo = q6k_lo(sb, j, klo);
                hi = q6k_lo(sb, j, khi);
                // pairs as deq_q4 orders them: (4g, 4g+2), (4g+1, 4g+3), then
                // the same +16; code 4g+i is in pair i&1 (2 + (i&1) for +16),
                // as its low (i < 2) or high element: bits 2p (+8 if high)
                const int p = i & 1, sh8 = 8 * (i >> 1);
                hq |= (uint32_t)q6k_hi(sb, j, klo) << (2 * p + sh8);
                hq |= (uint32_t)q6k_hi(sb, j, khi) << (2 * (2 + p) + sh8);
            }
            w |= (uint32_t)(lo | (hi << 4)) << (8 * i);
        }
        words[bi] = w;
        hbits[bi >> 1] |= hq << (16 * (bi & 1));
    }
    uint32_t *dst = (uint32_t *)(t.qs + ((size_t)cell * 64 + lane) * 16);
    for (int i = 0; i < 4; i++) dst[i] = words[i];
    if constexpr (DT == DT_Q6_K) {
        t.qh[((size_t)cell * 64 + lane) * 2] = hbits[0];
        t.qh[((size_t)cell * 64 + lane) * 2 + 1] = hbits[1];
    }
    if (g == 0) {
        uint32_t rec[4] = {0u, 0u, 0u, 0u};
        if constexpr (DT == DT_Q4_K) {
            rec[0] = (uint32_t)sb[0] | ((uint32_t)sb[1] << 8) | ((uint32_t)sb[2] << 16) | ((uint32_t)sb[3] << 24);
            for (int bi = 0; bi < 4; bi++) {
                int sc, mn;
                q4k_scale_min(sb, (b0 + bi) & 7, &sc, &mn);
                rec[1 + (bi >> 1)] |= (uint32_t)(sc | (mn << 8)) << (16 * (bi & 1));
            }
        } else {
            rec[0] = (uint32_t)sb[208] | ((uint32_t)sb[209] << 8);
            for (int bi = 0; bi < 4; bi++) {
                const int j = (b0 + bi) & 7;
                const uint32_t pair = (uint32_t)sb[192 + 2 * j] | ((uint32_t)sb[192 + 2 * j + 1] << 8);
                rec[1 + (bi >> 1)] |= pair << (16 * (bi & 1));
            }
        }
        uint32_t *rd = (uint32_t *)((uint8_t *)t.d + ((size_t)cell * 16 + c) * 16);
        for (int i = 0; i < 4; i++) rd[i] = rec[i];
    }
}

int launch_repack(const QTensor &t, const uint8_t *raw, int rows, int row0,
                  int mode, int part, hipStream_t s)
{
    if (rows <= 0) return 0;
    const int R = 16 / t.fold;
    const int d0 = mode == 0 ? row0 : 2 * row0 + part;
    const int d1 = mode == 0 ? row0 + rows - 1 : 2 * (row0 + rows - 1) + part;
    const int tile0 = d0 / R, tiles = d1 / R - tile0 + 1;
    if (tile0 < 0 || tile0 + tiles > t.row_tiles) return -6;
    const long total = (long)tiles * t.block_quads * 64;
    const unsigned grid = (unsigned)((total + 255) / 256);
#define REPACK(DTV) hipLaunchKernelGGL(k_repack<DTV>, dim3(grid), dim3(256), 0, s, raw, rows, row0, mode, part, t, tile0, tiles)
    switch (t.dtype) {
    case DT_Q4_0: REPACK(DT_Q4_0); break;
    case DT_Q5_0: REPACK(DT_Q5_0); break;
    case DT_Q8_0: REPACK(DT_Q8_0); break;
    case DT_Q4_K: hipLaunchKernelGGL(k_repack_k<DT_Q4_K>, dim3(grid), dim3(256), 0, s, raw, rows, row0, mode, part, t, tile0, tiles); break;
    case DT_Q6_K: hipLaunchKernelGGL(k_repack_k<DT_Q6_K>, dim3(grid), dim3(256), 0, s, raw, rows, row0, mode, part, t, tile0, tiles); break;
    default: return -4;
    }
#undef REPACK
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int DT>
__device__ void block_values(const QTensor &t, int row, int b, float *dst)
{
    for (int g = 0; g < 4; g++) block_values_g<DT>(t, row, b, g, dst);
}

template <int DT>
__global__ void k_dequant(QTensor t, float *__restrict__ out)
{
    long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int nb = t.cols / 32;
    long total = (long)t.rows * nb;
    if (gid >= total) return;
    int row = (int)(gid / nb), b = (int)(gid % nb);
    block_values<DT>(t, row, b, out + (size_t)row * t.cols + (size_t)b * 32);
}

int launch_dequant(const QTensor &t, float *out, hipStream_t s)
{
    long total = (long)t.rows * (t.cols / 32);
    unsigned grid = (unsigned)((total + 255) / 256);
    switch (t.dtype) {
    case DT_Q4_0: hipLaunchKernelGGL(k_dequant<DT_Q4_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q5_0: hipLaunchKernelGGL(k_dequant<DT_Q5_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_dequant<DT_Q8_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q4_K: hipLaunchKernelGGL(k_dequant<DT_Q4_K>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q6_K: hipLaunchKernelGGL(k_dequant<DT_Q6_K>, dim3(grid), dim3(256), 0, s, t, out); break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Embedding rows for n vectors: x[s][:] = dequant(row token[s]), plus the
// first consumer's operand and its per-block sums of squares.  Four threads
// per block (one per lane group).  Work-group (0, s) also clears vector s's
// argmax slots for the LM head that ends the step.
template <int DT>
__global__ __launch_bounds__(256) void k_embed(QTensor t, const int32_t *__restrict__ token,
                                               int token_stride, float *__restrict__ x,
                                               int x_stride, ActOut o,
                                               unsigned long long *__restrict__ argmax, int n)
{
    const int s = blockIdx.y;
    if (s >= n) return;
    const int tok = token[s * token_stride];
    if (argmax && blockIdx.x == 0)
        for (int i = threadIdx.x; i < ARGMAX_SLOTS; i += blockDim.x) argmax[(size_t)s * ARGMAX_SLOTS + i] = 0ull;
    embed_group<DT, StPlain>(t, tok, blockIdx.x * blockDim.x + threadIdx.x, x + (size_t)s * x_stride, o, s);
}

int launch_embed(const QTensor &t, const int32_t *token, int token_stride, float *x,
                 int x_stride, const ActOut &o, unsigned long long *argmax, int n, hipStream_t s)
{
    const int nb = t.cols / 32;
    dim3 grid((nb * 4 + 255) / 256, n);
    switch (t.dtype) {
    case DT_Q4_0: hipLaunchKernelGGL(k_embed<DT_Q4_0>, grid, dim3(256), 0, s, t, token, token_stride, x, x_stride, o, argmax, n); break;
    case DT_Q5_0: hipLaunchKernelGGL(k_embed<DT_Q5_0>, grid, dim3(256), 0, s, t, token, token_stride, x, x_stride, o, argmax, n); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_embed<DT_Q8_0>, grid, dim3(256), 0, s, t, token, token_stride, x, x_stride, o, argmax, n); break;
    case DT_Q4_K: hipLaunchKernelGGL(k_embed<DT_Q4_K>, grid, dim3(256), 0, s, t, token, token_stride, x, x_stride, o, argmax, n); break;
    case DT_Q6_K: hipLaunchKernelGGL(k_embed<DT_Q6_K>, grid, dim3(256), 0, s, t, token, token_stride, x, x_stride, o, argmax, n); break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
