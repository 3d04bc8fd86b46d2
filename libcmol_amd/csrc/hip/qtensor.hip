// qtensor.hip — upload-time repack of GGUF blocks into the quad-tile layout,
// bit-exact dequantisation from that layout, and the embedding-row gather.
#include "common.h"
#include "kernels.h"

// One thread per (tile, quad, lane): gathers the lane's codes for 4 blocks,
// its Q5_0 fifth-bit byte per block, and (lanes 0..15) the row's 4 scales.
template <int DT>
__global__ void k_repack(const uint8_t *__restrict__ raw, int rows, int nb,
                         int row0, int BQ, uint8_t *__restrict__ qs,
                         uint16_t *__restrict__ dsc, uint32_t *__restrict__ qh,
                         int tile0, int tiles)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES, BB = QFmt<DT>::BLOCK_BYTES;
    long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long total = (long)tiles * BQ * 64;
    if (gid >= total) return;
    int lane = (int)(gid & 63);
    long cell = (gid >> 6) + (long)tile0 * BQ;   // t * BQ + q
    int q = (int)(cell % BQ);
    int t = (int)(cell / BQ);
    int r16 = lane & 15, g = lane >> 4;
    int grow = t * 16 + r16;            // row within the destination tensor
    int srow = grow - row0;             // row within this part
    uint8_t out[LB];
    uint32_t hword = 0;
    uint16_t dv[4];
    for (int bi = 0; bi < 4; bi++) {
        int b = q * 4 + bi;
        bool valid = srow >= 0 && srow < rows && b < nb;
        const uint8_t *src = raw + ((size_t)(valid ? srow : 0) * nb + (valid ? b : 0)) * BB;
        dv[bi] = valid ? (uint16_t)(src[0] | (src[1] << 8)) : 0;
        if constexpr (DT == DT_Q8_0) {
            for (int j = 0; j < 8; j++) out[bi * 8 + j] = valid ? src[2 + 8 * g + j] : 0;
        } else if constexpr (DT == DT_Q4_0) {
            for (int j = 0; j < 4; j++) out[bi * 4 + j] = valid ? src[2 + 4 * g + j] : 0;
        } else {
            for (int j = 0; j < 4; j++) out[bi * 4 + j] = valid ? src[6 + 4 * g + j] : 0;
            uint32_t qhw = valid ? (uint32_t)src[2] | ((uint32_t)src[3] << 8) |
                                   ((uint32_t)src[4] << 16) | ((uint32_t)src[5] << 24)
                                 : 0u;
            // byte layout expected by deq_q5: bit p = fifth bit of pair p's
            // low element, bit 4+p = fifth bit of its high element
            int base = 4 * g;
            uint32_t hb = 0;
            hb |= ((qhw >> (base + 0)) & 1u) << 0;        // p0 lo: lo(b0)
            hb |= ((qhw >> (base + 2)) & 1u) << 4;        // p0 hi: lo(b2)
            hb |= ((qhw >> (base + 1)) & 1u) << 1;        // p1 lo: lo(b1)
            hb |= ((qhw >> (base + 3)) & 1u) << 5;        // p1 hi: lo(b3)
            hb |= ((qhw >> (16 + base + 0)) & 1u) << 2;   // p2 lo: hi(b0)
            hb |= ((qhw >> (16 + base + 2)) & 1u) << 6;   // p2 hi: hi(b2)
            hb |= ((qhw >> (16 + base + 1)) & 1u) << 3;   // p3 lo: hi(b1)
            hb |= ((qhw >> (16 + base + 3)) & 1u) << 7;   // p3 hi: hi(b3)
            hword |= hb << (8 * bi);
        }
    }
    // Only rows of this part are written; the tensor is zero-filled before
    // the first part, which covers padding rows beyond every part.
    if (srow < 0 || srow >= rows) return;
    uint8_t *dst = qs + ((size_t)cell * 64 + lane) * LB;
    for (int j = 0; j < LB; j += 4)
        *(uint32_t *)(dst + j) = (uint32_t)out[j] | ((uint32_t)out[j + 1] << 8) |
                                 ((uint32_t)out[j + 2] << 16) | ((uint32_t)out[j + 3] << 24);
    if constexpr (DT == DT_Q5_0) qh[(size_t)cell * 64 + lane] = hword;
    if (g == 0) {
        uint16_t *dd = dsc + (size_t)cell * 64 + r16 * 4;
        for (int bi = 0; bi < 4; bi++) dd[bi] = dv[bi];
    }
}

// Interleave mode: destination row 2i+p comes from part p row i.
template <int DT>
__global__ void k_repack_il(const uint8_t *__restrict__ raw, int rows, int nb,
                            int row0, int part, int BQ, uint8_t *__restrict__ qs,
                            uint16_t *__restrict__ dsc, uint32_t *__restrict__ qh,
                            int tile0, int tiles)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES, BB = QFmt<DT>::BLOCK_BYTES;
    long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long total = (long)tiles * BQ * 64;
    if (gid >= total) return;
    int lane = (int)(gid & 63);
    long cell = (gid >> 6) + (long)tile0 * BQ;
    int q = (int)(cell % BQ);
    int t = (int)(cell / BQ);
    int r16 = lane & 15, g = lane >> 4;
    int grow = t * 16 + r16;
    if ((grow & 1) != part) return;
    int srow = (grow >> 1) - row0;
    if (srow < 0 || srow >= rows) return;
    uint8_t out[LB];
    uint32_t hword = 0;
    uint16_t dv[4];
    for (int bi = 0; bi < 4; bi++) {
        int b = q * 4 + bi;
        bool valid = b < nb;
        const uint8_t *src = raw + ((size_t)srow * nb + (valid ? b : 0)) * BB;
        dv[bi] = valid ? (uint16_t)(src[0] | (src[1] << 8)) : 0;
        if constexpr (DT == DT_Q8_0) {
            for (int j = 0; j < 8; j++) out[bi * 8 + j] = valid ? src[2 + 8 * g + j] : 0;
        } else if constexpr (DT == DT_Q4_0) {
            for (int j = 0; j < 4; j++) out[bi * 4 + j] = valid ? src[2 + 4 * g + j] : 0;
        } else {
            for (int j = 0; j < 4; j++) out[bi * 4 + j] = valid ? src[6 + 4 * g + j] : 0;
            uint32_t qhw = valid ? (uint32_t)src[2] | ((uint32_t)src[3] << 8) |
                                   ((uint32_t)src[4] << 16) | ((uint32_t)src[5] << 24)
                                 : 0u;
            int base = 4 * g;
            uint32_t hb = 0;
            hb |= ((qhw >> (base + 0)) & 1u) << 0;
            hb |= ((qhw >> (base + 2)) & 1u) << 4;
            hb |= ((qhw >> (base + 1)) & 1u) << 1;
            hb |= ((qhw >> (base + 3)) & 1u) << 5;
            hb |= ((qhw >> (16 + base + 0)) & 1u) << 2;
            hb |= ((qhw >> (16 + base + 2)) & 1u) << 6;
            hb |= ((qhw >> (16 + base + 1)) & 1u) << 3;
            hb |= ((qhw >> (16 + base + 3)) & 1u) << 7;
            hword |= hb << (8 * bi);
        }
    }
    uint8_t *dst = qs + ((size_t)cell * 64 + lane) * LB;
    for (int j = 0; j < LB; j += 4)
        *(uint32_t *)(dst + j) = (uint32_t)out[j] | ((uint32_t)out[j + 1] << 8) |
                                 ((uint32_t)out[j + 2] << 16) | ((uint32_t)out[j + 3] << 24);
    if constexpr (DT == DT_Q5_0) qh[(size_t)cell * 64 + lane] = hword;
    if (g == 0) {
        uint16_t *dd = dsc + (size_t)cell * 64 + r16 * 4;
        for (int bi = 0; bi < 4; bi++) dd[bi] = dv[bi];
    }
}

int launch_repack(const QTensor &t, const uint8_t *raw, int rows, int row0,
                  int mode, int part, hipStream_t s)
{
    if (rows <= 0) return 0;
    int d0 = mode == 0 ? row0 : 2 * row0 + part;
    int d1 = mode == 0 ? row0 + rows - 1 : 2 * (row0 + rows - 1) + part;
    int tile0 = d0 / 16, tiles = d1 / 16 - tile0 + 1;
    if (tile0 < 0 || tile0 + tiles > t.row_tiles) return -6;
    long total = (long)tiles * t.block_quads * 64;
    int threads = 256;
    unsigned grid = (unsigned)((total + threads - 1) / threads);
    int nb = t.cols / 32;
#define REPACK(DTV)                                                                       \
    if (mode == 0)                                                                        \
        hipLaunchKernelGGL(k_repack<DTV>, dim3(grid), dim3(threads), 0, s, raw, rows, nb, \
                           row0, t.block_quads, t.qs, t.d, t.qh, tile0, tiles);            \
    else                                                                                  \
        hipLaunchKernelGGL(k_repack_il<DTV>, dim3(grid), dim3(threads), 0, s, raw, rows,  \
                           nb, row0, part, t.block_quads, t.qs, t.d, t.qh, tile0, tiles);
    switch (t.dtype) {
    case DT_Q4_0: REPACK(DT_Q4_0); break;
    case DT_Q5_0: REPACK(DT_Q5_0); break;
    case DT_Q8_0: REPACK(DT_Q8_0); break;
    default: return -4;
    }
#undef REPACK
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Decoded value of one block: 32 floats in natural k order, computed through
// the same lane decoders the GEMM uses, times the fp32 scale.
template <int DT>
__device__ void block_values(const QTensor &t, int row, int b, float *dst, int dst_stride)
{
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    int tt = row >> 4, r16 = row & 15, q = b >> 2, bi = b & 3;
    size_t cell = (size_t)tt * t.block_quads + q;
    float d = f16_bits_to_f32(t.d[cell * 64 + r16 * 4 + bi]);
    for (int g = 0; g < 4; g++) {
        int lane = g * 16 + r16;
        const u32x4 *p = (const u32x4 *)(t.qs + (cell * 64 + lane) * LB);
        u32x4 c0 = p[0], c1 = LB == 32 ? p[1] : u32x4{0, 0, 0, 0};
        uint32_t h = DT == DT_Q5_0 ? t.qh[cell * 64 + lane] : 0u;
        f16x8 v = deq_block<DT>(c0, c1, h, bi);
        for (int e = 0; e < 8; e++)
            dst[kmap(DT, g, e) * dst_stride] = mul_scale_x86(d, (float)v[e]);
    }
}

template <int DT>
__global__ void k_dequant(QTensor t, float *__restrict__ out)
{
    long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int nb = t.cols / 32;
    long total = (long)t.rows * nb;
    if (gid >= total) return;
    int row = (int)(gid / nb), b = (int)(gid % nb);
    block_values<DT>(t, row, b, out + (size_t)row * t.cols + (size_t)b * 32, 1);
}

int launch_dequant(const QTensor &t, float *out, hipStream_t s)
{
    long total = (long)t.rows * (t.cols / 32);
    unsigned grid = (unsigned)((total + 255) / 256);
    switch (t.dtype) {
    case DT_Q4_0: hipLaunchKernelGGL(k_dequant<DT_Q4_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q5_0: hipLaunchKernelGGL(k_dequant<DT_Q5_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_dequant<DT_Q8_0>, dim3(grid), dim3(256), 0, s, t, out); break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Embedding rows for n vectors: x[s][:] = dequant(row token[s]).  Thread per
// block.  Also clears each vector's argmax slots for the LM head that ends
// the step.
template <int DT>
__global__ void k_embed(QTensor t, const int32_t *__restrict__ token, int token_stride,
                        float *__restrict__ x, int x_stride,
                        unsigned long long *__restrict__ argmax, int n)
{
    int s = blockIdx.y;
    if (s >= n) return;
    int nb = t.cols / 32;
    int tok = token[s * token_stride];
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < ARGMAX_SLOTS; i += blockDim.x) argmax[(size_t)s * ARGMAX_SLOTS + i] = 0ull;
    if (tok < 0 || tok >= t.rows) tok = 0;
    for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += gridDim.x * blockDim.x)
        block_values<DT>(t, tok, b, x + (size_t)s * x_stride + (size_t)b * 32, 1);
}

int launch_embed(const QTensor &t, const int32_t *token, int token_stride, float *x,
                 int x_stride, unsigned long long *argmax, int n, hipStream_t s)
{
    int nb = t.cols / 32;
    dim3 grid((nb + 63) / 64, n);
    switch (t.dtype) {
    case DT_Q4_0: hipLaunchKernelGGL(k_embed<DT_Q4_0>, grid, dim3(64), 0, s, t, token, token_stride, x, x_stride, argmax, n); break;
    case DT_Q5_0: hipLaunchKernelGGL(k_embed<DT_Q5_0>, grid, dim3(64), 0, s, t, token, token_stride, x, x_stride, argmax, n); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_embed<DT_Q8_0>, grid, dim3(64), 0, s, t, token, token_stride, x, x_stride, argmax, n); break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
