// qtensor_impl.h — reading the quad-tile layout element by element: the
// position of a (row, block) in the tiles, decoded block values (bit-exact
// with the reference's dequantisation) and the embedding-row gather shared
// by k_embed and the persistent decode kernel.
#pragma once
#include "common.h"
#include "kernels.h"

// Position of a destination tensor element in the tiled layout.
struct CellPos {
    size_t cell;   // t * BQ + q
    int col;       // MFMA column 0..15
    int bi;        // block within the quad
};

__device__ inline CellPos cell_pos(const QTensor &t, int row, int b)
{
    const int R = 16 / t.fold, BQ = t.block_quads;
    const int part = b / (4 * BQ), bq = b - part * 4 * BQ;
    CellPos p;
    p.cell = (size_t)(row / R) * BQ + (bq >> 2);
    p.col = part * R + row % R;
    p.bi = bq & 3;
    return p;
}

// Decoded values of lane group g of one block: val[e] is input
// 32b + kmap(DT, g, e), computed through the same lane decoders the matvec
// uses, times the fp32 scale.
template <int DT>
__device__ inline void block_vals8(const QTensor &t, int row, int b, int g, float val[8])
{
#pragma clang fp contract(off)
    constexpr int LB = QFmt<DT>::LANE_BYTES;
    const CellPos cp = cell_pos(t, row, b);
    if constexpr (is_kquant(DT)) {
        // the reference's arithmetic with x86 NaN rules: Q4_K
        // (d*sc)*q - dmin*mn, Q6_K (d*scale16)*(q - 32)
        const int lane = g * 16 + cp.col;
        u32x4 c0, c1;
        typename QScale<DT>::T sv;
        uint32_t h;
        q_load<DT>(t, cp.cell, cp.col, lane, c0, c1, sv, h);
        const f16x8 v = deq_block<DT>(c0, c1, h, cp.bi);
        const uint32_t pr = (sv[1 + (cp.bi >> 1)] >> (16 * (cp.bi & 1))) & 0xFFFFu;
        if constexpr (DT == DT_Q4_K) {
            const float db = mul_x86(f16_bits_to_f32(sv[0] & 0xFFFFu), (float)(pr & 0xFFu));
            const float mb = mul_x86(f16_bits_to_f32(sv[0] >> 16), (float)(pr >> 8));
#pragma unroll
            for (int e = 0; e < 8; e++) val[e] = sub_x86(mul_x86(db, (float)v[e] + 8.0f), mb);
        } else {
            const float d = f16_bits_to_f32(sv[0] & 0xFFFFu);
            const float dl = mul_x86(d, (float)(int8_t)(pr & 0xFFu));
            const float dh = mul_x86(d, (float)(int8_t)(pr >> 8));
#pragma unroll
            for (int e = 0; e < 8; e++) val[e] = mul_x86(e < 4 ? dl : dh, (float)v[e]);
        }
        return;
    }
    const float d = f16_bits_to_f32(t.d[cp.cell * 64 + cp.col * 4 + cp.bi]);
    const int lane = g * 16 + cp.col;
    const u32x4 *p = (const u32x4 *)(t.qs + (cp.cell * 64 + lane) * LB);
    const u32x4 c0 = p[0], c1 = LB == 32 ? p[1] : u32x4{0, 0, 0, 0};
    const uint32_t h = DT == DT_Q5_0 ? t.qh[cp.cell * 64 + lane] : 0u;
    const f16x8 v = deq_block<DT>(c0, c1, h, cp.bi);
#pragma unroll
    for (int e = 0; e < 8; e++) val[e] = mul_scale_x86(d, (float)v[e]);
}

// The same values written at their natural k positions dst[0..31].
template <int DT>
__device__ void block_values_g(const QTensor &t, int row, int b, int g, float *dst)
{
    float val[8];
    block_vals8<DT>(t, row, b, g, val);
    for (int e = 0; e < 8; e++) dst[kmap(DT, g, e)] = val[e];
}

// Embedding gather for one vector s, one thread per (block, lane group):
// thread gid covers block gid/4, group gid%4 of row `tok` (out-of-range ids
// read row 0): x[32b + k] = value, the consumer operand of vector s, and the
// per-block sum of squares (the 4 threads of a block are consecutive lanes).
// Every lane of the wave must call it (shuffles).
template <int DT, typename M>
__device__ inline void embed_group(const QTensor &t, int tok, int gid, float *x, const ActOut &o, int s)
{
#pragma clang fp contract(off)
    const int nb = t.cols / 32;
    if (tok < 0 || tok >= t.rows) tok = 0;
    const int b = gid >> 2, g = gid & 3;
    float ss = 0.0f;
    if (b < nb) {
        float val[8];
        block_vals8<DT>(t, tok, b, g, val);
        for (int e = 0; e < 8; e++) {
            const int k = 32 * b + kmap(DT, g, e);
            if (x) M::st(x + k, val[e]);
            ss += val[e] * val[e];
            if (o.q) act_put<M>(o, s, k, val[e]);
        }
    }
    // per-block sum over the 4 lane groups (lanes 4b..4b+3 of the wave)
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    if (b < nb && g == 0 && o.ss) M::st(o.ss + (size_t)s * o.ss_stride + b, ss);
}
