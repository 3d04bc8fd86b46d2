/*
 * o_quant.c — oracle: fp16 conversion, block dequantisation and the two
 * reference matmul accumulation orders.  TEST INFRASTRUCTURE ONLY (see
 * oracle.h).  Compiled with -ffp-contract=off so that every product and
 * sum is rounded where the reference rounds it; fused multiply-adds are
 * written explicitly with fmaf() exactly where the reference's SIMD kernel
 * uses _mm512_fmadd_ps.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* IEEE binary16 -> binary32, exact for every input including subnormals,
 * infinities and NaN payloads (mantissa shifted left by 13).
 * Follows reference src/quant.c:38-63. */
float o_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t f = h & 0x3FFu;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7F800000u | (f << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0u) {
        bits = sign;
    } else {
        /* subnormal half: value = f * 2^-24; normalise the mantissa */
        int lead = 31 - __builtin_clz(f);          /* 0..9 */
        uint32_t mant = (f << (10 - lead)) & 0x3FFu;
        uint32_t exp32 = (uint32_t)(lead - 24 + 127);
        bits = sign | (exp32 << 23) | (mant << 13);
    }
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* Block geometry per dtype: values per block, bytes per block.
 * Reference src/quant.c:298-308 (+ Q4_0, absent there: 18-byte blocks). */
int o_block_params(int dtype, size_t *bsz)
{
    switch (dtype) {
    case O_F32:  *bsz = 4;  return 1;
    case O_F16:  *bsz = 2;  return 1;
    case O_Q4_0: *bsz = 18; return 32;
    case O_Q5_0: *bsz = 22; return 32;
    case O_Q8_0: *bsz = 34; return 32;
    default:     *bsz = 0;  return 0;
    }
}

/* Reference src/model.c:68-78 (+ Q4_0). */
size_t o_row_bytes(int k, int dtype)
{
    size_t bsz;
    int bs = o_block_params(dtype, &bsz);
    return bs ? (size_t)(k / bs) * bsz : 0;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q8_0: 2-byte fp16 scale + 32 int8; dst = d * q.  src/quant.c:166-170 */
static void deq_q8_0(const uint8_t *b, float *dst)
{
    float d = o_f16_to_f32(rd16(b));
    for (int i = 0; i < 32; i++) dst[i] = d * (float)(int8_t)b[2 + i];
}

/* Q5_0: fp16 d, qh[4] (bit j = 5th bit of value j), qs[16] low nibble =
 * value j, high nibble = value j+16; q - 16.  src/quant.c:152-164 */
static void deq_q5_0(const uint8_t *b, float *dst)
{
    float d = o_f16_to_f32(rd16(b));
    uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) |
                  ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int j = 0; j < 16; j++) {
        uint32_t byte = b[6 + j];
        int lo = (int)((byte & 0xFu) | (((qh >> j) & 1u) << 4));
        int hi = (int)((byte >> 4) | (((qh >> (j + 16)) & 1u) << 4));
        dst[j] = d * (float)(lo - 16);
        dst[j + 16] = d * (float)(hi - 16);
    }
}

/* Q4_0 (GGML layout, absent from the reference): fp16 d + qs[16]; value j
 * is the low nibble of qs[j], value j+16 the high nibble; q - 8.  Same
 * nibble order as Q5_0 without qh.  Pinned by transcoding to Q8_0. */
static void deq_q4_0(const uint8_t *b, float *dst)
{
    float d = o_f16_to_f32(rd16(b));
    for (int j = 0; j < 16; j++) {
        uint32_t byte = b[2 + j];
        dst[j] = d * (float)((int)(byte & 0xFu) - 8);
        dst[j + 16] = d * (float)((int)(byte >> 4) - 8);
    }
}

static void deq_block(const uint8_t *b, float *dst, int dtype)
{
    switch (dtype) {
    case O_Q4_0: deq_q4_0(b, dst); break;
    case O_Q5_0: deq_q5_0(b, dst); break;
    case O_Q8_0: deq_q8_0(b, dst); break;
    default: break;
    }
}

/* Reference src/quant.c:241-289.  NULL / n<=0 / unknown dtype: no-op. */
void o_dequant_row(const void *src, float *dst, int n, int dtype)
{
    if (!src || !dst || n <= 0) return;
    const uint8_t *s = (const uint8_t *)src;
    switch (dtype) {
    case O_F32:
        memcpy(dst, src, (size_t)n * 4);
        break;
    case O_F16:
        for (int i = 0; i < n; i++) dst[i] = o_f16_to_f32(rd16(s + 2 * i));
        break;
    case O_Q4_0: case O_Q5_0: case O_Q8_0: {
        size_t bsz;
        o_block_params(dtype, &bsz);
        for (int bi = 0; bi < n / 32; bi++) deq_block(s + bi * bsz, dst + bi * 32, dtype);
        break;
    }
    default:
        break;
    }
}

/* Horizontal sum in the order of GCC's _mm512_reduce_add_ps: fold the
 * upper 256 bits onto the lower, then 128, then lanes {2,3} onto {0,1},
 * then lane 1 onto lane 0. */
static float reduce16(const float *a)
{
    float t8[8], t4[4];
    for (int i = 0; i < 8; i++) t8[i] = a[8 + i] + a[i];
    for (int i = 0; i < 4; i++) t4[i] = t8[4 + i] + t8[i];
    float u0 = t4[0] + t4[2];
    float u1 = t4[1] + t4[3];
    return u0 + u1;
}

/* out[m*n] = A[m x k] . B[k x n]; B is k-major (B[ki*n+ni]), out[mi*n+ni].
 * order O_ORDER_SCALAR follows cmol_matmul_scalar (src/quant.c:334-376):
 *   one running float per output, acc = acc + w*x, no fusion.
 * order O_ORDER_AVX512 follows cmol_matmul_avx512 (src/quant.c:488-566):
 *   16 accumulator lanes; per 16 consecutive k, lane j += w[k]*x[k] fused;
 *   final reduce16; F32 tail (k % 16) added sequentially after the reduce;
 *   F16 weights use the sequential unfused sum. */
void o_matmul(float *out, const void *a, const float *b,
              int m, int k, int n, int dtype, int order)
{
    size_t bsz;
    int bs = o_block_params(dtype, &bsz);
    if (!bs) return;
    const uint8_t *ab = (const uint8_t *)a;
    size_t row_bytes = (size_t)(k / bs) * bsz;
    float tmp[32];

    for (int mi = 0; mi < m; mi++) {
        const uint8_t *row = ab + (size_t)mi * row_bytes;
        for (int ni = 0; ni < n; ni++) {
            if (dtype == O_F16 || (dtype == O_F32 && order == O_ORDER_SCALAR)) {
                float acc = 0.0f;
                for (int ki = 0; ki < k; ki++) {
                    float w = dtype == O_F16 ? o_f16_to_f32(rd16(row + 2 * ki))
                                             : ((const float *)row)[ki];
                    acc = acc + w * b[(size_t)ki * n + ni];
                }
                out[(size_t)mi * n + ni] = acc;
                continue;
            }
            if (order == O_ORDER_SCALAR) {
                float acc = 0.0f;
                for (int bi = 0; bi < k / 32; bi++) {
                    deq_block(row + bi * bsz, tmp, dtype);
                    for (int j = 0; j < 32; j++)
                        acc = acc + tmp[j] * b[(size_t)(bi * 32 + j) * n + ni];
                }
                out[(size_t)mi * n + ni] = acc;
                continue;
            }
            /* 16-lane order */
            float lane[16] = {0};
            if (dtype == O_F32) {
                const float *af = (const float *)row;
                int ki = 0;
                for (; ki + 15 < k; ki += 16)
                    for (int j = 0; j < 16; j++)
                        lane[j] = fmaf(af[ki + j], b[(size_t)(ki + j) * n + ni], lane[j]);
                float t = reduce16(lane);
                for (; ki < k; ki++) t = t + af[ki] * b[(size_t)ki * n + ni];
                out[(size_t)mi * n + ni] = t;
                continue;
            }
            for (int bi = 0; bi < k / 32; bi++) {
                deq_block(row + bi * bsz, tmp, dtype);
                for (int h = 0; h < 32; h += 16)
                    for (int j = 0; j < 16; j++)
                        lane[j] = fmaf(tmp[h + j], b[(size_t)(bi * 32 + h + j) * n + ni], lane[j]);
            }
            out[(size_t)mi * n + ni] = reduce16(lane);
        }
    }
}
