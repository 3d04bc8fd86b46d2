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

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow to
 * +-Inf, NaN stays a quiet NaN keeping the top payload bits.  No reference
 * counterpart (the reference caches K/V in fp32): it models the fp16 KV
 * cache of the multi-session configuration, where each K/V value is rounded
 * once when it is written. */
uint16_t o_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 (and Inf) */
    uint32_t h, rem, half;
    if (ax >= 0x38800000u) {                 /* normal: exponent rebias, 13 bits dropped */
        const uint32_t r = ax - 0x38000000u;
        h = r >> 13;
        rem = r & 0x1FFFu;
        half = 0x1000u;
    } else {                                 /* subnormal half: units of 2^-24 */
        const uint32_t e = ax >> 23;
        if (e < 102u) return (uint16_t)sign;  /* below 2^-25 */
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u, sh = 126u - e;   /* 14..24 */
        h = mant >> sh;
        rem = mant & ((1u << sh) - 1u);
        half = 1u << (sh - 1u);
    }
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* Block geometry per dtype: values per block, bytes per block.
 * Reference src/quant.c:298-308 (+ Q4_0, absent there: 18-byte blocks);
 * the K-quant super-blocks hold 256 values (src/quant.c:91-105). */
int o_block_params(int dtype, size_t *bsz)
{
    switch (dtype) {
    case O_F32:  *bsz = 4;  return 1;
    case O_F16:  *bsz = 2;  return 1;
    case O_Q4_0: *bsz = 18; return 32;
    case O_Q5_0: *bsz = 22; return 32;
    case O_Q8_0: *bsz = 34; return 32;
    case O_Q4_K: *bsz = 144; return 256;
    case O_Q6_K: *bsz = 210; return 256;
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

/* Q4_K super-block: fp16 d, fp16 dmin, 12 bytes packing eight 6-bit
 * scales and eight 6-bit mins, 128 bytes of nibbles.  Sub-block j takes
 * scale/min j (j < 4: low 6 bits of bytes j / j+4; j >= 4: the low / high
 * nibble of byte j+4 under the top two bits of bytes j-4 / j), and its 32
 * values are the low (j even) or high (j odd) nibbles of bytes
 * 32*(j/2) .. +31: value = (d*sc)*q - dmin*mn, products exact in fp32, one
 * rounding at the subtraction.  src/quant.c:92-97,113-132,172-195 */
static void q4k_scale_min(int j, const uint8_t *s, int *sc, int *mn)
{
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *mn = s[j + 4] & 0x3F;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void deq_q4_k(const uint8_t *b, float *dst)
{
    float d = o_f16_to_f32(rd16(b)), dmin = o_f16_to_f32(rd16(b + 2));
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min(j, b + 4, &sc, &mn);
        float db = d * (float)sc, mb = dmin * (float)mn;
        const uint8_t *q = b + 16 + 32 * (j / 2);
        int sh = (j & 1) ? 4 : 0;
        for (int k = 0; k < 32; k++) dst[32 * j + k] = db * (float)((q[k] >> sh) & 0xF) - mb;
    }
}

/* Q6_K super-block: ql[128], qh[64], int8 scales[16], fp16 d.  Value i (group
 * g = i/32, j = i%32): low nibble of ql[(g<4 ? 0 : 64) + 32*(g&1) + j]
 * (upper half when g&2), two high bits from qh[(g<4 ? 0 : 32) + j] at bit
 * 2*(g&3); value = (d*scales[i/16]) * (q - 32).  src/quant.c:99-105,197-231 */
static void deq_q6_k(const uint8_t *b, float *dst)
{
    float d = o_f16_to_f32(rd16(b + 208));
    for (int i = 0; i < 256; i++) {
        int g = i / 32, j = i % 32;
        int lo = (b[(g < 4 ? 0 : 64) + (g & 1) * 32 + j] >> ((g & 2) ? 4 : 0)) & 0xF;
        int hi = (b[128 + (g < 4 ? 0 : 32) + j] >> ((g & 3) * 2)) & 0x3;
        int q = (lo | (hi << 4)) - 32;
        dst[i] = d * (float)(int8_t)b[192 + i / 16] * (float)q;
    }
}

/* One block (32 values, or 256 for the K-quants) into dst. */
static void deq_block(const uint8_t *b, float *dst, int dtype)
{
    switch (dtype) {
    case O_Q4_0: deq_q4_0(b, dst); break;
    case O_Q5_0: deq_q5_0(b, dst); break;
    case O_Q8_0: deq_q8_0(b, dst); break;
    case O_Q4_K: deq_q4_k(b, dst); break;
    case O_Q6_K: deq_q6_k(b, dst); break;
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
    case O_Q4_0: case O_Q5_0: case O_Q8_0: case O_Q4_K: case O_Q6_K: {
        size_t bsz;
        int bs = o_block_params(dtype, &bsz);
        for (int bi = 0; bi < n / bs; bi++) deq_block(s + bi * bsz, dst + bi * bs, dtype);
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
    float tmp[256];

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
                for (int bi = 0; bi < k / bs; bi++) {
                    deq_block(row + bi * bsz, tmp, dtype);
                    for (int j = 0; j < bs; j++)
                        acc = acc + tmp[j] * b[(size_t)(bi * bs + j) * n + ni];
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
            for (int bi = 0; bi < k / bs; bi++) {
                deq_block(row + bi * bsz, tmp, dtype);
                for (int h = 0; h < bs; h += 16)
                    for (int j = 0; j < 16; j++)
                        lane[j] = fmaf(tmp[h + j], b[(size_t)(bi * bs + h + j) * n + ni], lane[j]);
            }
            out[(size_t)mi * n + ni] = reduce16(lane);
        }
    }
}
