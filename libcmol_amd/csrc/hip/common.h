// common.h — shared device types, the tiled weight layout and the
// per-format code-to-f16 decoders used by every gfx950 kernel of libcmol.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Global and LDS pointers for direct-to-LDS loads (global_load_lds).
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8)
#define WAITCNT_VM_LGKM0(N) (((N) & 15) | (((N) >> 4) << 14) | (7 << 4))

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum { DT_F32 = 0, DT_F16 = 1, DT_Q4_0 = 2, DT_Q5_0 = 6, DT_Q8_0 = 8, DT_Q4_K = 12, DT_Q6_K = 14 };

// Global-memory view of a generic pointer: accesses through the result
// compile to global_* instructions.  Used where the compiler cannot infer the
// address space itself (pointers read from memory), which would otherwise
// get flat_* accesses that also count against the LDS/scalar wait counter.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gptr(const T *p)
{
    return (const __attribute__((address_space(1))) T *)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gptr(T *p)
{
    return (__attribute__((address_space(1))) T *)p;
}

// Load of a 4-, 8- or 16-byte value (vector class types included) through
// gptr.
// Pins a launch argument in SGPRs at this point: the kernel-argument loads
// of every pinned value are then issued together and waited for once,
// instead of being sunk into the branches that first use them (each sunk
// group is another round trip before the weight loads go out).
template <typename T>
__device__ __forceinline__ void sgpr_pin(T v)
{
    asm volatile("" ::"s"(v));
}

// A pointer every lane holds the same value of, moved to scalar registers
// (loads through it can take the base from there: no per-lane 64-bit adds).
template <typename T>
__device__ __forceinline__ const T *uniform_ptr(const T *p)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T *)(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T ldg(const T *p)
{
    if constexpr (sizeof(T) == 16) return __builtin_bit_cast(T, *gptr((const u32x4 *)p));
    else if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, *gptr((const u32x2 *)p));
    else return __builtin_bit_cast(T, *gptr((const uint32_t *)p));
}

// ---------------------------------------------------------------------------
// Tiled weight layout ("quad tiles").
//
// A GGUF block tensor of M rows x K cols (nb = K/32 blocks per row) with fold
// F in {1, 2, 4, 8} is cut into RT = ceil(M/R) row tiles of R = 16/F rows
// and, along k, into F parts of BQ quads (4 blocks) each, BQ = ceil(ceil(nb/F)
// / 4); part p covers blocks [4*BQ*p, 4*BQ*(p+1)).  A (tile t, quad q) cell
// has 16 columns, the 16 B-operand columns of v_mfma_f32_16x16x32_f16:
//   column c -> weight row R*t + c % R, part c / R, blocks 4*BQ*(c/R)+4q+bi
// and every one of the 64 lanes of a wavefront owns the codes it feeds to
// the MFMA:  lane l -> column l % 16, k-group g = l / 16,
//   Q4_0/Q5_0: 16 bytes = dword g of the 16-byte nibble array of each of the
//              cell's 4 blocks (4 bytes per block)
//   Q8_0:      32 bytes = bytes 8g..8g+7 of the 32 int8 codes of each of the
//              4 blocks (8 bytes per block)
// so one wave-wide 16-byte (or 2x16-byte) load per lane moves a contiguous
// 1 KiB (2 KiB).  Scales: 16 columns x 4 blocks fp16 per cell (128 bytes),
// entry [column][block % 4].  Q5_0 fifth bits: one dword per lane per cell,
// byte (block % 4) holding the 8 fifth bits of the lane's 8 codes in pair
// order (see deq_q5).  Rows beyond M and blocks beyond nb are zero-filled.
// F = 1 is the plain layout (16 rows per tile); F > 1 lets a matrix with
// few rows spread over F times more work-groups at batch 1.
//
// k order inside a block for lane group g, element e (the same permutation is
// applied to the activation operand, so the MFMA contraction is unchanged):
//   Q4_0/Q5_0/Q4_K/Q6_K: e -> (e>=4 ? 16 : 0) + 4g + {0,2,1,3}[e&3]
//   Q8_0:                e -> 8g + e
//
// K-quants (super-blocks of 256 = 8 blocks of 32, so a quad never straddles
// two super-blocks): the "blocks" above are the 32-value sub-blocks.
//   Q4_K: codes as Q4_0 (nibble q, decoded as q - 8); no fifth-bit array.
//   Q6_K: low nibbles as Q4_0; the two high bits of the lane's 8 codes of a
//         block in 16 bits (bits 2p..2p+1: low element of pair p, bits
//         8+2p..: high element, pairs as deq_q4 orders them), two blocks per
//         dword, two dwords per lane per cell.
//   Scales: a 16-byte record per (cell, column) instead of 4 fp16 scales:
//     Q4_K: [d | dmin << 16, sc0 mn0 sc1 mn1, sc2 mn2 sc3 mn3, 0] (fp16 bits,
//           then the cell's four 6-bit scale/min pairs as bytes);
//     Q6_K: [d, s0 s0' s1 s1', s2 s2' s3 s3', 0] (int8 scales of the low and
//           high 16 values of each block).
// ---------------------------------------------------------------------------

__host__ __device__ inline bool fold_ok(int f) { return f == 1 || f == 2 || f == 4 || f == 8; }
// block quads per k part
__host__ __device__ inline int fold_quads(int nb, int f) { return ((nb + f - 1) / f + 3) / 4; }

template <int DT> struct QFmt;
template <> struct QFmt<DT_Q4_0> { static constexpr int LANE_BYTES = 16, BLOCK_BYTES = 18; };
template <> struct QFmt<DT_Q5_0> { static constexpr int LANE_BYTES = 16, BLOCK_BYTES = 22; };
template <> struct QFmt<DT_Q8_0> { static constexpr int LANE_BYTES = 32, BLOCK_BYTES = 34; };
template <> struct QFmt<DT_Q4_K> { static constexpr int LANE_BYTES = 16, BLOCK_BYTES = 144; };
template <> struct QFmt<DT_Q6_K> { static constexpr int LANE_BYTES = 16, BLOCK_BYTES = 210; };

__host__ __device__ constexpr bool is_kquant(int dt) { return dt == DT_Q4_K || dt == DT_Q6_K; }
__host__ __device__ inline int lane_bytes_of(int dt) { return dt == DT_Q8_0 ? 32 : 16; }
// bytes of one GGUF block (a 256-value super-block for the K-quants)
__host__ __device__ inline int block_bytes_of(int dt)
{
    return dt == DT_Q4_0 ? 18 : dt == DT_Q5_0 ? 22 : dt == DT_Q8_0 ? 34 : dt == DT_Q4_K ? 144
         : dt == DT_Q6_K ? 210 : 0;
}
__host__ __device__ inline int block_values_of(int dt) { return is_kquant(dt) ? 256 : 32; }

// position (0..31) inside a block of element e for lane group g
__host__ __device__ inline int kmap(int dt, int g, int e)
{
    if (dt == DT_Q8_0) return 8 * g + e;
    const int sub[4] = {0, 2, 1, 3};
    return (e >= 4 ? 16 : 0) + 4 * g + sub[e & 3];
}

__device__ inline f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

__device__ inline f16x8 pack8(f16x2 a, f16x2 b, f16x2 c, f16x2 d)
{
    f16x4 lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
    f16x4 hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Codes -> exact small integers in f16.  0x6400 | n is the f16 value 1024+n
// for n < 1024, so OR-ing a nibble/byte under that exponent and subtracting
// the bias in packed f16 yields the signed code exactly.

// Q4_0: dword D holds 8 nibbles; the low/high nibble of each 16-bit half is
// placed under the exponent of 1024 (0x6400): 1024 + n, or 1024 + 16 n for
// the upper nibble (rescaled by the packed fma), then the bias 1024 + 8 is
// removed.  Element order [n@0, n@16, n@8, n@24, n@4, n@20, n@12, n@28]
// (bit positions in D), which is the kmap order.  All steps are exact.
__device__ inline uint32_t magic_1024()
{
    uint32_t m = 0x64006400u;
    asm("" : "+v"(m));   // in a VGPR so and-or fuses; not volatile, so one copy serves every decode
    return m;
}

__device__ inline f16x8 deq_q4(uint32_t D)
{
    const uint32_t m = magic_1024();
    const f16x2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const f16x2 bias16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const uint32_t Dh = D >> 8;
    const uint32_t p0 = (D & 0x000F000Fu) | m;
    const uint32_t p1 = (Dh & 0x000F000Fu) | m;
    const uint32_t p2 = (D & 0x00F000F0u) | m;
    const uint32_t p3 = (Dh & 0x00F000F0u) | m;
    return pack8(as_h2(p0) + bias, as_h2(p1) + bias, as_h2(p2) * s16 + bias16,
                 as_h2(p3) * s16 + bias16);
}

// Q5_0: nibbles as Q4_0 plus fifth bits; hb = the lane's byte for this block
// (bit p: low element of pair p, bit 4+p: high element of pair p).
// value = (nibble | fifth << 4) - 16.
__device__ inline f16x8 deq_q5(uint32_t D, uint32_t hb)
{
    const uint32_t m = magic_1024();
    const f16x2 bias = {(_Float16)-1040.0f, (_Float16)-1040.0f};
    const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const f16x2 bias16 = {(_Float16)-80.0f, (_Float16)-80.0f};
    const uint32_t hs = ((hb & 0x0Fu) << 4) | ((hb & 0xF0u) << 16);
    const uint32_t Dh = D >> 8;
    const uint32_t p0 = (D & 0x000F000Fu) | m | (hs & 0x00100010u);
    const uint32_t p1 = (Dh & 0x000F000Fu) | m | ((hs >> 1) & 0x00100010u);
    const uint32_t p2 = (D & 0x00F000F0u) | m | ((hs << 2) & 0x01000100u);
    const uint32_t p3 = (Dh & 0x00F000F0u) | m | ((hs << 1) & 0x01000100u);
    return pack8(as_h2(p0) + bias, as_h2(p1) + bias, as_h2(p2) * s16 + bias16,
                 as_h2(p3) * s16 + bias16);
}

// Q6_K: nibbles as Q4_0 plus two high bits per code; hq = the lane's 16
// bits for this block (see the layout notes).  value = (nibble | hi << 4) - 32;
// 1024 + 16 * 63 < 2048 keeps the upper-nibble halves exact.
__device__ inline f16x8 deq_q6(uint32_t D, uint32_t hq)
{
    const uint32_t m = magic_1024();
    const f16x2 bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const f16x2 bias16 = {(_Float16)-96.0f, (_Float16)-96.0f};
    const uint32_t x = (hq & 0xFFu) | ((hq & 0xFF00u) << 8);
    const uint32_t Dh = D >> 8;
    const uint32_t p0 = (D & 0x000F000Fu) | m | ((x << 4) & 0x00300030u);
    const uint32_t p1 = (Dh & 0x000F000Fu) | m | ((x << 2) & 0x00300030u);
    const uint32_t p2 = (D & 0x00F000F0u) | m | ((x << 4) & 0x03000300u);
    const uint32_t p3 = (Dh & 0x00F000F0u) | m | ((x << 2) & 0x03000300u);
    return pack8(as_h2(p0) + bias, as_h2(p1) + bias, as_h2(p2) * s16 + bias16,
                 as_h2(p3) * s16 + bias16);
}

// Q8_0: two dwords of int8 codes; flip the sign bit (b+128 in 0..255),
// place each byte under the 0x64 exponent byte, subtract 1152.
__device__ inline f16x8 deq_q8(uint32_t D0, uint32_t D1)
{
    const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    D0 ^= 0x80808080u;
    D1 ^= 0x80808080u;
    uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, D0, 0x04010400u);
    uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, D0, 0x04030402u);
    uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, D1, 0x04010400u);
    uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, D1, 0x04030402u);
    return pack8(as_h2(p0) + bias, as_h2(p1) + bias, as_h2(p2) + bias, as_h2(p3) + bias);
}

// Decoded codes of block bi (0..3) of a quad from a lane's loaded data (h:
// Q5_0 fifth bits; Q6_K high bits of blocks 0,1 (c1[0]) and 2,3 (c1[1])).
template <int DT>
__device__ inline f16x8 deq_block(const u32x4 c0, const u32x4 c1, uint32_t h, int bi)
{
    if constexpr (DT == DT_Q4_0 || DT == DT_Q4_K) {
        return deq_q4(c0[bi]);
    } else if constexpr (DT == DT_Q6_K) {
        return deq_q6(c0[bi], (c1[bi >> 1] >> (16 * (bi & 1))) & 0xFFFFu);
    } else if constexpr (DT == DT_Q5_0) {
        return deq_q5(c0[bi], (h >> (8 * bi)) & 0xFFu);
    } else {
        uint32_t a = bi < 2 ? c0[2 * bi] : c1[2 * bi - 4];
        uint32_t b = bi < 2 ? c0[2 * bi + 1] : c1[2 * bi - 3];
        return deq_q8(a, b);
    }
}

// IEEE half -> float, exact, from bits (NaN payload moved as mantissa<<13).
__device__ inline float f16_bits_to_f32(uint32_t h)
{
    uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu, bits;
    if (e == 31u) bits = sign | 0x7F800000u | (f << 13);
    else if (e) bits = sign | ((e + 112u) << 23) | (f << 13);
    else if (!f) bits = sign;
    else {
        int lead = 31 - __builtin_clz(f);
        bits = sign | ((uint32_t)(lead + 103) << 23) | (((f << (10 - lead)) & 0x3FFu) << 13);
    }
    return __uint_as_float(bits);
}

// d * q with the result an x86 SSE multiply gives for special scales:
// NaN scale -> the quieted NaN itself; inf * 0 -> the x86 default NaN.
__device__ inline float mul_scale_x86(float d, float q)
{
    uint32_t db = __float_as_uint(d);
    if ((db & 0x7F800000u) == 0x7F800000u) {
        if (db & 0x007FFFFFu) return __uint_as_float(db | 0x00400000u);
        if (q == 0.0f) return __uint_as_float(0xFFC00000u);
    }
    return d * q;
}

// x86 SSE multiply / subtract (first operand a): a NaN operand comes out
// quieted, a's before b's; an invalid operation (inf * 0, inf - inf) gives
// the default NaN 0xFFC00000.  Used where the reference's dequantised values
// are matched bit for bit, special scales included.
__device__ inline bool nan_bits(float a) { return (__float_as_uint(a) & 0x7FFFFFFFu) > 0x7F800000u; }
__device__ inline float quieted(float a) { return __uint_as_float(__float_as_uint(a) | 0x00400000u); }
__device__ inline bool inf_bits(float a) { return (__float_as_uint(a) & 0x7FFFFFFFu) == 0x7F800000u; }

__device__ inline float mul_x86(float a, float b)
{
#pragma clang fp contract(off)
    if (nan_bits(a)) return quieted(a);
    if (nan_bits(b)) return quieted(b);
    if ((inf_bits(a) && b == 0.0f) || (inf_bits(b) && a == 0.0f)) return __uint_as_float(0xFFC00000u);
    return a * b;
}

__device__ inline float sub_x86(float a, float b)
{
#pragma clang fp contract(off)
    if (nan_bits(a)) return quieted(a);
    if (nan_bits(b)) return quieted(b);
    if (inf_bits(a) && inf_bits(b) && ((__float_as_uint(a) ^ __float_as_uint(b)) & 0x80000000u) == 0)
        return __uint_as_float(0xFFC00000u);
    return a - b;
}

// ---- reductions ------------------------------------------------------------
__device__ inline float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Orderable 64-bit key: larger float wins, ties go to the smaller index,
// NaN never wins.
__device__ inline unsigned long long argmax_key(float v, uint32_t idx)
{
    uint32_t u = __float_as_uint(v);
    uint32_t k = (v != v) ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    return ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__host__ __device__ inline uint32_t argmax_index(unsigned long long key)
{
    return 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull);
}
