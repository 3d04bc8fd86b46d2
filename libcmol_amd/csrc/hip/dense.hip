// dense.hip — the kernel seam's F32 and F16 weight products
// (src/quant.c:351-360 scalar, :506-530 AVX-512): out[m][n] = A[m][k] . B
// with A's rows as stored and B given transposed, x[n][k].  Each output
// follows the reference's AVX-512 kernel operation for operation, so the
// results are the CPU kernel's bit for bit:
//   * F32: sixteen accumulators, accumulator j taking k = 16c + j with a
//     fused multiply-add in c order; the horizontal sum in the order of
//     _mm512_reduce_add_ps (upper 256 bits onto the lower, then 128, then
//     lanes {2,3} onto {0,1}, then lane 1 onto lane 0); the k % 16 tail
//     added after it, each product rounded before its add;
//   * F16: one running sum over k in order, each product rounded before its
//     add (the reference's F16 branch is sequential in both kernels).
// A sixteen-lane group of a wave computes one F32 output (four per wave);
// an F16 output is one lane's sequential loop.  Throughput is not the
// point of this path: none of the model configurations has F16 or F32
// projection weights, and the model loader refuses them.
#include "common.h"
#include "kernels.h"

__global__ __launch_bounds__(256) void k_dense_f32(const float *a, const float *x, float *out, int m, int k, int n)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, j = lane & 15;
    const long o = ((long)blockIdx.x * 256 + threadIdx.x) / 16;   // output m * n + ni
    const bool act = o < (long)m * n;
    const int mi = act ? (int)(o / n) : 0, ni = act ? (int)(o % n) : 0;
    const float *ar = a + (size_t)mi * k, *xr = x + (size_t)ni * k;
    const int kc = k / 16;
    float acc = 0.0f;
    for (int c = 0; c < kc; c++) acc = fmaf(ar[16 * c + j], xr[16 * c + j], acc);
    // _mm512_reduce_add_ps: t8[i] = a[8+i] + a[i], t4[i] = t8[4+i] + t8[i],
    // then (t4[0] + t4[2]) + (t4[1] + t4[3]); lanes of the group hold a[j]
    const float t8 = __shfl_down(acc, 8, 16) + acc;   // valid in j < 8
    const float t4 = __shfl_down(t8, 4, 16) + t8;     // valid in j < 4
    const float u = __shfl_down(t4, 2, 16) + t4;      // j = 0: t4[2] + t4[0]; j = 1: t4[3] + t4[1]
    float t = __shfl_down(u, 1, 16) + u;              // j = 0: u1 + u0
    if (j == 0 && act) {
        for (int ki = 16 * kc; ki < k; ki++) {
            const float p = ar[ki] * xr[ki];
            t = t + p;
        }
        out[o] = t;
    }
}

__global__ __launch_bounds__(256) void k_dense_f16(const uint16_t *a, const float *x, float *out, int m, int k, int n)
{
#pragma clang fp contract(off)
    const long o = (long)blockIdx.x * 256 + threadIdx.x;
    if (o >= (long)m * n) return;
    const int mi = (int)(o / n), ni = (int)(o % n);
    const uint16_t *ar = a + (size_t)mi * k;
    const float *xr = x + (size_t)ni * k;
    float s = 0.0f;
    for (int ki = 0; ki < k; ki++) {
        const float p = (float)__builtin_bit_cast(_Float16, ar[ki]) * xr[ki];
        s = s + p;
    }
    out[o] = s;
}

int launch_matmul_dense(const void *a, int dtype, const float *x, float *out, int m, int k, int n, hipStream_t s)
{
    if (m < 1 || k < 1 || n < 1 || (dtype != 0 && dtype != 1)) return -6;
    const long outs = (long)m * n;
    if (dtype == 0) {
        const long blocks = (outs * 16 + 255) / 256;
        if (blocks > 0x7fffffffL) return -6;
        hipLaunchKernelGGL(k_dense_f32, dim3((unsigned)blocks), dim3(256), 0, s, (const float *)a, x, out, m, k, n);
    } else {
        const long blocks = (outs + 255) / 256;
        if (blocks > 0x7fffffffL) return -6;
        hipLaunchKernelGGL(k_dense_f16, dim3((unsigned)blocks), dim3(256), 0, s, (const uint16_t *)a, x, out, m, k,
                           n);
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
