// misc.hip — fills and KV-cache conversions used by load, tests and benches.
#include "common.h"
#include "kernels.h"

__device__ inline uint64_t mix64d(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Synthetic cache contents ~U(-1,1) for positions [0, n) of one layer slice
// [n_kv][max_ctx][d_head]; layers are handled by the caller's loop.
__global__ void k_kv_synth(void *kc, void *vc, int n_kv, int max_ctx, int d_head,
                           int n, int kv_f16, uint64_t seed)
{
    size_t total = (size_t)n_kv * n * d_head;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        int dd = (int)(i % d_head);
        size_t r = i / d_head;
        int pos = (int)(r % n), h = (int)(r / n);
        size_t idx = ((size_t)h * max_ctx + pos) * d_head + dd;
        uint64_t z = mix64d(seed ^ mix64d(idx));
        float a = (float)(int32_t)(z & 0xFFFFFF) * (1.0f / 8388608.0f) - 1.0f;
        float b = (float)(int32_t)((z >> 32) & 0xFFFFFF) * (1.0f / 8388608.0f) - 1.0f;
        if (kv_f16) {
            ((_Float16 *)kc)[idx] = (_Float16)a;
            ((_Float16 *)vc)[idx] = (_Float16)b;
        } else {
            ((float *)kc)[idx] = a;
            ((float *)vc)[idx] = b;
        }
    }
}

int launch_kv_synth(void *kc, void *vc, int n_kv, int max_ctx, int d_head,
                    int n_tokens, int kv_f16, uint64_t seed, hipStream_t s)
{
    size_t total = (size_t)n_kv * n_tokens * d_head;
    if (!total) return 0;
    unsigned grid = (unsigned)((total + 255) / 256);
    if (grid > 65535u * 4u) grid = 65535u * 4u;
    hipLaunchKernelGGL(k_kv_synth, dim3(grid), dim3(256), 0, s, kc, vc, n_kv, max_ctx,
                       d_head, n_tokens, kv_f16, seed);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Device cache slice [n_kv][max_ctx][d_head] -> reference layout
// [pos][n_kv][d_head] fp32 for positions [0, n).
__global__ void k_kv_to_ref(const void *src, float *dst, int n_kv, int max_ctx, int d_head,
                            int n, int kv_f16)
{
    size_t total = (size_t)n * n_kv * d_head;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        int dd = (int)(i % d_head);
        size_t r = i / d_head;
        int h = (int)(r % n_kv), pos = (int)(r / n_kv);
        size_t sidx = ((size_t)h * max_ctx + pos) * d_head + dd;
        dst[i] = kv_f16 ? (float)((const _Float16 *)src)[sidx] : ((const float *)src)[sidx];
    }
}

__global__ void k_kv_from_ref(const float *src, void *dst, int n_kv, int max_ctx, int d_head,
                              int n, int kv_f16)
{
    size_t total = (size_t)n * n_kv * d_head;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        int dd = (int)(i % d_head);
        size_t r = i / d_head;
        int h = (int)(r % n_kv), pos = (int)(r / n_kv);
        size_t didx = ((size_t)h * max_ctx + pos) * d_head + dd;
        if (kv_f16) ((_Float16 *)dst)[didx] = (_Float16)src[i];
        else ((float *)dst)[didx] = src[i];
    }
}

int launch_kv_convert(const void *src, float *dst, int n_kv, int max_ctx, int d_head,
                      int n, int kv_f16, int to_ref, hipStream_t s)
{
    (void)to_ref;
    size_t total = (size_t)n * n_kv * d_head;
    if (!total) return 0;
    unsigned grid = (unsigned)((total + 255) / 256);
    if (grid > 65535u * 4u) grid = 65535u * 4u;
    hipLaunchKernelGGL(k_kv_to_ref, dim3(grid), dim3(256), 0, s, src, dst, n_kv, max_ctx,
                       d_head, n, kv_f16);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_kv_import(const float *src, void *dst, int n_kv, int max_ctx, int d_head, int n,
                     int kv_f16, hipStream_t s)
{
    size_t total = (size_t)n * n_kv * d_head;
    if (!total) return 0;
    unsigned grid = (unsigned)((total + 255) / 256);
    if (grid > 65535u * 4u) grid = 65535u * 4u;
    hipLaunchKernelGGL(k_kv_from_ref, dim3(grid), dim3(256), 0, s, src, dst, n_kv, max_ctx,
                       d_head, n, kv_f16);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Operand rows of vector v of an n-vector operand (K inputs) -> a one-vector
// operand, plus that vector's sum-of-squares partials.
__global__ void k_act_extract(const _Float16 *src, int K, int n, int v, _Float16 *dst,
                              const float *ss_src, int ss_stride, int ss_count, float *ss_dst)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;   // (block, group) segment
    const int segs = (K / 32) * 4;
    if (i < segs) {
        const uint4 *s = (const uint4 *)(src + ((size_t)i * 2 * n + 2 * v) * 8);
        uint4 *d = (uint4 *)(dst + (size_t)i * 2 * 8);
        d[0] = s[0];
        d[1] = s[1];
    }
    if (ss_src && i < ss_count) ss_dst[i] = ss_src[(size_t)v * ss_stride + i];
}

int launch_act_extract(const _Float16 *src, int K, int n, int v, _Float16 *dst, const float *ss_src,
                       int ss_stride, int ss_count, float *ss_dst, hipStream_t s)
{
    const int segs = (K / 32) * 4;
    const int work = segs > ss_count ? segs : ss_count;
    hipLaunchKernelGGL(k_act_extract, dim3((work + 255) / 256), dim3(256), 0, s, src, K, n, v, dst,
                       ss_src, ss_stride, ss_count, ss_dst);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// dst[c][r] = src[r][c] for a rows x cols fp32 matrix (the host seam's
// k-major activations and [m][n] outputs against the matvec's [n][k]).
__global__ void k_transpose(const float *__restrict__ src, float *__restrict__ dst, int rows, int cols)
{
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) t[i][tx] = src[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[(size_t)c * rows + r] = t[tx][i];
    }
}

int launch_transpose(const float *src, float *dst, int rows, int cols, hipStream_t s)
{
    if (rows < 1 || cols < 1) return 0;
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, s, src, dst, rows, cols);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// out[i] = i for i < n.
__global__ void k_iota(int32_t *out, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = i;
}

int launch_iota(int32_t *out, int n, hipStream_t s)
{
    if (n < 1) return 0;
    hipLaunchKernelGGL(k_iota, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
