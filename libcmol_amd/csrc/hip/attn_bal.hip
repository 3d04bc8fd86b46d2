// attn_bal.hip — decode attention over balanced ranges for lock-step
// sessions over an fp16 cache (attn_bal_mf in attn_impl.h), and its merge;
// a translation unit of its own, so the split-grid kernels' code object is
// unchanged by it.
#include "attn_impl.h"

#include <algorithm>

#define BAL_THREADS 256

// four waves per piece, each on its own positions; held to four
// work-groups per CU at d_head <= 128 (the grid is sized for that many)
template <int DH>
__global__ __launch_bounds__(BAL_THREADS) __attribute__((amdgpu_waves_per_eu(DH <= 128 ? 4 : 1)))
void k_attn_bal(AttnArgs a)
{
    attn_bal_mf<DH, StPlain>(a, blockIdx.x, blockIdx.y);
}

template <int DH>
__global__ __launch_bounds__(BAL_THREADS) void k_attn_merge_bal(AttnArgs a)
{
    attn_merge_bal<DH, BAL_THREADS, StPlain>(a, blockIdx.x, blockIdx.y);
}

static int bal_cus()
{
    static const int c = [] {
        int d = 0, n = 0;
        if (hipGetDevice(&d) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess ||
            n < 1) {
            (void)hipGetLastError();
            n = 256;
        }
        return n;
    }();
    return c;
}

int attn_bal_wgs(int n, int n_kv, int d_head, int kv_f16, int max_splits)
{
    if (n < 2 || !kv_f16 || (d_head != 64 && d_head != 128 && d_head != 256) || max_splits < 2 ||
        max_splits + 1 > ATT_MAX_MERGE)
        return 0;
    const char *e = getenv("CMOL_ATTN_BAL");
    const long t = e ? atol(e) : (long)ATT_BAL_WGS_PER_CU * bal_cus();
    if (t <= 0) return 0;
    const long w = std::max(1L, t / n_kv - n), cap = (long)n * (max_splits - 1);
    return (int)std::min(w, cap);
}

int launch_attn_bal(const AttnArgs &a, hipStream_t s)
{
    // a piece count is at most one above the split count
    if (!a.kv_f16 || a.bal < 1 || a.max_splits + 1 > ATT_MAX_MERGE || (long)a.bal + a.n > (long)a.n * a.max_splits)
        return -4;
    const dim3 grid(a.n_kv, a.bal + a.n), mgrid(a.n_heads, a.n), block(BAL_THREADS);
    switch (a.d_head) {
    case 64:
        hipLaunchKernelGGL((k_attn_bal<64>), grid, block, 0, s, a);
        hipLaunchKernelGGL((k_attn_merge_bal<64>), mgrid, block, 0, s, a);
        break;
    case 128:
        hipLaunchKernelGGL((k_attn_bal<128>), grid, block, 0, s, a);
        hipLaunchKernelGGL((k_attn_merge_bal<128>), mgrid, block, 0, s, a);
        break;
    case 256:
        hipLaunchKernelGGL((k_attn_bal<256>), grid, block, 0, s, a);
        hipLaunchKernelGGL((k_attn_merge_bal<256>), mgrid, block, 0, s, a);
        break;
    default: return -4;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
