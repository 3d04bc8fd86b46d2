// attn.hip — the decode attention kernels over the work-group functions of
// attn_impl.h: one work-group of ATT_THREADS per (kv head, split, vector),
// then one per (query head, vector) to merge the splits.
#include "attn_impl.h"

#define ATT_THREADS 256
// Positions per chunk of a 256-thread work-group (a split is a multiple).
#define ATT_CHUNK (ATT_THREADS / 4)

template <int DH, typename KT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a)
{
    attn_split<DH, KT, ATT_THREADS, StPlain>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_merge(AttnArgs a)
{
    attn_merge_head<DH, ATT_THREADS, StPlain>(a, blockIdx.x, blockIdx.y);
}

int attn_max_splits(int max_ctx, int split) { return (max_ctx + split - 1) / split; }

int launch_attn(const AttnArgs &a, hipStream_t s)
{
    const int G = a.n_heads / a.n_kv;
    if (G < 1 || G > ATT_MAX_G || a.n_heads % a.n_kv || a.split < 1 || a.split % ATT_CHUNK)
        return -4;
    if (a.max_splits > ATT_MAX_MERGE) return -4;
    dim3 grid(a.n_kv, a.max_splits, a.n), block(ATT_THREADS), mgrid(a.n_heads, a.n);
#define ATT(DHV)                                                                          \
    if (a.kv_f16) hipLaunchKernelGGL((k_attn<DHV, _Float16>), grid, block, 0, s, a);      \
    else hipLaunchKernelGGL((k_attn<DHV, float>), grid, block, 0, s, a);                  \
    if (a.max_splits > 1) hipLaunchKernelGGL((k_attn_merge<DHV>), mgrid, block, 0, s, a);
    switch (a.d_head) {
    case 16: ATT(16); break;
    case 32: ATT(32); break;
    case 64: ATT(64); break;
    case 128: ATT(128); break;
    case 256: ATT(256); break;
    default: return -4;
    }
#undef ATT
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
