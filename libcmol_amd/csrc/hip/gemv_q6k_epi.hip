// gemv_q6k_epi.hip — the one-group matvec kernels for Q6_K weights with
// the epilogue fixed at compile time (single-session decode).
#define GEMV_EPI_TU
#include "gemv_impl.h"

template int launch_gemv_epi<DT_Q6_K, 1>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q6_K, 2>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q6_K, 4>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q6_K, 8>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
