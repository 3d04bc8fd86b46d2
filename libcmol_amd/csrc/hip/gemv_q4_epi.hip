// gemv_q4_epi.hip — the one-group matvec kernels for Q4_0 weights with
// the epilogue fixed at compile time (single-session decode).
#define GEMV_EPI_TU
#include "gemv_impl.h"

template int launch_gemv_epi<DT_Q4_0, 1>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q4_0, 2>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q4_0, 4>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q4_0, 8>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q4_0, 16>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
