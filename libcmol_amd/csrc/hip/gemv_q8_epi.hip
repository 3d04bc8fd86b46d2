// gemv_q8_epi.hip — the one-group matvec kernels for Q8_0 weights with
// the epilogue fixed at compile time (single-session decode).
#define GEMV_EPI_TU
#include "gemv_impl.h"

template int launch_gemv_epi<DT_Q8_0, 1>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q8_0, 2>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q8_0, 4>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
template int launch_gemv_epi<DT_Q8_0, 8>(const GemvArgs &, const GemvShape &, int, int, hipStream_t);
