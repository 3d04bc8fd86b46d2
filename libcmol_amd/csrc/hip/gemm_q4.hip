// gemm_q4.hip — prompt GEMM kernels for Q4_0 weights.
#include "gemm_impl.h"

int launch_gemm_q4(const GemvArgs &a, int epi, hipStream_t s) { return launch_gemm_dt<DT_Q4_0>(a, epi, s); }
