// gemm_q5.hip — prompt GEMM kernels for Q5_0 weights.
#include "gemm_impl.h"

int launch_gemm_q5(const GemvArgs &a, int epi, hipStream_t s) { return launch_gemm_dt<DT_Q5_0>(a, epi, s); }
