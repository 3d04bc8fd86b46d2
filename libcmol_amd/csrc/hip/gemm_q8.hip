// gemm_q8.hip — prompt GEMM kernels for Q8_0 weights.
#include "gemm_impl.h"

int launch_gemm_q8(const GemvArgs &a, int epi, hipStream_t s) { return launch_gemm_dt<DT_Q8_0>(a, epi, s); }
