// gemm_q4k.hip — prompt GEMM kernels for Q4_K weights.
#include "gemm_impl.h"

int launch_gemm_q4k(const GemvArgs &a, int epi, hipStream_t s) { return launch_gemm_dt<DT_Q4_K>(a, epi, s); }
