// gemm_q6k.hip — prompt GEMM kernels for Q6_K weights.
#include "gemm_impl.h"

int launch_gemm_q6k(const GemvArgs &a, int epi, hipStream_t s) { return launch_gemm_dt<DT_Q6_K>(a, epi, s); }
