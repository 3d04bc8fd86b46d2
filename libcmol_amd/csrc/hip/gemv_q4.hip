// gemv_q4.hip — matvec kernels for Q4_0 weights.
#include "gemv_impl.h"

int launch_gemv_q4(const GemvArgs &a, int epi, hipStream_t s) { return launch_ng<DT_Q4_0>(a, epi, s); }
