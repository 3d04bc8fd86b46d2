// gemv_q5.hip — matvec kernels for Q5_0 weights.
#include "gemv_impl.h"

int launch_gemv_q5(const GemvArgs &a, int epi, hipStream_t s) { return launch_ng<DT_Q5_0>(a, epi, s); }
