// gemv_q8.hip — matvec kernels for Q8_0 weights.
#include "gemv_impl.h"

int launch_gemv_q8(const GemvArgs &a, int epi, hipStream_t s) { return launch_ng<DT_Q8_0>(a, epi, s); }
