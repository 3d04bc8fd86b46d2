// gemv_q4k.hip — matvec kernels for Q4_K weights.
#include "gemv_impl.h"

int launch_gemv_q4k(const GemvArgs &a, int epi, hipStream_t s) { return launch_ng<DT_Q4_K>(a, epi, s); }
