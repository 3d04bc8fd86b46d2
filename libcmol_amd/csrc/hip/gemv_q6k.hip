// gemv_q6k.hip — matvec kernels for Q6_K weights.
#include "gemv_impl.h"

int launch_gemv_q6k(const GemvArgs &a, int epi, hipStream_t s) { return launch_ng<DT_Q6_K>(a, epi, s); }
