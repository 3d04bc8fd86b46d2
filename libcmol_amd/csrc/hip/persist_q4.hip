// persist_q4.hip — the persistent decode kernel for Q4_0 layer weights.
#include "persist_impl.h"

int launch_persist_q4(const PkArgs &a, int nwg, int lds, hipStream_t s) { return launch_persist_dl<DT_Q4_0>(a, nwg, lds, s); }
int persist_capacity_q4(int d_head, int kv_f16, int lds) { return persist_capacity_dl<DT_Q4_0>(d_head, kv_f16, lds); }
