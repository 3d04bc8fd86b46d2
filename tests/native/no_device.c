/*
 * no_device.c — the device entry points the host code calls, answered as a
 * machine without a usable GPU answers them (CMOL_ERR_UNSUPPORTED), so the
 * C host of libcmol (parser, tokenizer, sampler, scheduler, pool, load error
 * paths) can be built alone under the sanitizers.  Test infrastructure only:
 * linked into tests/native/host_check, never into libcmol.so.
 */
#include <stddef.h>
#include <stdint.h>

#include "../../include/cmol_hip.h"

#define NODEV (-4) /* CMOL_ERR_UNSUPPORTED */

size_t cmolhip_arena_size(const cmolhip_ctx_t *c) { (void)c; return 0; }
cmolhip_ctx_t *cmolhip_model_ctx(cmolhip_model_t *m) { (void)m; return NULL; }
void cmolhip_model_destroy(cmolhip_model_t *m) { (void)m; }

int cmolhip_model_plan(const cmolhip_model_desc_t *d, size_t *bytes)
{
    (void)d;
    if (bytes) *bytes = 0;
    return NODEV;
}

int cmolhip_model_create(const cmolhip_model_desc_t *d, int dev, cmolhip_model_t **out)
{
    (void)d; (void)dev;
    if (out) *out = NULL;
    return NODEV;
}

int cmolhip_decode(cmolhip_model_t *m, int slot, int32_t tok, int32_t pos, float *lg, int32_t *am)
{
    (void)m; (void)slot; (void)tok; (void)pos; (void)lg; (void)am;
    return NODEV;
}

int cmolhip_decode_batch(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *toks,
                         const int32_t *pos, float *lg, int32_t *am)
{
    (void)m; (void)n; (void)slots; (void)toks; (void)pos; (void)lg; (void)am;
    return NODEV;
}

int cmolhip_decode_batch_each(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *toks,
                              const int32_t *pos, float *const *lg, int32_t *am)
{
    (void)m; (void)n; (void)slots; (void)toks; (void)pos; (void)lg; (void)am;
    return NODEV;
}

int cmolhip_prefill(cmolhip_model_t *m, int slot, const int32_t *toks, int n, int32_t pos0, float *lg,
                    int32_t *am)
{
    (void)m; (void)slot; (void)toks; (void)n; (void)pos0; (void)lg; (void)am;
    return NODEV;
}

int cmolhip_kv_fill_synthetic(cmolhip_model_t *m, int slot, int n, uint64_t seed)
{
    (void)m; (void)slot; (void)n; (void)seed;
    return NODEV;
}
