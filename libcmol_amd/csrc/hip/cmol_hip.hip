// cmol_hip.hip — C ABI of the gfx950 backend (include/cmol_hip.h).
//
// Owns the device context (one arena from one hipMalloc, one upload stream),
// quantised-tensor upload/repack, the standalone kernel entry points and the
// whole-model decode path: per-session streams and buffers, the per-session
// decode step captured once as a HIP graph at load, prefill, KV access.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <vector>

#include "../../../include/cmol_hip.h"
#include "common.h"
#include "kernels.h"

namespace {

constexpr int E_OK = 0, E_OOM = -1, E_INVALID = -3, E_UNSUPPORTED = -4, E_ARGS = -6, E_TRUNC = -8;
constexpr size_t ALIGN = 256;
// vectors per matvec/GEMM call (the operand preparation grid's y extent)
constexpr int GEMM_MAX_N = 65535;

int herr(hipError_t e)
{
    switch (e) {
    case hipSuccess: return E_OK;
    case hipErrorOutOfMemory: return E_OOM;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice:
    case hipErrorInsufficientDriver:
    case hipErrorNoBinaryForGpu: return E_UNSUPPORTED;
    default: return E_INVALID;
    }
}

#define HC(x)                                        \
    do {                                             \
        hipError_t e_ = (x);                         \
        if (e_ != hipSuccess) return herr(e_);       \
    } while (0)
#define RC(x)                                        \
    do {                                             \
        int r_ = (x);                                \
        if (r_ != 0) return r_;                      \
    } while (0)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct QLayout {
    size_t qs, d, qh;
    int rt, bq;
};

// Byte sizes of the tiled arrays: codes, scales (4 fp16 per column per cell,
// or a 16-byte record per column per cell for the K-quants), and the Q5_0
// fifth bits / Q6_K high bits.
bool qlayout(int dtype, int rows, int cols, int fold, QLayout *L)
{
    if (dtype != DT_Q4_0 && dtype != DT_Q5_0 && dtype != DT_Q8_0 && !is_kquant(dtype)) return false;
    if (rows <= 0 || cols <= 0 || cols % block_values_of(dtype) || !fold_ok(fold)) return false;
    const int R = 16 / fold;
    L->rt = (rows + R - 1) / R;
    L->bq = fold_quads(cols / 32, fold);
    size_t cells = (size_t)L->rt * L->bq;
    L->qs = cells * 64 * lane_bytes_of(dtype);
    L->d = is_kquant(dtype) ? cells * 16 * 16 : cells * 64 * 2;
    L->qh = dtype == DT_Q5_0 ? cells * 64 * 4 : dtype == DT_Q6_K ? cells * 64 * 8 : 0;
    return true;
}

size_t qbytes_aligned(int dtype, int rows, int cols, int fold)
{
    QLayout L;
    if (!qlayout(dtype, rows, cols, fold, &L)) return 0;
    return align_up(L.qs, ALIGN) + align_up(L.d, ALIGN) + align_up(L.qh, ALIGN);
}

QTensor to_qt(const cmolhip_qtensor_t &t)
{
    QTensor q;
    q.qs = (uint8_t *)t.qs;
    q.d = (uint16_t *)t.d;
    q.qh = (uint32_t *)t.qh;
    q.dtype = t.dtype;
    q.rows = t.rows;
    q.cols = t.cols;
    q.row_tiles = t.row_tiles;
    q.block_quads = t.block_quads;
    q.fold = t.fold;
    return q;
}

size_t raw_row_bytes(int dtype, int cols)
{
    int bb = block_bytes_of(dtype);
    return bb ? (size_t)(cols / block_values_of(dtype)) * bb : 0;
}

} // namespace

struct cmolhip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint8_t *arena = nullptr;
    size_t size = 0, used = 0;
    std::mutex mu;
};

// Scratch of the allocation-free entry point (cmolhip_gemm_noalloc): one
// array per device, in the code object, held until the process ends.  Host
// code never passes `scratch` itself (on the host the name is only a
// stand-in): each device's address is looked up once, with that device
// current, by resolve_scratch and kept in scratch_addr.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
constexpr int SCRATCH_MAX_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static uint8_t *scratch_addr[SCRATCH_MAX_DEVICES];
static std::mutex scratch_mu;

// Device address of `scratch` on `device` (current); nullptr on failure.
static uint8_t *resolve_scratch(int device)
{
    if (device < 0 || device >= SCRATCH_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> g(scratch_mu);
    if (!scratch_addr[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        scratch_addr[device] = (uint8_t *)ptr;
    }
    return scratch_addr[device];
}

static size_t arena_mark(cmolhip_ctx_t *c)
{
    std::lock_guard<std::mutex> g(c->mu);
    return c->used;
}
static void arena_release(cmolhip_ctx_t *c, size_t mark)
{
    std::lock_guard<std::mutex> g(c->mu);
    if (mark <= c->used) c->used = mark;
}
template <typename T>
static int arena_get(cmolhip_ctx_t *c, size_t count, T **p)
{
    return cmolhip_alloc(c, count * sizeof(T), ALIGN, (void **)p);
}

extern "C" {

int cmolhip_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int cmolhip_ctx_create(int device, size_t bytes, cmolhip_ctx_t **out)
{
    if (!out) return E_ARGS;
    *out = nullptr;
    int n = cmolhip_device_count();
    if (n <= 0 || device < 0 || device >= n) return E_UNSUPPORTED;
    HC(hipSetDevice(device));
    cmolhip_ctx_t *c = new (std::nothrow) cmolhip_ctx_t();
    if (!c) return E_OOM;
    c->device = device;
    if (!resolve_scratch(device)) {   // once per device, this device current
        delete c;
        return E_UNSUPPORTED;
    }
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return E_UNSUPPORTED;
    }
    if (bytes) {
        if (hipMalloc((void **)&c->arena, bytes) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipStreamDestroy(c->stream);
            delete c;
            return E_OOM;
        }
    }
    c->size = bytes;
    *out = c;
    return E_OK;
}

void cmolhip_ctx_destroy(cmolhip_ctx_t *c)
{
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamDestroy(c->stream);
    }
    if (c->arena) (void)hipFree(c->arena);
    delete c;
}

int cmolhip_alloc(cmolhip_ctx_t *c, size_t bytes, size_t align, void **dptr)
{
    if (!c || !dptr || (align & (align - 1))) return E_ARGS;
    if (align < ALIGN) align = ALIGN;
    std::lock_guard<std::mutex> g(c->mu);
    size_t start = align_up(c->used, align);
    if (start > c->size || bytes > c->size - start) return E_OOM;
    *dptr = c->arena + start;
    c->used = start + bytes;
    return E_OK;
}

size_t cmolhip_arena_used(const cmolhip_ctx_t *c) { return c ? c->used : 0; }
size_t cmolhip_arena_size(const cmolhip_ctx_t *c) { return c ? c->size : 0; }

int cmolhip_memcpy_h2d(cmolhip_ctx_t *c, void *dst, const void *src, size_t n)
{
    if (!c || (!dst && n) || (!src && n)) return E_ARGS;
    HC(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
    HC(hipStreamSynchronize(c->stream));
    return E_OK;
}

int cmolhip_memcpy_d2h(cmolhip_ctx_t *c, void *dst, const void *src, size_t n)
{
    if (!c || (!dst && n) || (!src && n)) return E_ARGS;
    HC(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
    HC(hipStreamSynchronize(c->stream));
    return E_OK;
}

int cmolhip_memcpy_d2d(cmolhip_ctx_t *c, void *dst, const void *src, size_t n)
{
    if (!c || (!dst && n) || (!src && n)) return E_ARGS;
    HC(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, c->stream));
    return E_OK;
}

int cmolhip_synchronize(cmolhip_ctx_t *c)
{
    if (!c) return E_ARGS;
    HC(hipStreamSynchronize(c->stream));
    return E_OK;
}

void *cmolhip_stream(cmolhip_ctx_t *c) { return c ? (void *)c->stream : nullptr; }

size_t cmolhip_qtensor_bytes(int dtype, int rows, int cols, int fold)
{
    return qbytes_aligned(dtype, rows, cols, fold);
}

int cmolhip_qtensor_upload(cmolhip_ctx_t *c, int dtype, int cols, int fold, int n_parts,
                           const void *const *parts, const int32_t *part_rows, int mode,
                           void *staging, size_t staging_bytes, cmolhip_qtensor_t *out)
{
    if (!c || !parts || !part_rows || !out || n_parts < 1 || !staging) return E_ARGS;
    if (mode != CMOLHIP_PARTS_CONCAT && mode != CMOLHIP_PARTS_INTERLEAVE) return E_ARGS;
    if (mode == CMOLHIP_PARTS_INTERLEAVE && (n_parts != 2 || part_rows[0] != part_rows[1]))
        return E_ARGS;
    long rows = 0;
    for (int p = 0; p < n_parts; p++) {
        if (!parts[p] || part_rows[p] <= 0) return E_ARGS;
        rows += part_rows[p];
    }
    if (rows > (1L << 30)) return E_ARGS;
    QLayout L;
    if (!qlayout(dtype, (int)rows, cols, fold, &L)) return E_UNSUPPORTED;
    cmolhip_qtensor_t t{};
    RC(cmolhip_alloc(c, L.qs, ALIGN, &t.qs));
    RC(cmolhip_alloc(c, L.d, ALIGN, &t.d));
    if (L.qh) RC(cmolhip_alloc(c, L.qh, ALIGN, &t.qh));
    t.dtype = dtype;
    t.rows = (int)rows;
    t.cols = cols;
    t.row_tiles = L.rt;
    t.block_quads = L.bq;
    t.fold = fold;
    HC(hipMemsetAsync(t.qs, 0, L.qs, c->stream));
    HC(hipMemsetAsync(t.d, 0, L.d, c->stream));
    if (L.qh) HC(hipMemsetAsync(t.qh, 0, L.qh, c->stream));
    const QTensor q = to_qt(t);
    const size_t rb = raw_row_bytes(dtype, cols);
    const long chunk = (long)(staging_bytes / rb);
    if (chunk < 1) return E_OOM;
    long row0 = 0;
    for (int p = 0; p < n_parts; p++) {
        for (long r = 0; r < part_rows[p]; r += chunk) {
            long nr = part_rows[p] - r < chunk ? part_rows[p] - r : chunk;
            HC(hipMemcpyAsync(staging, (const uint8_t *)parts[p] + (size_t)r * rb, (size_t)nr * rb,
                              hipMemcpyHostToDevice, c->stream));
            int dst0 = mode == CMOLHIP_PARTS_CONCAT ? (int)(row0 + r) : (int)r;
            RC(launch_repack(q, (const uint8_t *)staging, (int)nr, dst0, mode, p, c->stream));
            HC(hipStreamSynchronize(c->stream));
        }
        row0 += part_rows[p];
    }
    *out = t;
    return E_OK;
}

int cmolhip_dequant(cmolhip_ctx_t *c, const cmolhip_qtensor_t *t, float *dout)
{
    if (!c || !t || !dout) return E_ARGS;
    RC(launch_dequant(to_qt(*t), dout, c->stream));
    HC(hipStreamSynchronize(c->stream));
    return E_OK;
}

size_t cmolhip_act_bytes(int cols, int n) { return (cols > 0 && n > 0) ? act_bytes(cols, n) : 0; }

int cmolhip_act_prepare(cmolhip_ctx_t *c, const float *dx, int n, int cols, int dtype,
                        const float *norm_w, void *op, float *ss)
{
    if (!c || !dx || !op || n < 1 || n > GEMM_MAX_N || cols < 32 || cols % 32) return E_ARGS;
    if (dtype != DT_Q4_0 && dtype != DT_Q5_0 && dtype != DT_Q8_0 && !is_kquant(dtype)) return E_UNSUPPORTED;
    ActOut o{};
    o.q = (_Float16 *)op;
    o.dt = dtype;
    o.nrows = 2 * n;
    o.norm_w = norm_w;
    o.ss = ss;
    o.ss_stride = cols / 32;
    return launch_act_prep(dx, cols, cols, n, o, c->stream);
}

int cmolhip_gemm_prepared(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const void *op, int n,
                          const float *ss, float eps, float *dy)
{
    return cmolhip_gemm_prepared_timed(c, w, op, n, ss, eps, dy, nullptr, nullptr);
}

} // extern "C"

// dy[n][rows] = W . op for a prepared operand: up to 32 vectors stream the
// weights once through the matvec (k-split partial sums in part, part_cap
// floats), more run the tiled MFMA GEMM.
static int launch_product(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const void *op, int n,
                          const float *ss, float eps, float *dy, float *part, size_t part_cap,
                          void *ev_start, void *ev_stop)
{
    GemvArgs a{};
    a.w = to_qt(*w);
    a.in.q = (const _Float16 *)op;
    a.in.nrows = 2 * n;
    a.in.ss = ss;
    a.in.ss_count = w->cols / 32;
    a.in.ss_stride = w->cols / 32;
    a.in.eps = eps;
    a.out = dy;
    a.out_stride = w->rows;
    a.n = n;
    a.ev_start = (hipEvent_t)ev_start;
    a.ev_stop = (hipEvent_t)ev_stop;
    a.part = part;
    a.part_cap = part_cap;
    return n <= 32 ? launch_gemv(a, EPI_STORE, c->stream) : launch_gemm(a, EPI_STORE, c->stream);
}

extern "C" {

int cmolhip_gemm_prepared_timed(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const void *op,
                                int n, const float *ss, float eps, float *dy, void *ev_start,
                                void *ev_stop)
{
    if (!c || !w || !op || !dy || n < 1 || n > GEMM_MAX_N || (!ev_start != !ev_stop)) return E_ARGS;
    // the arena space of k-split partial sums is released at once: later
    // work on this stream runs after the kernels
    const size_t mark = arena_mark(c);
    const size_t pf = n <= 32 ? gemv_part_floats(to_qt(*w), n) : gemm_part_floats(to_qt(*w), n);
    float *part = nullptr;
    int rc = pf ? arena_get(c, pf, &part) : E_OK;
    if (rc == E_OK) rc = launch_product(c, w, op, n, ss, eps, dy, part, pf, ev_start, ev_stop);
    arena_release(c, mark);
    return rc;
}

int cmolhip_gemm(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const float *dx, float *dy, int n,
                 const float *norm_w, float eps)
{
    if (!c || !w || !dx || !dy || n < 1 || n > GEMM_MAX_N) return E_ARGS;
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        void *op = nullptr;
        float *ss = nullptr;
        if ((rc = cmolhip_alloc(c, act_bytes(w->cols, n), ALIGN, &op))) break;
        if (norm_w && (rc = arena_get(c, (size_t)n * (w->cols / 32), &ss))) break;
        if ((rc = cmolhip_act_prepare(c, dx, n, w->cols, w->dtype, norm_w, op, ss))) break;
        rc = cmolhip_gemm_prepared(c, w, op, n, ss, eps, dy);
    } while (0);
    arena_release(c, mark);
    return rc;
}

size_t cmolhip_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

int cmolhip_gemm_noalloc(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const float *dx, float *dy, int n,
                         const float *norm_w, float eps)
{
    if (!c || !w || !dx || !dy || n < 1 || n > GEMM_MAX_N || w->cols < 32 || w->cols % 32) return E_ARGS;
    uint8_t *base = scratch_addr[c->device];   // resolved when c was created
    if (!base) return E_UNSUPPORTED;
    // scratch layout: operand | sum-of-squares partials | k-split partial sums
    const size_t op_b = align_up(act_bytes(w->cols, n), ALIGN);
    const size_t ss_b = norm_w ? align_up((size_t)n * (w->cols / 32) * 4, ALIGN) : 0;
    const size_t pf = n <= 32 ? gemv_part_floats(to_qt(*w), n) : gemm_part_floats(to_qt(*w), n);
    if (op_b + ss_b + pf * 4 > NOALLOC_SCRATCH_BYTES) return E_ARGS;   // beyond the fixed scratch
    float *ss = norm_w ? (float *)(base + op_b) : nullptr;
    float *part = pf ? (float *)(base + op_b + ss_b) : nullptr;
    RC(cmolhip_act_prepare(c, dx, n, w->cols, w->dtype, norm_w, base, ss));
    return launch_product(c, w, base, n, ss, eps, dy, part, pf, nullptr, nullptr);
}

// F32 / F16 weights: rows of k values, any k (src/quant.c:246-256)
static int matmul_dense_host(cmolhip_ctx_t *c, float *out, const void *a, const float *b, int m, int k, int n,
                             int dtype)
{
    const size_t esz = dtype == 0 ? 4 : 2;
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        void *da = nullptr;
        float *db = nullptr, *dx = nullptr, *dy = nullptr;
        if ((rc = cmolhip_alloc(c, esz * (size_t)m * k, ALIGN, &da))) break;
        if ((rc = arena_get(c, (size_t)k * n, &db))) break;
        if ((rc = arena_get(c, (size_t)k * n, &dx))) break;
        if ((rc = arena_get(c, (size_t)m * n, &dy))) break;
        if ((rc = cmolhip_memcpy_h2d(c, da, a, esz * (size_t)m * k))) break;
        if ((rc = cmolhip_memcpy_h2d(c, db, b, (size_t)k * n * 4))) break;
        if ((rc = launch_transpose(db, dx, k, n, c->stream))) break;
        if (launch_matmul_dense(da, dtype, dx, dy, m, k, n, c->stream)) {
            rc = E_ARGS;
            break;
        }
        if ((rc = cmolhip_memcpy_d2h(c, out, dy, (size_t)m * n * 4))) break;
    } while (0);
    arena_release(c, mark);
    return rc;
}

int cmolhip_matmul_host(cmolhip_ctx_t *c, float *out, const void *a, const float *b, int m, int k,
                        int n, int dtype)
{
    if ((dtype == 0 || dtype == 1) && c && out && a && b && m >= 1 && k >= 1 && n >= 1 && n <= GEMM_MAX_N)
        return matmul_dense_host(c, out, a, b, m, k, n, dtype);
    if (!c || !out || !a || !b || m < 1 || k < 32 || k % 32 || n < 1 || n > GEMM_MAX_N) return E_ARGS;
    if (!qbytes_aligned(dtype, m, k, 1)) return E_UNSUPPORTED;
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        const size_t rb = raw_row_bytes(dtype, k);
        void *staging = nullptr;
        float *dx = nullptr, *dy = nullptr;
        cmolhip_qtensor_t t{};
        if ((rc = cmolhip_alloc(c, rb * (size_t)m, ALIGN, &staging))) break;
        const size_t big = (size_t)(k > m ? k : m) * n;   // each buffer holds either side
        if ((rc = arena_get(c, big, &dx))) break;
        if ((rc = arena_get(c, big, &dy))) break;
        const void *parts[1] = {a};
        const int32_t rows[1] = {m};
        if ((rc = cmolhip_qtensor_upload(c, dtype, k, 1, 1, parts, rows, CMOLHIP_PARTS_CONCAT, staging,
                                         rb * (size_t)m, &t)))
            break;
        // B[k][n] -> x[n][k] and y[n][m] -> out[m][n] on the device: the
        // call allocates no host memory
        if ((rc = cmolhip_memcpy_h2d(c, dy, b, (size_t)k * n * 4))) break;
        if ((rc = launch_transpose(dy, dx, k, n, c->stream))) break;
        if ((rc = cmolhip_gemm(c, &t, dx, dy, n, nullptr, 0.0f))) break;
        if ((rc = launch_transpose(dy, dx, n, m, c->stream))) break;
        if ((rc = cmolhip_memcpy_d2h(c, out, dx, (size_t)m * n * 4))) break;
    } while (0);
    arena_release(c, mark);
    return rc;
}

int cmolhip_attn_decode(cmolhip_ctx_t *c, int n, const float *q, const void *kcache,
                        const void *vcache, const int32_t *seqlen, int n_heads, int n_kv, int d_head,
                        int max_ctx, int kv_f16, int split, float *out)
{
    if (!c || n < 1 || !q || !kcache || !vcache || !seqlen || !out || n_kv < 1 || n_heads < n_kv ||
        n_heads % n_kv || max_ctx < 1 || split < 0 || split % 32 ||
        (split % 64 && d_head != 64 && d_head != 128))
        return E_ARGS;
    if (!split) split = 64;
    const int G = n_heads / n_kv, ms = attn_max_splits(max_ctx, split);
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        float *pm, *pl, *po;
        int32_t *ids;
        const size_t np = (size_t)n * n_kv * ms * G;
        if ((rc = arena_get(c, np, &pm)) || (rc = arena_get(c, np, &pl)) ||
            (rc = arena_get(c, np * d_head, &po)) || (rc = arena_get(c, (size_t)n, &ids)))
            break;
        if ((rc = launch_iota(ids, n, c->stream))) break;   // cache i belongs to session i
        AttnArgs a{};
        a.q = q;
        a.q_stride = n_heads * d_head;
        a.kv.k_base = (void *)kcache;
        a.kv.v_base = (void *)vcache;
        a.kv.slot_stride = (size_t)n_kv * max_ctx * d_head;
        a.kv.layer_off = 0;
        a.kv.slot_ids = ids;
        a.seqlen = seqlen;
        a.seqlen_stride = 1;
        a.n = n;
        a.n_heads = n_heads;
        a.n_kv = n_kv;
        a.d_head = d_head;
        a.max_ctx = max_ctx;
        a.kv_f16 = kv_f16;
        a.split = split;
        a.max_splits = ms;
        a.bal = attn_bal_wgs(n, n_kv, d_head, kv_f16, ms);
        a.pm = pm;
        a.pl = pl;
        a.po = po;
        a.out = out;
        a.out_stride = n_heads * d_head;
        if ((rc = launch_attn(a, c->stream))) break;
        if (hipStreamSynchronize(c->stream) != hipSuccess) rc = E_INVALID;
    } while (0);
    arena_release(c, mark);
    return rc;
}

} // extern "C"

// ---------------------------------------------------------------------------
// Whole-model decode path
// ---------------------------------------------------------------------------
namespace {

struct MLayer {
    // q|k|v rows in runs of parts that share a format (one tensor per run;
    // a single run unless the GGUF mixes formats, e.g. a Q6_K attn_v)
    cmolhip_qtensor_t qkv[3]{};
    int qkv_row0[3]{}, n_qkv = 1;
    cmolhip_qtensor_t o{}, gu{}, down{};
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;   // per-head QK-norm weights [d_head] or null
    int rope_on = 1;
};

// Device buffers of one decode batch of up to `cap` activation vectors.
struct Batch {
    int cap = 0;
    hipStream_t st = nullptr;
    int32_t *steps = nullptr;       // device [cap][3] {token, pos, seqlen}
    int32_t *slot_ids = nullptr;    // device [cap]: KV slot of each vector
    float *x = nullptr, *q = nullptr, *logits = nullptr;
    _Float16 *op_qkv = nullptr, *op_o = nullptr, *op_gu = nullptr, *op_dn = nullptr,
             *op_lm = nullptr;      // consumer operands (kernels.h)
    float *ss_a = nullptr, *ss_b = nullptr;   // sum-of-squares partials [cap][d]
    unsigned long long *argmax = nullptr;     // [cap][ARGMAX_SLOTS]
    float *pm = nullptr, *pl = nullptr, *po = nullptr;
    float *part = nullptr;                    // k-split partial sums of batched matvecs
    size_t part_cap = 0;                      // floats at part
    float *qkv_raw = nullptr;                 // QK-norm models: [cap][d + 2 kvd] q|k|v rows
    int32_t *h_steps = nullptr;               // pinned [cap][3]
    int32_t *h_slots = nullptr;               // pinned [cap]
    unsigned long long *h_argmax = nullptr;   // pinned [cap][ARGMAX_SLOTS]
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    // the shared batch: one captured step per vector count (index n - 1;
    // null where capture failed: that count launches from the stream)
    std::vector<hipGraphExec_t> gexec_n;
    std::mutex mu;
};

// Buffers of a batched prompt pass of up to `cap` tokens of one session
// (shared by the sessions; prefills are serialised by `mu`).
struct Prefill {
    int cap = 0;
    int split = 1024, max_splits = 1;         // attention splits of the pass
    int32_t *steps = nullptr;                 // device [cap][3] {token, pos, seqlen}
    int32_t *slot_ids = nullptr;              // device [cap]
    float *x = nullptr, *q = nullptr;
    _Float16 *op_qkv = nullptr, *op_o = nullptr, *op_gu = nullptr, *op_dn = nullptr,
             *op_lm = nullptr;
    float *ss_a = nullptr, *ss_b = nullptr;   // [cap][d]
    float *pm = nullptr, *pl = nullptr, *po = nullptr;
    float *qkv_raw = nullptr;                 // QK-norm models: [cap][d + 2 kvd]
    _Float16 *kv_hl = nullptr;                // prompt attention: high/low f16 copy of one layer's cache
    float *part = nullptr;                    // split-K partial sums of the prompt GEMMs
    size_t part_cap = 0;                      // floats at part
    int32_t *h_steps = nullptr;               // pinned [cap][3]
    int32_t *h_slots = nullptr;               // pinned [cap]
    std::mutex mu;
};

constexpr int ATTN_SPLIT_MIN = 64, ATTN_SPLIT_MAX = 1024;

// Prompts of up to this many tokens run through the matvec kernels as one
// lock-step batch of the session's consecutive positions: at this size the
// tiled GEMM covers too few work-groups (a 1-token pass costs 5x a decode
// step at the 3B shape).
constexpr int PROMPT_MATVEC_MAX = 8;

// Vectors of the shared lock-step batch: every session, and short prompts.
int multi_cap(const cmolhip_hparams_t &h)
{
    return h.max_sessions > PROMPT_MATVEC_MAX ? h.max_sessions : PROMPT_MATVEC_MAX;
}

int prefill_cap(const cmolhip_hparams_t &h)
{
    const int c = h.prefill_chunk > 0 ? h.prefill_chunk : 512;
    return c < h.max_ctx ? c : h.max_ctx;
}

// CMOL_PROMPT_ATTN=0: prompt passes use the split attention kernels
// (measurements).
bool prompt_attn_on()
{
    static const bool on = [] {
        const char *e = getenv("CMOL_PROMPT_ATTN");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Whether prompt passes of this model run the flash-style prompt attention
// (fp32 cache, d_head 64 / 128, at most 8 query heads per kv head).
bool prompt_attn_fits(const cmolhip_hparams_t &h)
{
    const int G = h.n_heads / h.n_kv_heads;
    return prompt_attn_on() && !h.kv_f16 && (h.d_head == 64 || h.d_head == 128) && G >= 1 && G <= 8;
}

// Positions per attention work-group in a prompt pass: the split kernels
// take at most 16 splits of at least 1024 positions; the prompt kernel, whose
// work-groups already share K/V across 64 query rows, at most 32 splits of
// at least 256 (more work-groups for a pass over a short prefix).
int prefill_split(const cmolhip_hparams_t &h)
{
    const bool pk = prompt_attn_fits(h);
    int s = (h.max_ctx + (pk ? 31 : 15)) / (pk ? 32 : 16);
    s = (s + 63) / 64 * 64;
    const int lo = pk ? 256 : 1024;
    return s < lo ? lo : s;
}

int pick_split(int max_ctx)
{
    const char *e = getenv("CMOL_ATTN_SPLIT");
    int s = e ? atoi(e) : max_ctx / 64;
    s = (s + 63) / 64 * 64;
    if (s < ATTN_SPLIT_MIN) s = ATTN_SPLIT_MIN;
    if (s > ATTN_SPLIT_MAX) s = ATTN_SPLIT_MAX;
    return s;
}

bool is_block_fmt(int dt) { return dt == DT_Q4_0 || dt == DT_Q5_0 || dt == DT_Q8_0 || is_kquant(dt); }

// Runs of consecutive q / k / v parts that share a format: run r covers
// parts first[r] .. first[r] + count[r] - 1 (rows of q, k, v: d, kvd, kvd),
// rows[r] output rows of format dt[r].  Each run is one uploaded tensor and
// one matvec launch per stage, so the arena plan, the upload and the k-split
// scratch all read their shapes from here.
struct QkvRuns {
    int n = 0;
    int first[3]{}, count[3]{}, rows[3]{}, dt[3]{};
};

QkvRuns qkv_runs(const cmolhip_layer_tensors_t &L, const cmolhip_hparams_t &h)
{
    const int dt[3] = {L.q.dtype, L.k.dtype, L.v.dtype};
    const int rows[3] = {h.d_model, h.n_kv_heads * h.d_head, h.n_kv_heads * h.d_head};
    QkvRuns R;
    for (int p = 0; p < 3; p++) {
        if (R.n && dt[p] == R.dt[R.n - 1]) {
            R.count[R.n - 1]++;
            R.rows[R.n - 1] += rows[p];
        } else {
            R.first[R.n] = p;
            R.count[R.n] = 1;
            R.rows[R.n] = rows[p];
            R.dt[R.n] = dt[p];
            R.n++;
        }
    }
    return R;
}

// Byte sizes of everything the model puts in the arena, in creation order.
struct Plan {
    std::vector<size_t> sizes;
    size_t staging = 0;
    void add(size_t b) { sizes.push_back(b); }
    size_t total() const
    {
        size_t t = ALIGN;
        for (size_t s : sizes) t += align_up(s, ALIGN);
        return t;
    }
};

void add_q(Plan &P, int dt, int rows, int cols, int fold)
{
    QLayout L;
    qlayout(dt, rows, cols, fold, &L);
    P.add(L.qs);
    P.add(L.d);
    if (L.qh) P.add(L.qh);
}

// k parts per tile for a projection: single-session models fold matrices
// with few rows until they make >= 192 row tiles at batch 1 (CMOL_FOLD_TILES
// overrides the target for measurements), as long as
// the parts stay whole quads (padding <= 1/16); batched models keep fold 1,
// whose tiles serve up to 8 vectors per MFMA.
int pick_fold(int rows, int cols, int max_sessions)
{
    if (max_sessions > 1) return 1;
    const int nb = cols / 32;
    int f = 1;
    static const int target = [] {
        const char *e = getenv("CMOL_FOLD_TILES");   // measurements
        const int v = e ? atoi(e) : 192;
        return v < 1 ? 1 : v;
    }();
    while (f < 8 && (rows + 16 / f - 1) / (16 / f) < target) {
        const int nf = 2 * f;
        if (nf * fold_quads(nb, nf) * 4 > nb + nb / 16) break;
        f = nf;
    }
    return f;
}

// k parts per tile for the persistent decode kernel, where a wave finishes
// its tiles alone: the largest fold whose padding stays within nb/16 blocks
// of the unfolded layout's (more, smaller tiles spread one matrix over the
// launch's waves).
int persist_fold(int cols)
{
    const int nb = cols / 32;
    const int base = 4 * fold_quads(nb, 1);
    for (int f = 8; f > 1; f >>= 1)
        if (4 * f * fold_quads(nb, f) <= base + nb / 16) return f;
    return 1;
}

// Layer weight format when the model's single session decodes with the
// persistent kernel, else 0.  Opt-in with CMOL_PERSIST=1 in the environment
// (one session, d_head 64 or 128, every layer matrix in one format): on
// MI355X its device-wide barriers cost about as much as the kernel
// boundaries of the decode graph they replace, and the graph stays faster.
int persist_format(const cmolhip_model_desc_t *d)
{
    const char *e = getenv("CMOL_PERSIST");
    if (!e || e[0] != '1') return 0;
    const cmolhip_hparams_t &h = d->hp;
    if (h.max_sessions != 1 || (h.d_head != 64 && h.d_head != 128)) return 0;
    const int dt = d->layers[0].q.dtype;
    if (dt != DT_Q4_0 && dt != DT_Q5_0 && dt != DT_Q8_0) return 0;   // no K-quant kernel
    for (int l = 0; l < h.n_layers; l++) {
        const cmolhip_layer_tensors_t &L = d->layers[l];
        if (L.q_norm.data || L.k_norm.data) return 0;   // no QK-norm stage
        if (L.q.dtype != dt || L.k.dtype != dt || L.v.dtype != dt || L.o.dtype != dt ||
            L.gate.dtype != dt || L.down.dtype != dt)
            return 0;
    }
    return dt;
}

// Fold of a layer matrix (rows x cols) of model d.
int layer_fold(const cmolhip_model_desc_t *d, int rows, int cols)
{
    return persist_format(d) ? persist_fold(cols) : pick_fold(rows, cols, d->hp.max_sessions);
}

} // namespace

extern "C" int cmolhip_pick_fold(int rows, int cols, int max_sessions)
{
    return (rows > 0 && cols > 0 && cols % 32 == 0) ? pick_fold(rows, cols, max_sessions) : 1;
}

namespace {

int validate_desc(const cmolhip_model_desc_t *d)
{
    if (!d || !d->layers || !d->rope_table) return E_ARGS;
    const cmolhip_hparams_t &h = d->hp;
    if (h.n_layers < 1 || h.n_heads < 1 || h.n_kv_heads < 1 || h.d_model < 32 || h.d_ffn < 32 ||
        h.vocab < 1 || h.max_ctx < 1 || h.max_sessions < 1 || h.max_sessions > 32)
        return E_ARGS;
    if (h.d_model % 32 || h.d_ffn % 32 || h.n_heads % h.n_kv_heads ||
        h.d_head * h.n_heads != h.d_model)
        return E_UNSUPPORTED;
    if ((h.d_head != 16 && h.d_head != 32 && h.d_head != 64 && h.d_head != 128 && h.d_head != 256) ||
        h.n_heads / h.n_kv_heads > 8)
        return E_UNSUPPORTED;
    const int kvd = h.n_kv_heads * h.d_head;
    auto chk = [](const cmolhip_host_tensor_t &t, int rows, int cols) {
        return t.data && t.rows == rows && t.cols == cols && is_block_fmt(t.dtype);
    };
    auto chk_norm = [](const cmolhip_host_tensor_t &t, int cols) {
        return t.data && t.dtype == DT_F32 && t.cols == cols && t.rows == 1;
    };
    if (!chk(d->embd, h.vocab, h.d_model)) return d->embd.data ? E_UNSUPPORTED : E_INVALID;
    if (d->lm_head.data && !chk(d->lm_head, h.vocab, h.d_model)) return E_UNSUPPORTED;
    if (!chk_norm(d->out_norm, h.d_model)) return E_INVALID;
    for (int l = 0; l < h.n_layers; l++) {
        const cmolhip_layer_tensors_t &L = d->layers[l];
        if (!L.q.data || !L.k.data || !L.v.data || !L.o.data || !L.gate.data || !L.up.data ||
            !L.down.data || !L.attn_norm.data || !L.ffn_norm.data)
            return E_INVALID;
        if (!chk(L.q, h.d_model, h.d_model) || !chk(L.k, kvd, h.d_model) ||
            !chk(L.v, kvd, h.d_model) || !chk(L.o, h.d_model, h.d_model) ||
            !chk(L.gate, h.d_ffn, h.d_model) || !chk(L.up, h.d_ffn, h.d_model) ||
            !chk(L.down, h.d_model, h.d_ffn))
            return E_UNSUPPORTED;
        // q, k and v may differ in format but share one activation operand,
        // whose k order differs for Q8_0; gate and up are interleaved rows
        const bool q8 = L.q.dtype == DT_Q8_0;
        if (q8 != (L.k.dtype == DT_Q8_0) || q8 != (L.v.dtype == DT_Q8_0) || L.gate.dtype != L.up.dtype)
            return E_UNSUPPORTED;
        if (!chk_norm(L.attn_norm, h.d_model) || !chk_norm(L.ffn_norm, h.d_model)) return E_INVALID;
        if ((L.q_norm.data && !chk_norm(L.q_norm, h.d_head)) || (L.k_norm.data && !chk_norm(L.k_norm, h.d_head)))
            return E_INVALID;
    }
    return E_OK;
}

// Whether any layer normalises q or k per head (attn_q_norm / attn_k_norm).
bool has_qk_norm(const cmolhip_model_desc_t *d)
{
    for (int l = 0; l < d->hp.n_layers; l++)
        if (d->layers[l].q_norm.data || d->layers[l].k_norm.data) return true;
    return false;
}

// Fold of the embedding / LM head (tied or not): the persistent kernel
// spreads the LM head like the layer matrices.
int head_fold(const cmolhip_model_desc_t *d) { return persist_format(d) ? persist_fold(d->hp.d_model) : 1; }

// Device view of the dimensions of a tiled tensor (no data), enough for
// gemv_part_floats.
QTensor shape_qt(int dt, int rows, int cols, int fold)
{
    QTensor t{};
    t.dtype = dt;
    t.rows = rows;
    t.cols = cols;
    t.fold = fold;
    t.row_tiles = (rows + 16 / fold - 1) / (16 / fold);
    t.block_quads = fold_quads(cols / 32, fold);
    return t;
}

// Every matvec launch of one decode step of model d, in launch order:
// f(dtype, rows, cols, fold).  q|k|v launch once per run of formats
// (enqueue_step, enqueue_qk_norm).
template <class F>
void for_each_step_matvec(const cmolhip_model_desc_t *d, F f)
{
    const cmolhip_hparams_t &h = d->hp;
    for (int l = 0; l < h.n_layers; l++) {
        const cmolhip_layer_tensors_t &L = d->layers[l];
        const QkvRuns R = qkv_runs(L, h);
        for (int r = 0; r < R.n; r++) f(R.dt[r], R.rows[r], h.d_model, layer_fold(d, R.rows[r], h.d_model));
        f(L.o.dtype, h.d_model, h.d_model, layer_fold(d, h.d_model, h.d_model));
        f(L.gate.dtype, 2 * h.d_ffn, h.d_model, layer_fold(d, 2 * h.d_ffn, h.d_model));
        f(L.down.dtype, h.d_model, h.d_ffn, layer_fold(d, h.d_model, h.d_ffn));
    }
    const cmolhip_host_tensor_t &lm = d->lm_head.data ? d->lm_head : d->embd;
    f(lm.dtype, h.vocab, h.d_model, head_fold(d));
}

// k-split scratch (floats) the matvecs of one step of n vectors need: the
// largest over the step's launches (they run one after another on one
// stream, so they share the buffer).
size_t step_part_floats(const cmolhip_model_desc_t *d, int n)
{
    size_t m = 0;
    for_each_step_matvec(d, [&](int dt, int rows, int cols, int fold) {
        const size_t f = gemv_part_floats(shape_qt(dt, rows, cols, fold), n);
        m = f > m ? f : m;
    });
    return m;
}

// Scratch for a batch of up to cap vectors: the largest step need over
// 1..cap (the split count depends on the batch size).
size_t batch_part_floats(const cmolhip_model_desc_t *d, int cap)
{
    size_t m = 0;
    for (int n = 1; n <= cap; n++) {
        const size_t f = step_part_floats(d, n);
        m = f > m ? f : m;
    }
    return m;
}

// Buffers of one batch, in allocation order (mirrored by build_batch).
void plan_batch(Plan &P, const cmolhip_model_desc_t *d, int cap, int ms)
{
    const cmolhip_hparams_t &h = d->hp;
    const size_t np = (size_t)h.n_kv_heads * ms * (h.n_heads / h.n_kv_heads);
    P.add((size_t)cap * 3 * 4);
    P.add((size_t)cap * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * h.vocab * 4);
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_ffn, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * ARGMAX_SLOTS * 8);
    P.add((size_t)cap * np * 4);
    P.add((size_t)cap * np * 4);
    P.add((size_t)cap * np * h.d_head * 4);
    P.add(batch_part_floats(d, cap) * 4);
    if (has_qk_norm(d)) P.add((size_t)cap * (h.d_model + 2 * h.n_kv_heads * h.d_head) * 4);
}

// Partial sums a prompt pass's split-K GEMMs may need: GEMM_KS_MAX ranges of
// the pass's tokens for the widest of q|k|v and the d_model-row matrices.
size_t prefill_part_floats(const cmolhip_hparams_t &h)
{
    const size_t rows = (size_t)h.d_model + 2 * (size_t)h.n_kv_heads * h.d_head;
    return (size_t)GEMM_KS_MAX * prefill_cap(h) * rows;
}

// Buffers of the prompt pass, in allocation order (mirrored by build_prefill).
void plan_prefill(Plan &P, const cmolhip_model_desc_t *d)
{
    const cmolhip_hparams_t &h = d->hp;
    const int cap = prefill_cap(h);
    const int ms = attn_max_splits(h.max_ctx, prefill_split(h));
    const size_t np = (size_t)h.n_kv_heads * ms * (h.n_heads / h.n_kv_heads);
    P.add((size_t)cap * 3 * 4);
    P.add((size_t)cap * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add(act_bytes(h.d_ffn, cap));
    P.add(act_bytes(h.d_model, cap));
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * h.d_model * 4);
    P.add((size_t)cap * np * 4);
    P.add((size_t)cap * np * 4);
    P.add((size_t)cap * np * h.d_head * 4);
    if (has_qk_norm(d)) P.add((size_t)cap * (h.d_model + 2 * h.n_kv_heads * h.d_head) * 4);
    if (prompt_attn_fits(h)) P.add(attn_prompt_kv_bytes(h.n_kv_heads, h.d_head, h.max_ctx));
    P.add(prefill_part_floats(h) * 4);
}


// Work-groups the persistent kernel will run with: one per CU of device 0
// (at most PK_MAX_WGS; 256 when no device is visible, for size estimates).
int persist_wgs()
{
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || cus < 1) {
        (void)hipGetLastError();
        cus = 256;
    }
    return cus < PK_MAX_WGS ? cus : PK_MAX_WGS;
}

// Attention splits of the persistent kernel: one item per work-group.
int persist_max_splits(const cmolhip_hparams_t &h) { return persist_wgs() / h.n_kv_heads; }

// CMOL_PERSIST_TRACE=1: the persistent kernel records per-stage times of
// every work-group (profiling; see cmolhip_persist_marks).
bool persist_tracing()
{
    const char *e = getenv("CMOL_PERSIST_TRACE");
    return e && e[0] == '1';
}

// Exchange floats of one layer and parity (q, kn, vn, partials, att, xa, h, xo).
size_t pk_ex_floats(const cmolhip_hparams_t &h)
{
    const size_t d = h.d_model, kvd = (size_t)h.n_kv_heads * h.d_head;
    const size_t part = (size_t)h.n_heads * persist_max_splits(h) * (h.d_head + 4);
    return d + 2 * kvd + part + 3 * d + h.d_ffn;
}

// Exchange buffers of the persistent kernel, in allocation order (mirrored
// by build_persist).
void plan_persist(Plan &P, const cmolhip_hparams_t &h)
{
    P.add(((size_t)2 * h.d_model + (size_t)2 * h.n_layers * pk_ex_floats(h)) * 4);   // x0, then every layer
    P.add((size_t)h.n_layers * sizeof(PkLayer));
    P.add(4);                                              // launch counter
    P.add(4);                                              // error flag
    if (persist_tracing()) {
        P.add(2 * 8);
        P.add((size_t)pk_stages(h.n_layers) * PK_MAX_WGS * PK_MARKS * 8);
    }
}

Plan make_plan(const cmolhip_model_desc_t *d)
{
    const cmolhip_hparams_t &h = d->hp;
    const int ms = attn_max_splits(h.max_ctx, pick_split(h.max_ctx));
    Plan P;
    size_t big = 0;
    auto upd = [&](const cmolhip_host_tensor_t &t) {
        size_t b = raw_row_bytes(t.dtype, t.cols) * (size_t)t.rows;
        if (b > big) big = b;
    };
    upd(d->embd);
    if (d->lm_head.data) upd(d->lm_head);
    for (int l = 0; l < h.n_layers; l++) {
        const auto &L = d->layers[l];
        upd(L.q); upd(L.k); upd(L.v); upd(L.o); upd(L.gate); upd(L.up); upd(L.down);
    }
    P.staging = big < ((size_t)64 << 20) ? big : ((size_t)64 << 20);
    P.add(P.staging);
    for (int l = 0; l < h.n_layers; l++) {
        const auto &L = d->layers[l];
        const QkvRuns R = qkv_runs(L, h);
        for (int r = 0; r < R.n; r++) add_q(P, R.dt[r], R.rows[r], h.d_model, layer_fold(d, R.rows[r], h.d_model));
        add_q(P, L.o.dtype, h.d_model, h.d_model, layer_fold(d, h.d_model, h.d_model));
        add_q(P, L.gate.dtype, 2 * h.d_ffn, h.d_model, layer_fold(d, 2 * h.d_ffn, h.d_model));
        add_q(P, L.down.dtype, h.d_model, h.d_ffn, layer_fold(d, h.d_model, h.d_ffn));
        P.add((size_t)h.d_model * 4);
        P.add((size_t)h.d_model * 4);
        if (L.q_norm.data) P.add((size_t)h.d_head * 4);
        if (L.k_norm.data) P.add((size_t)h.d_head * 4);
    }
    add_q(P, d->embd.dtype, h.vocab, h.d_model, head_fold(d));
    if (d->lm_head.data) add_q(P, d->lm_head.dtype, h.vocab, h.d_model, head_fold(d));
    P.add((size_t)h.d_model * 4);                                   // out_norm
    P.add((size_t)h.max_ctx * (h.d_head / 2) * 2 * 4);              // rope
    const size_t esz = h.kv_f16 ? 2 : 4;
    const size_t kv_elems = (size_t)h.max_sessions * h.n_layers * h.n_kv_heads * h.max_ctx * h.d_head;
    P.add(kv_elems * esz);
    P.add(kv_elems * esz);
    P.add((size_t)h.n_kv_heads * h.max_ctx * h.d_head * 4);         // scratch
    for (int s = 0; s < h.max_sessions; s++) plan_batch(P, d, 1, ms);
    plan_batch(P, d, multi_cap(h), ms);                             // lock-step batch
    plan_prefill(P, d);
    if (persist_format(d)) plan_persist(P, h);
    return P;
}

} // namespace

struct cmolhip_model {
    cmolhip_ctx_t *ctx = nullptr;
    cmolhip_hparams_t hp{};
    cmolhip_qtensor_t embd{}, lm{};
    float *out_norm = nullptr, *rope = nullptr, *scratch = nullptr;
    std::vector<MLayer> layers;
    void *kbase = nullptr, *vbase = nullptr;
    size_t slot_stride = 0, layer_stride = 0;
    int split = 64, max_splits = 1;
    std::vector<std::unique_ptr<Batch>> slots;   // one single-vector batch per session
    std::unique_ptr<Batch> multi;                // lock-step batch over sessions
    std::unique_ptr<Prefill> pf;                 // prompt passes
    std::mutex scratch_mu;
    bool use_graph = true;
    bool qk_norm = false;   // some layer normalises q or k per head
    int max_fold = 1;       // largest fold of the model's tensors
    // persistent single-session decode (pk_dt = layer format, 0: not used)
    int pk_dt = 0, pk_nwg = 0, pk_lds = 0;
    PkArgs pk{};                  // launch arguments but the per-step fields
    float *pk_ex = nullptr;       // exchange buffers of both parities
    size_t pk_ex_n = 0;           // floats at pk_ex
    int *h_pk_err = nullptr;      // pinned copy of pk.err
    unsigned pk_launches = 0;     // persistent launches since the last reset (exchange set = parity)
    int pk_giveups = 0;           // steps the graph redid after a persistent wait gave up
    unsigned long long *h_trace = nullptr;   // pinned copy of the last step's stage times
    int trace_n = 0;
};

namespace {

KVRef kvref(const cmolhip_model *m, const Batch &B, int layer)
{
    KVRef r;
    r.k_base = m->kbase;
    r.v_base = m->vbase;
    r.slot_stride = m->slot_stride;
    r.layer_off = (size_t)layer * m->layer_stride;
    r.slot_ids = B.slot_ids;
    return r;
}

ActOut act_out(_Float16 *q, int dt, int n, const float *norm_w, float *ss, int ss_stride)
{
    ActOut o{};
    o.q = q;
    o.dt = dt;
    o.nrows = 2 * n;
    o.norm_w = norm_w;
    o.ss = norm_w ? ss : nullptr;
    o.ss_stride = ss_stride;
    return o;
}

ActIn act_in(const _Float16 *q, int n, const float *ss, int count, int stride, float eps)
{
    ActIn i{};
    i.q = q;
    i.nrows = 2 * n;
    i.ss = ss;
    i.ss_count = count;
    i.ss_stride = stride;
    i.eps = eps;
    return i;
}

const cmolhip_qtensor_t &lm_tensor(const cmolhip_model *m) { return m->lm.qs ? m->lm : m->embd; }

// QKV of a QK-norm layer (src/attn.c:62-101): the matvec (or, for a prompt
// pass, the GEMM) stores the raw q|k|v rows of each vector into `raw`, then
// one stage normalises every q and k head, applies RoPE and writes q to
// g.out and k / v to the cache.  g carries the activation operand, q output,
// positions and the layer's RoPE switch.
int enqueue_qk_norm(const cmolhip_model *m, const MLayer &L, GemvArgs g, float *raw, const KVRef &kv, int n,
                    hipStream_t st, bool gemm)
{
    const cmolhip_hparams_t &hp = m->hp;
    const int stride = hp.d_model + 2 * hp.n_kv_heads * hp.d_head;
    QkArgs qa{};
    qa.q = g.out;
    qa.q_stride = g.out_stride;
    g.out_stride = stride;
    for (int r = 0; r < L.n_qkv; r++) {
        g.w = to_qt(L.qkv[r]);
        g.out = raw + L.qkv_row0[r];
        g.row_base = 0;
        RC(gemm ? launch_gemm(g, EPI_STORE, st) : launch_gemv(g, EPI_STORE, st));
    }
    qa.raw = raw;
    qa.raw_stride = stride;
    qa.qn_w = L.q_norm;
    qa.kn_w = L.k_norm;
    qa.eps = hp.rms_eps;
    qa.n = n;
    qa.n_heads = hp.n_heads;
    qa.n_kv = hp.n_kv_heads;
    qa.d_head = hp.d_head;
    qa.max_ctx = hp.max_ctx;
    qa.kv_f16 = hp.kv_f16;
    qa.rope_on = L.rope_on;
    qa.rope = m->rope;
    qa.pos = g.pos;
    qa.pos_stride = g.pos_stride;
    qa.kv = kv;
    return launch_qk_rope(qa, st);
}

// One decode step of n vectors of batch B (reference cmol_model_forward per
// vector): embedding, L x (QKV+RoPE+KV write, attention, Wo + residual,
// gate/up + SwiGLU, down + residual), LM head + argmax.
int enqueue_step(cmolhip_model *m, Batch &B, int n, hipStream_t st)
{
    const cmolhip_hparams_t &hp = m->hp;
    // sum-of-squares partials: one per 32 inputs from the embedding, one per
    // row tile from a residual epilogue; stride d covers both
    const int d = hp.d_model, kvd = hp.n_kv_heads * hp.d_head, P = d;
    const float eps = hp.rms_eps;
    RC(launch_embed(to_qt(m->embd), B.steps, 3, B.x, d,
                    act_out(B.op_qkv, m->layers[0].qkv[0].dtype, n, m->layers[0].attn_norm, B.ss_a, P),
                    B.argmax, n, st));
    int ss_count = d / 32;   // the embedding writes one partial per 32 inputs
    for (int l = 0; l < hp.n_layers; l++) {
        const MLayer &L = m->layers[l];
        GemvArgs g{};
        g.in = act_in(B.op_qkv, n, B.ss_a, ss_count, P, eps);
        g.out = B.q;
        g.out_stride = d;
        g.n = n;
        g.nq = d;
        g.nkv = kvd;
        g.d_head = hp.d_head;
        g.max_ctx = hp.max_ctx;
        g.kv_f16 = hp.kv_f16;
        g.rope_on = L.rope_on;
        g.rope = m->rope;
        g.kv = kvref(m, B, l);
        g.pos = B.steps + 1;
        g.pos_stride = 3;
        g.part = B.part;
        g.part_cap = B.part_cap;
        if (L.q_norm || L.k_norm) {
            RC(enqueue_qk_norm(m, L, g, B.qkv_raw, g.kv, n, st, false));
        } else {
            for (int r = 0; r < L.n_qkv; r++) {   // one launch per run of q|k|v formats
                g.w = to_qt(L.qkv[r]);
                g.row_base = L.qkv_row0[r];
                RC(launch_gemv(g, EPI_QKV, st));
            }
        }

        AttnArgs at{};
        at.q = B.q;
        at.q_stride = d;
        at.kv = kvref(m, B, l);
        at.seqlen = B.steps + 2;
        at.seqlen_stride = 3;
        at.n = n;
        at.n_heads = hp.n_heads;
        at.n_kv = hp.n_kv_heads;
        at.d_head = hp.d_head;
        at.max_ctx = hp.max_ctx;
        at.kv_f16 = hp.kv_f16;
        at.split = m->split;
        at.max_splits = m->max_splits;
        at.bal = attn_bal_wgs(n, hp.n_kv_heads, hp.d_head, hp.kv_f16, m->max_splits);
        at.pm = B.pm;
        at.pl = B.pl;
        at.po = B.po;
        at.out = nullptr;
        at.next = act_out(B.op_o, L.o.dtype, n, nullptr, nullptr, 0);
        RC(launch_attn(at, st));

        GemvArgs go{};
        go.w = to_qt(L.o);
        go.in = act_in(B.op_o, n, nullptr, 0, 0, eps);
        go.out = B.x;
        go.out_stride = d;
        go.n = n;
        go.next = act_out(B.op_gu, L.gu.dtype, n, L.ffn_norm, B.ss_b, P);
        go.part = B.part;
        go.part_cap = B.part_cap;
        RC(launch_gemv(go, EPI_RESID, st));

        GemvArgs gu{};
        gu.w = to_qt(L.gu);
        gu.in = act_in(B.op_gu, n, B.ss_b, L.o.row_tiles, P, eps);
        gu.out = nullptr;
        gu.n = n;
        gu.next = act_out(B.op_dn, L.down.dtype, n, nullptr, nullptr, 0);
        gu.part = B.part;
        gu.part_cap = B.part_cap;
        RC(launch_gemv(gu, EPI_SWIGLU, st));

        GemvArgs gd{};
        gd.w = to_qt(L.down);
        gd.in = act_in(B.op_dn, n, nullptr, 0, 0, eps);
        gd.out = B.x;
        gd.out_stride = d;
        gd.n = n;
        if (l + 1 < hp.n_layers)
            gd.next = act_out(B.op_qkv, m->layers[l + 1].qkv[0].dtype, n, m->layers[l + 1].attn_norm, B.ss_a, P);
        else
            gd.next = act_out(B.op_lm, lm_tensor(m).dtype, n, m->out_norm, B.ss_a, P);
        gd.part = B.part;
        gd.part_cap = B.part_cap;
        RC(launch_gemv(gd, EPI_RESID, st));
        ss_count = L.down.row_tiles;
    }
    GemvArgs gl{};
    gl.w = to_qt(lm_tensor(m));
    gl.in = act_in(B.op_lm, n, B.ss_a, ss_count, P, eps);
    gl.out = B.logits;
    gl.out_stride = hp.vocab;
    gl.n = n;
    gl.argmax = B.argmax;
    gl.part = B.part;
    gl.part_cap = B.part_cap;
    RC(launch_gemv(gl, EPI_LOGITS, st));
    return E_OK;
}

// One batched prompt pass of n tokens of one session (steps and slot ids
// already on the device): embedding, L x (QKV GEMM + RoPE + KV write, causal
// attention over the cache, Wo GEMM + residual, gate/up GEMM + SwiGLU, down
// GEMM + residual); with `last`, the final token's LM-head operand is
// extracted into the session's decode batch B and its logits computed there.
int enqueue_prefill(cmolhip_model *m, Prefill &F, Batch &B, int n, bool last, hipStream_t st)
{
    const cmolhip_hparams_t &hp = m->hp;
    const int d = hp.d_model, kvd = hp.n_kv_heads * hp.d_head, P = d;
    const float eps = hp.rms_eps;
    KVRef kv;
    kv.k_base = m->kbase;
    kv.v_base = m->vbase;
    kv.slot_stride = m->slot_stride;
    kv.slot_ids = F.slot_ids;
    RC(launch_embed(to_qt(m->embd), F.steps, 3, F.x, d,
                    act_out(F.op_qkv, m->layers[0].qkv[0].dtype, n, m->layers[0].attn_norm, F.ss_a, P),
                    nullptr, n, st));
    int ss_count = d / 32;
    const int tile_count = (d + 15) / 16;   // GEMM residual partials: one per 16 rows
    for (int l = 0; l < hp.n_layers; l++) {
        const MLayer &L = m->layers[l];
        kv.layer_off = (size_t)l * m->layer_stride;
        GemvArgs g{};
        g.in = act_in(F.op_qkv, n, F.ss_a, ss_count, P, eps);
        g.out = F.q;
        g.out_stride = d;
        g.n = n;
        g.nq = d;
        g.nkv = kvd;
        g.d_head = hp.d_head;
        g.max_ctx = hp.max_ctx;
        g.kv_f16 = hp.kv_f16;
        g.rope_on = L.rope_on;
        g.rope = m->rope;
        g.kv = kv;
        g.pos = F.steps + 1;
        g.pos_stride = 3;
        g.part = F.part;
        g.part_cap = F.part_cap;
        if (L.q_norm || L.k_norm) {
            RC(enqueue_qk_norm(m, L, g, F.qkv_raw, kv, n, st, true));
        } else {
            for (int r = 0; r < L.n_qkv; r++) {
                g.w = to_qt(L.qkv[r]);
                g.row_base = L.qkv_row0[r];
                RC(launch_gemm(g, EPI_QKV, st));
            }
        }

        AttnArgs at{};
        at.q = F.q;
        at.q_stride = d;
        at.kv = kv;
        at.seqlen = F.steps + 2;
        at.seqlen_stride = 3;
        at.n = n;
        at.n_heads = hp.n_heads;
        at.n_kv = hp.n_kv_heads;
        at.d_head = hp.d_head;
        at.max_ctx = hp.max_ctx;
        at.kv_f16 = hp.kv_f16;
        at.split = F.split;
        at.max_splits = F.max_splits;
        at.pm = F.pm;
        at.pl = F.pl;
        at.po = F.po;
        at.out = nullptr;
        at.next = act_out(F.op_o, L.o.dtype, n, nullptr, nullptr, 0);
        // the pass's tokens share every K/V tile (flash style on MFMA); other
        // shapes and fp16 caches take the split kernels
        if (prompt_attn_on() && launch_attn_prompt(at, F.kv_hl, F.h_steps[3 * (n - 1) + 2], st) == 0) {
        } else {
            RC(launch_attn(at, st));
        }

        GemvArgs go{};
        go.w = to_qt(L.o);
        go.in = act_in(F.op_o, n, nullptr, 0, 0, eps);
        go.out = F.x;
        go.out_stride = d;
        go.n = n;
        go.next = act_out(F.op_gu, L.gu.dtype, n, L.ffn_norm, F.ss_b, P);
        go.part = F.part;
        go.part_cap = F.part_cap;
        RC(launch_gemm(go, EPI_RESID, st));

        GemvArgs gu{};
        gu.w = to_qt(L.gu);
        gu.in = act_in(F.op_gu, n, F.ss_b, tile_count, P, eps);
        gu.out = nullptr;
        gu.n = n;
        gu.next = act_out(F.op_dn, L.down.dtype, n, nullptr, nullptr, 0);
        gu.part = F.part;
        gu.part_cap = F.part_cap;
        RC(launch_gemm(gu, EPI_SWIGLU, st));

        GemvArgs gd{};
        gd.w = to_qt(L.down);
        gd.in = act_in(F.op_dn, n, nullptr, 0, 0, eps);
        gd.out = F.x;
        gd.out_stride = d;
        gd.n = n;
        if (l + 1 < hp.n_layers)
            gd.next = act_out(F.op_qkv, m->layers[l + 1].qkv[0].dtype, n, m->layers[l + 1].attn_norm, F.ss_a, P);
        else
            gd.next = act_out(F.op_lm, lm_tensor(m).dtype, n, m->out_norm, F.ss_a, P);
        gd.part = F.part;
        gd.part_cap = F.part_cap;
        RC(launch_gemm(gd, EPI_RESID, st));
        ss_count = tile_count;
    }
    if (!last) return E_OK;
    // LM head for the last token only, through the session's decode buffers
    RC(launch_act_extract(F.op_lm, d, n, n - 1, B.op_lm, F.ss_a, P, ss_count, B.ss_a, st));
    HC(hipMemsetAsync(B.argmax, 0, ARGMAX_SLOTS * sizeof(unsigned long long), st));
    GemvArgs gl{};
    gl.w = to_qt(lm_tensor(m));
    gl.in = act_in(B.op_lm, 1, B.ss_a, ss_count, ss_count, eps);
    gl.out = B.logits;
    gl.out_stride = hp.vocab;
    gl.n = 1;
    gl.argmax = B.argmax;
    RC(launch_gemv(gl, EPI_LOGITS, st));
    return E_OK;
}

int upload_norm(cmolhip_ctx_t *c, const cmolhip_host_tensor_t &t, float **dst)
{
    RC(arena_get(c, (size_t)t.cols, dst));
    return cmolhip_memcpy_h2d(c, *dst, t.data, (size_t)t.cols * 4);
}

int upload_q(cmolhip_ctx_t *c, int n, const cmolhip_host_tensor_t *const *ts, int mode, int fold,
             void *stg, size_t stg_bytes, cmolhip_qtensor_t *out)
{
    const void *parts[3];
    int32_t rows[3];
    for (int i = 0; i < n; i++) {
        parts[i] = ts[i]->data;
        rows[i] = ts[i]->rows;
    }
    return cmolhip_qtensor_upload(c, ts[0]->dtype, ts[0]->cols, fold, n, parts, rows, mode, stg, stg_bytes, out);
}

int build_batch(cmolhip_model *m, Batch &B, int cap, size_t part_floats)
{
    cmolhip_ctx_t *c = m->ctx;
    const cmolhip_hparams_t &h = m->hp;
    const size_t np = (size_t)h.n_kv_heads * m->max_splits * (h.n_heads / h.n_kv_heads);
    B.cap = cap;
    RC(arena_get(c, (size_t)cap * 3, &B.steps));
    RC(arena_get(c, (size_t)cap, &B.slot_ids));
    RC(arena_get(c, (size_t)cap * h.d_model, &B.x));
    RC(arena_get(c, (size_t)cap * h.d_model, &B.q));
    RC(arena_get(c, (size_t)cap * h.vocab, &B.logits));
    _Float16 **ops[5] = {&B.op_qkv, &B.op_o, &B.op_gu, &B.op_dn, &B.op_lm};
    const int opk[5] = {h.d_model, h.d_model, h.d_model, h.d_ffn, h.d_model};
    for (int i = 0; i < 5; i++) {
        const size_t nb = act_bytes(opk[i], cap);
        RC(cmolhip_alloc(c, nb, ALIGN, (void **)ops[i]));
    }
    RC(arena_get(c, (size_t)cap * h.d_model, &B.ss_a));
    RC(arena_get(c, (size_t)cap * h.d_model, &B.ss_b));
    RC(arena_get(c, (size_t)cap * ARGMAX_SLOTS, &B.argmax));
    RC(arena_get(c, (size_t)cap * np, &B.pm));
    RC(arena_get(c, (size_t)cap * np, &B.pl));
    RC(arena_get(c, (size_t)cap * np * h.d_head, &B.po));
    if (part_floats) RC(arena_get(c, part_floats, &B.part));
    B.part_cap = part_floats;
    if (m->qk_norm) RC(arena_get(c, (size_t)cap * (h.d_model + 2 * h.n_kv_heads * h.d_head), &B.qkv_raw));
    HC(hipMemsetAsync(B.steps, 0, (size_t)cap * 12, c->stream));
    HC(hipStreamCreateWithFlags(&B.st, hipStreamNonBlocking));
    HC(hipHostMalloc((void **)&B.h_steps, (size_t)cap * 3 * 4, hipHostMallocDefault));
    HC(hipHostMalloc((void **)&B.h_slots, (size_t)cap * 4, hipHostMallocDefault));
    HC(hipHostMalloc((void **)&B.h_argmax, (size_t)cap * ARGMAX_SLOTS * 8, hipHostMallocDefault));
    return E_OK;
}

int build_prefill(cmolhip_model *m, Prefill &F)
{
    cmolhip_ctx_t *c = m->ctx;
    const cmolhip_hparams_t &h = m->hp;
    F.cap = prefill_cap(h);
    F.split = prefill_split(h);
    F.max_splits = attn_max_splits(h.max_ctx, F.split);
    const int cap = F.cap;
    const size_t np = (size_t)h.n_kv_heads * F.max_splits * (h.n_heads / h.n_kv_heads);
    RC(arena_get(c, (size_t)cap * 3, &F.steps));
    RC(arena_get(c, (size_t)cap, &F.slot_ids));
    RC(arena_get(c, (size_t)cap * h.d_model, &F.x));
    RC(arena_get(c, (size_t)cap * h.d_model, &F.q));
    _Float16 **ops[5] = {&F.op_qkv, &F.op_o, &F.op_gu, &F.op_dn, &F.op_lm};
    const int opk[5] = {h.d_model, h.d_model, h.d_model, h.d_ffn, h.d_model};
    for (int i = 0; i < 5; i++) RC(cmolhip_alloc(c, act_bytes(opk[i], cap), ALIGN, (void **)ops[i]));
    RC(arena_get(c, (size_t)cap * h.d_model, &F.ss_a));
    RC(arena_get(c, (size_t)cap * h.d_model, &F.ss_b));
    RC(arena_get(c, (size_t)cap * np, &F.pm));
    RC(arena_get(c, (size_t)cap * np, &F.pl));
    RC(arena_get(c, (size_t)cap * np * h.d_head, &F.po));
    if (m->qk_norm) RC(arena_get(c, (size_t)cap * (h.d_model + 2 * h.n_kv_heads * h.d_head), &F.qkv_raw));
    if (prompt_attn_fits(h))
        RC(arena_get(c, attn_prompt_kv_bytes(h.n_kv_heads, h.d_head, h.max_ctx) / sizeof(_Float16), &F.kv_hl));
    F.part_cap = prefill_part_floats(h);
    RC(arena_get(c, F.part_cap, &F.part));
    HC(hipHostMalloc((void **)&F.h_steps, (size_t)cap * 3 * 4, hipHostMallocDefault));
    HC(hipHostMalloc((void **)&F.h_slots, (size_t)cap * 4, hipHostMallocDefault));
    return E_OK;
}

int persist_capacity(int dt, int d_head, int kv_f16, int lds)
{
    switch (dt) {
    case DT_Q4_0: return persist_capacity_q4(d_head, kv_f16, lds);
    case DT_Q5_0: return persist_capacity_q5(d_head, kv_f16, lds);
    case DT_Q8_0: return persist_capacity_q8(d_head, kv_f16, lds);
    default: return 0;
    }
}

int launch_persist(int dt, const PkArgs &a, int nwg, int lds, hipStream_t s)
{
    switch (dt) {
    case DT_Q4_0: return launch_persist_q4(a, nwg, lds, s);
    case DT_Q5_0: return launch_persist_q5(a, nwg, lds, s);
    case DT_Q8_0: return launch_persist_q8(a, nwg, lds, s);
    default: return E_UNSUPPORTED;
    }
}

// Every exchange buffer of both parities filled with PK_POISON, the launch
// counter and error flag cleared (at creation, and after a launch whose wait
// gave up).
int persist_reset(cmolhip_model *m, hipStream_t st)
{
    m->pk_launches = 0;   // the next launch uses exchange set 0
    HC(hipMemsetD32Async((hipDeviceptr_t)m->pk_ex, (int)PK_POISON, m->pk_ex_n, st));
    HC(hipMemsetAsync(m->pk.err, 0, 4, st));
    return E_OK;
}

// Exchange buffers and launch arguments of the persistent kernel (after the
// weights and caches exist).  The kernel stays off (pk_dt = 0) when the
// device cannot keep a work-group per CU resident with its LDS needs.
int build_persist(cmolhip_model *m, int dt)
{
    cmolhip_ctx_t *c = m->ctx;
    const cmolhip_hparams_t &h = m->hp;
    const size_t d = h.d_model, kvd = (size_t)h.n_kv_heads * h.d_head, exn = pk_ex_floats(h);
    const int ms = persist_max_splits(h);
    std::vector<PkLayer> ly(h.n_layers);
    int opb = 0;
    auto need = [&](const cmolhip_qtensor_t &t) {
        const int b = pk_op_bytes(t.fold, t.block_quads);
        opb = b > opb ? b : opb;
    };
    // the embedding rows of both parities, then every layer's exchange
    // vectors: one block, filled with PK_POISON as a whole
    float *ex = nullptr;
    RC(arena_get(c, 2 * d + (size_t)2 * h.n_layers * exn, &ex));
    m->pk_ex = ex;
    m->pk_ex_n = 2 * d + (size_t)2 * h.n_layers * exn;
    float *const x0 = ex;
    ex += 2 * d;
    for (int l = 0; l < h.n_layers; l++) {
        const MLayer &L = m->layers[l];
        PkLayer &Y = ly[l];
        Y.qkv = to_qt(L.qkv[0]);   // one run: the persistent kernel needs uniform formats
        Y.o = to_qt(L.o);
        Y.gu = to_qt(L.gu);
        Y.down = to_qt(L.down);
        need(L.qkv[0]);
        need(L.o);
        need(L.gu);
        need(L.down);
        Y.attn_norm = L.attn_norm;
        Y.ffn_norm = L.ffn_norm;
        Y.rope_on = L.rope_on;
        Y.kv_off = (size_t)l * m->layer_stride;
        for (int p = 0; p < 2; p++) {
            float *b = ex + ((size_t)p * h.n_layers + l) * exn;
            PkEx &E = Y.ex[p];
            E.q = b;
            b += d;
            E.kn = b;
            b += kvd;
            E.vn = b;
            b += kvd;
            E.part = b;
            b += (size_t)h.n_heads * ms * (h.d_head + 4);
            E.att = b;
            b += d;
            E.xa = b;
            b += d;
            E.xo = b;
            b += d;
            E.h = b;
        }
    }
    const cmolhip_qtensor_t &lm = lm_tensor(m);
    need(lm);
    PkArgs &a = m->pk;
    a.n_layers = h.n_layers;
    a.embd = to_qt(m->embd);
    a.lm = to_qt(lm);
    a.out_norm = m->out_norm;
    a.rope = m->rope;
    a.x0 = x0;
    PkLayer *dl = nullptr;
    RC(cmolhip_alloc(c, ly.size() * sizeof(PkLayer), ALIGN, (void **)&dl));
    RC(cmolhip_memcpy_h2d(c, dl, ly.data(), ly.size() * sizeof(PkLayer)));
    a.layers = dl;
    a.k_base = m->kbase;
    a.v_base = m->vbase;
    a.slot_stride = m->slot_stride;
    a.d = h.d_model;
    a.n_heads = h.n_heads;
    a.n_kv = h.n_kv_heads;
    a.d_head = h.d_head;
    a.d_ffn = h.d_ffn;
    a.max_ctx = h.max_ctx;
    a.kv_f16 = h.kv_f16;
    a.max_splits = ms;
    a.op_bytes = opb;
    a.eps = h.rms_eps;
    RC(cmolhip_alloc(c, 4, ALIGN, (void **)&a.err));
    RC(persist_reset(m, c->stream));
    HC(hipHostMalloc((void **)&m->h_pk_err, 4, hipHostMallocDefault));
    if (persist_tracing()) {
        RC(arena_get(c, 2, &a.trace));
        RC(arena_get(c, (size_t)pk_stages(h.n_layers) * PK_MAX_WGS * PK_MARKS, &a.marks));
        HC(hipHostMalloc((void **)&m->h_trace, 2 * 8, hipHostMallocDefault));
    }
    const int G = h.n_heads / h.n_kv_heads;
    const int lds = pk_lds(opb, h.d_model, h.d_head, h.kv_f16, G, ms).total;
    const int nwg = persist_capacity(dt, h.d_head, h.kv_f16, lds);
    // every work-group at most one attention item and one merge item; the io
    // threads' operand share within PK_MAXI items
    int max_tiles = 0;   // tiles of one matrix per mac wave (the LM head finishes its tiles in registers)
    for (const PkLayer &Y : ly)
        for (const QTensor *t : {&Y.qkv, &Y.o, &Y.gu, &Y.down}) {
            const int w = PK_MAC * persist_wgs(), n = (t->row_tiles + w - 1) / w;
            max_tiles = n > max_tiles ? n : max_tiles;
        }
    const bool fits = nwg == persist_wgs() && (size_t)ms * h.n_kv_heads <= (size_t)nwg && max_tiles <= PK_ZW_TILES &&
                      h.n_heads * (h.d_head / PK_MSLICE) <= nwg && h.d_head % PK_MSLICE == 0 &&
                      h.d_ffn / 8 <= PK_MAXI * 64 * PK_IO && h.d_model / 8 <= PK_MAXI * 64 * PK_IO &&
                      ms * 9 <= 12 * 64 * PK_IO && G <= ATT_MAX_G;
    if (nwg < 1 || !fits) return E_OK;   // stays off
    m->pk_dt = dt;
    m->pk_nwg = nwg;
    m->pk_lds = lds;
    return E_OK;
}

// Steps whose persistent wait gave up before the model stays on the graph.
constexpr int PK_GIVEUP_MAX = 4;

// One decode step of the single session with the persistent kernel (the
// step record is already on its way to B.steps on B.st).
int run_persist(cmolhip_model *m, Batch &B)
{
    PkArgs a = m->pk;
    a.par = (int)(m->pk_launches & 1u);   // launches are serialised by the session's lock
    m->pk_launches++;
    a.step = B.steps;
    a.slot_id = B.slot_ids;
    a.logits = B.logits;
    a.argmax = B.argmax;
    RC(launch_persist(m->pk_dt, a, m->pk_nwg, m->pk_lds, B.st));
    HC(hipMemcpyAsync(m->h_pk_err, a.err, 4, hipMemcpyDeviceToHost, B.st));
    if (a.trace) {
        m->trace_n = 2;
        HC(hipMemcpyAsync(m->h_trace, a.trace, 2 * 8, hipMemcpyDeviceToHost, B.st));
    }
    return E_OK;
}

// After the step's synchronisation: a wait that gave up leaves the step's
// outputs invalid and the exchange buffers in an unknown state; they are
// poisoned again for the next step.
int persist_check(cmolhip_model *m, Batch &B)
{
    if (!*m->h_pk_err) return E_OK;
    RC(persist_reset(m, B.st));
    HC(hipStreamSynchronize(B.st));
    *m->h_pk_err = 0;
    return E_UNSUPPORTED;
}

int build_model(cmolhip_model *m, const cmolhip_model_desc_t *d, const Plan &P)
{
    cmolhip_ctx_t *c = m->ctx;
    const cmolhip_hparams_t &h = d->hp;
    void *stg = nullptr;
    RC(cmolhip_alloc(c, P.staging, ALIGN, &stg));
    m->qk_norm = has_qk_norm(d);
    m->layers.resize(h.n_layers);
    for (int l = 0; l < h.n_layers; l++) {
        const cmolhip_layer_tensors_t &T = d->layers[l];
        MLayer &L = m->layers[l];
        const cmolhip_host_tensor_t *qkv[3] = {&T.q, &T.k, &T.v};
        const QkvRuns R = qkv_runs(T, h);
        L.n_qkv = R.n;
        for (int r = 0, row0 = 0; r < R.n; r++) {
            L.qkv_row0[r] = row0;
            RC(upload_q(c, R.count[r], qkv + R.first[r], CMOLHIP_PARTS_CONCAT,
                        layer_fold(d, R.rows[r], h.d_model), stg, P.staging, &L.qkv[r]));
            row0 += R.rows[r];
        }
        const cmolhip_host_tensor_t *o[1] = {&T.o};
        RC(upload_q(c, 1, o, CMOLHIP_PARTS_CONCAT, layer_fold(d, h.d_model, h.d_model), stg,
                    P.staging, &L.o));
        const cmolhip_host_tensor_t *gu[2] = {&T.gate, &T.up};
        RC(upload_q(c, 2, gu, CMOLHIP_PARTS_INTERLEAVE, layer_fold(d, 2 * h.d_ffn, h.d_model), stg,
                    P.staging, &L.gu));
        const cmolhip_host_tensor_t *dn[1] = {&T.down};
        RC(upload_q(c, 1, dn, CMOLHIP_PARTS_CONCAT, layer_fold(d, h.d_model, h.d_ffn), stg,
                    P.staging, &L.down));
        RC(upload_norm(c, T.attn_norm, &L.attn_norm));
        RC(upload_norm(c, T.ffn_norm, &L.ffn_norm));
        if (T.q_norm.data) RC(upload_norm(c, T.q_norm, &L.q_norm));
        if (T.k_norm.data) RC(upload_norm(c, T.k_norm, &L.k_norm));
        L.rope_on = !(h.no_rope_interval > 0 && (l + 1) % h.no_rope_interval == 0);
    }
    const cmolhip_host_tensor_t *e[1] = {&d->embd};
    RC(upload_q(c, 1, e, CMOLHIP_PARTS_CONCAT, head_fold(d), stg, P.staging, &m->embd));
    if (d->lm_head.data) {
        const cmolhip_host_tensor_t *lh[1] = {&d->lm_head};
        RC(upload_q(c, 1, lh, CMOLHIP_PARTS_CONCAT, head_fold(d), stg, P.staging, &m->lm));
    }
    RC(upload_norm(c, d->out_norm, &m->out_norm));
    auto fold_of = [&](const cmolhip_qtensor_t &t) { m->max_fold = t.fold > m->max_fold ? t.fold : m->max_fold; };
    for (const MLayer &L : m->layers) {
        for (int r = 0; r < L.n_qkv; r++) fold_of(L.qkv[r]);
        fold_of(L.o);
        fold_of(L.gu);
        fold_of(L.down);
    }
    fold_of(m->embd);
    if (m->lm.qs) fold_of(m->lm);
    const size_t rope_n = (size_t)h.max_ctx * (h.d_head / 2) * 2;
    RC(arena_get(c, rope_n, &m->rope));
    RC(cmolhip_memcpy_h2d(c, m->rope, d->rope_table, rope_n * 4));
    const size_t esz = h.kv_f16 ? 2 : 4;
    m->layer_stride = (size_t)h.n_kv_heads * h.max_ctx * h.d_head;
    m->slot_stride = m->layer_stride * h.n_layers;
    const size_t kv_elems = m->slot_stride * h.max_sessions;
    RC(cmolhip_alloc(c, kv_elems * esz, ALIGN, &m->kbase));
    RC(cmolhip_alloc(c, kv_elems * esz, ALIGN, &m->vbase));
    HC(hipMemsetAsync(m->kbase, 0, kv_elems * esz, c->stream));
    HC(hipMemsetAsync(m->vbase, 0, kv_elems * esz, c->stream));
    RC(arena_get(c, (size_t)h.n_kv_heads * h.max_ctx * h.d_head, &m->scratch));
    m->split = pick_split(h.max_ctx);
    m->max_splits = attn_max_splits(h.max_ctx, m->split);
    for (int s = 0; s < h.max_sessions; s++) {
        m->slots.emplace_back(new Batch());
        Batch &B = *m->slots.back();
        RC(build_batch(m, B, 1, batch_part_floats(d, 1)));
        const int32_t sid = s;
        RC(cmolhip_memcpy_h2d(c, B.slot_ids, &sid, 4));
    }
    m->multi.reset(new Batch());
    RC(build_batch(m, *m->multi, multi_cap(h), batch_part_floats(d, multi_cap(h))));
    m->pf.reset(new Prefill());
    RC(build_prefill(m, *m->pf));
    if (persist_format(d)) RC(build_persist(m, persist_format(d)));
    HC(hipStreamSynchronize(c->stream));
    if (m->use_graph) {
        for (auto &sp : m->slots) {
            Batch &B = *sp;
            HC(hipStreamBeginCapture(B.st, hipStreamCaptureModeThreadLocal));
            int rc = enqueue_step(m, B, 1, B.st);
            hipError_t ce = hipStreamEndCapture(B.st, &B.graph);
            if (rc) return rc;
            HC(ce);
            HC(hipGraphInstantiate(&B.gexec, B.graph, nullptr, nullptr, 0));
        }
        // the shared batch: every per-step input (tokens, positions, cache
        // slots) lives in device buffers, so one capture per vector count
        // replays any step of that size
        Batch &M = *m->multi;
        M.gexec_n.assign(M.cap, nullptr);
        for (int n = 1; n <= M.cap; n++) {
            hipGraph_t gr = nullptr;
            if (hipStreamBeginCapture(M.st, hipStreamCaptureModeThreadLocal) != hipSuccess) break;
            const int rc = enqueue_step(m, M, n, M.st);
            const hipError_t ce = hipStreamEndCapture(M.st, &gr);
            if (rc == E_OK && ce == hipSuccess && gr) {
                if (hipGraphInstantiate(&M.gexec_n[n - 1], gr, nullptr, nullptr, 0) != hipSuccess)
                    M.gexec_n[n - 1] = nullptr;
            }
            if (gr) (void)hipGraphDestroy(gr);
            (void)hipGetLastError();   // a failed capture leaves that count on stream launches
        }
    }
    return E_OK;
}

unsigned long long reduce_slots(const unsigned long long *k)
{
    unsigned long long best = 0;
    for (int i = 0; i < ARGMAX_SLOTS; i++) best = k[i] > best ? k[i] : best;
    return best;
}

// One step of the shared batch over its first n vectors: the captured
// graph of that count, else stream launches.
int run_multi(cmolhip_model *m, Batch &B, int n)
{
    if (n >= 1 && n <= (int)B.gexec_n.size() && B.gexec_n[n - 1]) {
        HC(hipGraphLaunch(B.gexec_n[n - 1], B.st));
        return E_OK;
    }
    return enqueue_step(m, B, n, B.st);
}

int run_single(cmolhip_model *m, Batch &B)
{
    if (B.gexec) {
        HC(hipGraphLaunch(B.gexec, B.st));
        return E_OK;
    }
    return enqueue_step(m, B, 1, B.st);
}

int finish(cmolhip_model *m, Batch &B, int n, float *logits_host, int32_t *argmax,
           float *const *logits_each = nullptr)
{
    HC(hipMemcpyAsync(B.h_argmax, B.argmax, (size_t)n * ARGMAX_SLOTS * 8, hipMemcpyDeviceToHost, B.st));
    const size_t V = m->hp.vocab;
    if (logits_host) HC(hipMemcpyAsync(logits_host, B.logits, n * V * 4, hipMemcpyDeviceToHost, B.st));
    if (logits_each)
        for (int i = 0; i < n; i++)
            if (logits_each[i])
                HC(hipMemcpyAsync(logits_each[i], B.logits + i * V, V * 4, hipMemcpyDeviceToHost, B.st));
    HC(hipStreamSynchronize(B.st));
    if (argmax)
        for (int i = 0; i < n; i++)
            argmax[i] = (int32_t)argmax_index(reduce_slots(B.h_argmax + (size_t)i * ARGMAX_SLOTS));
    return E_OK;
}

void destroy_batch(Batch &B)
{
    if (B.st) (void)hipStreamSynchronize(B.st);
    if (B.gexec) (void)hipGraphExecDestroy(B.gexec);
    for (hipGraphExec_t e : B.gexec_n)
        if (e) (void)hipGraphExecDestroy(e);
    if (B.graph) (void)hipGraphDestroy(B.graph);
    if (B.st) (void)hipStreamDestroy(B.st);
    if (B.h_steps) (void)hipHostFree(B.h_steps);
    if (B.h_slots) (void)hipHostFree(B.h_slots);
    if (B.h_argmax) (void)hipHostFree(B.h_argmax);
}

int decode_batch(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *tokens, const int32_t *pos,
                 float *logits_host, float *const *logits_each, int32_t *argmax);

// A short prompt of session `slot` as one lock-step step of the matvec path:
// vector i is tokens[i] at pos0 + i in the same cache.  The QKV kernel writes
// every vector's K/V before the attention kernel reads positions < pos + 1,
// so vector i attends to the prompt's earlier tokens as in a causal pass.
// Outputs (logits, argmax) are the last vector's.
int prompt_by_matvec(cmolhip_model_t *m, int slot, const int32_t *tokens, int n, int32_t pos0,
                     float *logits_host, int32_t *argmax)
{
    Batch &B = *m->multi;
    if (n > B.cap) return E_ARGS;
    std::lock_guard<std::mutex> g(B.mu);   // same order as decode_batch: batch, then slot
    std::lock_guard<std::mutex> gs(m->slots[slot]->mu);
    for (int i = 0; i < n; i++) {
        B.h_steps[3 * i + 0] = tokens[i];
        B.h_steps[3 * i + 1] = pos0 + i;
        B.h_steps[3 * i + 2] = pos0 + i + 1;
        B.h_slots[i] = slot;
    }
    HC(hipMemcpyAsync(B.steps, B.h_steps, (size_t)n * 12, hipMemcpyHostToDevice, B.st));
    HC(hipMemcpyAsync(B.slot_ids, B.h_slots, (size_t)n * 4, hipMemcpyHostToDevice, B.st));
    RC(run_multi(m, B, n));
    const size_t V = m->hp.vocab;
    HC(hipMemcpyAsync(B.h_argmax, B.argmax + (size_t)(n - 1) * ARGMAX_SLOTS, ARGMAX_SLOTS * 8,
                      hipMemcpyDeviceToHost, B.st));
    if (logits_host)
        HC(hipMemcpyAsync(logits_host, B.logits + (n - 1) * V, V * 4, hipMemcpyDeviceToHost, B.st));
    HC(hipStreamSynchronize(B.st));
    if (argmax) *argmax = (int32_t)argmax_index(reduce_slots(B.h_argmax));
    return E_OK;
}

} // namespace

extern "C" {

int cmolhip_model_plan(const cmolhip_model_desc_t *desc, size_t *device_bytes)
{
    if (!device_bytes) return E_ARGS;
    RC(validate_desc(desc));
    *device_bytes = make_plan(desc).total();
    return E_OK;
}

size_t cmolhip_gemv_scratch_floats(int dtype, int rows, int cols, int fold, int n)
{
    if (!is_block_fmt(dtype) || rows < 1 || cols < 32 || cols % 32 || n < 1 || n > 32 ||
        (fold != 1 && fold != 2 && fold != 4 && fold != 8))
        return 0;
    return gemv_part_floats(shape_qt(dtype, rows, cols, fold), n);
}

int cmolhip_batch_scratch_floats(const cmolhip_model_desc_t *desc, int cap, size_t *floats)
{
    if (!floats || cap < 1 || cap > 32) return E_ARGS;
    RC(validate_desc(desc));
    *floats = batch_part_floats(desc, cap);
    return E_OK;
}

int cmolhip_model_create(const cmolhip_model_desc_t *desc, int device, cmolhip_model_t **out)
{
    if (!out) return E_ARGS;
    *out = nullptr;
    RC(validate_desc(desc));
    Plan P = make_plan(desc);
    cmolhip_model *m = new (std::nothrow) cmolhip_model();
    if (!m) return E_OOM;
    m->hp = desc->hp;
    const char *g = getenv("CMOL_HIP_GRAPH");
    m->use_graph = !(g && g[0] == '0');
    int rc = cmolhip_ctx_create(device, P.total(), &m->ctx);
    if (rc == E_OK) rc = build_model(m, desc, P);
    if (rc != E_OK) {
        cmolhip_model_destroy(m);
        return rc;
    }
    *out = m;
    return E_OK;
}

void cmolhip_model_destroy(cmolhip_model_t *m)
{
    if (!m) return;
    if (m->ctx) (void)hipSetDevice(m->ctx->device);
    for (auto &sp : m->slots) destroy_batch(*sp);
    if (m->multi) destroy_batch(*m->multi);
    if (m->pf) {
        if (m->pf->h_steps) (void)hipHostFree(m->pf->h_steps);
        if (m->pf->h_slots) (void)hipHostFree(m->pf->h_slots);
    }
    if (m->h_pk_err) (void)hipHostFree(m->h_pk_err);
    if (m->h_trace) (void)hipHostFree(m->h_trace);
    cmolhip_ctx_destroy(m->ctx);
    delete m;
}

cmolhip_ctx_t *cmolhip_model_ctx(cmolhip_model_t *m) { return m ? m->ctx : nullptr; }

void *cmolhip_session_stream(cmolhip_model_t *m, int slot)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size()) return nullptr;
    return (void *)m->slots[slot]->st;
}

int cmolhip_decode(cmolhip_model_t *m, int slot, int32_t token, int32_t pos, float *logits_host,
                   int32_t *argmax)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size()) return E_ARGS;
    if (token < 0 || token >= m->hp.vocab || pos < 0 || pos >= m->hp.max_ctx) return E_ARGS;
    Batch &B = *m->slots[slot];
    std::lock_guard<std::mutex> g(B.mu);
    B.h_steps[0] = token;
    B.h_steps[1] = pos;
    B.h_steps[2] = pos + 1;
    HC(hipMemcpyAsync(B.steps, B.h_steps, 12, hipMemcpyHostToDevice, B.st));
    if (m->pk_dt) {
        RC(run_persist(m, B));
        RC(finish(m, B, 1, logits_host, argmax));
        const int rc = persist_check(m, B);
        if (rc != E_UNSUPPORTED) return rc;
        // a wait gave up (a slow or contended step): the decode graph redoes
        // the step from the record already in B.steps (it rewrites the same
        // cache row); after PK_GIVEUP_MAX such steps the model stays on the graph
        if (++m->pk_giveups >= PK_GIVEUP_MAX) m->pk_dt = 0;
    }
    RC(run_single(m, B));
    return finish(m, B, 1, logits_host, argmax);
}

int cmolhip_model_persistent(cmolhip_model_t *m) { return m && m->pk_dt ? 1 : 0; }

int cmolhip_persist_marks(cmolhip_model_t *m, uint64_t *out, size_t cap)
{
    if (!m || !out) return E_ARGS;
    if (!m->pk.marks || !m->trace_n) return 0;
    const size_t n = (size_t)pk_stages(m->hp.n_layers) * m->pk_nwg * PK_MARKS;
    if (cap < n) return E_TRUNC;
    HC(hipMemcpy(out, m->pk.marks, n * 8, hipMemcpyDeviceToHost));
    return m->pk_nwg;
}

int cmolhip_persist_trace(cmolhip_model_t *m, uint64_t *out, int cap)
{
    if (!m || !out || cap < 0) return E_ARGS;
    if (!m->h_trace) return 0;
    const int n = m->trace_n < cap ? m->trace_n : cap;
    for (int i = 0; i < n; i++) out[i] = m->h_trace[i];
    return n;
}

int cmolhip_prefill(cmolhip_model_t *m, int slot, const int32_t *tokens, int n, int32_t pos0,
                    float *logits_host, int32_t *argmax)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size() || !tokens || n < 1) return E_ARGS;
    if (pos0 < 0 || (long)pos0 + n > m->hp.max_ctx) return E_ARGS;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->hp.vocab) return E_ARGS;
    if (n == 1) return cmolhip_decode(m, slot, tokens[0], pos0, logits_host, argmax);
    // a few tokens run as one lock-step matvec step (its MFMA rows hold
    // 2 n fold <= 64 operand rows), longer prompts as GEMM passes
    if (n <= PROMPT_MATVEC_MAX && n * m->max_fold <= 32)
        return prompt_by_matvec(m, slot, tokens, n, pos0, logits_host, argmax);
    Batch &B = *m->slots[slot];
    Prefill &F = *m->pf;
    std::lock_guard<std::mutex> g(B.mu);
    std::lock_guard<std::mutex> gf(F.mu);
    for (int i = 0; i < F.cap; i++) F.h_slots[i] = slot;
    HC(hipMemcpyAsync(F.slot_ids, F.h_slots, (size_t)F.cap * 4, hipMemcpyHostToDevice, B.st));
    for (int c0 = 0; c0 < n; c0 += F.cap) {
        const int nc = n - c0 < F.cap ? n - c0 : F.cap;
        // the pinned step records are reused: wait for the previous pass's copy
        if (c0) HC(hipStreamSynchronize(B.st));
        for (int i = 0; i < nc; i++) {
            F.h_steps[3 * i + 0] = tokens[c0 + i];
            F.h_steps[3 * i + 1] = pos0 + c0 + i;
            F.h_steps[3 * i + 2] = pos0 + c0 + i + 1;
        }
        HC(hipMemcpyAsync(F.steps, F.h_steps, (size_t)nc * 12, hipMemcpyHostToDevice, B.st));
        RC(enqueue_prefill(m, F, B, nc, c0 + nc == n, B.st));
    }
    return finish(m, B, 1, logits_host, argmax);
}

int cmolhip_decode_batch(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *tokens,
                         const int32_t *pos, float *logits_host, int32_t *argmax)
{
    return decode_batch(m, n, slots, tokens, pos, logits_host, nullptr, argmax);
}

int cmolhip_decode_batch_each(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *tokens,
                              const int32_t *pos, float *const *logits_each, int32_t *argmax)
{
    return decode_batch(m, n, slots, tokens, pos, nullptr, logits_each, argmax);
}

} // extern "C"

namespace {

int decode_batch(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *tokens, const int32_t *pos,
                 float *logits_host, float *const *logits_each, int32_t *argmax)
{
    if (!m || n < 1 || n > m->hp.max_sessions || !slots || !tokens || !pos) return E_ARGS;
    for (int i = 0; i < n; i++) {
        if (slots[i] < 0 || slots[i] >= (int)m->slots.size()) return E_ARGS;
        if (tokens[i] < 0 || tokens[i] >= m->hp.vocab || pos[i] < 0 || pos[i] >= m->hp.max_ctx)
            return E_ARGS;
        for (int j = 0; j < i; j++)
            if (slots[j] == slots[i]) return E_ARGS;
    }
    Batch &B = *m->multi;
    std::lock_guard<std::mutex> g(B.mu);
    // the KV caches of these sessions are written: exclude their own decodes,
    // locking the slots in ascending order (fixed arrays: a step allocates
    // nothing)
    int order[32];
    for (int i = 0; i < n; i++) {
        int j = i;
        for (; j > 0 && order[j - 1] > slots[i]; j--) order[j] = order[j - 1];
        order[j] = slots[i];
    }
    for (int i = 0; i < n; i++) m->slots[order[i]]->mu.lock();
    struct Unlock {
        cmolhip_model_t *m;
        const int *order;
        int n;
        ~Unlock()
        {
            for (int i = n - 1; i >= 0; i--) m->slots[order[i]]->mu.unlock();
        }
    } unlock{m, order, n};
    for (int i = 0; i < n; i++) {
        B.h_steps[3 * i + 0] = tokens[i];
        B.h_steps[3 * i + 1] = pos[i];
        B.h_steps[3 * i + 2] = pos[i] + 1;
        B.h_slots[i] = slots[i];
    }
    HC(hipMemcpyAsync(B.steps, B.h_steps, (size_t)n * 12, hipMemcpyHostToDevice, B.st));
    HC(hipMemcpyAsync(B.slot_ids, B.h_slots, (size_t)n * 4, hipMemcpyHostToDevice, B.st));
    RC(run_multi(m, B, n));
    return finish(m, B, n, logits_host, argmax, logits_each);
}

} // namespace

extern "C" {

int cmolhip_kv_download(cmolhip_model_t *m, int slot, int layer, int n, float *k_out, float *v_out)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size() || layer < 0 || layer >= m->hp.n_layers ||
        n < 0 || n > m->hp.max_ctx || !k_out || !v_out)
        return E_ARGS;
    const cmolhip_hparams_t &h = m->hp;
    const size_t esz = h.kv_f16 ? 2 : 4;
    const size_t off = ((size_t)slot * m->slot_stride + (size_t)layer * m->layer_stride) * esz;
    const size_t cnt = (size_t)n * h.n_kv_heads * h.d_head;
    std::lock_guard<std::mutex> g(m->scratch_mu);
    hipStream_t st = m->ctx->stream;
    HC(hipStreamSynchronize(m->slots[slot]->st));
    HC(hipStreamSynchronize(m->multi->st));
    for (int w = 0; w < 2; w++) {
        const uint8_t *src = (const uint8_t *)(w ? m->vbase : m->kbase) + off;
        RC(launch_kv_convert(src, m->scratch, h.n_kv_heads, h.max_ctx, h.d_head, n, h.kv_f16, 1, st));
        RC(cmolhip_memcpy_d2h(m->ctx, w ? v_out : k_out, m->scratch, cnt * 4));
    }
    return E_OK;
}

int cmolhip_kv_upload(cmolhip_model_t *m, int slot, int layer, int n, const float *k_in,
                      const float *v_in)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size() || layer < 0 || layer >= m->hp.n_layers ||
        n < 0 || n > m->hp.max_ctx || !k_in || !v_in)
        return E_ARGS;
    const cmolhip_hparams_t &h = m->hp;
    const size_t esz = h.kv_f16 ? 2 : 4;
    const size_t off = ((size_t)slot * m->slot_stride + (size_t)layer * m->layer_stride) * esz;
    const size_t cnt = (size_t)n * h.n_kv_heads * h.d_head;
    std::lock_guard<std::mutex> g(m->scratch_mu);
    hipStream_t st = m->ctx->stream;
    HC(hipStreamSynchronize(m->slots[slot]->st));
    HC(hipStreamSynchronize(m->multi->st));
    for (int w = 0; w < 2; w++) {
        uint8_t *dst = (uint8_t *)(w ? m->vbase : m->kbase) + off;
        RC(cmolhip_memcpy_h2d(m->ctx, m->scratch, w ? v_in : k_in, cnt * 4));
        RC(launch_kv_import(m->scratch, dst, h.n_kv_heads, h.max_ctx, h.d_head, n, h.kv_f16, st));
        HC(hipStreamSynchronize(st));
    }
    return E_OK;
}

int cmolhip_kv_fill_synthetic(cmolhip_model_t *m, int slot, int n, uint64_t seed)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size() || n < 0 || n > m->hp.max_ctx) return E_ARGS;
    const cmolhip_hparams_t &h = m->hp;
    const size_t esz = h.kv_f16 ? 2 : 4;
    hipStream_t st = m->ctx->stream;
    HC(hipStreamSynchronize(m->slots[slot]->st));
    HC(hipStreamSynchronize(m->multi->st));
    for (int l = 0; l < h.n_layers; l++) {
        const size_t off = ((size_t)slot * m->slot_stride + (size_t)l * m->layer_stride) * esz;
        RC(launch_kv_synth((uint8_t *)m->kbase + off, (uint8_t *)m->vbase + off, h.n_kv_heads,
                           h.max_ctx, h.d_head, n, h.kv_f16, seed + (uint64_t)l * 0x9E37ull, st));
    }
    HC(hipStreamSynchronize(st));
    return E_OK;
}

} // extern "C"
