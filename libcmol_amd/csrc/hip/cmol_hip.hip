// cmol_hip.hip — C ABI of the gfx950 backend (include/cmol_hip.h).
//
// Owns the device context (one arena from one hipMalloc, one upload stream),
// quantised-tensor upload/repack, the standalone kernel entry points and the
// whole-model decode path: per-session streams and buffers, the per-session
// decode step captured once as a HIP graph at load, prefill, KV access.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <vector>

#include "../../../include/cmol_hip.h"
#include "common.h"
#include "kernels.h"

namespace {

constexpr int E_OK = 0, E_OOM = -1, E_INVALID = -3, E_UNSUPPORTED = -4, E_ARGS = -6;
constexpr size_t ALIGN = 256;

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

bool qlayout(int dtype, int rows, int cols, QLayout *L)
{
    if (dtype != DT_Q4_0 && dtype != DT_Q5_0 && dtype != DT_Q8_0) return false;
    if (rows <= 0 || cols <= 0 || cols % 32) return false;
    L->rt = (rows + 15) / 16;
    L->bq = (cols / 32 + 3) / 4;
    size_t cells = (size_t)L->rt * L->bq;
    L->qs = cells * 64 * lane_bytes_of(dtype);
    L->d = cells * 64 * 2;
    L->qh = dtype == DT_Q5_0 ? cells * 64 * 4 : 0;
    return true;
}

size_t qbytes_aligned(int dtype, int rows, int cols)
{
    QLayout L;
    if (!qlayout(dtype, rows, cols, &L)) return 0;
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
    return q;
}

size_t raw_row_bytes(int dtype, int cols)
{
    int bb = block_bytes_of(dtype);
    return bb ? (size_t)(cols / 32) * bb : 0;
}

} // namespace

struct cmolhip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint8_t *arena = nullptr;
    size_t size = 0, used = 0;
    std::mutex mu;
};

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
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return E_UNSUPPORTED;
    }
    if (bytes) {
        if (hipMalloc((void **)&c->arena, bytes) != hipSuccess) {
            (void)hipGetLastError();
            hipStreamDestroy(c->stream);
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
    hipSetDevice(c->device);
    if (c->stream) {
        hipStreamSynchronize(c->stream);
        hipStreamDestroy(c->stream);
    }
    if (c->arena) hipFree(c->arena);
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

size_t cmolhip_qtensor_bytes(int dtype, int rows, int cols) { return qbytes_aligned(dtype, rows, cols); }

int cmolhip_qtensor_upload(cmolhip_ctx_t *c, int dtype, int cols, int n_parts,
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
    if (!qlayout(dtype, (int)rows, cols, &L)) return E_UNSUPPORTED;
    cmolhip_qtensor_t t{};
    RC(cmolhip_alloc(c, L.qs, ALIGN, &t.qs));
    RC(cmolhip_alloc(c, L.d, ALIGN, &t.d));
    if (L.qh) RC(cmolhip_alloc(c, L.qh, ALIGN, &t.qh));
    t.dtype = dtype;
    t.rows = (int)rows;
    t.cols = cols;
    t.row_tiles = L.rt;
    t.block_quads = L.bq;
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

int cmolhip_gemm(cmolhip_ctx_t *c, const cmolhip_qtensor_t *w, const float *dx, float *dy, int n,
                 const float *norm_w, float eps)
{
    if (!c || !w || !dx || !dy || n < 1 || n > 32) return E_ARGS;
    for (int i = 0; i < n; i++) {
        GemvArgs a{};
        a.w = to_qt(*w);
        a.x = dx + (size_t)i * w->cols;
        a.x_stride = w->cols;
        a.norm_w = norm_w;
        a.eps = eps;
        a.out = dy + (size_t)i * w->rows;
        a.out_stride = w->rows;
        a.n = 1;
        RC(launch_gemv(a, EPI_STORE, c->stream));
    }
    return E_OK;
}

int cmolhip_matmul_host(cmolhip_ctx_t *c, float *out, const void *a, const float *b, int m, int k,
                        int n, int dtype)
{
    if (!c || !out || !a || !b || m < 1 || k < 32 || k % 32 || n < 1 || n > 32) return E_ARGS;
    if (!qbytes_aligned(dtype, m, k)) return E_UNSUPPORTED;
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        const size_t rb = raw_row_bytes(dtype, k);
        void *staging = nullptr;
        float *dx = nullptr, *dy = nullptr;
        cmolhip_qtensor_t t{};
        if ((rc = cmolhip_alloc(c, rb * (size_t)m, ALIGN, &staging))) break;
        if ((rc = arena_get(c, (size_t)k * n, &dx))) break;
        if ((rc = arena_get(c, (size_t)m * n, &dy))) break;
        const void *parts[1] = {a};
        const int32_t rows[1] = {m};
        if ((rc = cmolhip_qtensor_upload(c, dtype, k, 1, parts, rows, CMOLHIP_PARTS_CONCAT, staging,
                                         rb * (size_t)m, &t)))
            break;
        std::vector<float> xt((size_t)k * n), yt((size_t)m * n);
        for (int ki = 0; ki < k; ki++)
            for (int ni = 0; ni < n; ni++) xt[(size_t)ni * k + ki] = b[(size_t)ki * n + ni];
        if ((rc = cmolhip_memcpy_h2d(c, dx, xt.data(), xt.size() * 4))) break;
        if ((rc = cmolhip_gemm(c, &t, dx, dy, n, nullptr, 0.0f))) break;
        if ((rc = cmolhip_memcpy_d2h(c, yt.data(), dy, yt.size() * 4))) break;
        for (int mi = 0; mi < m; mi++)
            for (int ni = 0; ni < n; ni++) out[(size_t)mi * n + ni] = yt[(size_t)ni * m + mi];
    } while (0);
    arena_release(c, mark);
    return rc;
}

int cmolhip_attn_decode(cmolhip_ctx_t *c, int n, const float *q, const void *kcache,
                        const void *vcache, const int32_t *seqlen, int n_heads, int n_kv, int d_head,
                        int max_ctx, int kv_f16, float *out)
{
    if (!c || n < 1 || !q || !kcache || !vcache || !seqlen || !out || n_kv < 1 || n_heads < n_kv ||
        n_heads % n_kv || max_ctx < 1)
        return E_ARGS;
    const int G = n_heads / n_kv, split = 64, ms = attn_max_splits(max_ctx, split);
    const size_t mark = arena_mark(c);
    int rc = E_OK;
    do {
        float *pm, *pl, *po;
        int32_t *ids;
        const size_t np = (size_t)n * n_kv * ms * G;
        if ((rc = arena_get(c, np, &pm)) || (rc = arena_get(c, np, &pl)) ||
            (rc = arena_get(c, np * d_head, &po)) || (rc = arena_get(c, (size_t)n, &ids)))
            break;
        std::vector<int32_t> hid(n);
        for (int i = 0; i < n; i++) hid[i] = i;
        if ((rc = cmolhip_memcpy_h2d(c, ids, hid.data(), (size_t)n * 4))) break;
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
    cmolhip_qtensor_t qkv{}, o{}, gu{}, down{};
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    int rope_on = 1;
};

struct MSlot {
    hipStream_t st = nullptr;
    int32_t *step = nullptr;      // device {token, pos, seqlen}
    int32_t *steps = nullptr;     // device prompt step records [max_ctx][3]
    int32_t *slot_id = nullptr;   // device: this slot's index
    float *x = nullptr, *q = nullptr, *ao = nullptr, *h = nullptr, *logits = nullptr;
    unsigned long long *argmax = nullptr;
    float *pm = nullptr, *pl = nullptr, *po = nullptr;
    int32_t *h_steps = nullptr;   // pinned host [max_ctx][3]
    unsigned long long *h_argmax = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    std::mutex mu;
};

constexpr int ATTN_SPLIT_MIN = 64, ATTN_SPLIT_MAX = 256;

int pick_split(int max_ctx)
{
    int s = max_ctx / 64;
    s = (s + 63) / 64 * 64;
    if (s < ATTN_SPLIT_MIN) s = ATTN_SPLIT_MIN;
    if (s > ATTN_SPLIT_MAX) s = ATTN_SPLIT_MAX;
    return s;
}

bool is_block_fmt(int dt) { return dt == DT_Q4_0 || dt == DT_Q5_0 || dt == DT_Q8_0; }

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

void add_q(Plan &P, int dt, int rows, int cols)
{
    QLayout L;
    qlayout(dt, rows, cols, &L);
    P.add(L.qs);
    P.add(L.d);
    if (L.qh) P.add(L.qh);
}

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
        if (L.q.dtype != L.k.dtype || L.q.dtype != L.v.dtype || L.gate.dtype != L.up.dtype)
            return E_UNSUPPORTED;
        if (!chk_norm(L.attn_norm, h.d_model) || !chk_norm(L.ffn_norm, h.d_model)) return E_INVALID;
        if (L.q_norm.data || L.k_norm.data) return E_UNSUPPORTED;
    }
    return E_OK;
}

Plan make_plan(const cmolhip_model_desc_t *d)
{
    const cmolhip_hparams_t &h = d->hp;
    const int kvd = h.n_kv_heads * h.d_head, G = h.n_heads / h.n_kv_heads;
    const int ms = attn_max_splits(h.max_ctx, pick_split(h.max_ctx));
    Plan P;
    // staging: largest raw tensor, capped (uploads are chunked)
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
        add_q(P, L.q.dtype, h.d_model + 2 * kvd, h.d_model);
        add_q(P, L.o.dtype, h.d_model, h.d_model);
        add_q(P, L.gate.dtype, 2 * h.d_ffn, h.d_model);
        add_q(P, L.down.dtype, h.d_model, h.d_ffn);
        P.add((size_t)h.d_model * 4);
        P.add((size_t)h.d_model * 4);
    }
    add_q(P, d->embd.dtype, h.vocab, h.d_model);
    if (d->lm_head.data) add_q(P, d->lm_head.dtype, h.vocab, h.d_model);
    P.add((size_t)h.d_model * 4);                                   // out_norm
    P.add((size_t)h.max_ctx * (h.d_head / 2) * 2 * 4);              // rope
    const size_t esz = h.kv_f16 ? 2 : 4;
    const size_t kv_elems = (size_t)h.max_sessions * h.n_layers * h.n_kv_heads * h.max_ctx * h.d_head;
    P.add(kv_elems * esz);
    P.add(kv_elems * esz);
    P.add((size_t)h.n_kv_heads * h.max_ctx * h.d_head * 4);         // scratch
    const size_t np = (size_t)h.n_kv_heads * ms * G;
    for (int s = 0; s < h.max_sessions; s++) {
        P.add(16);
        P.add((size_t)h.max_ctx * 3 * 4);
        P.add(4);
        P.add((size_t)h.d_model * 4);
        P.add((size_t)h.d_model * 4);
        P.add((size_t)h.d_model * 4);
        P.add((size_t)h.d_ffn * 4);
        P.add((size_t)h.vocab * 4);
        P.add(8 * ARGMAX_SLOTS);
        P.add(np * 4);
        P.add(np * 4);
        P.add(np * h.d_head * 4);
    }
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
    std::vector<std::unique_ptr<MSlot>> slots;
    std::mutex scratch_mu;
    bool use_graph = true;
};

namespace {

KVRef kvref(const cmolhip_model *m, const MSlot &S, int layer)
{
    KVRef r;
    r.k_base = m->kbase;
    r.v_base = m->vbase;
    r.slot_stride = m->slot_stride;
    r.layer_off = (size_t)layer * m->layer_stride;
    r.slot_ids = S.slot_id;
    return r;
}

int enqueue_decode(cmolhip_model *m, MSlot &S, hipStream_t st)
{
    const cmolhip_hparams_t &hp = m->hp;
    const int d = hp.d_model, kvd = hp.n_kv_heads * hp.d_head;
    RC(launch_embed(to_qt(m->embd), S.step, 3, S.x, d, S.argmax, 1, st));
    for (int l = 0; l < hp.n_layers; l++) {
        const MLayer &L = m->layers[l];
        GemvArgs g{};
        g.w = to_qt(L.qkv);
        g.x = S.x;
        g.x_stride = d;
        g.norm_w = L.attn_norm;
        g.eps = hp.rms_eps;
        g.out = S.q;
        g.out_stride = d;
        g.n = 1;
        g.nq = d;
        g.nkv = kvd;
        g.d_head = hp.d_head;
        g.max_ctx = hp.max_ctx;
        g.kv_f16 = hp.kv_f16;
        g.rope_on = L.rope_on;
        g.rope = m->rope;
        g.kv = kvref(m, S, l);
        g.pos = S.step + 1;
        g.pos_stride = 3;
        RC(launch_gemv(g, EPI_QKV, st));

        AttnArgs at{};
        at.q = S.q;
        at.q_stride = d;
        at.kv = kvref(m, S, l);
        at.seqlen = S.step + 2;
        at.seqlen_stride = 3;
        at.n = 1;
        at.n_heads = hp.n_heads;
        at.n_kv = hp.n_kv_heads;
        at.d_head = hp.d_head;
        at.max_ctx = hp.max_ctx;
        at.kv_f16 = hp.kv_f16;
        at.split = m->split;
        at.max_splits = m->max_splits;
        at.pm = S.pm;
        at.pl = S.pl;
        at.po = S.po;
        at.out = S.ao;
        at.out_stride = d;
        RC(launch_attn(at, st));

        GemvArgs go{};
        go.w = to_qt(L.o);
        go.x = S.ao;
        go.x_stride = d;
        go.out = S.x;
        go.out_stride = d;
        go.n = 1;
        RC(launch_gemv(go, EPI_RESID, st));

        GemvArgs gu{};
        gu.w = to_qt(L.gu);
        gu.x = S.x;
        gu.x_stride = d;
        gu.norm_w = L.ffn_norm;
        gu.eps = hp.rms_eps;
        gu.out = S.h;
        gu.out_stride = hp.d_ffn;
        gu.n = 1;
        RC(launch_gemv(gu, EPI_SWIGLU, st));

        GemvArgs gd{};
        gd.w = to_qt(L.down);
        gd.x = S.h;
        gd.x_stride = hp.d_ffn;
        gd.out = S.x;
        gd.out_stride = d;
        gd.n = 1;
        RC(launch_gemv(gd, EPI_RESID, st));
    }
    GemvArgs gl{};
    gl.w = to_qt(m->lm.qs ? m->lm : m->embd);
    gl.x = S.x;
    gl.x_stride = d;
    gl.norm_w = m->out_norm;
    gl.eps = hp.rms_eps;
    gl.out = S.logits;
    gl.out_stride = hp.vocab;
    gl.n = 1;
    gl.argmax = S.argmax;
    RC(launch_gemv(gl, EPI_LOGITS, st));
    return E_OK;
}

int upload_norm(cmolhip_ctx_t *c, const cmolhip_host_tensor_t &t, float **dst)
{
    RC(arena_get(c, (size_t)t.cols, dst));
    return cmolhip_memcpy_h2d(c, *dst, t.data, (size_t)t.cols * 4);
}

int upload_q(cmolhip_ctx_t *c, int n, const cmolhip_host_tensor_t *const *ts, int mode, void *stg,
             size_t stg_bytes, cmolhip_qtensor_t *out)
{
    const void *parts[3];
    int32_t rows[3];
    for (int i = 0; i < n; i++) {
        parts[i] = ts[i]->data;
        rows[i] = ts[i]->rows;
    }
    return cmolhip_qtensor_upload(c, ts[0]->dtype, ts[0]->cols, n, parts, rows, mode, stg, stg_bytes, out);
}

int build_model(cmolhip_model *m, const cmolhip_model_desc_t *d, const Plan &P)
{
    cmolhip_ctx_t *c = m->ctx;
    const cmolhip_hparams_t &h = d->hp;
    const int kvd = h.n_kv_heads * h.d_head, G = h.n_heads / h.n_kv_heads;
    void *stg = nullptr;
    RC(cmolhip_alloc(c, P.staging, ALIGN, &stg));
    m->layers.resize(h.n_layers);
    for (int l = 0; l < h.n_layers; l++) {
        const cmolhip_layer_tensors_t &T = d->layers[l];
        MLayer &L = m->layers[l];
        const cmolhip_host_tensor_t *qkv[3] = {&T.q, &T.k, &T.v};
        RC(upload_q(c, 3, qkv, CMOLHIP_PARTS_CONCAT, stg, P.staging, &L.qkv));
        const cmolhip_host_tensor_t *o[1] = {&T.o};
        RC(upload_q(c, 1, o, CMOLHIP_PARTS_CONCAT, stg, P.staging, &L.o));
        const cmolhip_host_tensor_t *gu[2] = {&T.gate, &T.up};
        RC(upload_q(c, 2, gu, CMOLHIP_PARTS_INTERLEAVE, stg, P.staging, &L.gu));
        const cmolhip_host_tensor_t *dn[1] = {&T.down};
        RC(upload_q(c, 1, dn, CMOLHIP_PARTS_CONCAT, stg, P.staging, &L.down));
        RC(upload_norm(c, T.attn_norm, &L.attn_norm));
        RC(upload_norm(c, T.ffn_norm, &L.ffn_norm));
        L.rope_on = !(h.no_rope_interval > 0 && (l + 1) % h.no_rope_interval == 0);
    }
    (void)kvd;
    const cmolhip_host_tensor_t *e[1] = {&d->embd};
    RC(upload_q(c, 1, e, CMOLHIP_PARTS_CONCAT, stg, P.staging, &m->embd));
    if (d->lm_head.data) {
        const cmolhip_host_tensor_t *lh[1] = {&d->lm_head};
        RC(upload_q(c, 1, lh, CMOLHIP_PARTS_CONCAT, stg, P.staging, &m->lm));
    }
    RC(upload_norm(c, d->out_norm, &m->out_norm));
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
    const size_t np = (size_t)h.n_kv_heads * m->max_splits * G;
    for (int s = 0; s < h.max_sessions; s++) {
        m->slots.emplace_back(new MSlot());
        MSlot &S = *m->slots.back();
        RC(arena_get(c, 4, &S.step));
        RC(arena_get(c, (size_t)h.max_ctx * 3, &S.steps));
        RC(arena_get(c, 1, &S.slot_id));
        RC(arena_get(c, (size_t)h.d_model, &S.x));
        RC(arena_get(c, (size_t)h.d_model, &S.q));
        RC(arena_get(c, (size_t)h.d_model, &S.ao));
        RC(arena_get(c, (size_t)h.d_ffn, &S.h));
        RC(arena_get(c, (size_t)h.vocab, &S.logits));
        RC(arena_get(c, ARGMAX_SLOTS, &S.argmax));
        RC(arena_get(c, np, &S.pm));
        RC(arena_get(c, np, &S.pl));
        RC(arena_get(c, np * h.d_head, &S.po));
        HC(hipMemsetAsync(S.step, 0, 16, c->stream));
        int32_t sid = s;
        RC(cmolhip_memcpy_h2d(c, S.slot_id, &sid, 4));
        HC(hipStreamCreateWithFlags(&S.st, hipStreamNonBlocking));
        HC(hipHostMalloc((void **)&S.h_steps, (size_t)h.max_ctx * 3 * 4, hipHostMallocDefault));
        HC(hipHostMalloc((void **)&S.h_argmax, 8 * ARGMAX_SLOTS, hipHostMallocDefault));
    }
    HC(hipStreamSynchronize(c->stream));
    if (m->use_graph) {
        for (auto &sp : m->slots) {
            MSlot &S = *sp;
            HC(hipStreamBeginCapture(S.st, hipStreamCaptureModeThreadLocal));
            int rc = enqueue_decode(m, S, S.st);
            hipError_t ce = hipStreamEndCapture(S.st, &S.graph);
            if (rc) return rc;
            HC(ce);
            HC(hipGraphInstantiate(&S.gexec, S.graph, nullptr, nullptr, 0));
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

int run_step(cmolhip_model *m, MSlot &S)
{
    if (S.gexec) {
        HC(hipGraphLaunch(S.gexec, S.st));
        return E_OK;
    }
    return enqueue_decode(m, S, S.st);
}

int finish_step(cmolhip_model *m, MSlot &S, float *logits_host, int32_t *argmax)
{
    HC(hipMemcpyAsync(S.h_argmax, S.argmax, 8 * ARGMAX_SLOTS, hipMemcpyDeviceToHost, S.st));
    if (logits_host)
        HC(hipMemcpyAsync(logits_host, S.logits, (size_t)m->hp.vocab * 4, hipMemcpyDeviceToHost, S.st));
    HC(hipStreamSynchronize(S.st));
    if (argmax) *argmax = (int32_t)argmax_index(reduce_slots(S.h_argmax));
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
    if (m->ctx) hipSetDevice(m->ctx->device);
    for (auto &sp : m->slots) {
        MSlot &S = *sp;
        if (S.st) hipStreamSynchronize(S.st);
        if (S.gexec) hipGraphExecDestroy(S.gexec);
        if (S.graph) hipGraphDestroy(S.graph);
        if (S.st) hipStreamDestroy(S.st);
        if (S.h_steps) hipHostFree(S.h_steps);
        if (S.h_argmax) hipHostFree(S.h_argmax);
    }
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
    MSlot &S = *m->slots[slot];
    std::lock_guard<std::mutex> g(S.mu);
    S.h_steps[0] = token;
    S.h_steps[1] = pos;
    S.h_steps[2] = pos + 1;
    HC(hipMemcpyAsync(S.step, S.h_steps, 12, hipMemcpyHostToDevice, S.st));
    RC(run_step(m, S));
    return finish_step(m, S, logits_host, argmax);
}

int cmolhip_prefill(cmolhip_model_t *m, int slot, const int32_t *tokens, int n, int32_t pos0,
                    float *logits_host, int32_t *argmax)
{
    if (!m || slot < 0 || slot >= (int)m->slots.size() || !tokens || n < 1) return E_ARGS;
    if (pos0 < 0 || (long)pos0 + n > m->hp.max_ctx) return E_ARGS;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->hp.vocab) return E_ARGS;
    MSlot &S = *m->slots[slot];
    std::lock_guard<std::mutex> g(S.mu);
    for (int i = 0; i < n; i++) {
        S.h_steps[3 * i + 0] = tokens[i];
        S.h_steps[3 * i + 1] = pos0 + i;
        S.h_steps[3 * i + 2] = pos0 + i + 1;
    }
    HC(hipMemcpyAsync(S.steps, S.h_steps, (size_t)n * 12, hipMemcpyHostToDevice, S.st));
    for (int i = 0; i < n; i++) {
        HC(hipMemcpyAsync(S.step, S.steps + 3 * i, 12, hipMemcpyDeviceToDevice, S.st));
        RC(run_step(m, S));
    }
    return finish_step(m, S, logits_host, argmax);
}

int cmolhip_decode_batch(cmolhip_model_t *m, int n, const int32_t *slots, const int32_t *tokens,
                         const int32_t *pos, float *logits_host, int32_t *argmax)
{
    if (!m || n < 1 || !slots || !tokens || !pos) return E_ARGS;
    for (int i = 0; i < n; i++) {
        if (slots[i] < 0 || slots[i] >= (int)m->slots.size()) return E_ARGS;
        if (tokens[i] < 0 || tokens[i] >= m->hp.vocab || pos[i] < 0 || pos[i] >= m->hp.max_ctx)
            return E_ARGS;
        for (int j = 0; j < i; j++)
            if (slots[j] == slots[i]) return E_ARGS;
    }
    for (int i = 0; i < n; i++) {
        MSlot &S = *m->slots[slots[i]];
        S.mu.lock();
        S.h_steps[0] = tokens[i];
        S.h_steps[1] = pos[i];
        S.h_steps[2] = pos[i] + 1;
        hipError_t e = hipMemcpyAsync(S.step, S.h_steps, 12, hipMemcpyHostToDevice, S.st);
        int rc = e == hipSuccess ? run_step(m, S) : herr(e);
        if (rc == E_OK) {
            e = hipMemcpyAsync(S.h_argmax, S.argmax, 8 * ARGMAX_SLOTS, hipMemcpyDeviceToHost, S.st);
            if (e == hipSuccess && logits_host)
                e = hipMemcpyAsync(logits_host + (size_t)i * m->hp.vocab, S.logits,
                                   (size_t)m->hp.vocab * 4, hipMemcpyDeviceToHost, S.st);
            rc = herr(e);
        }
        if (rc != E_OK) {
            for (int j = 0; j <= i; j++) {
                hipStreamSynchronize(m->slots[slots[j]]->st);
                m->slots[slots[j]]->mu.unlock();
            }
            return rc;
        }
    }
    int rc = E_OK;
    for (int i = 0; i < n; i++) {
        MSlot &S = *m->slots[slots[i]];
        if (hipStreamSynchronize(S.st) != hipSuccess) rc = E_INVALID;
        if (argmax) argmax[i] = (int32_t)argmax_index(reduce_slots(S.h_argmax));
        S.mu.unlock();
    }
    return rc;
}

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
    hipStreamSynchronize(m->slots[slot]->st);
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
    hipStreamSynchronize(m->slots[slot]->st);
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
    hipStreamSynchronize(m->slots[slot]->st);
    for (int l = 0; l < h.n_layers; l++) {
        const size_t off = ((size_t)slot * m->slot_stride + (size_t)l * m->layer_stride) * esz;
        RC(launch_kv_synth((uint8_t *)m->kbase + off, (uint8_t *)m->vbase + off, h.n_kv_heads,
                           h.max_ctx, h.d_head, n, h.kv_f16, seed + (uint64_t)l * 0x9E37ull, st));
    }
    HC(hipStreamSynchronize(st));
    return E_OK;
}

} // extern "C"
