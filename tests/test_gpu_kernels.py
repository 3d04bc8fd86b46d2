"""Kernel-level parity of the gfx950 path against the oracle (CPU restatement
of the reference): bit-exact dequantisation, matvec and attention within
|a-b| <= 1e-4 + 1e-3*|b| (fp32 accumulate)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.qdata import random_blocks

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-4, 1e-3


def assert_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = ~(np.abs(got - want) <= ATOL + RTOL * np.abs(want))
    bad &= ~(np.isnan(got) & np.isnan(want))
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst "
                           f"{np.max(np.abs(got - want)[bad]):.3g}")


@pytest.fixture(scope="module")
def ctx(gpu):
    c = gpu.Ctx(2 << 30)   # one bump arena for the module's tensors
    yield c
    c.close()


@pytest.mark.parametrize("dtype", [2, 6, 8])
@pytest.mark.parametrize("shape,fold", [((16, 128), 1), ((37, 96), 1), ((64, 2048), 1), ((3, 4096), 1),
                                        ((37, 96), 2), ((64, 2048), 4), ((21, 1344), 8), ((5, 160), 4)])
def test_dequant_bit_exact(ctx, dtype, shape, fold):
    """Every fold of the tiled layout dequantises to the reference rows."""
    rows, cols = shape
    raw = random_blocks(dtype, rows, cols, seed=rows * 7 + cols + dtype)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.dequant(t)
    want = np.stack([O.dequant_row(raw[r], cols, dtype) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [2, 6, 8])
def test_dequant_special_scales_bit_exact(ctx, dtype):
    rows, cols = 48, 256
    raw = random_blocks(dtype, rows, cols, seed=11 + dtype, special=True)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.dequant(t)
    want = np.stack([O.dequant_row(raw[r], cols, dtype) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [2, 6, 8])
@pytest.mark.parametrize("fold", [1, 4])
def test_upload_concat_interleave_chunked(ctx, dtype, fold):
    """Row-concatenated and row-interleaved uploads, staged in small chunks,
    dequantise to the stacked / interleaved reference rows."""
    cols = 160
    a = random_blocks(dtype, 40, cols, seed=1)
    b = random_blocks(dtype, 24, cols, seed=2)
    c = random_blocks(dtype, 24, cols, seed=3)
    bb = a.shape[1]
    t = ctx.qtensor([a, b, c], dtype, cols, [40, 24, 24], mode=0, staging_bytes=bb * 5, fold=fold)
    want = np.concatenate([a, b, c])
    got = ctx.dequant(t)
    ref = np.stack([O.dequant_row(want[r], cols, dtype) for r in range(want.shape[0])])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    t2 = ctx.qtensor([b, c], dtype, cols, [24, 24], mode=1, staging_bytes=bb * 7, fold=fold)
    got2 = ctx.dequant(t2)
    il = np.empty((48, bb), np.uint8)
    il[0::2], il[1::2] = b, c
    ref2 = np.stack([O.dequant_row(il[r], cols, dtype) for r in range(48)])
    assert np.array_equal(got2.view(np.uint32), ref2.view(np.uint32))


@pytest.mark.parametrize("dtype,rows,cols,fold", [
    (8, 64, 256, 1), (6, 48, 960, 1), (2, 96, 576, 1), (8, 49152 // 16, 576, 1), (2, 320, 2560, 1),
    (2, 11008, 2048, 1), (2, 2048, 11008, 1), (8, 1024, 2048, 1), (6, 2560, 960, 1),
    (2, 2048, 2048, 4), (2, 2048, 11008, 4), (2, 3072, 2048, 4), (8, 576, 576, 8),
    (6, 960, 960, 2), (2, 130, 4096, 8)])
def test_gemv_matches_oracle(ctx, dtype, rows, cols, fold):
    raw = random_blocks(dtype, rows, cols, seed=rows + cols + dtype)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.gemm(t, x)[0]
    want = O.matmul(raw, x, rows, cols, dtype, O.AVX512)[:, 0]
    assert_close(got, want, f"gemv q{dtype} {rows}x{cols} fold {fold}")


@pytest.mark.parametrize("dtype,rows,cols,fold,n", [
    (2, 256, 2048, 1, 3), (2, 256, 2048, 1, 8), (2, 128, 11008, 1, 8), (2, 200, 2048, 1, 17),
    (8, 96, 960, 1, 32), (6, 160, 2560, 1, 16), (2, 512, 2048, 4, 2), (2, 512, 2048, 4, 4),
    (2, 64, 2048, 2, 4), (8, 48, 576, 8, 2),
    # operands beyond the LDS budget on grids of at most one work-group per
    # CU: read by the waves straight from L2 (partial row tiles included)
    (8, 160, 8192, 1, 8), (6, 100, 11008, 1, 5), (2, 70, 16384, 1, 7), (2, 2048, 11008, 1, 6),
    # more row tiles than CUs with such an operand: staged in chunks
    (2, 4112, 11008, 1, 8), (8, 4100, 8192, 1, 3),
    # 9-32 vectors where the batched plan would split k: groups of 8 on
    # grid.y of the one-group kernel (full and ragged last groups; the 3B
    # QKV / Wo and 360M QKV / down shapes)
    (2, 3072, 2048, 1, 32), (2, 2048, 2048, 1, 32), (2, 2048, 2048, 1, 20), (2, 3072, 2048, 1, 27),
    (6, 1600, 960, 1, 16), (6, 960, 2560, 1, 13), (8, 1000, 576, 1, 9)])
def test_gemv_batched_matches_oracle(ctx, dtype, rows, cols, fold, n):
    """Several activation vectors per launch (multi-session decode), including
    operands staged in chunks or read from L2 (n * cols too large for one LDS
    copy)."""
    raw = random_blocks(dtype, rows, cols, seed=rows * 3 + cols + n)
    x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.gemm(t, x)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"gemm q{dtype} {rows}x{cols} fold {fold} n {n}")


@pytest.mark.parametrize("dtype,rows,cols,fold,n", [
    (2, 2048, 11040, 1, 8), (8, 160, 8288, 1, 8), (6, 100, 11008 + 32, 1, 5)])
def test_gemv_direct_padding_ignores_stale_operand(ctx, dtype, rows, cols, fold, n):
    """The operand read straight from L2 (beyond the LDS budget, at most one
    work-group per CU) with k/32 not a multiple of 4: the last quad's
    padding blocks have no operand rows, and the buffer past the last real
    block holds f16 NaN before the operand is prepared.  The result must not
    see them."""
    import ctypes as C
    import libcmol_amd.native as native
    raw = random_blocks(dtype, rows, cols, seed=rows + 9 * cols + n)
    x = np.random.default_rng(n + 3).standard_normal((n, cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    L = native.lib()
    nbytes = L.cmolhip_act_bytes(cols, n)
    quads = (cols // 32 + 3) // 4
    op = ctx.alloc(quads * 4 * 128 * n + 4096)   # room for whole quads, stale NaN throughout
    ctx.h2d(op, np.full((quads * 4 * 128 * n + 4096) // 2, 0x7E00, np.uint16))
    assert nbytes <= quads * 4 * 128 * n + 4096
    dx = ctx.upload(x)
    native.check(L.cmolhip_act_prepare(ctx.h, C.c_void_p(dx), n, cols, dtype, None, C.c_void_p(op), None),
                 "act_prepare")
    dy = ctx.alloc(n * rows * 4)
    ctx.gemm_prepared(t, op, n, None, dy)
    native.check(L.cmolhip_synchronize(ctx.h), "sync")
    got = ctx.d2h(dy, (n, rows), np.float32)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, dtype, O.AVX512).T
    assert np.isfinite(got).all(), "padding blocks read stale NaN operand bytes"
    assert_close(got, want, f"direct gemv q{dtype} {rows}x{cols} n {n}")


@pytest.mark.parametrize("dtype,rows,cols,fold,n", [
    (2, 384, 2048, 1, 33), (2, 256, 2048, 1, 64), (2, 300, 2048, 1, 130), (8, 576, 576, 1, 200),
    (6, 320, 960, 1, 97), (6, 2560, 960, 1, 64), (2, 2048, 11008, 4, 65), (2, 3072, 2048, 4, 128),
    (8, 200, 576, 8, 70), (6, 960, 960, 2, 96), (2, 37, 4096, 1, 40), (2, 512, 2048, 1, 512),
    (6, 1664, 960, 2, 640), (8, 2176, 576, 1, 600), (2, 2100, 2048, 4, 700),
    # split-K (tiles short of two work-groups per CU): the 3B down / Wo /
    # QKV shapes at a 512-token pass, a ragged token tile, fold 2
    (2, 2048, 11008, 1, 512), (2, 2048, 2048, 1, 512), (2, 3072, 2048, 1, 448), (2, 2048, 11008, 2, 300)])
def test_gemm_tiled_matches_oracle(ctx, dtype, rows, cols, fold, n):
    """More than 32 vectors run the tiled MFMA GEMM (prompt prefill): partial
    row and vector tiles, folded weights read in place, and padding blocks.
    Shapes with more than 128 tiles of 64 vectors x 128 rows take the
    eight-wave work-groups (the last three), the others the four-wave ones;
    k ranges of 960 and 576 end in partial quads."""
    raw = random_blocks(dtype, rows, cols, seed=rows * 5 + cols + n)
    x = np.random.default_rng(n + 1).standard_normal((n, cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.gemm(t, x)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"tiled gemm q{dtype} {rows}x{cols} fold {fold} n {n}")


@pytest.mark.parametrize("dtype,rows,cols,n", [(6, 256, 960, 80), (2, 2048, 2048, 200)])
def test_gemm_tiled_rmsnorm_prologue(ctx, dtype, rows, cols, n):
    """The GEMM applies the RMSNorm scale from the operand's sums of squares
    (the second shape splits k: the finish kernel applies it)."""
    raw = random_blocks(dtype, rows, cols, seed=9)
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((n, cols)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.gemm(t, x, norm_w=w, eps=1e-6)
    xn = np.stack([O.rms_norm(xi, w, 1e-6) for xi in x])
    want = O.matmul(raw, np.ascontiguousarray(xn.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"tiled gemm with rmsnorm {rows}x{cols} n {n}")


@pytest.mark.parametrize("dtype,rows,cols,n", [
    (2, 3072, 2048, 32), (2, 2048, 11008, 32), (2, 22016, 2048, 32), (6, 960, 2560, 16),
    (8, 576, 576, 24), (2, 300, 2048, 9), (6, 1600, 960, 16), (8, 4104, 576, 12),
    (2, 22016, 2048, 21), (8, 16404, 1024, 32), (6, 16400, 960, 32)])
def test_gemv_batched_groups_match_oracle(ctx, dtype, rows, cols, n):
    """9..32 vectors: vector groups of 8, operand slices staged once per
    work-group, k splits summed by the finish kernel; partial row tiles and
    partial vector groups included.  Unsplit shapes of 17-32 vectors that
    need more than one round of work-groups (the 22016-row ones and the last
    two) take the sixteen-wave kernel with vector groups of 16, including a
    partial group, a partial row tile and a k range ending in a partial quad."""
    raw = random_blocks(dtype, rows, cols, seed=rows + 7 * cols + n)
    x = np.random.default_rng(n + 3).standard_normal((n, cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.gemm(t, x)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"batched gemv q{dtype} {rows}x{cols} n {n}")


def test_gemv_batched_groups_rmsnorm(ctx):
    """The batched path applies each vector's RMSNorm scale (in place and in
    the k-split finish)."""
    rng = np.random.default_rng(17)
    for rows, cols, n in ((512, 2048, 20), (256, 11008, 16)):
        raw = random_blocks(2, rows, cols, seed=rows + n)
        x = (rng.standard_normal((n, cols)) * 2).astype(np.float32)
        w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
        t = ctx.qtensor([raw], 2, cols, [rows])
        got = ctx.gemm(t, x, norm_w=w, eps=1e-6)
        xn = np.stack([O.rms_norm(xi, w, 1e-6) for xi in x])
        want = O.matmul(raw, np.ascontiguousarray(xn.T), rows, cols, 2, O.AVX512).T
        assert_close(got, want, f"batched gemv rmsnorm {rows}x{cols} n {n}")


@pytest.mark.parametrize("rows,cols,n", [(256, 2048, 1), (192, 11008, 8)])
def test_gemv_rmsnorm_prologue(ctx, rows, cols, n):
    """RMSNorm scale of each vector from the staged sum-of-squares partials
    (n=8 over 11008 inputs: operand read from L2)."""
    dtype = 2
    raw = random_blocks(dtype, rows, cols, seed=9 + n)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((n, cols)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.gemm(t, x, norm_w=w, eps=1e-6)
    xn = np.stack([O.rms_norm(xi, w, 1e-6) for xi in x])
    want = O.matmul(raw, np.ascontiguousarray(xn.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"gemv with RMSNorm prologue n {n}")


def test_gemv_reference_kats(ctx):
    """Reference tests/test_quant.c:272-320: Q8_0 known answers 1.0, 6.0, 11.0."""
    def blk(d, qs):
        b = np.zeros(34, np.uint8)
        b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
        for i, v in qs.items():
            b[2 + i] = np.uint8(np.int8(v).view(np.uint8))
        return b
    a = np.stack([blk(1.0, {0: 1}), blk(3.0, {1: 1})])
    x = np.zeros(32, np.float32); x[0], x[1] = 1.0, 2.0
    t = ctx.qtensor([a], 8, 32, [2])
    assert ctx.gemm(t, x)[0].tolist() == [1.0, 6.0]
    a2 = np.concatenate([blk(1.0, {0: 5}), blk(2.0, {0: 3})])[None]
    x2 = np.zeros(64, np.float32); x2[0] = x2[32] = 1.0
    t2 = ctx.qtensor([a2], 8, 64, [1])
    assert ctx.gemm(t2, x2)[0].tolist() == [11.0]


@pytest.mark.parametrize("n_heads,n_kv,d_head,lens,split,kv_f16", [
    (9, 3, 64, [1, 17, 160], 64, 0), (16, 4, 128, [2304, 5, 700], 64, 0),
    (15, 5, 64, [64, 1024], 64, 0), (4, 4, 128, [333], 64, 0),
    (16, 4, 128, [2304, 5, 700, 1], 256, 0), (16, 4, 128, [3000, 64, 65, 129], 192, 1),
    (9, 3, 64, [1, 17, 160, 999], 1024, 1), (4, 2, 16, [70, 3], 128, 0),
    (8, 1, 32, [300], 64, 1), (8, 8, 256, [200, 77], 128, 0),
    # fp16 caches through the MFMA score phase: one, two, four and eight
    # query heads per kv head, d_head 64 / 128 / 256, ragged chunk tails
    (16, 4, 128, [4096, 1, 257, 1500], 256, 1), (4, 4, 128, [513, 64], 256, 1),
    (8, 4, 64, [77, 700], 256, 1), (8, 8, 256, [200, 77], 128, 1), (16, 2, 128, [1000, 3], 320, 1),
    # splits of 32-position chunks (single-session decode): head-per-wave kernel
    (16, 4, 128, [2048, 1, 31, 33, 97], 32, 0), (9, 3, 64, [100, 2], 32, 1), (16, 4, 128, [700, 65], 96, 1),
    # a long context: 79 splits in one merge
    (4, 2, 128, [5000, 40], 64, 0)])
def test_attention_matches_oracle(ctx, gpu, n_heads, n_kv, d_head, lens, split, kv_f16):
    """Ragged lengths across splits of one or several 64- (or 32-) position
    chunks, fp32 and fp16 caches (the oracle reads the same rounded fp16
    values; the fp16 path scores on MFMA with the query split into exact f16
    halves)."""
    n = len(lens)
    max_ctx = max(lens)
    rng = np.random.default_rng(n_heads * 100 + d_head + split)
    q = rng.standard_normal((n, n_heads * d_head)).astype(np.float32)
    kc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float32)
    vc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float32)
    if kv_f16:
        kc16, vc16 = kc.astype(np.float16), vc.astype(np.float16)
        kc, vc = kc16.astype(np.float32), vc16.astype(np.float32)
        dk, dv = ctx.upload(kc16), ctx.upload(vc16)
    else:
        dk, dv = ctx.upload(kc), ctx.upload(vc)
    sl = np.array(lens, np.int32)
    dq, ds = ctx.upload(q), ctx.upload(sl)
    dout = ctx.alloc(q.nbytes)
    import ctypes as C
    gpu.check(gpu.lib().cmolhip_attn_decode(ctx.h, n, C.c_void_p(dq), C.c_void_p(dk), C.c_void_p(dv),
                                            C.c_void_p(ds), n_heads, n_kv, d_head, max_ctx, kv_f16,
                                            split, C.c_void_p(dout)), "attn")
    got = ctx.d2h(dout, q.shape, np.float32)
    for i, L in enumerate(lens):
        # oracle cache layout: [pos][n_kv][d_head]
        kref = np.ascontiguousarray(kc[i].transpose(1, 0, 2)[:L])
        vref = np.ascontiguousarray(vc[i].transpose(1, 0, 2)[:L])
        want = O.attention(q[i], kref, vref, L, n_heads, n_kv, d_head)
        assert_close(got[i], want, f"attention session {i} len {L} split {split}")


def attention_case(ctx, gpu, n_heads, n_kv, d_head, lens, split, kv_f16, seed, q_scale=1.0):
    n = len(lens)
    max_ctx = max(lens)
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((n, n_heads * d_head)) * q_scale).astype(np.float32)
    kc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float32)
    vc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float32)
    if kv_f16:
        kc16, vc16 = kc.astype(np.float16), vc.astype(np.float16)
        kc, vc = kc16.astype(np.float32), vc16.astype(np.float32)
        dk, dv = ctx.upload(kc16), ctx.upload(vc16)
    else:
        dk, dv = ctx.upload(kc), ctx.upload(vc)
    dq, ds = ctx.upload(q), ctx.upload(np.array(lens, np.int32))
    dout = ctx.alloc(q.nbytes)
    import ctypes as C
    gpu.check(gpu.lib().cmolhip_attn_decode(ctx.h, n, C.c_void_p(dq), C.c_void_p(dk), C.c_void_p(dv),
                                            C.c_void_p(ds), n_heads, n_kv, d_head, max_ctx, kv_f16,
                                            split, C.c_void_p(dout)), "attn")
    got = ctx.d2h(dout, q.shape, np.float32)
    for i, L in enumerate(lens):
        kref = np.ascontiguousarray(kc[i].transpose(1, 0, 2)[:L])
        vref = np.ascontiguousarray(vc[i].transpose(1, 0, 2)[:L])
        want = O.attention(q[i], kref, vref, L, n_heads, n_kv, d_head)
        assert_close(got[i], want, f"attention session {i} len {L} split {split}")


def test_attention_decode_rejects_bad_arguments(ctx, gpu):
    """Shapes the decode attention cannot take fail with an error code before
    any attention kernel runs: no vectors, query heads not a multiple of the
    kv heads, splits that are not whole 32-position chunks (or 32-position
    chunks at a d_head other than 64 / 128), a d_head without a kernel and
    more than 8 query heads per kv head; a valid call afterwards still
    matches the oracle."""
    import ctypes as C
    L = gpu.lib()
    dq = ctx.upload(np.zeros(16 * 256, np.float32))
    dk = ctx.upload(np.zeros(4 * 64 * 256, np.float32))
    dv = ctx.upload(np.zeros(4 * 64 * 256, np.float32))
    ds = ctx.upload(np.array([10], np.int32))
    dout = ctx.alloc(16 * 256 * 4)

    def call(n, n_heads, n_kv, d_head, split):
        return L.cmolhip_attn_decode(ctx.h, n, C.c_void_p(dq), C.c_void_p(dk), C.c_void_p(dv), C.c_void_p(ds),
                                     n_heads, n_kv, d_head, 64, 0, split, C.c_void_p(dout))

    assert call(0, 4, 4, 64, 64) == gpu.CMOL_ERR_ARGS        # no vectors
    assert call(1, 6, 4, 64, 64) == gpu.CMOL_ERR_ARGS        # 6 query heads over 4 kv heads
    assert call(1, 4, 4, 64, 48) == gpu.CMOL_ERR_ARGS        # not whole 32-position chunks
    assert call(1, 4, 4, 256, 32) == gpu.CMOL_ERR_ARGS       # 32-position chunks at d_head 256
    assert call(1, 4, 4, 48, 64) == gpu.CMOL_ERR_UNSUPPORTED  # no d_head 48 kernel
    assert call(1, 16, 1, 16, 64) == gpu.CMOL_ERR_UNSUPPORTED  # 16 query heads per kv head
    attention_case(ctx, gpu, 8, 2, 64, [10, 3], 64, 0, seed=5)


# Balanced ranges over an fp16 cache: CMOL_ATTN_BAL = total work-groups, so
# bal = total / n_kv - n ranges per kv head (at most n * (splits - 1)); small
# grids cut contexts into several pieces (and ranges across several
# contexts), large ones clamp the range to the split; None: the default grid.
_R = np.random.default_rng(99)
BAL_CASES = [
    (16, 4, 128, [4096, 1, 257, 1500], 256, None), (16, 4, 128, [4096, 1, 257, 1500], 256, "44"),
    (16, 4, 128, [4096, 1, 257, 1500], 256, "100000"), (8, 4, 64, [77, 700, 3, 64, 65, 129], 64, "36"),
    (8, 8, 256, [200, 77, 513], 128, "40"), (16, 2, 128, [1000, 3, 2000], 64, "14"),
    (4, 4, 128, [513, 64], 256, "20"), (12, 4, 128, [1, 1, 1, 300, 2], 64, "32"),
    (4, 2, 64, [int(x) for x in _R.integers(1, 300, 70)], 64, "200"),
    (4, 2, 64, [int(x) for x in _R.integers(1, 300, 70)], 64, None),
    (16, 4, 128, [int(x) for x in _R.integers(400, 3000, 9)], 128, "48"),
]


@pytest.mark.parametrize("n_heads,n_kv,d_head,lens,split,kv_f16,bal", [
    (16, 4, 128, [4096, 1, 257, 1500], 256, 1, None),   # balanced ranges
    (16, 4, 128, [4096, 1, 257, 1500], 256, 1, "0"),    # fp16 split grid
    (8, 4, 64, [900, 33, 2], 64, 1, None),
    (16, 4, 128, [2048, 5, 700], 64, 0, None),          # fp32 cache: head-per-wave kernel
    (9, 3, 64, [1000, 65], 64, 0, None)])
def test_attention_peaked_scores_match_oracle(ctx, gpu, monkeypatch, n_heads, n_kv, d_head, lens, split, kv_f16, bal):
    """Queries scaled by 8 (score standard deviation 8 instead of 1): the
    running maximum moves often and far (the lazily rescaled softmax of the
    fp16 kernels rescales many times), and most weights underflow on the
    hardware exponential; every kernel still matches the oracle."""
    if bal is None:
        monkeypatch.delenv("CMOL_ATTN_BAL", raising=False)
    else:
        monkeypatch.setenv("CMOL_ATTN_BAL", bal)
    attention_case(ctx, gpu, n_heads, n_kv, d_head, lens, split, kv_f16, seed=len(lens) * 17 + d_head, q_scale=8.0)


@pytest.mark.parametrize("n_heads,n_kv,d_head,lens,split,bal", BAL_CASES)
def test_attention_balanced_matches_oracle(ctx, gpu, monkeypatch, n_heads, n_kv, d_head, lens, split, bal):
    """Decode attention over the balanced ranges (one work-group per piece of
    a context cut by the ranges, pieces merged per vector): every vector
    against the oracle, over mixes of long, short, length-1 and 70
    contexts."""
    if bal is None:
        monkeypatch.delenv("CMOL_ATTN_BAL", raising=False)
    else:
        monkeypatch.setenv("CMOL_ATTN_BAL", bal)
    attention_case(ctx, gpu, n_heads, n_kv, d_head, lens, split, 1, seed=len(lens) * 31 + d_head + split)


def test_attention_balanced_equals_split_grid_closely(ctx, gpu, monkeypatch):
    """The balanced ranges and the one-work-group-per-split grid give the
    same outputs up to fp32 summation order (same inputs, both paths)."""
    import ctypes as C
    n_heads, n_kv, d_head, split = 16, 4, 128, 256
    lens = [5000, 17, 900, 2600, 1]
    n, max_ctx = len(lens), max(lens)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((n, n_heads * d_head)).astype(np.float32)
    kc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float16)
    vc = rng.standard_normal((n, n_kv, max_ctx, d_head)).astype(np.float16)
    dk, dv, dq = ctx.upload(kc), ctx.upload(vc), ctx.upload(q)
    ds = ctx.upload(np.array(lens, np.int32))
    outs = []
    for bal in ("0", "60"):
        monkeypatch.setenv("CMOL_ATTN_BAL", bal)
        dout = ctx.alloc(q.nbytes)
        gpu.check(gpu.lib().cmolhip_attn_decode(ctx.h, n, C.c_void_p(dq), C.c_void_p(dk), C.c_void_p(dv),
                                                C.c_void_p(ds), n_heads, n_kv, d_head, max_ctx, 1, split,
                                                C.c_void_p(dout)), "attn")
        outs.append(ctx.d2h(dout, q.shape, np.float32))
    assert np.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-6)


# ---- K-quants (Q4_K = 12, Q6_K = 14): super-blocks of 256 ------------------
KQ_DEQ = [((16, 256), 1), ((37, 512), 1), ((64, 2048), 4), ((21, 1024), 8), ((5, 768), 2),
          ((130, 2048), 1)]


@pytest.mark.parametrize("dtype", [12, 14])
@pytest.mark.parametrize("shape,fold", KQ_DEQ)
def test_kquant_dequant_bit_exact(ctx, dtype, shape, fold):
    """Every fold of the tiled K-quant layout dequantises to the reference
    rows bit for bit."""
    rows, cols = shape
    raw = random_blocks(dtype, rows, cols, seed=rows * 7 + cols + dtype)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.dequant(t)
    want = np.stack([O.dequant_row(raw[r], cols, dtype) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [12, 14])
def test_kquant_dequant_special_scales_bit_exact(ctx, dtype):
    """fp16 super-block scales from the IEEE special set (zeros, subnormals,
    max, inf, NaN payloads): the reference's x86 results, NaNs included."""
    rows, cols = 48, 512
    raw = random_blocks(dtype, rows, cols, seed=11 + dtype, special=True)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.dequant(t)
    want = np.stack([O.dequant_row(raw[r], cols, dtype) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [12, 14])
def test_kquant_upload_concat_interleave_chunked(ctx, dtype):
    cols = 512
    a, b, c = (random_blocks(dtype, r, cols, seed=s) for r, s in ((40, 1), (24, 2), (24, 3)))
    bb = a.shape[1]
    t = ctx.qtensor([a, b, c], dtype, cols, [40, 24, 24], mode=0, staging_bytes=bb * 5, fold=4)
    want = np.concatenate([a, b, c])
    ref = np.stack([O.dequant_row(want[r], cols, dtype) for r in range(want.shape[0])])
    assert np.array_equal(ctx.dequant(t).view(np.uint32), ref.view(np.uint32))
    t2 = ctx.qtensor([b, c], dtype, cols, [24, 24], mode=1, staging_bytes=bb * 7)
    il = np.empty((48, bb), np.uint8)
    il[0::2], il[1::2] = b, c
    ref2 = np.stack([O.dequant_row(il[r], cols, dtype) for r in range(48)])
    assert np.array_equal(ctx.dequant(t2).view(np.uint32), ref2.view(np.uint32))


@pytest.mark.parametrize("dtype", [12, 14])
@pytest.mark.parametrize("rows,cols,fold,n", [
    (64, 256, 1, 1), (2048, 2048, 4, 1), (3072, 2048, 4, 1), (11008, 2048, 1, 1), (2048, 11008, 4, 1),
    (300, 1024, 8, 1), (96, 768, 2, 1), (256, 2048, 1, 3), (512, 2048, 4, 2), (256, 2048, 1, 8),
    (300, 2048, 1, 17), (2048, 11008, 1, 32), (384, 2048, 1, 40), (2048, 11008, 4, 65),
    (300, 2048, 1, 130), (2048, 11008, 1, 8), (90, 16384, 1, 5)])
def test_kquant_gemv_gemm_match_oracle(ctx, dtype, rows, cols, fold, n):
    """Q4_K / Q6_K through the matvec (n <= 8), the vector-group kernel
    (9..32) and the tiled GEMM (> 32), folded and unfolded, against the
    oracle in the reference's AVX-512 order."""
    raw = random_blocks(dtype, rows, cols, seed=rows * 5 + cols + n + dtype)
    x = np.random.default_rng(n + dtype).standard_normal((n, cols)).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows], fold=fold)
    got = ctx.gemm(t, x)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"q{dtype} {rows}x{cols} fold {fold} n {n}")


@pytest.mark.parametrize("dtype", [12, 14])
@pytest.mark.parametrize("n", [1, 20, 64])
def test_kquant_rmsnorm_prologue(ctx, dtype, n):
    rows, cols = 512, 2048
    raw = random_blocks(dtype, rows, cols, seed=9 + n)
    rng = np.random.default_rng(11 + n)
    x = (rng.standard_normal((n, cols)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    t = ctx.qtensor([raw], dtype, cols, [rows])
    got = ctx.gemm(t, x, norm_w=w, eps=1e-6)
    xn = np.stack([O.rms_norm(xi, w, 1e-6) for xi in x])
    want = O.matmul(raw, np.ascontiguousarray(xn.T), rows, cols, dtype, O.AVX512).T
    assert_close(got, want, f"q{dtype} rmsnorm n {n}")


# ---- sizes of the measured configurations --------------------------------
@pytest.fixture
def big_ctx(gpu):
    c = gpu.Ctx(3 << 30)
    yield c
    c.close()


@pytest.mark.parametrize("rows,cols", [(11008, 2048), (2048, 11008)])
def test_ffn_shapes_full_size(gpu, big_ctx, rows, cols):
    """The isolated matvec configuration at its size: SmolLM3-3B FFN matrices
    of weights ~N(0, 0.02) quantised to Q4_0, activations ~N(0, 1).  The
    whole tensor dequantises bit-exactly in the single-session fold and in
    fold 1; the matvec at batch 1 and 8 matches the oracle."""
    from libcmol_amd import synth
    w = synth.normal(rows * cols, 4242 + rows, 0, 0.02)
    raw = synth.quantize(2, w).reshape(rows, cols // 32 * 18)
    want_deq = np.stack([O.dequant_row(raw[r], cols, 2) for r in range(rows)])
    folds = sorted({1, gpu.lib().cmolhip_pick_fold(rows, cols, 1)})
    x = np.random.default_rng(7).standard_normal((8, cols)).astype(np.float32)
    want = O.matmul(raw, np.ascontiguousarray(x.T), rows, cols, 2, O.AVX512).T
    for fold in folds:
        t = big_ctx.qtensor([raw], 2, cols, [rows], fold=fold)
        got = big_ctx.dequant(t)
        assert np.array_equal(got.view(np.uint32), want_deq.view(np.uint32)), f"fold {fold}"
        assert_close(big_ctx.gemm(t, x[:1]), want[:1], f"{rows}x{cols} fold {fold} n 1")
        if fold == 1:
            assert_close(big_ctx.gemm(t, x), want, f"{rows}x{cols} fold {fold} n 8")


@pytest.mark.parametrize("rows,cols,fold", [(11008, 2048, 1), (2048, 11008, 1), (2048, 11008, 2),
                                            (3072, 2048, 1)])
def test_gemm_tiled_prompt_size_matches_oracle(gpu, big_ctx, rows, cols, fold):
    """The prompt GEMM at a 2048-token prompt on the SmolLM3-3B projection
    shapes.  Each token's output depends only on its own activation vector,
    so 64 of the 2048 tokens (the first, the last and 62 drawn) are compared
    with the oracle."""
    n = 2048
    raw = random_blocks(2, rows, cols, seed=rows + 3 * cols + fold)
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    t = big_ctx.qtensor([raw], 2, cols, [rows], fold=fold)
    got = big_ctx.gemm(t, x)
    pick = np.unique(np.concatenate([[0, n - 1], rng.choice(n, 62, replace=False)]))
    want = O.matmul(raw, np.ascontiguousarray(x[pick].T), rows, cols, 2, O.AVX512).T
    assert_close(got[pick], want, f"tiled gemm {rows}x{cols} fold {fold} n {n}")


# ---- the reference's kernel seam (src/cmol_internal.h:175-182) -----------
@pytest.mark.parametrize("dtype,m,k", [(2, 96, 256), (6, 64, 512), (8, 130, 288), (12, 48, 512),
                                       (14, 40, 768)])
@pytest.mark.parametrize("n", [1, 3, 40])
def test_matmul_host_seam_matches_oracle(gpu, ctx, dtype, m, k, n):
    """cmolhip_matmul_host takes what cmol_matmul_fn_t takes: host pointers,
    raw GGUF rows A[m][k], B k-major [k][n], out [m][n]; its result matches
    the oracle's cmol_matmul order within 1e-4 + 1e-3*|ref|."""
    L = gpu.lib()
    raw = np.ascontiguousarray(random_blocks(dtype, m, k, seed=m * 11 + k + dtype))
    b = np.random.default_rng(n + k).standard_normal((k, n)).astype(np.float32)
    out = np.zeros((m, n), np.float32)
    gpu.check(L.cmolhip_matmul_host(ctx.h, gpu.ptr(out), gpu.ptr(raw), gpu.ptr(b), m, k, n, dtype),
              "matmul_host")
    want = O.matmul(raw, b, m, k, dtype, O.AVX512)
    assert_close(out, want, f"seam q{dtype} {m}x{k} n {n}")


def test_matmul_host_seam_rejects_bad_arguments(gpu, ctx):
    L = gpu.lib()
    raw = np.zeros((4, 18), np.uint8)
    b = np.zeros((32, 1), np.float32)
    out = np.zeros((4, 1), np.float32)
    args = (gpu.ptr(out), gpu.ptr(raw), gpu.ptr(b))
    assert L.cmolhip_matmul_host(ctx.h, *args, 4, 31, 1, 2) == gpu.CMOL_ERR_ARGS
    assert L.cmolhip_matmul_host(ctx.h, *args, 4, 32, 0, 2) == gpu.CMOL_ERR_ARGS
    assert L.cmolhip_matmul_host(ctx.h, None, raw.ctypes.data, b.ctypes.data, 4, 32, 1, 2) == gpu.CMOL_ERR_ARGS
    assert L.cmolhip_matmul_host(ctx.h, *args, 4, 32, 1, 3) == gpu.CMOL_ERR_UNSUPPORTED
    assert L.cmolhip_matmul_host(ctx.h, *args, 4, 0, 1, 0) == gpu.CMOL_ERR_ARGS   # F32, k = 0


def test_matmul_host_seam_f32_reference_kats(gpu, ctx):
    """The reference's own F32 matmul checks (tests/test_quant.c:210-261):
    m=3, k=4, n=1 and m=2, k=4, n=2, exact."""
    L = gpu.lib()
    a = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0]], np.float32)
    b = np.array([5, 7, 0, 0], np.float32).reshape(4, 1)
    out = np.zeros((3, 1), np.float32)
    gpu.check(L.cmolhip_matmul_host(ctx.h, gpu.ptr(out), gpu.ptr(a), gpu.ptr(b), 3, 4, 1, 0), "f32 kat")
    assert out.ravel().tolist() == [5.0, 7.0, 12.0]
    a2 = np.ascontiguousarray(a[:2])
    b2 = np.array([1, 2, 3, 4, 0, 0, 0, 0], np.float32).reshape(4, 2)
    out2 = np.zeros((2, 2), np.float32)
    gpu.check(L.cmolhip_matmul_host(ctx.h, gpu.ptr(out2), gpu.ptr(a2), gpu.ptr(b2), 2, 4, 2, 0), "f32 kat n2")
    assert out2.ravel().tolist() == [1.0, 2.0, 3.0, 4.0]


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("m,k,n", [(7, 4, 1), (33, 100, 3), (64, 2048, 1), (130, 515, 5), (16, 16, 40),
                                   (5, 31, 2), (300, 4096, 1)])
def test_matmul_host_seam_dense_bit_exact(gpu, ctx, dtype, m, k, n):
    """F32 and F16 weights through the seam (src/quant.c:351-360, 506-530):
    bit-identical to the oracle's AVX-512-order restatement (sixteen fused
    accumulators, the _mm512_reduce_add_ps tree, an unfused tail; F16 one
    unfused running sum), for any k, F16 rows including subnormal halves."""
    L = gpu.lib()
    rng = np.random.default_rng(m * 1000 + k * 7 + n + dtype)
    if dtype == 0:
        a = rng.standard_normal((m, k)).astype(np.float32)
    else:
        a = rng.standard_normal((m, k)).astype(np.float16)
        sub = rng.random((m, k)) < 0.05   # subnormal halves
        a[sub] = (rng.integers(1, 1024, int(sub.sum())).astype(np.uint16)).view(np.float16)
        a = a.view(np.uint16)
    a = np.ascontiguousarray(a)
    b = rng.standard_normal((k, n)).astype(np.float32)
    out = np.zeros((m, n), np.float32)
    gpu.check(L.cmolhip_matmul_host(ctx.h, gpu.ptr(out), gpu.ptr(a), gpu.ptr(b), m, k, n, dtype), "dense seam")
    want = O.matmul(a.view(np.uint8), b, m, k, dtype, O.AVX512)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), \
        f"dtype {dtype} {m}x{k} n {n}: max diff {np.abs(out - want).max():.3g}"
