"""The allocation-free product (cmolhip_gemm_noalloc): the same result as
cmolhip_gemm, bit for bit (same kernels, scratch in the fixed per-GPU array
instead of the context arena), on consecutive calls of shrinking size, and a
clear refusal of a call whose scratch would not fit."""
import ctypes as C

import numpy as np
import pytest

import libcmol_amd.native as native
from tests.qdata import random_blocks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(gpu):
    c = gpu.Ctx(1 << 30)
    yield c
    c.close()


def noalloc(ctx, t, x, norm_w, eps=1e-5):
    L = native.lib()
    n = x.shape[0]
    dx = ctx.upload(np.ascontiguousarray(x, np.float32))
    dy = ctx.alloc(n * t.rows * 4)
    ctx.h2d(dy, np.full(n * t.rows, np.nan, np.float32))
    dn = ctx.upload(np.ascontiguousarray(norm_w, np.float32)) if norm_w is not None else None
    rc = L.cmolhip_gemm_noalloc(ctx.h, C.byref(t), C.c_void_p(dx), C.c_void_p(dy), n,
                                C.c_void_p(dn) if dn else None, eps)
    native.check(L.cmolhip_synchronize(ctx.h), "sync")
    return rc, ctx.d2h(dy, (n, t.rows), np.float32)


# consecutive calls, each smaller than the one before: the tiled GEMM with an
# RMSNorm prologue, the batched matvec splitting k (partial sums in the
# scratch), a plain matvec
CALLS = [(2, 2048, 2048, 40, True), (12, 2048, 2048, 24, True), (8, 192, 256, 3, False)]


def test_noalloc_matches_gemm_on_consecutive_calls(ctx):
    L = native.lib()
    assert L.cmolhip_noalloc_scratch_bytes() == 16 << 20
    assert L.cmolhip_gemv_scratch_floats(12, 2048, 2048, 1, 24) > 0   # the second call splits k
    rng = np.random.default_rng(8)
    for i, (dt, rows, cols, n, norm) in enumerate(CALLS):
        raw = random_blocks(dt, rows, cols, seed=100 + i)
        t = ctx.qtensor([raw], dt, cols, [rows])
        x = rng.standard_normal((n, cols)).astype(np.float32)
        w = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32) if norm else None
        want = ctx.gemm(t, x, norm_w=w)
        rc, got = noalloc(ctx, t, x, w)
        assert rc == 0, (i, rc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}"


def test_noalloc_refuses_oversized_scratch(ctx):
    """4096 vectors of 2048 inputs need a 32 MiB operand: refused with
    CMOL_ERR_ARGS, nothing written; the next call in bounds still works."""
    raw = random_blocks(2, 64, 2048, seed=5)
    t = ctx.qtensor([raw], 2, 2048, [64])
    x = np.ones((4096, 2048), np.float32)
    rc, got = noalloc(ctx, t, x, None)
    assert rc == native.CMOL_ERR_ARGS
    assert np.isnan(got).all()
    x2 = np.random.default_rng(1).standard_normal((2, 2048)).astype(np.float32)
    rc, got = noalloc(ctx, t, x2, None)
    assert rc == 0
    want = ctx.gemm(t, x2)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_direct_padding_after_nan_call(ctx):
    """A call whose operand ends in f16 NaN (11136 inputs, NaN in the last
    96), then one of 11040 inputs at the same vector count: the second reads
    its operand straight from L2, and the padding blocks of its last quad sit
    where the first call left NaN in the scratch.  Its result must equal
    cmolhip_gemm's bit for bit."""
    rng = np.random.default_rng(21)
    raw0 = random_blocks(2, 2048, 11136, seed=31)
    t0 = ctx.qtensor([raw0], 2, 11136, [2048])
    x0 = rng.standard_normal((8, 11136)).astype(np.float32)
    x0[:, -96:] = np.nan
    rc, _ = noalloc(ctx, t0, x0, None)
    assert rc == 0
    raw = random_blocks(2, 2048, 11040, seed=32)
    t = ctx.qtensor([raw], 2, 11040, [2048])
    x = rng.standard_normal((8, 11040)).astype(np.float32)
    want = ctx.gemm(t, x)
    rc, got = noalloc(ctx, t, x, None)
    assert rc == 0
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
