"""GPU parity of the fp32 MFMA GEMM seam (kernels.rs:49-108) and the matmul
backward (ops_matmul.rs:62-74) against the oracle, on the benchmark sweep:
M = 2048, K, N in {256, 1024, 4096}, A ~ N(0,1) from Rng(1), B ~ N(0,0.02)
from Rng(2), dC ~ N(0,1) from Rng(3).

Tolerance (written here, not tuned per case): the MFMA sums the products in a
different order from the reference's p-ascending loop, so each element may
differ by rounding only: |gpu - oracle| <= 1e-5 * sum_p |a_ip b_pj|.
"""
import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as O

pytestmark = pytest.mark.gpu

M = 2048
SIZES = (256, 1024, 4096)
_cache = {}


def sweep_inputs(k, n):
    key = (k, n)
    if key not in _cache:
        a = O.randn((M, k), 1.0, O.rng(1))
        b = O.randn((k, n), 0.02, O.rng(2))
        dc = O.randn((M, n), 1.0, O.rng(3))
        _cache.clear()
        _cache[key] = (a, b, dc)
    return _cache[key]


def bound(a, b):
    return 1e-5 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30


def check(got, want, bnd, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float(np.max(err / bnd))
    rel = float(np.max(err) / max(np.max(np.abs(want)), 1e-30))
    print(f"  {what}: max err/bound {worst:.3g}, max|diff|/max|ref| {rel:.3g}", flush=True)
    assert np.all(np.isfinite(got)), what
    assert worst <= 1.0, what


def test_hand_calculation_exact(ctx, goldens):
    g = goldens["gemm_hand"]
    a = np.array(g["a"], np.float32).reshape(2, 3)
    b = np.array(g["b"], np.float32).reshape(3, 2)
    want = np.array(g["c"], np.float32).reshape(2, 2)
    for form, aa, bb in (("nn", a, b), ("nt", a, np.array(g["bt"], np.float32).reshape(2, 3)),
                         ("tn", np.array(g["at"], np.float32).reshape(3, 2), b)):
        A, B, C = ctx.to_device(aa), ctx.to_device(bb), ctx.empty((2, 2))
        mh.gemm(ctx, form, A, B, C, 2, 3, 2)
        assert np.array_equal(C.numpy(), want), form


@pytest.mark.parametrize("k", SIZES)
@pytest.mark.parametrize("n", SIZES)
def test_sweep_forward_and_backward(ctx, k, n):
    print(f"\n[gemm sweep] M={M} K={k} N={n}", flush=True)
    a, b, dc = sweep_inputs(k, n)
    A, B, DC = ctx.to_device(a), ctx.to_device(b), ctx.to_device(dc)
    C, DA, DB = ctx.empty((M, n)), ctx.empty((M, k)), ctx.empty((k, n))
    mh.gemm(ctx, "nn", A, B, C, M, k, n)
    mh.matmul_backward(ctx, A, B, DC, M, k, n, da=DA, db=DB)
    c_ref = O.gemm("nn", a, b, M, k, n)
    da_ref, db_ref = O.matmul_backward(a, b, dc, M, k, n)
    check(C.numpy(), c_ref, bound(a, b), "C = A.B")
    check(DA.numpy(), da_ref, bound(dc, b.T), "dA = dC.B^T")
    check(DB.numpy(), db_ref, bound(a.T, dc), "dB = A^T.dC")
    for x in (A, B, DC, C, DA, DB):
        x.free()


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (12, 16, 32), (33, 17, 65),
                                   (129, 250, 131), (64, 4097, 40), (300, 8, 1000),
                                   (2048, 128, 4096),
                                   # the 128x128 kernel's load ring (3 slots, unrolled by 6)
                                   # with 1, 3, 6 and 7 K-tiles, the last with ragged edges
                                   (2048, 16, 4096), (2048, 48, 4096), (2048, 96, 4096),
                                   (2050, 112, 4100),
                                   # short-K shapes of the tiny preset and its edges
                                   (2048, 128, 384), (2048, 352, 128), (2047, 480, 97),
                                   (2000, 481, 50), (65, 33, 700),
                                   # 384 and 448 tiles of 128x128 on 256 CUs: the last
                                   # 128 / 192 run as 2 / 4 K-pieces + tail_reduce
                                   # (ragged edges and a short last piece in the first)
                                   (3000, 1000, 2000), (3584, 1024, 2048)])
@pytest.mark.parametrize("form", ["nn", "nt", "tn"])
def test_ragged_shapes_and_accumulate(ctx, m, k, n, form):
    print(f"\n[gemm ragged] {form} m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    aa = a if form != "tn" else np.ascontiguousarray(a.T)
    bb = b if form != "nt" else np.ascontiguousarray(b.T)
    A, B = ctx.to_device(aa), ctx.to_device(bb)
    C = ctx.to_device(c0)
    mh.gemm(ctx, form, A, B, C, m, k, n, accumulate=True)
    want = O.gemm(form, aa, bb, m, k, n, c=c0)
    check(C.numpy(), want, bound(a, b) + 1e-6 * np.abs(c0), f"{form} accumulate")
    mh.gemm(ctx, form, A, B, C, m, k, n, accumulate=False)
    check(C.numpy(), O.gemm(form, aa, bb, m, k, n), bound(a, b), f"{form} store")
    for x in (A, B, C):
        x.free()


GUARD = 0x7FC0DEAD  # the reference's guard value (kernels_avx.rs:374)
MIN_POSITIVE = np.float32(1.17549435e-38)

# Shapes that route the seam to each kernel path (gemm.hip's dispatch on a
# 256-CU MI355X): the 128x128 kernel with interior and edge tiles; the 64x64
# kernel with a partial K step; the 32x32 K-split kernel in one workgroup
# (nn; nt and tn of this shape split K across two workgroups); the K-split
# kernel split across workgroups plus splitk_reduce; the 128x128 kernel split
# along K plus splitk_reduce.
SPECIAL_PATHS = [
    ("128x128 tiles, interior and edges", 1100, 48, 4100),
    ("64x64 tiles, partial K step", 2048, 500, 1024),
    # K beyond 1024 on the 64x64 tiles (at most 2^29 multiply-adds): 4 splits
    # of 16 K-steps, the last one short, summed by each tile's last split
    ("64x64 tiles, K 2000 in 4 splits summed by the last split", 256, 2000, 1024),
    ("32x32 K-split tiles", 2048, 344, 128),
    ("32x32 K-split over 8 workgroups + reduce", 256, 2048, 256),
    ("128x128 split 8 ways along K + reduce", 1024, 8192, 1024),
    ("128x128 whole tiles + K-pieces of the last tiles + tail_reduce", 3000, 1000, 2000),
]


def special_operands(m, k, n, seed):
    """Integer-valued A [m,k], B [k,n], C0 [m,n] (every sum exact in f32, so
    the result does not depend on the summation order) with special values
    planted: the reference's case a=[0,-0,inf,1,NaN,-2] x b=[-0,0,3,-inf,1,
    MIN_POSITIVE] (kernels_avx.rs:355-357) in the last two rows, the last
    three k and the last two columns (edge tiles, the K tail); a row of -0
    against a positive column (the sum is -0: +0 stored, C's -0 kept when
    accumulating); a row of subnormal and MIN_POSITIVE multiples; C0 with
    -0, inf and NaN."""
    r = np.random.default_rng(seed)
    a = r.integers(-3, 4, (m, k)).astype(np.float32)
    b = r.integers(-3, 4, (k, n)).astype(np.float32)
    c0 = r.integers(-5, 6, (m, n)).astype(np.float32)
    i0, p0, j0 = m - 2, k - 3, n - 2
    a[i0:i0 + 2, :] = 0.0
    b[:, j0:j0 + 2] = 0.0
    a[i0:i0 + 2, p0:p0 + 3] = np.array([0.0, -0.0, np.inf, 1.0, np.nan, -2.0],
                                       np.float32).reshape(2, 3)
    b[p0:p0 + 3, j0:j0 + 2] = np.array([-0.0, 0.0, 3.0, -np.inf, 1.0, MIN_POSITIVE],
                                       np.float32).reshape(3, 2)
    # a row of -0 and a column of positives: every product -0
    i1, j1 = m // 2, 1
    a[i1, :] = -0.0
    b[:, j1] = r.integers(1, 4, k).astype(np.float32)
    c0[i1, j1] = -0.0
    c0[i1, j1 + 1] = 0.0
    # tiny values only (no integer to absorb them): subnormal and MIN_POSITIVE
    # multiples, exact in f32 in any order
    i2 = 3
    a[i2, :] = 0.0
    a[i2, 0] = MIN_POSITIVE / np.float32(4)   # subnormal operand
    a[i2, k // 2] = MIN_POSITIVE
    c0[0, 0], c0[0, 1], c0[0, 2] = -0.0, np.inf, np.nan
    return a, b, c0


def same_bits(got, want):
    g, w = got.view(np.uint32), want.view(np.uint32)
    return (g == w) | (np.isnan(got) & np.isnan(want))


@pytest.mark.parametrize("path,m,k,n", SPECIAL_PATHS, ids=[p[0] for p in SPECIAL_PATHS])
@pytest.mark.parametrize("form", ["nn", "nt", "tn"])
def test_special_values_and_guard_bands_on_every_kernel_path(ctx, path, m, k, n, form):
    # kernels_avx.rs:351-366: special values follow the scalar rules bit for
    # bit (NaN matches NaN); :368-390: C written between guard values that
    # must survive. C sits at a 256-byte offset (vector stores) and at a
    # 4-byte one (element stores) inside a buffer of guards.
    print(f"\n[gemm special] {path}: {form} m={m} k={k} n={n}", flush=True)
    a, b, c0 = special_operands(m, k, n, m + k + n)
    aa = a if form != "tn" else np.ascontiguousarray(a.T)
    bb = b if form != "nt" else np.ascontiguousarray(b.T)
    A, B = ctx.to_device(aa), ctx.to_device(bb)
    G = 64
    buf = ctx.empty((m * n + 2 * G + 1,))
    with np.errstate(invalid="ignore"):
        want_store = O.gemm(form, aa, bb, m, k, n, threads=16)
        want_acc = O.gemm(form, aa, bb, m, k, n, c=c0, threads=16)
    nonfinite = int(np.sum(~np.isfinite(want_acc)))
    negzero = int(np.sum((want_acc == 0) & np.signbit(want_acc)))
    print(f"  reference: {nonfinite} non-finite, {negzero} -0 in the accumulated result",
          flush=True)
    assert nonfinite > 0 and negzero > 0
    for off in (G, G + 1):
        for accumulate, want in ((False, want_store), (True, want_acc)):
            host = np.full(buf.size, 0, np.uint32) + GUARD
            host = host.view(np.float32)
            host[off:off + m * n] = c0.ravel()
            buf.upload(host)
            mh.gemm(ctx, form, A, B, buf.offset(off), m, k, n, accumulate=accumulate)
            out = buf.numpy()
            got = out[off:off + m * n].reshape(m, n)
            ok = same_bits(got, want)
            bad = np.argwhere(~ok)
            assert ok.all(), (off, accumulate, bad[:5].tolist(),
                              [(float(got[i, j]), float(want[i, j])) for i, j in bad[:5]])
            guards = np.concatenate([out[:off], out[off + m * n:]]).view(np.uint32)
            assert np.all(guards == GUARD), (off, accumulate, "a guard value was overwritten")
    for x in (A, B, buf):
        x.free()


def test_special_values_propagate(ctx):
    # NaN and inf in A reach exactly the rows they touch (kernels_avx.rs:351-366).
    rng = np.random.default_rng(11)
    a = rng.standard_normal((40, 24)).astype(np.float32)
    b = rng.standard_normal((24, 36)).astype(np.float32)
    a[3, 5] = np.nan
    a[7, 2] = np.inf
    A, B, C = ctx.to_device(a), ctx.to_device(b), ctx.empty((40, 36))
    mh.gemm(ctx, "nn", A, B, C, 40, 24, 36)
    c = C.numpy()
    assert np.all(np.isnan(c[3]))
    assert np.all(~np.isfinite(c[7]))
    ok = np.ones(40, bool)
    ok[[3, 7]] = False
    assert np.all(np.isfinite(c[ok]))


def test_batched_matmul(ctx):
    # ops_matmul.rs:87-96: every matrix of the batch is an independent product.
    rng = np.random.default_rng(12)
    a = rng.standard_normal((6, 33, 20)).astype(np.float32)
    b = rng.standard_normal((6, 20, 47)).astype(np.float32)
    out = mh.matmul(ctx, ctx.to_device(a), ctx.to_device(b)).numpy()
    for i in range(6):
        check(out[i], O.gemm("nn", a[i], b[i], 33, 20, 47), bound(a[i], b[i]), f"batch {i}")


def test_shared_rhs_matmul_flattens_leading_axes(ctx):
    rng = np.random.default_rng(13)
    a = rng.standard_normal((2, 3, 9, 16)).astype(np.float32)
    b = rng.standard_normal((16, 5)).astype(np.float32)
    out = mh.matmul(ctx, ctx.to_device(a), ctx.to_device(b)).numpy()
    assert out.shape == (2, 3, 9, 5)
    check(out.reshape(-1, 5), O.gemm("nn", a.reshape(-1, 16), b, 54, 16, 5),
          bound(a.reshape(-1, 16), b), "flattened")


def test_matmul_backward_need_flags(ctx):
    rng = np.random.default_rng(14)
    a = rng.standard_normal((64, 32)).astype(np.float32)
    b = rng.standard_normal((32, 48)).astype(np.float32)
    dc = rng.standard_normal((64, 48)).astype(np.float32)
    A, B, DC = ctx.to_device(a), ctx.to_device(b), ctx.to_device(dc)
    DA = ctx.empty((64, 32))
    mh.matmul_backward(ctx, A, B, DC, 64, 32, 48, da=DA, db=None)
    da_ref, _ = O.matmul_backward(a, b, dc, 64, 32, 48, need_b=False)
    check(DA.numpy(), da_ref, bound(dc, b.T), "dA only")
    DB = ctx.empty((32, 48))
    mh.matmul_backward(ctx, None, B, DC, 64, 32, 48, da=None, db=None)  # nothing requested
    with pytest.raises(mh.ArgumentError):
        mh.matmul_backward(ctx, None, B, DC, 64, 32, 48, da=None, db=DB)  # dB needs A


def test_shape_errors(ctx):
    A = ctx.empty((4, 4))
    with pytest.raises(mh.ShapeError):
        mh.gemm(ctx, "nn", A, A, A, 0, 4, 4)
    with pytest.raises(mh.ArgumentError):
        mh.gemm(ctx, "nn", None, A, A, 4, 4, 4)
