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
                                   (2000, 481, 50), (65, 33, 700)])
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
