"""mmh_gemm_noalloc against mmh_gemm_nn/nt/tn through the C ABI: the same
kernels and split choices, with the split-K partials in the library's fixed
per-GPU array instead of an allocated workspace, so the results must be the
same bits. Two calls in a row, the second with a smaller input (the array
keeps the first call's partials, which must not leak into the second), and
a product whose partials do not fit is refused before anything runs.
"""
import ctypes

import numpy as np
import pytest

import midman_hip as mh

pytestmark = pytest.mark.gpu

FORMS = {"nn": 0, "nt": 1, "tn": 2}


def run(ctx, fn, form, a, b, c0, m, k, n, accumulate):
    A, B, C = ctx.to_device(a), ctx.to_device(b), ctx.to_device(c0)
    if fn == "noalloc":
        st = mh.lib().mmh_gemm_noalloc(ctx.handle, FORMS[form], A.ptr, B.ptr, C.ptr, m, k, n,
                                       1 if accumulate else 0)
    else:
        st = getattr(mh.lib(), f"mmh_gemm_{form}")(ctx.handle, A.ptr, B.ptr, C.ptr, m, k, n,
                                                   1 if accumulate else 0)
    mh.check(st)
    out = C.numpy()
    for x in (A, B, C):
        x.free()
    return out


def operands(form, m, k, n, seed):
    r = np.random.default_rng(seed)
    a = r.standard_normal((k, m) if form == "tn" else (m, k)).astype(np.float32)
    b = r.standard_normal((n, k) if form == "nt" else (k, n)).astype(np.float32)
    c0 = r.standard_normal((m, n)).astype(np.float32)
    return a, b, c0


@pytest.mark.parametrize("form,first,second", [
    # dB = A^T dC of the benchmark sweep (a 2048-long reduction into 256 x 256:
    # split across workgroups), then a smaller split product
    ("tn", (256, 2048, 256), (128, 1024, 96)),
    # the 128x128 kernel split along K (16 tiles), then the K-split kernel
    ("nn", (512, 8192, 512), (300, 2000, 200)),
    ("nt", (256, 4096, 1024), (64, 512, 64)),
    # the sweep's largest partials (16 MiB: dB 4096 x 256 from 2048 rows, 4
    # splits), then the smallest sweep dB
    ("tn", (4096, 2048, 256), (256, 2048, 256)),
    # the sweep's 1 GFLOP dB products: 64x64 tiles, 4 splits summed by each
    # tile's last split (the counters in the static set)
    ("tn", (256, 2048, 1024), (1024, 2048, 256)),
])
@pytest.mark.parametrize("accumulate", [False, True])
def test_noalloc_matches_the_allocating_entry_point(ctx, form, first, second, accumulate):
    print(f"\n[gemm_noalloc] {form} {first} then {second} accumulate={accumulate}", flush=True)
    for i, (m, k, n) in enumerate((first, second)):
        a, b, c0 = operands(form, m, k, n, seed=m + k + n + i)
        want = run(ctx, "alloc", form, a, b, c0, m, k, n, accumulate)
        got = run(ctx, "noalloc", form, a, b, c0, m, k, n, accumulate)
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (form, m, k, n)


def test_noalloc_unsplit_product_and_errors(ctx):
    # a product that fills the chip takes no split: any size is accepted
    a, b, c0 = operands("nn", 2048, 256, 4096, 7)
    want = run(ctx, "alloc", "nn", a, b, c0, 2048, 256, 4096, False)
    got = run(ctx, "noalloc", "nn", a, b, c0, 2048, 256, 4096, False)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # partials over the 16 MiB array: 1152 x 2048 (144 tiles of 128 x 128)
    # from a 2048-long reduction splits 2 ways, 18.9 MB of partials; refused,
    # the output untouched
    m, k, n = 1152, 2048, 2048
    A, B = ctx.empty((m, k)), ctx.empty((k, n))
    C = ctx.to_device(np.full((m, n), 3.0, np.float32))
    st = mh.lib().mmh_gemm_noalloc(ctx.handle, 0, A.ptr, B.ptr, C.ptr, m, k, n, 0)
    assert st == mh.ERR_SHAPE, st
    assert "scratch holds" in mh.last_error()
    assert np.all(C.numpy() == 3.0)
    lib = mh.lib()
    assert lib.mmh_gemm_noalloc(ctx.handle, 3, A.ptr, B.ptr, C.ptr, 4, 4, 4, 0) == mh.ERR_ARGUMENT
    assert lib.mmh_gemm_noalloc(ctx.handle, 0, None, B.ptr, C.ptr, 4, 4, 4, 0) == mh.ERR_ARGUMENT
    assert lib.mmh_gemm_noalloc(ctx.handle, 0, A.ptr, B.ptr, C.ptr, 0, 4, 4, 0) == mh.ERR_SHAPE
    assert lib.mmh_gemm_noalloc(424242, 0, A.ptr, B.ptr, C.ptr, 4, 4, 4, 0) == mh.ERR_ARGUMENT
    for x in (A, B, C):
        x.free()


@pytest.mark.parametrize("accumulate", [False, True])
def test_noalloc_tail_balanced_product(ctx, accumulate):
    # tiles = CUs + 16 of 128 x 128 (2048 columns): the last 16 tiles are cut
    # along K into 8 pieces (8 MiB of partials, inside the array) and summed
    # in piece order by tail_reduce, on both entry points; then a smaller
    # split product through the same array
    _, cus = ctx.device_info()
    m, k, n = 128 * (cus // 16 + 1), 2048, 2048
    print(f"\n[gemm_noalloc tail] nn {m}x{k}x{n} ({cus} CUs) accumulate={accumulate}", flush=True)
    for i, (form, mm, kk, nn) in enumerate((("nn", m, k, n), ("tn", 128, 1024, 96))):
        a, b, c0 = operands(form, mm, kk, nn, seed=11 + i)
        want = run(ctx, "alloc", form, a, b, c0, mm, kk, nn, accumulate)
        got = run(ctx, "noalloc", form, a, b, c0, mm, kk, nn, accumulate)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (form, mm, kk, nn)


def test_noalloc_refuses_tail_pieces_over_the_array(ctx):
    # tiles = CUs + (CUs / 2 + 1): the tail takes 8 pieces per tile, about
    # 66 MiB of partials on 256 CUs: the allocating entry point runs it, the
    # no-alloc one refuses it (never a different split) and leaves C alone
    _, cus = ctx.device_info()
    tiles_n = 11
    rows = -(-(cus + cus // 2 + 1) // tiles_n)
    m, k, n = 128 * rows, 2048, 128 * tiles_n
    print(f"\n[gemm_noalloc tail refusal] nn {m}x{k}x{n}", flush=True)
    A, B = ctx.empty((m, k)), ctx.empty((k, n))
    C = ctx.to_device(np.full((m, n), 3.0, np.float32))
    st = mh.lib().mmh_gemm_noalloc(ctx.handle, 0, A.ptr, B.ptr, C.ptr, m, k, n, 0)
    assert st == mh.ERR_SHAPE, st
    assert "tail pieces" in mh.last_error()
    assert np.all(C.numpy() == 3.0)
    for x in (A, B, C):
        x.free()
