"""GPU parity of the layer ops (midman-nn/src/lib.rs:45-56 surface) against
the oracle, plus the reference's closed forms and error kinds.

Tolerances, stated per op:
  embedding, rope tables, apply_rope, add: bit-exact.
  rms_norm: 4e-6 relative. The sum of squares runs in a different order
            (the reference's sequential f32 sum over d terms is itself off by
            up to ~d*2^-24 relative); the rest rounds as the reference rounds.
  causal_attention: |diff| <= 2e-5 * max|v| + 1e-5 * |ref| (online softmax and
            MFMA dot order).
  attention_forward / swiglu: |diff| <= 1e-4 * max|ref| per tensor (three or
            four chained GEMMs).
  block_forward: the block's change out - x within 2e-4 of its max|ref|
            (two norms and both sublayers chained), out itself within 1e-5.
  cross_entropy: 1e-4 relative to the oracle (the north-star loss
            tolerance; the reference's sequential f32 sum of V exponentials
            drifts by up to ~1e-5 relative at V = 1e5) and 2e-6 relative to a
            float64 evaluation.
"""
import math

import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as O

pytestmark = pytest.mark.gpu


def rel_max(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.mark.parametrize("d", [128, 256, 512, 1024, 2048, 4096])
def test_embedding_row_kernels_bit_exact(ctx, d):
    # the row-per-workgroup gathers (1, 2, 4 or 8 rows per workgroup), with a
    # row count that leaves the last workgroup partly empty
    print(f"\n[embedding] d={d}", flush=True)
    table = O.randn((300, d), 1.0, O.rng(d))
    ids = np.random.default_rng(d).integers(0, 300, size=257).astype(np.int32)
    out = mh.embedding(ctx, ctx.to_device(table), ids)
    assert np.array_equal(out.numpy(), O.embedding(table, ids))


def test_embedding_bit_exact_and_index_error(ctx):
    print("\n[embedding]", flush=True)
    table = O.randn((300, 48), 0.02, O.rng(5))
    ids = np.random.default_rng(0).integers(0, 300, size=257).astype(np.int32)
    T = ctx.to_device(table)
    out = mh.embedding(ctx, T, ids)
    assert np.array_equal(out.numpy(), O.embedding(table, ids))
    # odd width takes the scalar path
    t2 = O.randn((10, 7), 1.0, O.rng(6))
    assert np.array_equal(mh.embedding(ctx, ctx.to_device(t2), [9, 0, 3]).numpy(), t2[[9, 0, 3]])
    before = out.numpy()
    with pytest.raises(mh.IndexOutOfRange):
        mh.embedding(ctx, T, np.array([1, 300], np.int32), out=out)
    with pytest.raises(mh.IndexOutOfRange):
        mh.embedding(ctx, T, np.array([-1], np.int32), out=out)
    assert np.array_equal(out.numpy(), before)  # nothing ran


@pytest.mark.parametrize("rows,d", [(1, 2), (5, 64), (33, 100), (4096, 2048), (17, 1023)])
def test_rms_norm(ctx, rows, d):
    print(f"\n[rms_norm] rows={rows} d={d}", flush=True)
    x = O.randn((rows, d), 1.0, O.rng(rows + d))
    w = O.randn((d,), 1.0, O.rng(d))
    got = mh.rms_norm(ctx, ctx.to_device(x), ctx.to_device(w), 1e-5).numpy()
    want = O.rms_norm(x, w, 1e-5)
    np.testing.assert_allclose(got, want, rtol=4e-6, atol=0)


def test_rms_norm_known_row_and_errors(ctx, goldens):
    g = goldens["rms_norm_row"]
    y = mh.rms_norm(ctx, ctx.to_device(np.array([g["x"]], np.float32)),
                    ctx.to_device(np.array(g["w"], np.float32)), g["eps"]).numpy()
    r = math.sqrt(12.5)
    assert abs(y[0, 0] - 3 / r) < 1e-6 and abs(y[0, 1] - 8 / r) < 1e-6
    x = ctx.to_device(np.ones((2, 4), np.float32))
    with pytest.raises(mh.ArgumentError):
        mh.rms_norm(ctx, x, ctx.to_device(np.ones(4, np.float32)), 0.0)
    with pytest.raises(mh.ShapeError):
        mh.rms_norm(ctx, x, ctx.to_device(np.ones(3, np.float32)), 1e-5)


@pytest.mark.parametrize("hd,t", [(8, 16), (16, 128), (128, 2048), (64, 1000)])
def test_rope_tables_and_apply_bit_exact(ctx, hd, t):
    print(f"\n[rope] hd={hd} t={t}", flush=True)
    tabs = mh.RotaryTables(ctx, hd, t, 10000.0)
    cos, sin = O.rope_tables(hd, t, 10000.0)
    assert np.array_equal(tabs.cos.numpy(), cos) and np.array_equal(tabs.sin.numpy(), sin)
    x = O.randn((3, 2, min(t, 300), hd), 1.0, O.rng(hd))
    got = mh.apply_rope(ctx, ctx.to_device(x), tabs).numpy()
    assert np.array_equal(got, O.apply_rope(x, cos, sin))


ATTN_CASES = [
    # B, H, Hkv, T, hd
    (1, 2, 1, 2, 8),
    (2, 2, 1, 12, 8),
    (2, 4, 4, 32, 16),
    (1, 4, 2, 33, 16),
    (8, 4, 4, 256, 32),
    (2, 16, 16, 100, 64),
    (1, 16, 8, 1024, 128),
    (1, 16, 8, 2048, 128),  # the large preset's max_seq_len
    (2, 16, 8, 77, 128),
    (3, 6, 3, 1, 64),
    (2, 4, 2, 1, 128),  # a lone position in the 16-row kernel
    # odd counts of 128-row query blocks (the middle one has no partner)
    (1, 4, 2, 300, 128),
    (8, 16, 8, 300, 64),
    (16, 8, 8, 260, 32),
    # the key-split kernel's 8-wave form (blocks of more than 4 key tiles)
    (2, 4, 2, 200, 64),
    (1, 2, 1, 150, 16),
    # other even widths (config.rs:130-135 takes any), on the next kernel
    # width through zero-padded heads: key-split, paired and 16-row kernels
    (2, 4, 2, 37, 6),
    (1, 4, 2, 130, 24),
    (2, 2, 1, 300, 48),
    (1, 4, 4, 200, 96),
    (4, 16, 8, 512, 48),
    (2, 16, 8, 1024, 96),
    (1, 3, 1, 9, 2),
]


@pytest.mark.parametrize("B,H,Hkv,T,hd", ATTN_CASES)
def test_causal_attention(ctx, B, H, Hkv, T, hd):
    print(f"\n[attention] B={B} H={H} Hkv={Hkv} T={T} hd={hd}", flush=True)
    r = O.rng(B * 1000 + T)
    q = O.randn((B, H, T, hd), 1.0, r)
    k = O.randn((B, Hkv, T, hd), 1.0, r)
    v = O.randn((B, Hkv, T, hd), 1.0, r)
    got = mh.causal_attention(ctx, ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)).numpy()
    want = O.causal_attention(q, k, v)
    err = np.abs(got.astype(np.float64) - want)
    tol = 2e-5 * np.max(np.abs(v)) + 1e-5 * np.abs(want)
    print(f"  max|diff| {err.max():.3g} (max|v| {np.abs(v).max():.3g})", flush=True)
    assert np.all(err <= tol)


def test_attention_known_answer(ctx, goldens):
    g = goldens["attention_scale"]
    shp = g["shape"]
    q, k, v = (np.array(g[n], np.float32).reshape(shp) for n in ("q", "k", "v"))
    out = mh.causal_attention(ctx, ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)).numpy()
    w0 = 1.0 / (1.0 + math.exp(-1.0))
    want = np.array([1, 0, 0, 0, w0, 1 - w0, 0, 0], np.float32).reshape(shp)
    assert np.all(np.abs(out - want) < 1e-6)


def test_attention_rejects_bad_shapes(ctx):
    q = ctx.empty((1, 3, 4, 8))
    k = ctx.empty((1, 2, 4, 8))
    with pytest.raises(mh.ShapeError):
        mh.causal_attention(ctx, q, k, k)
    # every even head width up to 128 is taken (test_causal_attention); an
    # odd width (no rotation pairs) and one above 128 are refused before any
    # launch
    for hd in (7, 130):
        q2 = ctx.empty((1, 2, 4, hd))
        k2 = ctx.empty((1, 2, 4, hd))
        with pytest.raises(mh.ShapeError):
            mh.causal_attention(ctx, q2, k2, k2)


@pytest.mark.parametrize("B,T,d,H,Hkv", [(2, 12, 16, 2, 1), (2, 64, 256, 4, 2),
                                         (1, 300, 2048, 16, 8)])
def test_attention_forward(ctx, B, T, d, H, Hkv):
    print(f"\n[attention_forward] B={B} T={T} d={d} H={H} Hkv={Hkv}", flush=True)
    hd, kv = d // H, Hkv * (d // H)
    r = O.rng(d + T)
    x = O.randn((B, T, d), 1.0, r)
    wq, wk, wv = O.randn((d, d), 0.02, r), O.randn((d, kv), 0.02, r), O.randn((d, kv), 0.02, r)
    wo = O.randn((d, d), 0.02, r)
    tabs = mh.RotaryTables(ctx, hd, T, 10000.0)
    cos, sin = O.rope_tables(hd, T, 10000.0)
    dev = [ctx.to_device(a) for a in (x, wq, wk, wv, wo)]
    got = mh.attention_forward(ctx, dev[0], *dev[1:], H, Hkv, tabs).numpy()
    want = O.attention_forward(x, wq, wk, wv, wo, cos, sin, H, Hkv)
    e = rel_max(got, want)
    print(f"  max|diff|/max|ref| {e:.3g}", flush=True)
    assert e <= 1e-4


@pytest.mark.parametrize("B,T,d,H,Hkv,ff", [
    (2, 12, 16, 2, 1, 24), (2, 64, 256, 4, 2, 176), (1, 100, 128, 1, 1, 344),
    # the benchmark's block config (d 1024, 16 heads of 64, SwiGLU 2816, B8
    # T1024), both kv-head counts; heads of 64 columns rotated in the 128x128
    # GEMM's epilogue
    (8, 1024, 1024, 16, 16, 2816), (8, 1024, 1024, 16, 8, 2816),
    # heads of 128 (the large preset's), QKV at 512 tiles of 128x128: rotated
    # in the epilogue, with no K split; then 2049 rows (a last row tile of
    # one row, ragged sequences)
    (2, 1024, 2048, 16, 8, 512), (3, 683, 2048, 16, 8, 512)])
def test_block_forward(ctx, B, T, d, H, Hkv, ff):
    """DecoderBlock::forward (block.rs:77-81) against the oracle's block, on the
    benchmark block config's inputs: x ~ N(0,1) from Rng(0), then q, k, v, o,
    gate, up, down ~ N(0,0.02) from the same stream, norm weights 1."""
    print(f"\n[block_forward] B={B} T={T} d={d} H={H} Hkv={Hkv} ff={ff} Rng(0)", flush=True)
    hd, kv = d // H, Hkv * (d // H)
    c = O.config(1, d, 1, H, Hkv, ff, T)
    r = O.rng(0)
    x = O.randn((B, T, d), 1.0, r)
    parts = [np.ones(d, np.float32), O.randn((d, d), 0.02, r), O.randn((d, kv), 0.02, r),
             O.randn((d, kv), 0.02, r), O.randn((d, d), 0.02, r), np.ones(d, np.float32),
             O.randn((d, ff), 0.02, r), O.randn((d, ff), 0.02, r), O.randn((ff, d), 0.02, r)]
    bw = np.concatenate([p.reshape(-1) for p in parts])
    tabs = mh.RotaryTables(ctx, hd, T, 10000.0)
    cos, sin = O.rope_tables(hd, T, 10000.0)
    dx, dw = ctx.to_device(x), ctx.to_device(bw)
    got = mh.block_forward(ctx, dx, dw, H, Hkv, ff, 1e-5, tabs).numpy()
    want = O.block_forward(c, bw, cos, sin, x)
    e = rel_max(got - x, want.astype(np.float64) - x)
    print(f"  change: max|diff|/max|ref| {e:.3g}", flush=True)
    assert e <= 2e-4
    assert rel_max(got, want) <= 1e-5
    # in place: out = x
    again = mh.block_forward(ctx, dx, dw, H, Hkv, ff, 1e-5, tabs, out=dx).numpy()
    assert np.array_equal(again, got)


def test_block_forward_rejects_bad_arguments(ctx):
    tabs = mh.RotaryTables(ctx, 8, 4, 10000.0)
    x = ctx.to_device(np.zeros((1, 4, 16), np.float32))
    w = ctx.to_device(np.zeros(16 * 200, np.float32))
    with pytest.raises(mh.ShapeError):
        mh.block_forward(ctx, x, w, 3, 1, 8, 1e-5, tabs)   # 16 % 3
    with pytest.raises(mh.ShapeError):
        mh.block_forward(ctx, x, w, 2, 3, 8, 1e-5, tabs)   # 2 % 3
    with pytest.raises(mh.ArgumentError):
        mh.block_forward(ctx, x, w, 2, 1, 8, 0.0, tabs)    # eps
    with pytest.raises(mh.ArgumentError):
        mh.block_forward(ctx, x, w, 2, 1, 0, 1e-5, tabs)   # d_ff


@pytest.mark.parametrize("rows,d,ff", [(1, 1, 1), (64, 64, 176), (2048, 128, 344), (1024, 2048, 5632)])
def test_swiglu(ctx, rows, d, ff):
    print(f"\n[swiglu] rows={rows} d={d} ff={ff}", flush=True)
    r = O.rng(rows + ff)
    x = O.randn((rows, d), 1.0, r)
    wg, wu, wd = O.randn((d, ff), 0.02, r), O.randn((d, ff), 0.02, r), O.randn((ff, d), 0.02, r)
    dev = [ctx.to_device(a) for a in (x, wg, wu, wd)]
    got = mh.swiglu(ctx, *dev).numpy()
    want = O.swiglu(x, wg, wu, wd)
    e = rel_max(got, want)
    print(f"  max|diff|/max|ref| {e:.3g}", flush=True)
    assert e <= 1e-4


def test_swiglu_known_value(ctx, goldens):
    g = goldens["swiglu_value"]
    one = lambda v: ctx.to_device(np.array([[v]], np.float32))
    out = mh.swiglu(ctx, one(g["x"]), one(g["wg"]), one(g["wu"]), one(g["wd"])).numpy()
    assert abs(out[0, 0] - 2.0 / (1.0 + math.exp(-2.0)) * 12.0) < 1e-5


def test_add_bit_exact(ctx):
    a = O.randn((1001,), 1.0, O.rng(1))
    b = O.randn((1001,), 1.0, O.rng(2))
    got = mh.add(ctx, ctx.to_device(a), ctx.to_device(b)).numpy()
    assert np.array_equal(got, a + b)


@pytest.mark.parametrize("n,v", [(1, 2), (7, 5), (2048, 4096), (4096, 32000), (3, 100003)])
def test_cross_entropy(ctx, n, v):
    print(f"\n[cross_entropy] n={n} v={v}", flush=True)
    r = O.rng(n + v)
    logits = O.randn((n, v), 3.0, r)
    targets = np.random.default_rng(n).integers(0, v, size=n).astype(np.int32)
    got = mh.cross_entropy(ctx, ctx.to_device(logits), targets)
    want = O.cross_entropy(logits, targets)
    L = logits.astype(np.float64)
    m = L.max(1, keepdims=True)
    f64 = float(np.mean(np.log(np.exp(L - m).sum(1)) + m[:, 0] - L[np.arange(n), targets]))
    print(f"  gpu {got:.7f} oracle {want:.7f} float64 {f64:.7f}", flush=True)
    assert abs(got - want) <= 1e-4 * abs(want), (got, want)
    assert abs(got - f64) <= 2e-6 * abs(f64), (got, f64)


def test_cross_entropy_known_values_and_errors(ctx):
    L = lambda a: ctx.to_device(np.array(a, np.float32))
    assert abs(mh.cross_entropy(ctx, L([[0.0, 0.0]]), [0]) - math.log(2)) < 1e-6
    assert mh.cross_entropy(ctx, L([[20.0, 0, 0]]), [0]) < 1e-6
    assert abs(mh.cross_entropy(ctx, L([[0.0, 0], [50, -50]]), [1, 0]) - math.log(2) / 2) < 1e-6
    with pytest.raises(mh.IndexOutOfRange):
        mh.cross_entropy(ctx, L([[0.0, 0.0, 0.0]]), [3])
    with pytest.raises(mh.ShapeError):
        mh.cross_entropy(ctx, L([[0.0, 0.0, 0.0]]), [0, 1])


def test_mfma_peak_probe_is_a_plausible_ceiling(ctx):
    """The diagnostic MFMA probe runs and reports a rate under the published
    157.3 TFLOP/s fp32 matrix peak (it cannot exceed the peak clock's rate)."""
    tf = ctx.mfma_peak_tflops()
    print(f"\n  fp32 MFMA probe: {tf:.1f} TFLOP/s", flush=True)
    assert 50.0 < tf <= 157.3 * 1.02


# ---- outputs stay inside their buffers (kernels_avx.rs:368-390 on the device) ----

GUARD = 0x7FC0DEAD
G = 64


class Fenced:
    """A device buffer of n floats at a given word offset inside a larger one
    filled with the guard value."""

    def __init__(self, ctx, n, off, init=None):
        self.n, self.off = n, off
        self.buf = ctx.empty((n + off + G,))
        host = (np.zeros(self.buf.size, np.uint32) + GUARD).view(np.float32)
        if init is not None:
            host[off:off + n] = np.asarray(init, np.float32).ravel()
        self.buf.upload(host)
        self.ptr = self.buf.offset(off)

    def check(self, what):
        out = self.buf.numpy()
        guards = np.concatenate([out[:self.off], out[self.off + self.n:]]).view(np.uint32)
        assert np.all(guards == GUARD), f"{what}: a guard word was overwritten"
        return out[self.off:self.off + self.n]


@pytest.mark.parametrize("off", [G, G + 1])
def test_op_outputs_stay_inside_their_buffers(ctx, off):
    print(f"\n[guards] op outputs at word offset {off}", flush=True)
    L = mh.lib()
    # rms_norm rows: the vector path (d % 4 == 0) and the generic one
    for rows, d in ((33, 2048), (7, 1023), (5, 64)):
        x = O.randn((rows, d), 1.0, O.rng(d))
        w = O.randn((d,), 1.0, O.rng(d + 1))
        X, W = ctx.to_device(x), ctx.to_device(w)
        out = Fenced(ctx, rows * d, off)
        mh.check(L.mmh_rms_norm(ctx.handle, X.ptr, W.ptr, rows, d, 1e-5, out.ptr))
        got = out.check(f"rms_norm {rows}x{d}").reshape(rows, d)
        np.testing.assert_allclose(got, O.rms_norm(x, w, 1e-5), rtol=4e-6, atol=0)
    # embedding rows: float4 rows and an odd width
    for V, d, n in ((300, 48, 257), (10, 7, 9)):
        table = O.randn((V, d), 0.02, O.rng(V))
        ids = np.random.default_rng(V).integers(0, V, n).astype(np.int32)
        T = ctx.to_device(table)
        out = Fenced(ctx, n * d, off)
        mh.check(L.mmh_embedding(ctx.handle, T.ptr, V, d, mh._ip(ids), n, out.ptr))
        assert np.array_equal(out.check(f"embedding {V}x{d}").reshape(n, d), table[ids])
    # attention output: each kernel (16-row strips at hd 128 and 64 when the
    # output is 16-byte aligned, the 32-row paired blocks when it is not, the
    # key-split kernel for small grids), ragged T
    for B, H, Hkv, T, hd in ((1, 4, 2, 300, 128), (8, 8, 4, 520, 64), (2, 4, 4, 77, 64),
                             (4, 4, 4, 130, 32), (2, 2, 1, 12, 8)):
        r = O.rng(B * 100 + T)
        q = O.randn((B, H, T, hd), 1.0, r)
        k = O.randn((B, Hkv, T, hd), 1.0, r)
        v = O.randn((B, Hkv, T, hd), 1.0, r)
        Q, K, Vd = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
        out = Fenced(ctx, B * H * T * hd, off)
        mh.check(L.mmh_causal_attention(ctx.handle, Q.ptr, K.ptr, Vd.ptr, B, H, Hkv, T, hd,
                                        out.ptr))
        got = out.check(f"attention B{B} H{H} T{T} hd{hd}").reshape(B, H, T, hd)
        want = O.causal_attention(q, k, v)
        assert np.all(np.abs(got - want) <= 2e-5 * np.max(np.abs(v)) + 1e-5 * np.abs(want))
    # apply_rope and add
    tabs = mh.RotaryTables(ctx, 64, 40, 10000.0)
    cos, sin = O.rope_tables(64, 40, 10000.0)
    # (device buffers are held in names: a temporary's memory is freed and
    # reused by the next allocation)
    x = O.randn((3, 40, 64), 1.0, O.rng(9))
    X = ctx.to_device(x)
    out = Fenced(ctx, x.size, off)
    mh.check(L.mmh_apply_rope(ctx.handle, X.ptr, 3, 40, 64, tabs.cos.ptr, tabs.sin.ptr, out.ptr))
    assert np.array_equal(out.check("apply_rope").reshape(x.shape), O.apply_rope(x, cos, sin))
    a, b = O.randn((1001,), 1.0, O.rng(1)), O.randn((1001,), 1.0, O.rng(2))
    A, B = ctx.to_device(a), ctx.to_device(b)
    out = Fenced(ctx, 1001, off)
    mh.check(L.mmh_add(ctx.handle, A.ptr, B.ptr, out.ptr, 1001))
    assert np.array_equal(out.check("add"), a + b)
