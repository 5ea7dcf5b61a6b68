"""Device backward, clip, AdamW and schedule against the oracle and the
reference's own goldens (MI355X; everything runs through libmidman_hip.so).

Tolerances (the device sums in MFMA order, the reference sequentially):
  * per parameter: max|g_dev - g_ref| <= 2e-3 * max|g_ref| of that parameter;
  * loss: 1e-5 relative; global norm: 1e-4 relative (the reference's own
    tolerance for these goldens is 1e-4, engine.test.mjs:108-110);
  * op backward: attention 2e-4 of the largest gradient, RMSNorm 1e-5 relative,
    cross entropy 1e-5 of 1/N; RoPE backward bit-exact.
"""
import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as mo

pytestmark = pytest.mark.gpu

LAB = [12, 16, 2, 2, 1, 32, 16, 10000.0, 1e-5, 1]
HYPER = [0.03, 0.003, 15, 150, 0.01, 1.0, 0.9, 0.99]

# name: (config, batch, seq, init std); head dims 4..128, GQA, tied and untied,
# sequence lengths that are not multiples of the 32-row tiles.
CASES = {
    "lab_hd8_gqa": (LAB, 2, 12, 0.3),
    "wiring_hd4_tied": ([13, 16, 3, 4, 2, 24, 8, 10000.0, 1e-5, 1], 2, 5, 0.3),
    "wiring_hd4_untied_seq1": ([13, 16, 3, 4, 2, 24, 8, 10000.0, 1e-5, 0], 3, 1, 0.3),
    "smoke_hd16": (mh.PRESETS["smoke"], 2, 32, 0.1),
    "hd32_gqa_t70": ([97, 128, 2, 4, 2, 96, 96, 10000.0, 1e-5, 1], 2, 70, 0.1),
    "hd64_untied_t130": ([301, 256, 2, 4, 2, 200, 160, 10000.0, 1e-5, 0], 1, 130, 0.08),
    "hd128_gqa_t100": ([301, 256, 1, 2, 1, 136, 160, 10000.0, 1e-5, 1], 2, 100, 0.08),
    # the down projection's backward (SwiGLU-backward epilogue) at 352 tiles of
    # 128x128 on 256 CUs: its last 96 tiles run as K-pieces plus tail_reduce
    "tail_pieces_d512_t2048": ([64, 512, 1, 4, 4, 2816, 2048, 10000.0, 1e-5, 1], 1, 2048, 0.05),
    # head widths the attention kernels take through zero-padded heads (6 on
    # 8, 24 on 32, 48 and 96 on 64 and 128), GQA, tied and untied
    "hd6_gqa": ([20, 12, 2, 2, 1, 16, 16, 10000.0, 1e-5, 1], 2, 13, 0.3),
    "hd24_gqa": ([97, 96, 2, 4, 2, 64, 64, 10000.0, 1e-5, 1], 2, 40, 0.1),
    "hd48_untied": ([101, 96, 1, 2, 1, 80, 100, 10000.0, 1e-5, 0], 2, 70, 0.1),
    "hd96_t130": ([64, 192, 1, 2, 2, 128, 160, 10000.0, 1e-5, 1], 1, 130, 0.08),
}


def ocfg(config):
    return mo.config(*[int(x) for x in config[:7]], theta=config[7], eps=config[8],
                     tie=bool(config[9]))


def check_grads(got, want, c, tol=2e-3, what="", skip=()):
    for i, (off, size, _) in enumerate(mo.param_segments(c)):
        if i in skip:
            continue
        g, w = got[off:off + size], want[off:off + size]
        scale = float(np.abs(w).max())
        err = float(np.abs(g - w).max())
        assert err <= tol * scale + 1e-30, f"{what} parameter {i}: {err} vs scale {scale}"


@pytest.mark.parametrize("name", list(CASES))
def test_backward_matches_oracle(ctx, name):
    config, batch, seq, std = CASES[name]
    print(f"\n[case] backward {name} B{batch} T{seq}", flush=True)
    c = ocfg(config)
    w = mo.init_weights(c, mo.rng(11), std=std)
    r = np.random.default_rng(12)
    x = r.integers(0, c.vocab_size, batch * seq).astype(np.int32)
    y = r.integers(0, c.vocab_size, batch * seq).astype(np.int32)
    want_loss, want = mo.forward_backward(c, w, x, y, batch, seq)
    m = mh.Model.from_weights(ctx, config, w)
    try:
        loss = m.backward(x, y, batch, seq)
        got = m.grads()
        norm = m.grad_norm()
    finally:
        m.close()
    assert abs(loss - want_loss) <= 1e-5 * abs(want_loss), (loss, want_loss)
    # One position: the softmax is over a single score, so q and k do not reach
    # the output and the reference's gradient is exactly 0 (wiring.rs:290-306).
    # The device forms dS = P (dP - rowsum(dO O)) with the two sums in different
    # orders, so its q/k gradients are zero up to rounding.
    qk = {i for i in range(1, 9 * c.n_layers + 1) if (i - 1) % 9 in (1, 2)} if seq == 1 else set()
    check_grads(got, want, c, what=name, skip=qk)
    # the device's f64 norm of its own gradients, and against the oracle's
    own = float(np.sqrt((got.astype(np.float64) ** 2).sum()))
    assert abs(norm - own) <= 1e-6 * own
    ref = mo.global_norm(want)
    assert abs(norm - ref) <= 1e-4 * ref, (norm, ref)
    segs = mo.param_segments(c)
    for i in qk:
        off, size, _ = segs[i]
        assert np.abs(want[off:off + size]).max() == 0.0
        assert np.abs(got[off:off + size]).max() <= 1e-6 * norm


ATTN_SHAPES = [  # B, H, Hkv, T, hd
    (1, 2, 1, 33, 4), (2, 4, 2, 70, 8), (1, 2, 2, 64, 16), (2, 4, 1, 100, 32),
    (1, 4, 2, 130, 64), (1, 2, 1, 200, 128), (1, 1, 1, 1, 64), (2, 2, 2, 257, 128),
    # grids of at least one 128-row block per CU take the block kernels (the
    # shapes above, the strip kernels) also for heads of 64 and 32
    (4, 16, 8, 512, 64), (8, 8, 8, 512, 32),
    # the large preset's heads at its training shape and at its max_seq_len
    (4, 16, 8, 1024, 128), (1, 16, 8, 2048, 128),
    # a lone position and a single partial tile at hd 128 (the 16-row kernels)
    (1, 2, 1, 1, 128), (2, 4, 2, 17, 128),
    # other even widths, on the next kernel width through zero-padded heads
    (1, 2, 1, 45, 6), (2, 4, 2, 100, 24), (1, 4, 2, 130, 48), (1, 2, 1, 257, 96),
    (4, 16, 8, 512, 48), (1, 3, 1, 9, 2),
]


@pytest.mark.parametrize("shape", ATTN_SHAPES)
def test_attention_backward_matches_oracle(ctx, shape):
    B, H, Hkv, T, hd = shape
    print(f"\n[case] attention backward {shape}", flush=True)
    r = np.random.default_rng(sum(shape))
    q = r.standard_normal((B, H, T, hd)).astype(np.float32)
    k = r.standard_normal((B, Hkv, T, hd)).astype(np.float32)
    v = r.standard_normal((B, Hkv, T, hd)).astype(np.float32)
    g = r.standard_normal((B, H, T, hd)).astype(np.float32)
    want = mo.causal_attention_backward(q, k, v, g)
    got = mh.causal_attention_backward(ctx, ctx.to_device(q), ctx.to_device(k),
                                       ctx.to_device(v), ctx.to_device(g))
    for name, a, b in zip(("dq", "dk", "dv"), got, want):
        a = a.numpy()
        if T == 1 and name != "dv":
            # a lone position: the softmax is constant in q and k, the reference's
            # gradient is exactly 0 and the device's is 0 up to the rounding of
            # dP - rowsum(dO O), whose two sums run in different orders
            assert np.abs(b).max() == 0.0
            assert np.abs(a).max() <= 1e-6 * float(np.abs(g).max() * np.abs(v).max()) * hd
            continue
        scale = float(np.abs(b).max())
        assert np.abs(a - b).max() <= 2e-4 * scale, (name, float(np.abs(a - b).max()), scale)


# (1029 and 4099 rows: 4 and 16 rows per workgroup with a ragged last
# workgroup; 2049 x 4096: 8 rows per workgroup at the widest rows)
@pytest.mark.parametrize("rows,d", [(7, 16), (33, 64), (64, 2048), (9, 4096), (5, 100),
                                    (3, 4100), (1029, 256), (4099, 512), (2049, 4096)])
def test_rms_norm_backward_matches_oracle(ctx, rows, d):
    r = np.random.default_rng(rows * 7 + d)
    x = r.standard_normal((rows, d)).astype(np.float32)
    w = (1 + 0.2 * r.standard_normal(d)).astype(np.float32)
    dy = r.standard_normal((rows, d)).astype(np.float32)
    want_dx, want_dw = mo.rms_norm_backward(x, w, dy, 1e-5)
    dx, dw = mh.rms_norm_backward(ctx, ctx.to_device(x), ctx.to_device(w), ctx.to_device(dy), 1e-5)
    dx, dw = dx.numpy(), dw.numpy()
    assert np.abs(dx - want_dx).max() <= 1e-5 * np.abs(want_dx).max()
    assert np.abs(dw - want_dw).max() <= 1e-5 * np.abs(want_dw).max() * np.sqrt(rows)


def test_rope_backward_is_bit_exact(ctx):
    r = np.random.default_rng(5)
    for hd, t in ((4, 9), (16, 33), (64, 100), (128, 64), (6, 20), (24, 50), (96, 31)):
        tables = mh.RotaryTables(ctx, hd, 128)
        cos, sin = mo.rope_tables(hd, 128)
        dy = r.standard_normal((3, t, hd)).astype(np.float32)
        got = mh.apply_rope_backward(ctx, ctx.to_device(dy), tables).numpy()
        want = mo.rope_backward(dy, cos, sin)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), hd


@pytest.mark.parametrize("n,v", [(4, 7), (16, 4096), (3, 32000), (5, 1001)])
def test_cross_entropy_backward_matches_oracle(ctx, n, v):
    r = np.random.default_rng(n + v)
    z = (3 * r.standard_normal((n, v))).astype(np.float32)
    t = r.integers(0, v, n).astype(np.int32)
    want = mo.cross_entropy_backward(z, t)
    loss, got = mh.cross_entropy_backward(ctx, ctx.to_device(z), t)
    assert np.abs(got.numpy() - want).max() <= 1e-5 / n
    assert abs(loss - mo.cross_entropy(z, t)) <= 1e-4 * abs(loss)


@pytest.mark.parametrize("rows,d,ff", [(1, 1, 1), (7, 16, 24), (64, 64, 176), (300, 128, 344),
                                        (1024, 2048, 5632)])
def test_swiglu_backward_matches_oracle(ctx, rows, d, ff):
    """The op-level swiglu backward against the oracle's closures: silu*mul
    backward (bit-exact elementwise) between matmul backwards."""
    print(f"\n[swiglu backward] rows={rows} d={d} ff={ff}", flush=True)
    r = mo.rng(rows + d + ff)
    x = mo.randn((rows, d), 1.0, r)
    wg, wu, wd = mo.randn((d, ff), 0.02, r), mo.randn((d, ff), 0.02, r), mo.randn((ff, d), 0.02, r)
    dout = mo.randn((rows, d), 1.0, r)
    dev = [ctx.to_device(a) for a in (x, wg, wu, wd, dout)]
    dx, dwg, dwu, dwd = (t.numpy() for t in mh.swiglu_backward(ctx, *dev))
    # oracle: the closures of mlp.rs:20-24 in reverse
    g = mo.gemm("nn", x, wg, rows, d, ff)
    u = mo.gemm("nn", x, wu, rows, d, ff)
    h = (g * (1.0 / (1.0 + np.exp(-g.astype(np.float64))))).astype(np.float32) * u
    dh, want_dwd = mo.matmul_backward(h, wd, dout, rows, ff, d)
    dg, du = mo.silu_mul_backward(g, u, dh)
    dx_g, want_dwg = mo.matmul_backward(x, wg, dg, rows, d, ff)
    dx_u, want_dwu = mo.matmul_backward(x, wu, du, rows, d, ff)
    want_dx = dx_g + dx_u
    for got, want, name in [(dx, want_dx, "dx"), (dwg, want_dwg, "dwg"), (dwu, want_dwu, "dwu"),
                            (dwd, want_dwd, "dwd")]:
        scale = max(float(np.max(np.abs(want))), 1e-30)
        e = float(np.max(np.abs(got.astype(np.float64) - want))) / scale
        print(f"  {name}: max|diff|/max|ref| {e:.3g}", flush=True)
        assert e <= 2e-4, name


@pytest.mark.parametrize("n,vocab,d", [(1, 1, 1), (13, 7, 16), (4096, 32000, 64), (777, 50, 300)])
def test_embedding_backward_is_bit_exact(ctx, n, vocab, d):
    """Rows added per id in position order, untouched rows zero: the oracle's
    bits (ops_shape.rs:261-269)."""
    r = np.random.default_rng(n + vocab)
    ids = r.integers(0, vocab, n).astype(np.int32)
    dy = r.standard_normal((n, d), dtype=np.float32)
    got = mh.embedding_backward(ctx, ids, ctx.to_device(dy), vocab).numpy()
    want = mo.embedding_backward(ids, dy, vocab)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(mh.IndexOutOfRange):
        mh.embedding_backward(ctx, np.array([vocab], np.int32), ctx.to_device(dy[:1]), vocab)


def test_lab_goldens_on_device(ctx, goldens):
    g = goldens["lab_native"]
    lab = mh.Lab(ctx, g["config"], g["hyper"], g["seed"], g["batch"], g["seq"])
    try:
        assert list(lab.inputs[: g["seq"]]) == g["inputs0"]
        losses, norms, lrs, stopped = lab.step(5)
        assert stopped is None
        for i in range(5):
            assert abs(losses[i] - g["losses"][i]) <= g["tol"] * g["losses"][i], (i, losses[i])
            assert abs(norms[i] - g["grad_norms"][i]) <= g["tol"] * g["grad_norms"][i], (i, norms[i])
        assert abs(lrs[0] - 0.03 / 15) <= 1e-5 * 0.03 / 15
        g150 = goldens["lab_native_150"]
        rest, _, lrs2, stopped = lab.step(g150["steps"] - 5)
        assert stopped is None and len(rest) == g150["steps"] - 5
        assert rest[-1] < g150["below_fraction_of_first"] * losses[0]
        rel = abs(rest[-1] - g150["final_loss"]) / g150["final_loss"]
        assert rel <= g150["final_loss_rel_tol"], (rest[-1], rel)
        _, acc, pred = lab.eval()
        assert acc >= g150["min_accuracy"]
        assert np.array_equal(pred, lab.targets)
        assert lab.model.optimizer_steps() == g150["steps"]
    finally:
        lab.close()


def test_train_steps_match_oracle(ctx):
    config = mh.PRESETS["smoke"]
    c = ocfg(config)
    print("\n[case] smoke 4 training steps vs oracle", flush=True)
    want_losses, want_norms, _, want_w = mo.lab_train(c, HYPER, 7, 2, 32, 4, want_weights=True)
    lab = mh.Lab(ctx, config, HYPER, 7, 2, 32)
    try:
        losses, norms, _, stopped = lab.step(4)
        w = lab.model.weights()
    finally:
        lab.close()
    assert stopped is None
    np.testing.assert_allclose(losses, want_losses, rtol=1e-5)
    np.testing.assert_allclose(norms, want_norms, rtol=1e-4)
    # AdamW moves each weight by at most ~lr per step; gradient rounding can
    # flip the direction of a near-zero gradient's step, nothing more.
    assert np.abs(w - want_w).max() <= 2 * 4 * HYPER[0]
    assert np.median(np.abs(w - want_w)) <= 1e-6


def test_training_is_deterministic(ctx):
    config = [97, 128, 2, 4, 2, 96, 96, 10000.0, 1e-5, 1]
    c = ocfg(config)
    w0 = mo.init_weights(c, mo.rng(3), std=0.1)
    r = np.random.default_rng(4)
    x = r.integers(0, 97, 2 * 64).astype(np.int32)
    y = r.integers(0, 97, 2 * 64).astype(np.int32)
    out = []
    for _ in range(2):
        m = mh.Model.from_weights(ctx, config, w0)
        try:
            m.set_optimizer(0.9, 0.99, 1e-8, 0.01, 1.0)
            rec = [m.train_step(x, y, 2, 64, 0.01) for _ in range(3)]
            out.append((rec, m.weights(), m.grads()))
        finally:
            m.close()
    assert out[0][0] == out[1][0]
    assert np.array_equal(out[0][1], out[1][1])
    assert np.array_equal(out[0][2], out[1][2])


def test_non_finite_step_changes_nothing(ctx):
    config = LAB
    c = ocfg(config)
    w = mo.init_weights(c, mo.rng(2024))
    w[5] = np.nan  # in the embedding table: the loss becomes NaN
    x = np.array([0, 1, 2, 3], np.int32)
    y = np.array([1, 2, 3, 4], np.int32)
    m = mh.Model.from_weights(ctx, config, w)
    try:
        m.set_optimizer(0.9, 0.99, 1e-8, 0.01, 1.0)
        with pytest.raises(mh.Stopped):
            m.train_step(x, y, 1, 4, 0.01)
        after = m.weights()
        assert np.array_equal(np.isnan(after), np.isnan(w))
        assert np.array_equal(after[~np.isnan(w)], w[~np.isnan(w)])
        assert m.optimizer_steps() == 0
        with pytest.raises(mh.ArgumentError):
            m.train_step(x, y, 1, 4, float("nan"))
        with pytest.raises(mh.ArgumentError):
            m.set_optimizer(1.0, 0.99, 1e-8, 0.01, 1.0)
        with pytest.raises(mh.IndexOutOfRange):
            m.train_step(np.array([0, 1, 2, 12], np.int32), y, 1, 4, 0.01)
    finally:
        m.close()


def test_large_widths_backward_matches_oracle(ctx):
    """One block at the large preset's widths (d 2048, 16 heads / 8 kv heads of
    128, ff 5632, V 32000), B1 T128."""
    config = [32000, 2048, 1, 16, 8, 5632, 2048, 10000.0, 1e-5, 1]
    c = ocfg(config)
    print("\n[case] large widths backward B1 T128", flush=True)
    w = mo.init_weights(c, mo.rng(0), std=0.02)
    r = np.random.default_rng(1)
    x = r.integers(0, 32000, 128).astype(np.int32)
    y = r.integers(0, 32000, 128).astype(np.int32)
    want_loss, want = mo.forward_backward(c, w, x, y, 1, 128)
    m = mh.Model.from_weights(ctx, config, w)
    try:
        loss = m.backward(x, y, 1, 128)
        got = m.grads()
    finally:
        m.close()
    assert abs(loss - want_loss) <= 1e-5 * abs(want_loss)
    check_grads(got, want, c, what="large")
