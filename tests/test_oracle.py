"""Pins the CPU oracle (oracle/mm_oracle.c) before it is trusted as the checker.

Each test checks one oracle function against a value the reference's own files
hold (tests/golden/reference_goldens.json), against the reference's own C twin
built from its sources into oracle/_ref, or against what the mathematics
fixes (closed forms, float64 brute force, finite differences, invariants),
chosen so that a dropped term, a wrong sign or index or a transposed operand
fails.
"""
import math

import numpy as np
import pytest

import mm_oracle as O


# ---- RNG: rng.rs:127-157 ------------------------------------------------------

def test_rng_next_u64_known_answers(goldens):
    for seed, want in goldens["rng_next_u64"].items():
        if seed.startswith("_"):
            continue
        r = O.rng(int(seed))
        got = [O.lib().mmo_rng_next_u64(r) for _ in range(4)]
        assert got == [int(w, 16) for w in want]


def test_rng_below_and_next_f32_known_answers(goldens):
    r = O.rng(7)
    assert [O.lib().mmo_rng_below(r, 10) for _ in range(8)] == goldens["rng_below_seed7_n10"]["values"]
    r = O.rng(5)
    for want in goldens["rng_next_f32_seed5"]["values"]:
        assert abs(O.lib().mmo_rng_next_f32(r) - want) < 1e-7


def test_normal_pairs_and_spare_order():
    # normal(): the first call returns r*cos(theta), caches r*sin(theta) (rng.rs:74-84).
    r1, r2 = O.rng(3), O.rng(3)
    u1 = 1.0 - O.lib().mmo_rng_next_f64(r2)
    u2 = O.lib().mmo_rng_next_f64(r2)
    rad = math.sqrt(-2.0 * math.log(u1))
    th = 2 * math.pi * u2
    a, b = O.lib().mmo_rng_normal(r1), O.lib().mmo_rng_normal(r1)
    assert a == np.float32(rad * math.cos(th))
    assert b == np.float32(rad * math.sin(th))


def test_normal_moments():
    x = O.normals(O.rng(2024), 200_000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1.0) < 0.02


# ---- config: presets.rs:125-138 -------------------------------------------------

def test_param_counts(goldens):
    for name, want in goldens["param_counts"].items():
        if name.startswith("_"):
            continue
        assert O.param_count(O.preset(name)) == want, name


def test_config_validation():
    assert O.lib().mmo_config_validate(O.config(12, 16, 2, 3, 1, 32, 16)) == O.ERR_CONFIG
    assert O.lib().mmo_config_validate(O.config(12, 18, 2, 2, 1, 32, 16)) == O.ERR_CONFIG  # hd 9
    assert O.lib().mmo_config_validate(O.config(12, 16, 2, 2, 1, 32, 16)) == O.OK


# ---- whole chain: init + forward + loss, pinned by the native goldens ----------

def lab_case(goldens, key):
    g = goldens[key]
    c = O.config(*g["config"][:7], g["config"][7], g["config"][8], bool(g["config"][9]))
    w, x, y = O.lab_setup(c, g["seed"], g["batch"], g["seq"])
    return g, c, w, x, y


def test_lab_golden_loss_and_tokens(goldens):
    g, c, w, x, y = lab_case(goldens, "lab_native")
    assert list(x[: g["seq"]]) == g["inputs0"]
    assert list(y[: g["seq"] - 1]) == g["inputs0"][1:]
    loss, _ = O.forward_loss(c, w, x, y, g["batch"], g["seq"])
    assert abs(loss - g["losses"][0]) / g["losses"][0] < 1e-6, loss


def test_smoke_golden_first_loss(goldens):
    g, c, w, x, y = lab_case(goldens, "smoke_first_loss")
    loss, _ = O.forward_loss(c, w, x, y, g["batch"], g["seq"])
    assert round(loss, g["printed_decimals"]) == g["loss"], loss


def test_golden_fails_when_a_term_is_dropped(goldens):
    # The golden is sensitive enough to catch a plausible mistake: zero the
    # residual projections (o_proj, down_proj) and the loss moves.
    g, c, w, x, y = lab_case(goldens, "lab_native")
    v = O.weight_views(c, w)
    w2 = w.copy()
    v2 = O.weight_views(c, w2)
    for l in range(c.n_layers):
        v2[f"blocks.{l}.attn.o_proj.weight"][...] = 0
    loss, _ = O.forward_loss(c, w2, x, y, g["batch"], g["seq"])
    assert abs(loss - g["losses"][0]) > 1e-4
    assert v["embed_tokens.weight"].shape == (12, 16)


def test_init_draw_order_and_scales():
    c = O.preset("smoke")
    r = O.rng(0)
    w = O.init_weights(c, r)
    v = O.weight_views(c, w)
    # embed is the first draw: it equals randn(V*d) of a fresh stream
    e = O.normals(O.rng(0), 256 * 64, 0.02)
    assert np.array_equal(v["embed_tokens.weight"].ravel(), e)
    assert np.all(v["blocks.0.attn_norm.weight"] == 1) and np.all(v["final_norm.weight"] == 1)
    out_std = np.float32(0.02) / np.sqrt(np.float32(2 * c.n_layers))
    for name, want in [("blocks.1.attn.q_proj.weight", 0.02), ("blocks.1.mlp.down_proj.weight", out_std)]:
        s = float(np.std(v[name]))
        assert abs(s - want) / want < 0.1, (name, s, want)


@pytest.mark.parametrize("cfg", [
    # an untied head, a vocabulary and widths that are not powers of two, and
    # (below) tensors past the 2^20-pair chunk
    (257, 1118, 1, 13, 1, 301, 16, 10000.0, 1e-5, False),
    (32000, 2048, 1, 16, 8, 5632, 16, 10000.0, 1e-5, True),
])
def test_threaded_init_equals_sequential(cfg):
    c = O.config(*cfg)
    seq = O.init_weights(c, O.rng(5), threads=1)
    r = O.rng(5)
    par = O.init_weights(c, r, threads=8)
    assert np.array_equal(seq.view(np.uint32), par.view(np.uint32))
    # the stream continues identically afterwards (spare included)
    r1 = O.rng(5)
    O.init_weights(c, r1, threads=1)
    assert np.array_equal(O.normals(r1, 7), O.normals(r, 7))


# ---- GEMM: ops_matmul.rs:137-156, the reference's own C twin, brute force -------

def test_gemm_hand_calculation(goldens):
    g = goldens["gemm_hand"]
    a = np.array(g["a"], np.float32).reshape(2, 3)
    b = np.array(g["b"], np.float32).reshape(3, 2)
    want = np.array(g["c"], np.float32).reshape(2, 2)
    assert np.array_equal(O.gemm("nn", a, b, 2, 3, 2), want)
    assert np.array_equal(O.gemm("nt", a, np.array(g["bt"], np.float32).reshape(2, 3), 2, 3, 2), want)
    assert np.array_equal(O.gemm("tn", np.array(g["at"], np.float32).reshape(3, 2), b, 2, 3, 2), want)


def test_gemm_bit_identical_to_reference_c_twin():
    ref = O.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    rng = np.random.default_rng(0)
    for n in (1, 5, 17, 33, 96, 130):
        a = rng.standard_normal((n, n)).astype(np.float32)
        b = rng.standard_normal((n, n)).astype(np.float32)
        c = np.empty((n, n), np.float32)
        ref.mmb_matmul_ikj(O.fp(a), O.fp(b), O.fp(c), n)  # i-k-j, same per-element order
        got = O.gemm("nn", a, b, n, n, n, threads=3)
        assert np.array_equal(got.view(np.uint32), c.view(np.uint32)), n


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 33, 41), (64, 17, 5), (130, 70, 260)])
def test_gemm_forms_against_float64(m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    bound = 1e-5 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30
    for form, aa, bb in (("nn", a, b), ("nt", a, b.T.copy()), ("tn", a.T.copy(), b)):
        got = O.gemm(form, aa, bb, m, k, n)
        assert np.all(np.abs(got - want) <= bound), form
    # accumulate semantics: C += A.B
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    got = O.gemm("nn", a, b, m, k, n, c=c0)
    assert np.all(np.abs(got - (c0 + want)) <= bound + 1e-6 * np.abs(c0))


def test_gemm_order_is_sequential_in_p():
    # gemm_nt equals the dot-product form bit for bit (ops_matmul.rs:240-273).
    rng = np.random.default_rng(5)
    a = (rng.standard_normal((3, 50)) * [1e-3, 1.0, 1e3][1]).astype(np.float32)
    b = rng.standard_normal((4, 50)).astype(np.float32)
    got = O.gemm("nt", a, b, 3, 50, 4)
    for i in range(3):
        for j in range(4):
            s = np.float32(0)
            for p in range(50):
                s = np.float32(s + np.float32(a[i, p] * b[j, p]))
            assert got[i, j] == s


def test_gemm_thread_count_does_not_change_bits():
    rng = np.random.default_rng(9)
    a = rng.standard_normal((67, 300)).astype(np.float32)
    b = rng.standard_normal((300, 91)).astype(np.float32)
    one = O.gemm("nn", a, b, 67, 300, 91, threads=1)
    many = O.gemm("nn", a, b, 67, 300, 91, threads=7)
    assert np.array_equal(one, many)


def test_matmul_backward_finite_differences():
    # loss = sum(W * (A.B)); dL/dA = W.B^T, dL/dB = A^T.W (ops_matmul.rs:62-74)
    rng = np.random.default_rng(1)
    rows, k, n = 5, 4, 3
    a = rng.standard_normal((rows, k))
    b = rng.standard_normal((k, n))
    wt = rng.standard_normal((rows, n))
    da, db = O.matmul_backward(a, b, wt, rows, k, n)
    f = lambda A, B: float(np.sum(wt * (A @ B)))
    eps = 1e-3
    for (i, j) in [(0, 0), (2, 3), (4, 1)]:
        ap, am = a.copy(), a.copy()
        ap[i, j] += eps
        am[i, j] -= eps
        fd = (f(ap, b) - f(am, b)) / (2 * eps)
        assert abs(fd - da[i, j]) < 1e-4 * max(1, abs(fd))
    for (i, j) in [(0, 0), (3, 2), (1, 1)]:
        bp, bm = b.copy(), b.copy()
        bp[i, j] += eps
        bm[i, j] -= eps
        fd = (f(a, bp) - f(a, bm)) / (2 * eps)
        assert abs(fd - db[i, j]) < 1e-4 * max(1, abs(fd))
    da_only, db_none = O.matmul_backward(a, b, wt, rows, k, n, need_b=False)
    assert db_none is None and np.array_equal(da_only, da)


def test_matmul_backward_against_float64():
    rng = np.random.default_rng(2)
    rows, k, n = 96, 40, 72
    a = rng.standard_normal((rows, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal((k, n))).astype(np.float32)
    dc = rng.standard_normal((rows, n)).astype(np.float32)
    da, db = O.matmul_backward(a, b, dc, rows, k, n)
    A, B, G = (x.astype(np.float64) for x in (a, b, dc))
    assert np.all(np.abs(da - G @ B.T) <= 1e-5 * (np.abs(G) @ np.abs(B.T)) + 1e-30)
    assert np.all(np.abs(db - A.T @ G) <= 1e-5 * (np.abs(A.T) @ np.abs(G)) + 1e-30)


# ---- layer ops: closed forms and invariants ---------------------------------------

def test_rms_norm_known_rows(goldens):
    g = goldens["rms_norm_row"]
    y = O.rms_norm(np.array([g["x"]], np.float32), np.array(g["w"], np.float32), g["eps"])
    r = math.sqrt(12.5)
    assert abs(y[0, 0] - 3 / r) < 1e-6 and abs(y[0, 1] - 8 / r) < 1e-6
    g = goldens["rms_norm_eps"]
    y = O.rms_norm(np.array([g["x"]], np.float32), np.ones(2, np.float32), g["eps"])
    assert np.all(np.abs(y - g["want"]) < g["tol"])


def test_rms_norm_reference_c_twin_close():
    ref = O.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(4)
    x = rng.standard_normal((16, 64)).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    c = np.empty_like(x)
    ref.mmb_rms_norm(O.fp(x), O.fp(w), O.fp(c), 16, 64, 1e-5)
    # the C twin divides by dim and uses 1/sqrtf; the tensor path multiplies by
    # 1/len and uses powf(-0.5): equal within a few ulp, not bit for bit.
    np.testing.assert_allclose(O.rms_norm(x, w, 1e-5), c, rtol=3e-7 * 8, atol=0)


def test_rope_formula_and_norm():
    cos, sin = O.rope_tables(8, 6, 10000.0)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    for pos in range(6):
        for i in range(4):
            ang = pos * 10000.0 ** (-i / 4)
            assert cos[pos, i] == np.float32(math.cos(ang)) and sin[pos, i] == np.float32(math.sin(ang))
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 3, 6, 8)).astype(np.float32)
    y = O.apply_rope(x, cos, sin)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # rotate-half formula (rope.rs:320-331): first half x1 c - x2 s, second x2 c + x1 s
    t = 3
    want0 = x[0, 0, t, 1] * cos[t, 1] - x[0, 0, t, 5] * sin[t, 1]
    want1 = x[0, 0, t, 5] * cos[t, 1] + x[0, 0, t, 1] * sin[t, 1]
    assert y[0, 0, t, 1] == np.float32(want0) and y[0, 0, t, 5] == np.float32(want1)


@pytest.mark.parametrize("hd", [8, 6, 24])
def test_rope_relative_position(hd):
    # q_i . k_j depends on i - j only (rope.rs:351-368)
    cos, sin = O.rope_tables(hd, 16, 10000.0)
    rng = np.random.default_rng(1)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    Q = O.apply_rope(np.tile(q, (16, 1))[None], cos, sin)[0]
    K = O.apply_rope(np.tile(k, (16, 1))[None], cos, sin)[0]
    assert abs(float(Q[5] @ K[2]) - float(Q[9] @ K[6])) < 1e-4


def test_attention_score_scaling(goldens):
    g = goldens["attention_scale"]
    shp = g["shape"]
    q, k, v = (np.array(g[n], np.float32).reshape(shp) for n in ("q", "k", "v"))
    out = O.causal_attention(q, k, v)
    w0 = 1.0 / (1.0 + math.exp(-1.0))
    want = np.array([1, 0, 0, 0, w0, 1 - w0, 0, 0], np.float32).reshape(shp)
    assert np.all(np.abs(out - want) < 1e-6)


@pytest.mark.parametrize("hd", [8, 6, 24, 48])
def test_attention_against_float64_softmax_and_gqa(hd):
    # head widths the device runs on its own kernels (8) and through padded
    # heads (6, 24, 48): the oracle's loops take any width
    rng = np.random.default_rng(3 + hd)
    B, H, Hkv, T = 2, 4, 2, 9
    q = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, hd)).astype(np.float32)
    out = O.causal_attention(q, k, v)
    # GQA = attention over copied heads (attention.rs:411-429)
    kx = np.repeat(k, H // Hkv, axis=1)
    vx = np.repeat(v, H // Hkv, axis=1)
    assert np.array_equal(out, O.causal_attention(q, kx, vx))
    s = (q.astype(np.float64) @ kx.astype(np.float64).transpose(0, 1, 3, 2)) / math.sqrt(hd)
    s = s + np.triu(np.full((T, T), -1e9), 1)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(out, p @ vx, rtol=1e-5, atol=1e-6)
    # a single position attends only to itself (attention.rs:296-303)
    assert np.allclose(out[:, :, 0], vx[:, :, 0], atol=1e-6)


def test_swiglu_known_value(goldens):
    g = goldens["swiglu_value"]
    one = lambda v: np.array([[v]], np.float32)
    out = O.swiglu(one(g["x"]), one(g["wg"]), one(g["wu"]), one(g["wd"]))
    silu2 = 2.0 / (1.0 + math.exp(-2.0))
    assert abs(out[0, 0] - silu2 * 12.0) < 1e-5


def test_cross_entropy_known_values(goldens):
    assert abs(O.cross_entropy(np.zeros((1, 2)), [0]) - math.log(2)) < 1e-6
    assert O.cross_entropy(np.array([[20.0, 0, 0]]), [0]) < 1e-6
    assert abs(O.cross_entropy(np.array([[0.0, 0], [50, -50]]), [1, 0]) - math.log(2) / 2) < 1e-6
    with pytest.raises(IndexError):
        O.cross_entropy(np.zeros((2, 3)), [0, 3])


def test_embedding_gathers_and_rejects_out_of_range():
    t = np.arange(12, dtype=np.float32).reshape(4, 3)
    assert np.array_equal(O.embedding(t, [3, 0, 3]), t[[3, 0, 3]])
    with pytest.raises(IndexError):
        O.embedding(t, [4])


# ---- whole-model invariants (wiring.rs:123-217) -------------------------------------

def small(tie=True):
    return O.config(13, 16, 2, 4, 2, 24, 8, 10000.0, 1e-5, tie)


def test_causality_prefix_and_batch_independence():
    c = small()
    w = O.init_weights(c, O.rng(1), std=0.3)
    ids = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.int32)
    full = O.forward(c, w, ids, 1, 8)
    for kk in range(1, 8):
        pre = O.forward(c, w, ids[:kk], 1, kk)
        assert np.allclose(pre[0], full[0, :kk], atol=1e-5)
    other = np.array([0, 7, 7, 2, 1, 1, 1, 1], np.int32)
    both = O.forward(c, w, np.concatenate([ids, other]), 2, 8)
    assert np.allclose(both[0], full[0], atol=1e-5)


def test_batch_loss_is_mean_of_sequences():
    c = small(tie=False)
    w = O.init_weights(c, O.rng(6), std=0.3)
    a, b = np.array([1, 5, 2, 8, 3]), np.array([12, 0, 7, 7, 4])
    ta, tb = np.array([5, 2, 8, 3, 6]), np.array([0, 7, 7, 4, 10])
    la, _ = O.forward_loss(c, w, a, ta, 1, 5)
    lb, _ = O.forward_loss(c, w, b, tb, 1, 5)
    lab, _ = O.forward_loss(c, w, np.concatenate([a, b]), np.concatenate([ta, tb]), 2, 5)
    assert abs(lab - (la + lb) / 2) < 1e-5


def test_fresh_model_loss_near_ln_vocab():
    c = O.preset("smoke")
    w, x, y = O.lab_setup(c, 0, 2, 32)
    loss, _ = O.forward_loss(c, w, x, y, 2, 32)
    assert abs(loss - math.log(256)) < 0.1
