"""ctypes binding of the CPU oracle (oracle/libmm_oracle.so).

TEST INFRASTRUCTURE ONLY. The oracle restates the reference's CPU algorithm
(midman-ai, Rust) op for op and is the parity checker for the HIP path and
the CPU timing baseline. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product never does.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MM_ORACLE_LIB selects another build of the same source (the sanitizer build).
_LIB_PATH = os.environ.get("MM_ORACLE_LIB") or os.path.join(_HERE, "libmm_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libmmb_ref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

OK, ERR_ARGUMENT, ERR_CONFIG, ERR_SHAPE, ERR_INDEX = 0, -1, -2, -3, -4
PRESETS = ("smoke", "tiny", "small", "base", "medium", "large")


class Rng(ctypes.Structure):
    """mmo_rng: xoshiro256** state plus the cached Box-Muller spare."""

    _fields_ = [("s", ctypes.c_uint64 * 4), ("has_spare", ctypes.c_int32),
                ("spare", ctypes.c_float)]


class Config(ctypes.Structure):
    """mmo_config, the reference ModelConfig (config.rs:20-43)."""

    _fields_ = [("vocab_size", _i64), ("d_model", _i64), ("n_layers", _i64),
                ("n_heads", _i64), ("n_kv_heads", _i64), ("d_ff", _i64),
                ("max_seq_len", _i64), ("rope_theta", ctypes.c_float),
                ("norm_eps", ctypes.c_float), ("tie_embeddings", ctypes.c_int32)]

    def as_list(self):
        """The reference's 10-field config order (ffi.rs:68-79)."""
        return [self.vocab_size, self.d_model, self.n_layers, self.n_heads,
                self.n_kv_heads, self.d_ff, self.max_seq_len, float(self.rope_theta),
                float(self.norm_eps), int(self.tie_embeddings)]

    @property
    def head_dim(self):
        return self.d_model // self.n_heads

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        R = ctypes.POINTER(Rng)
        C = ctypes.POINTER(Config)
        sig = {
            "mmo_rng_seed": (None, [R, ctypes.c_uint64]),
            "mmo_rng_next_u64": (ctypes.c_uint64, [R]),
            "mmo_rng_next_f32": (ctypes.c_float, [R]),
            "mmo_rng_next_f64": (ctypes.c_double, [R]),
            "mmo_rng_normal": (ctypes.c_float, [R]),
            "mmo_rng_below": (ctypes.c_uint64, [R, ctypes.c_uint64]),
            "mmo_rng_fork": (None, [R, ctypes.c_uint64, R]),
            "mmo_rng_shuffle_u64": (None, [R, ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.c_uint64]),
            "mmo_permutation": (None, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.POINTER(ctypes.c_uint64)]),
            "mmo_randn": (None, [R, _f32p, _i64, ctypes.c_float]),
            "mmo_config_validate": (_i32, [C]),
            "mmo_param_count": (_i64, [C]),
            "mmo_preset": (_i32, [_i32, C]),
            "mmo_init_weights": (_i32, [C, ctypes.c_float, R, _f32p, _i64]),
            "mmo_init_weights_mt": (_i32, [C, ctypes.c_float, R, _f32p, _i64, _i32]),
            "mmo_lab_tokens": (None, [R, _i64, _i64, _i64, _i32p, _i32p]),
            "mmo_gemm_nn": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i32]),
            "mmo_gemm_nt": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i32]),
            "mmo_gemm_tn": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i32]),
            "mmo_matmul_backward": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64,
                                           _i64, _i32]),
            "mmo_embedding": (_i32, [_f32p, _i64, _i64, _i32p, _i64, _f32p]),
            "mmo_rms_norm": (None, [_f32p, _f32p, _i64, _i64, ctypes.c_float, _f32p]),
            "mmo_rope_tables": (None, [_i64, _i64, ctypes.c_float, _f32p, _f32p]),
            "mmo_apply_rope": (None, [_f32p, _i64, _i64, _i64, _f32p, _f32p, _f32p]),
            "mmo_causal_attention": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                            _i64, _f32p, _i32]),
            "mmo_attention_forward": (None, [_f32p] * 7 + [_i64] * 5 + [_f32p, _i32]),
            "mmo_swiglu": (None, [_f32p] * 4 + [_i64] * 3 + [_f32p, _i32]),
            "mmo_cross_entropy": (_i32, [_f32p, _i32p, _i64, _i64, _f32p]),
            "mmo_cross_entropy_rows": (_i32, [_f32p, _i32p, _i64, _i64, _f32p]),
            "mmo_block_forward": (_i32, [C, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _f32p,
                                         _i32]),
            "mmo_forward": (_i32, [C, _f32p, _i32p, _i64, _i64, _f32p, _i32]),
            "mmo_forward_loss": (_i32, [C, _f32p, _i32p, _i32p, _i64, _i64, _f32p, _f32p,
                                        _i32]),
            "mmo_cross_entropy_backward": (_i32, [_f32p, _i32p, _i64, _i64, ctypes.c_float,
                                                  _f32p]),
            "mmo_embedding_backward": (None, [_i32p, _i64, _f32p, _i64, _f32p]),
            "mmo_rms_norm_backward": (None, [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float,
                                             _f32p, _f32p]),
            "mmo_rope_backward": (None, [_f32p, _i64, _i64, _i64, _f32p, _f32p, _f32p]),
            "mmo_causal_attention_backward": (None, [_f32p] * 4 + [_i64] * 5 + [_f32p] * 3
                                              + [_i32]),
            "mmo_silu_mul_backward": (None, [_f32p, _f32p, _f32p, _i64, _f32p, _f32p]),
            "mmo_param_segments": (_i64, [C, _i64p, _i64p, _i32p]),
            "mmo_forward_backward": (_i32, [C, _f32p, _i32p, _i32p, _i64, _i64, _f32p, _f32p,
                                            _i32]),
            "mmo_global_norm": (ctypes.c_float, [_f32p, _i64]),
            "mmo_clip_global_norm": (_i32, [_f32p, _i64, ctypes.c_float, _f32p]),
            "mmo_warmup_cosine_lr": (ctypes.c_float, [ctypes.c_float, ctypes.c_float,
                                                      ctypes.c_uint64, ctypes.c_uint64,
                                                      ctypes.c_uint64]),
            "mmo_adamw_step": (_i32, [C, _f32p, _f32p, _f32p, _f32p] + [ctypes.c_float] * 5
                               + [ctypes.POINTER(ctypes.c_uint64)]),
            "mmo_adamw_update": (None, [_f32p] * 4 + [_i64, _i32, ctypes.c_uint64]
                                 + [ctypes.c_float] * 5),
            "mmo_lab_train": (_i32, [C, ctypes.POINTER(ctypes.c_double), ctypes.c_uint64,
                                     _i64, _i64, _i64, _f32p, _f32p, _f32p, _f32p, _i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def default_threads():
    return max(1, min(8, os.cpu_count() or 1))


def fp(a):
    """float32 pointer of a C-contiguous array (or NULL for None)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def ip(a):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i32p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


# ---- rng -----------------------------------------------------------------

def rng(seed):
    r = Rng()
    lib().mmo_rng_seed(ctypes.byref(r), seed)
    return r


def normals(r, n, std=1.0):
    """Tensor::randn(n, std) drawn from r (std * normal() in f32)."""
    out = np.empty(n, np.float32)
    lib().mmo_randn(ctypes.byref(r), fp(out), n, std)
    return out


def randn(shape, std, r):
    """Tensor::randn(shape, std, rng) (tensor.rs:158-162)."""
    return normals(r, int(np.prod(shape)), std).reshape(shape)


# ---- config / init -------------------------------------------------------

def preset(name):
    c = Config()
    assert lib().mmo_preset(PRESETS.index(name), ctypes.byref(c)) == OK
    return c


def config(vocab, d, layers, heads, kv_heads, ff, max_seq, theta=10000.0, eps=1e-5, tie=True):
    return Config(vocab, d, layers, heads, kv_heads, ff, max_seq, theta, eps, 1 if tie else 0)


def param_count(c):
    return lib().mmo_param_count(ctypes.byref(c))


def init_weights(c, r, std=0.02, threads=None):
    """MidManModel::with_init_std's draws (model.rs:51-83); threads > 1 spreads
    the Box-Muller arithmetic over threads (same bits, tested)."""
    n = param_count(c)
    w = np.empty(n, np.float32)
    threads = threads or default_threads()
    if threads > 1:
        st = lib().mmo_init_weights_mt(ctypes.byref(c), std, ctypes.byref(r), fp(w), n, threads)
    else:
        st = lib().mmo_init_weights(ctypes.byref(c), std, ctypes.byref(r), fp(w), n)
    if st != OK:
        raise ValueError(f"mmo_init_weights status {st}")
    return w


def lab_tokens(r, vocab, batch, seq):
    inputs = np.empty(batch * seq, np.int32)
    targets = np.empty(batch * seq, np.int32)
    lib().mmo_lab_tokens(ctypes.byref(r), vocab, batch, seq, ip(inputs), ip(targets))
    return inputs, targets


def lab_setup(c, seed, batch, seq, std=0.02, threads=None):
    """Lab::new / overfit.rs memorize: weights then tokens from one stream."""
    r = rng(seed)
    w = init_weights(c, r, std, threads)
    inputs, targets = lab_tokens(r, c.vocab_size, batch, seq)
    return w, inputs, targets


def weight_views(c, w):
    """Named views into the flat reference-order parameter vector."""
    d, ff, kv, V = c.d_model, c.d_ff, c.kv_dim, c.vocab_size
    out, o = {}, 0

    def take(name, shape):
        nonlocal o
        n = int(np.prod(shape))
        out[name] = w[o:o + n].reshape(shape)
        o += n

    take("embed_tokens.weight", (V, d))
    for l in range(c.n_layers):
        p = f"blocks.{l}."
        take(p + "attn_norm.weight", (d,))
        take(p + "attn.q_proj.weight", (d, d))
        take(p + "attn.k_proj.weight", (d, kv))
        take(p + "attn.v_proj.weight", (d, kv))
        take(p + "attn.o_proj.weight", (d, d))
        take(p + "mlp_norm.weight", (d,))
        take(p + "mlp.gate_proj.weight", (d, ff))
        take(p + "mlp.up_proj.weight", (d, ff))
        take(p + "mlp.down_proj.weight", (ff, d))
    take("final_norm.weight", (d,))
    if not c.tie_embeddings:
        take("lm_head.weight", (d, V))
    assert o == w.size
    return out


# ---- ops -----------------------------------------------------------------

def gemm(form, a, b, m, k, n, c=None, threads=None):
    """C (+)= op(A) op(B); form in nn/nt/tn with the reference layouts."""
    a, b = f32(a), f32(b)
    out = np.zeros((m, n), np.float32) if c is None else f32(c).copy()
    getattr(lib(), f"mmo_gemm_{form}")(fp(a), fp(b), fp(out), m, k, n,
                                       threads or default_threads())
    return out


def matmul_backward(a, b, dc, rows, k, n, need_a=True, need_b=True, threads=None):
    a, b, dc = f32(a), f32(b), f32(dc)
    da = np.empty((rows, k), np.float32) if need_a else None
    db = np.empty((k, n), np.float32) if need_b else None
    lib().mmo_matmul_backward(fp(a), fp(b), fp(dc), fp(da), fp(db), rows, k, n,
                              threads or default_threads())
    return da, db


def embedding(table, ids):
    table, ids = f32(table), i32(ids)
    V, d = table.shape
    out = np.empty((ids.size, d), np.float32)
    st = lib().mmo_embedding(fp(table), V, d, ip(ids), ids.size, fp(out))
    if st != OK:
        raise IndexError(f"embedding status {st}")
    return out


def rms_norm(x, w, eps):
    x, w = f32(x), f32(w)
    d = x.shape[-1]
    out = np.empty_like(x)
    lib().mmo_rms_norm(fp(x), fp(w), x.size // d, d, eps, fp(out))
    return out


def rope_tables(hd, max_seq, theta=10000.0):
    half = hd // 2
    cos = np.empty((max_seq, half), np.float32)
    sin = np.empty((max_seq, half), np.float32)
    lib().mmo_rope_tables(hd, max_seq, theta, fp(cos), fp(sin))
    return cos, sin


def apply_rope(x, cos, sin):
    """x [..., T, hd]"""
    x = f32(x)
    t, hd = x.shape[-2], x.shape[-1]
    out = np.empty_like(x)
    lib().mmo_apply_rope(fp(x), x.size // (t * hd), t, hd, fp(f32(cos)), fp(f32(sin)), fp(out))
    return out


def causal_attention(q, k, v, threads=None):
    q, k, v = f32(q), f32(k), f32(v)
    B, H, T, hd = q.shape
    out = np.empty_like(q)
    lib().mmo_causal_attention(fp(q), fp(k), fp(v), B, H, k.shape[1], T, hd, fp(out),
                               threads or default_threads())
    return out


def attention_forward(x, wq, wk, wv, wo, cos, sin, heads, kv_heads, threads=None):
    x = f32(x)
    B, T, d = x.shape
    out = np.empty_like(x)
    lib().mmo_attention_forward(fp(x), fp(f32(wq)), fp(f32(wk)), fp(f32(wv)), fp(f32(wo)),
                                fp(f32(cos)), fp(f32(sin)), B, T, d, heads, kv_heads, fp(out),
                                threads or default_threads())
    return out


def swiglu(x, wg, wu, wd, threads=None):
    x = f32(x)
    d = x.shape[-1]
    ff = wg.shape[1]
    out = np.empty_like(x)
    lib().mmo_swiglu(fp(x), fp(f32(wg)), fp(f32(wu)), fp(f32(wd)), x.size // d, d, ff,
                     fp(out), threads or default_threads())
    return out


def cross_entropy(logits, targets):
    logits, targets = f32(logits), i32(targets)
    n, v = logits.shape
    loss = ctypes.c_float()
    st = lib().mmo_cross_entropy(fp(logits), ip(targets), n, v, ctypes.byref(loss))
    if st != OK:
        raise IndexError(f"cross_entropy status {st}")
    return loss.value


def cross_entropy_rows(logits, targets):
    logits, targets = f32(logits), i32(targets)
    n, v = logits.shape
    out = np.empty(n, np.float32)
    st = lib().mmo_cross_entropy_rows(fp(logits), ip(targets), n, v, fp(out))
    if st != OK:
        raise IndexError(f"cross_entropy status {st}")
    return out


def block_forward(c, block_w, cos, sin, x, threads=None):
    x = f32(x)
    B, T, d = x.shape
    out = np.empty_like(x)
    st = lib().mmo_block_forward(ctypes.byref(c), fp(f32(block_w)), fp(f32(cos)),
                                 fp(f32(sin)), fp(x), B, T, fp(out),
                                 threads or default_threads())
    assert st == OK, st
    return out


def forward(c, w, ids, batch, seq, threads=None):
    ids = i32(ids)
    logits = np.empty((batch, seq, c.vocab_size), np.float32)
    st = lib().mmo_forward(ctypes.byref(c), fp(w), ip(ids), batch, seq, fp(logits),
                           threads or default_threads())
    if st != OK:
        raise ValueError(f"forward status {st}")
    return logits


def forward_loss(c, w, ids, targets, batch, seq, want_logits=True, threads=None):
    ids, targets = i32(ids), i32(targets)
    logits = np.empty((batch, seq, c.vocab_size), np.float32) if want_logits else None
    loss = ctypes.c_float()
    st = lib().mmo_forward_loss(ctypes.byref(c), fp(w), ip(ids), ip(targets), batch, seq,
                                fp(logits), ctypes.byref(loss), threads or default_threads())
    if st != OK:
        raise ValueError(f"forward_loss status {st}")
    return loss.value, logits


# ---- backward and training step ---------------------------------------------

def cross_entropy_backward(logits, targets, g=1.0):
    logits, targets = f32(logits), i32(targets)
    n, v = logits.shape
    out = np.empty_like(logits)
    st = lib().mmo_cross_entropy_backward(fp(logits), ip(targets), n, v, g, fp(out))
    if st != OK:
        raise IndexError(f"cross_entropy_backward status {st}")
    return out


def embedding_backward(ids, g, vocab):
    """dtable [V,d] from the gradient rows g [N,d] (rows added in id order)."""
    ids, g = i32(ids), f32(g)
    d = g.shape[-1]
    out = np.zeros((vocab, d), np.float32)
    lib().mmo_embedding_backward(ip(ids), ids.size, fp(g), d, fp(out))
    return out


def rms_norm_backward(x, w, dy, eps):
    """(dx share of the norm, dw)."""
    x, w, dy = f32(x), f32(w), f32(dy)
    d = x.shape[-1]
    dx = np.empty_like(x)
    dw = np.empty(d, np.float32)
    lib().mmo_rms_norm_backward(fp(x), fp(w), fp(dy), x.size // d, d, eps, fp(dx), fp(dw))
    return dx, dw


def rope_backward(dy, cos, sin):
    dy = f32(dy)
    hd = dy.shape[-1]
    t = dy.shape[-2]
    out = np.empty_like(dy)
    lib().mmo_rope_backward(fp(dy), dy.size // (t * hd), t, hd, fp(f32(cos)), fp(f32(sin)),
                            fp(out))
    return out


def causal_attention_backward(q, k, v, dout, threads=None):
    q, k, v, dout = f32(q), f32(k), f32(v), f32(dout)
    B, H, T, hd = q.shape
    hkv = k.shape[1]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().mmo_causal_attention_backward(fp(q), fp(k), fp(v), fp(dout), B, H, hkv, T, hd,
                                        fp(dq), fp(dk), fp(dv), threads or default_threads())
    return dq, dk, dv


def silu_mul_backward(gate, up, dh):
    gate, up, dh = f32(gate), f32(up), f32(dh)
    dg, du = np.empty_like(gate), np.empty_like(up)
    lib().mmo_silu_mul_backward(fp(gate), fp(up), fp(dh), gate.size, fp(dg), fp(du))
    return dg, du


def param_segments(c):
    """[(offset, size, rank)] of the flat parameter layout."""
    off = np.zeros(9 * c.n_layers + 3, np.int64)
    size = np.zeros_like(off)
    rank = np.zeros(off.size, np.int32)
    n = lib().mmo_param_segments(ctypes.byref(c), off.ctypes.data_as(_i64p),
                                 size.ctypes.data_as(_i64p), ip(rank))
    assert n > 0, n
    return [(int(off[i]), int(size[i]), int(rank[i])) for i in range(n)]


def forward_backward(c, w, ids, targets, batch, seq, threads=None):
    """(loss, grads) with grads in the flat layout of w."""
    ids, targets = i32(ids), i32(targets)
    grads = np.empty(param_count(c), np.float32)
    loss = ctypes.c_float()
    st = lib().mmo_forward_backward(ctypes.byref(c), fp(w), ip(ids), ip(targets), batch, seq,
                                    ctypes.byref(loss), fp(grads),
                                    threads or default_threads())
    if st != OK:
        raise ValueError(f"forward_backward status {st}")
    return loss.value, grads


def global_norm(g):
    g = f32(g)
    return lib().mmo_global_norm(fp(g), g.size)


def warmup_cosine_lr(max_lr, min_lr, warmup, total, step):
    return lib().mmo_warmup_cosine_lr(max_lr, min_lr, warmup, total, step)


def adamw_step(c, w, g, m, v, lr, beta1, beta2, eps, weight_decay, steps):
    """Updates w, m, v in place; returns the new step count."""
    cnt = ctypes.c_uint64(steps)
    st = lib().mmo_adamw_step(ctypes.byref(c), fp(w), fp(f32(g)), fp(m), fp(v), lr, beta1,
                              beta2, eps, weight_decay, ctypes.byref(cnt))
    if st != OK:
        raise ValueError(f"adamw status {st}")
    return cnt.value


def adamw_update(w, g, m, v, decays, t, lr, beta1, beta2, eps, weight_decay):
    """One parameter's AdamW update at step t (from 1), in place."""
    lib().mmo_adamw_update(fp(w), fp(f32(g)), fp(m), fp(v), w.size, int(decays), t, lr, beta1,
                           beta2, eps, weight_decay)


def lab_train(c, hyper, seed, batch, seq, steps, want_weights=False, threads=None):
    """(losses, grad_norms, lrs, final weights or None) of Lab::step."""
    h = (ctypes.c_double * 8)(*[float(x) for x in hyper])
    losses = np.zeros(steps, np.float32)
    norms = np.zeros(steps, np.float32)
    lrs = np.zeros(steps, np.float32)
    w = np.empty(param_count(c), np.float32) if want_weights else None
    st = lib().mmo_lab_train(ctypes.byref(c), h, seed, batch, seq, steps, fp(losses),
                             fp(norms), fp(lrs), fp(w), threads or default_threads())
    if st != OK:
        raise ValueError(f"lab_train status {st}")
    return losses, norms, lrs, w


# ---- token shards, sequences and the batcher (midman-data) -----------------

SHARD_MAGIC = b"MMTOKENS"
SHARD_HEADER = 32  # shard.rs:22-23: magic 8, four u32, one u64
SHARD_CHECKSUM = 32


def shard_width(vocab):
    """shard.rs:28-34: 2 bytes per id up to 65,536 ids, else 4."""
    return 2 if vocab <= 65536 else 4


def shard_bytes(vocab, eos, tokens):
    """TokenShard::to_bytes (shard.rs:112-135): header, little-endian ids, and
    the SHA-256 of everything before it (hashlib)."""
    import hashlib
    import struct
    w = shard_width(vocab)
    t = np.asarray(tokens, dtype=np.uint32)
    body = SHARD_MAGIC + struct.pack("<IIIIQ", 1, w, vocab, eos, t.size) + \
        t.astype("<u2" if w == 2 else "<u4").tobytes()
    return body + hashlib.sha256(body).digest()


def shard_parse(data):
    """TokenShard::from_bytes (shard.rs:146-223) restated: returns (vocab, eos,
    tokens) or raises ValueError whose text holds the reference's reason."""
    import hashlib
    import struct
    if len(data) < SHARD_HEADER + SHARD_CHECKSUM:
        raise ValueError(f"{len(data)} bytes is shorter than the smallest shard, 64")
    if data[:8] != SHARD_MAGIC:
        raise ValueError("the file does not start with `MMTOKENS`")
    version, width, vocab, eos, count = struct.unpack("<IIIIQ", data[8:32])
    if version != 1:
        raise ValueError(f"token shard version {version} is not supported")
    if vocab == 0:
        raise ValueError("the vocabulary size is 0")
    if width != shard_width(vocab):
        raise ValueError(f"token width {width} is not the one for a vocabulary of {vocab} ids")
    if eos >= vocab:
        raise ValueError(f"the end-of-text id {eos} is not below the vocabulary size {vocab}")
    if count * width + SHARD_HEADER + SHARD_CHECKSUM != len(data):
        raise ValueError(f"{count} tokens of {width} bytes do not make a file of "
                         f"{len(data)} bytes")
    body = len(data) - SHARD_CHECKSUM
    if hashlib.sha256(data[:body]).digest() != data[body:]:
        raise ValueError("the checksum does not match: the file is damaged")
    t = np.frombuffer(data[SHARD_HEADER:body], "<u2" if width == 2 else "<u4").astype(np.uint32)
    bad = np.nonzero(t >= vocab)[0]
    if bad.size:
        at = int(bad[0])
        raise ValueError(f"token {int(t[at])} at position {at} is not below the vocabulary "
                         f"size {vocab}")
    return vocab, eos, t


def sequence_windows(shard_tokens, seq_len):
    """Sequences::new + window (batch.rs:45-104): the window starts of every
    sequence, as (shard index, first token) pairs in sequence order."""
    out = []
    for s, t in enumerate(shard_tokens):
        n = len(t)
        if n > seq_len:
            out += [(s, i * seq_len) for i in range((n - 1) // seq_len)]
    return out


def permutation(n, seed, epoch):
    """permutation() of batch.rs:244-248 through the C restatement."""
    out = np.empty(n, dtype=np.uint64)
    lib().mmo_permutation(n, seed, epoch,
                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))
    return out


def batches(shard_tokens, seq_len, batch, seed, count):
    """The first `count` batches of Batcher::new(..).next_batch() (batch.rs:161-239):
    a list of (inputs, targets, epoch, index), ids as uint32 arrays."""
    wins = sequence_windows(shard_tokens, seq_len)
    n = len(wins)
    per = n // batch
    if batch == 0 or n < batch:
        raise ValueError("fewer sequences than one batch")
    out, epoch, nxt = [], 0, 0
    order = permutation(n, seed, 0)
    for _ in range(count):
        if nxt == per:
            epoch, nxt = epoch + 1, 0
            order = permutation(n, seed, epoch)
        rows = [wins[int(i)] for i in order[nxt * batch:(nxt + 1) * batch]]
        w = np.stack([np.asarray(shard_tokens[s][a:a + seq_len + 1], np.uint32)
                      for s, a in rows])
        out.append((w[:, :seq_len].reshape(-1), w[:, 1:].reshape(-1), epoch, nxt))
        nxt += 1
    return out


def eval_rows(n, batch_size, max_batches):
    """Trainer::evaluate's choice of sequences (trainer.rs:236-249): a list of
    batches, each a list of sequence indices."""
    batch = min(batch_size, n)
    nb = min(max_batches, n // batch)
    rows = nb * batch
    return [[(b * batch + r) * n // rows for r in range(batch)] for b in range(nb)]


# ---- the reference's own C twins (oracle/_ref) -----------------------------

def ref_lib():
    """benches/midman-bench/c/baseline_kernels.c built into oracle/_ref, or None."""
    if not os.path.exists(_REF_PATH):
        return None
    L = ctypes.CDLL(_REF_PATH)
    sz = ctypes.c_size_t
    L.mmb_matmul_ikj.argtypes = [_f32p, _f32p, _f32p, sz]
    L.mmb_matmul_ijk.argtypes = [_f32p, _f32p, _f32p, sz]
    L.mmb_softmax_rows.argtypes = [_f32p, _f32p, sz, sz]
    L.mmb_silu.argtypes = [_f32p, _f32p, sz]
    L.mmb_rms_norm.argtypes = [_f32p, _f32p, _f32p, sz, sz, ctypes.c_float]
    L.mmb_adamw_update.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, ctypes.c_int] + \
        [ctypes.c_float] * 5
    for n in ("mmb_matmul_ikj", "mmb_matmul_ijk", "mmb_softmax_rows", "mmb_silu",
              "mmb_rms_norm", "mmb_adamw_update"):
        getattr(L, n).restype = None
    return L
