"""Python host side of libmidman_hip.so, over its C ABI (include/midman_hip.h).

Mirrors the reference's operator surface for the decoder path
(midman-tensor matmul and its backward, midman-nn's rms_norm / apply_rope /
causal_attention / attention_forward / swiglu / embedding, cross_entropy, and
MidManModel::{new, forward, loss}) with the same argument meaning and the same
error kinds (midman-foundation/src/error.rs:18-65): a bad argument raises
ArgumentError, a bad config ConfigError, mismatched sizes ShapeError, an id or
target >= vocab IndexOutOfRange, and a HIP failure DeviceError.

There is no CPU fallback: if the library is not built, importing works but
every call raises LibraryMissing.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# MMH_LIB_PATH selects another build of the library (the host-only sanitizer
# build, midman-ai_amd/build_sanitized.py, which has no device entry points).
LIB_PATH = os.environ.get("MMH_LIB_PATH") or os.path.join(_PKG_DIR, "libmidman_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_DIR), "include", "midman_hip.h")

OK, STOPPED = 0, 1
ERR_ARGUMENT, ERR_CONFIG, ERR_SHAPE, ERR_INDEX, ERR_OTHER, ERR_DEVICE, ERR_PANIC = (
    -1, -2, -3, -4, -5, -6, -99)


class MidmanError(Exception):
    """A non-zero status from the library, with its message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class ArgumentError(MidmanError, ValueError):
    pass


class ConfigError(MidmanError, ValueError):
    pass


class ShapeError(MidmanError, ValueError):
    pass


class IndexOutOfRange(MidmanError, IndexError):
    pass


class DeviceError(MidmanError, RuntimeError):
    pass


class LibraryMissing(RuntimeError):
    pass


_ERRORS = {ERR_ARGUMENT: ArgumentError, ERR_CONFIG: ConfigError, ERR_SHAPE: ShapeError,
           ERR_INDEX: IndexOutOfRange, ERR_DEVICE: DeviceError}

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p
_h = ctypes.c_int64
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> argtypes (all return int32 unless listed in _RESTYPES)
_SIGNATURES = {
    "mmh_abi_version": [],
    "mmh_error_ptr": [],
    "mmh_error_len": [],
    "mmh_context_create": [_i32, ctypes.POINTER(_h)],
    "mmh_context_destroy": [_h],
    "mmh_synchronize": [_h],
    "mmh_device_info": [_h, ctypes.c_char_p, ctypes.c_uint32, ctypes.POINTER(_i32)],
    "mmh_context_fused_slots": [_h, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "mmh_mfma_peak_probe": [_h, ctypes.POINTER(ctypes.c_double)],
    "mmh_alloc": [_h, ctypes.c_uint64, ctypes.POINTER(_vp)],
    "mmh_free": [_h, _vp],
    "mmh_upload": [_h, _vp, _vp, ctypes.c_uint64],
    "mmh_download": [_h, _vp, _vp, ctypes.c_uint64],
    "mmh_timer_start": [_h],
    "mmh_timer_stop": [_h, ctypes.POINTER(ctypes.c_float)],
    "mmh_randn": [ctypes.c_uint64, ctypes.c_float, _f32p, _i64],
    "mmh_gemm_nn": [_h, _vp, _vp, _vp, _i64, _i64, _i64, _i32],
    "mmh_gemm_nt": [_h, _vp, _vp, _vp, _i64, _i64, _i64, _i32],
    "mmh_gemm_tn": [_h, _vp, _vp, _vp, _i64, _i64, _i64, _i32],
    "mmh_gemm_noalloc": [_h, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i32],
    "mmh_matmul_batched": [_h, _vp, _vp, _vp, _i64, _i64, _i64, _i64],
    "mmh_matmul_backward": [_h, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64],
    "mmh_embedding": [_h, _vp, _i64, _i64, _i32p, _i64, _vp],
    "mmh_rms_norm": [_h, _vp, _vp, _i64, _i64, ctypes.c_float, _vp],
    "mmh_rope_tables": [_h, _i64, _i64, ctypes.c_float, _vp, _vp],
    "mmh_apply_rope": [_h, _vp, _i64, _i64, _i64, _vp, _vp, _vp],
    "mmh_causal_attention": [_h, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp],
    "mmh_attention_forward": [_h, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                              _i64, _vp],
    "mmh_block_forward": [_h, _vp, _vp, _vp, _vp] + [_i64] * 6 + [ctypes.c_float, _vp],
    "mmh_swiglu": [_h, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "mmh_add": [_h, _vp, _vp, _vp, _i64],
    "mmh_cross_entropy": [_h, _vp, _i32p, _i64, _i64, _f32p],
    "mmh_model_create": [_h, ctypes.POINTER(ctypes.c_double), _f32p, _i64, ctypes.POINTER(_h)],
    "mmh_model_create_seeded": [_h, ctypes.POINTER(ctypes.c_double), ctypes.c_uint64,
                                ctypes.c_float, ctypes.POINTER(_h)],
    "mmh_model_lab_tokens": [_h, _i64, _i64, _i32p, _i32p],
    "mmh_model_param_count": [_h, ctypes.POINTER(_i64)],
    "mmh_model_download_weights": [_h, _f32p, _i64],
    "mmh_model_forward": [_h, _i32p, _i64, _i64, _f32p],
    "mmh_model_loss": [_h, _i32p, _i32p, _i64, _i64, _f32p],
    "mmh_model_forward_loss": [_h, _i32p, _i32p, _i64, _i64, _f32p, _f32p],
    "mmh_model_destroy": [_h],
    "mmh_model_check_guards": [_h, ctypes.POINTER(ctypes.c_uint64)],
    "mmh_model_stage": [_h, _i32p, _i32p, _i64, _i64],
    "mmh_model_run_staged": [_h, _i64, _i64],
    "mmh_model_read_loss": [_h, _f32p],
    "mmh_model_set_forward_path": [_h, _i32],
    "mmh_model_last_forward_fused": [_h, _i32p],
    "mmh_model_fused_fallbacks": [_h, ctypes.POINTER(_i64), _i32p],
    "mmh_model_inject_fused_error": [_h, _i32],
    "mmh_model_fused_duration": [_h, _i64, _i64, _i32, _f32p, _f32p],
    "mmh_model_profile": [_h, _i64, _i64, _f32p, _i32p],
    "mmh_rms_norm_backward": [_h, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp, _vp],
    "mmh_apply_rope_backward": [_h, _vp, _i64, _i64, _i64, _vp, _vp, _vp],
    "mmh_causal_attention_backward": [_h, _vp, _vp, _vp, _vp] + [_i64] * 5 + [_vp] * 3,
    "mmh_cross_entropy_backward": [_h, _vp, _i32p, _i64, _i64, _vp, _f32p],
    "mmh_swiglu_backward": [_h] + [_vp] * 5 + [_i64] * 3 + [_vp] * 4,
    "mmh_embedding_backward": [_h, _i32p, _i64, _vp, _i64, _i64, _vp],
    "mmh_tensorfile_create": [ctypes.POINTER(_h)],
    "mmh_tensorfile_parse": [ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(_h)],
    "mmh_tensorfile_push": [_h, ctypes.c_char_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64),
                            ctypes.c_int32, _f32p, ctypes.c_uint64],
    "mmh_tensorfile_set_metadata": [_h, ctypes.c_char_p, ctypes.c_uint32, ctypes.c_char_p,
                                    ctypes.c_uint32],
    "mmh_tensorfile_count": [_h, ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "mmh_tensorfile_tensor": [_h, _i64, ctypes.c_char_p, ctypes.c_uint32,
                              ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32),
                              ctypes.POINTER(ctypes.c_uint64), ctypes.c_int32,
                              ctypes.POINTER(ctypes.c_uint64)],
    "mmh_tensorfile_read": [_h, _i64, _f32p, ctypes.c_uint64],
    "mmh_tensorfile_metadata": [_h, _i64, ctypes.c_char_p, ctypes.c_uint32,
                                ctypes.POINTER(ctypes.c_uint32), ctypes.c_char_p,
                                ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)],
    "mmh_tensorfile_serialize": [_h, ctypes.c_char_p, ctypes.c_uint64,
                                 ctypes.POINTER(ctypes.c_uint64)],
    "mmh_tensorfile_destroy": [_h],
    "mmh_model_save_checkpoint": [_h, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                  ctypes.POINTER(ctypes.c_char_p), _i64],
    "mmh_model_load_checkpoint": [_h, ctypes.c_char_p],
    "mmh_model_create_from_checkpoint": [_h, ctypes.POINTER(ctypes.c_double), ctypes.c_char_p,
                                         ctypes.POINTER(_h)],
    "mmh_model_backward": [_h, _i32p, _i32p, _i64, _i64, _f32p],
    "mmh_model_download_grads": [_h, _f32p, _i64],
    "mmh_model_grad_norm": [_h, _f32p],
    "mmh_model_set_optimizer": [_h] + [ctypes.c_float] * 5,
    "mmh_model_train_step": [_h, _i32p, _i32p, _i64, _i64, ctypes.c_float, _f32p, _f32p],
    "mmh_model_stage_train": [_h, _i32p, _i32p, _i64, _i64],
    "mmh_model_train_staged": [_h, _i64, _i64, ctypes.c_float, _f32p, _f32p],
    "mmh_model_optimizer_steps": [_h, ctypes.POINTER(ctypes.c_uint64)],
    "mmh_warmup_cosine_lr": [ctypes.c_float, ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64,
                             ctypes.c_uint64, _f32p],
    "mmh_sha256": [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p],
    "mmh_sha256_new": [ctypes.POINTER(_h)],
    "mmh_sha256_update": [_h, ctypes.c_char_p, ctypes.c_uint64],
    "mmh_sha256_finalize": [_h, ctypes.c_char_p],
    "mmh_sha256_select": [_i32, ctypes.POINTER(_i32)],
    "mmh_shard_create": [ctypes.c_uint32, ctypes.c_uint32, _u32p, ctypes.c_uint64,
                         ctypes.POINTER(_h)],
    "mmh_shard_parse": [ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(_h)],
    "mmh_shard_load": [ctypes.c_char_p, ctypes.POINTER(_h)],
    "mmh_shard_save": [_h, ctypes.c_char_p],
    "mmh_shard_info": [_h, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                       ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32),
                       ctypes.POINTER(ctypes.c_uint64)],
    "mmh_shard_tokens": [_h, _u32p, ctypes.c_uint64],
    "mmh_shard_serialize": [_h, ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
    "mmh_shard_destroy": [_h],
    "mmh_sequences_create": [ctypes.POINTER(_h), _i64, ctypes.c_uint64, ctypes.POINTER(_h)],
    "mmh_sequences_info": [_h, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                           ctypes.POINTER(_i64)],
    "mmh_sequences_window": [_h, ctypes.c_uint64, _u32p],
    "mmh_sequences_destroy": [_h],
    "mmh_batcher_create": [_h, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(_h)],
    "mmh_batcher_info": [_h] + [ctypes.POINTER(ctypes.c_uint64)] * 5,
    "mmh_batcher_seek": [_h, ctypes.c_uint64, ctypes.c_uint64],
    "mmh_batcher_next": [_h, _u32p, _u32p, ctypes.POINTER(ctypes.c_uint64),
                         ctypes.POINTER(ctypes.c_uint64)],
    "mmh_batcher_destroy": [_h],
    "mmh_model_train_next": [_h, _h, ctypes.c_float, _f32p, _f32p,
                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "mmh_model_evaluate": [_h, _h, ctypes.c_uint64, ctypes.c_uint64, _f32p,
                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
}

PROFILE_CLASSES = ("embedding", "rms_norm", "gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_down",
                   "gemm_head", "attention", "loss")
_RESTYPES = {"mmh_abi_version": ctypes.c_uint32, "mmh_error_ptr": ctypes.c_void_p,
             "mmh_error_len": ctypes.c_uint32}

_lib = None


def lib():
    """The loaded libmidman_hip.so; raises LibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built (run python midman-ai_amd/build.py); "
                "there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:  # only a host-only build lacks symbols; calling one raises
                continue
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _i32)
        _lib = L
    return _lib


def last_error() -> str:
    L = lib()
    n = L.mmh_error_len()
    p = L.mmh_error_ptr()
    return ctypes.string_at(p, n).decode("utf-8", "replace") if n else ""


def check(status: int) -> int:
    if status < 0:
        raise _ERRORS.get(status, MidmanError)(status, last_error())
    return status


def abi_version() -> int:
    return lib().mmh_abi_version()


def randn(shape, std: float, seed: int) -> np.ndarray:
    """Tensor::randn(shape, std, &mut Rng::seed_from_u64(seed)) on the host."""
    shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,)
    out = np.empty(shape, np.float32)
    check(lib().mmh_randn(seed, std, out.ctypes.data_as(_f32p), out.size))
    return out


def warmup_cosine_lr(max_lr: float, min_lr: float, warmup_steps: int, total_steps: int,
                     step: int) -> float:
    """WarmupCosine::new(..).lr(step) (schedule.rs:25-66)."""
    out = ctypes.c_float()
    check(lib().mmh_warmup_cosine_lr(max_lr, min_lr, warmup_steps, total_steps, step,
                                     ctypes.byref(out)))
    return out.value


class Stopped(MidmanError):
    """A training step that did not run because the loss or the gradient norm
    was not finite (lab.rs:268-271, clip.rs:48-50); nothing was changed."""


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _ip(a: np.ndarray):
    return a.ctypes.data_as(_i32p)


class Context:
    """One GPU and one HIP stream (mmh_context_*)."""

    def __init__(self, device: int = 0):
        h = _h()
        check(lib().mmh_context_create(device, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if getattr(self, "handle", 0):
            check(lib().mmh_context_destroy(self.handle))
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self):
        check(lib().mmh_synchronize(self.handle))

    def device_info(self):
        buf = ctypes.create_string_buffer(256)
        cu = _i32()
        check(lib().mmh_device_info(self.handle, buf, 256, ctypes.byref(cu)))
        return buf.value.decode(), cu.value

    def fused_slots(self):
        """(teams, round_robin): whether the fused forward runs on this
        context, and whether its workgroups take their team slots from the
        dispatch order (True) or from one atomic each (False)."""
        teams, rr = _i32(), _i32()
        check(lib().mmh_context_fused_slots(self.handle, ctypes.byref(teams), ctypes.byref(rr)))
        return bool(teams.value), bool(rr.value)

    def mfma_peak_tflops(self) -> float:
        """The fp32 MFMA rate the chip sustains with no memory traffic (a
        diagnostic ceiling under the published peak)."""
        v = ctypes.c_double()
        check(lib().mmh_mfma_peak_probe(self.handle, ctypes.byref(v)))
        return v.value

    def empty(self, shape, dtype=np.float32) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def to_device(self, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = DeviceArray(self, a.shape, a.dtype)
        d.upload(a)
        return d

    def timer_start(self):
        check(lib().mmh_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        check(lib().mmh_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value


class DeviceArray:
    """A device buffer from mmh_alloc with a shape and dtype."""

    def __init__(self, ctx: Context, shape, dtype=np.float32):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        p = _vp()
        check(lib().mmh_alloc(ctx.handle, max(self.nbytes, 1), ctypes.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size == self.size, (a.shape, self.shape)
        check(lib().mmh_upload(self.ctx.handle, self.ptr, a.ctypes.data, self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().mmh_download(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr:
            check(lib().mmh_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and getattr(self.ctx, "handle", 0):
                lib().mmh_free(self.ctx.handle, self.ptr)
        except Exception:
            pass

    def offset(self, elements: int) -> int:
        return self.ptr + elements * self.dtype.itemsize


def _ptr(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceArray) else x


# ---- the GEMM seam: kernels.rs:49-84 -------------------------------------------

def gemm(ctx: Context, form: str, a, b, c, m: int, k: int, n: int, accumulate: bool = False):
    """C (+)= op(A) op(B) for form in {"nn", "nt", "tn"} (kernels.rs layouts)."""
    fn = {"nn": "mmh_gemm_nn", "nt": "mmh_gemm_nt", "tn": "mmh_gemm_tn"}[form]
    check(getattr(lib(), fn)(ctx.handle, _ptr(a), _ptr(b), _ptr(c), m, k, n,
                             1 if accumulate else 0))


def matmul(ctx: Context, a: DeviceArray, b: DeviceArray) -> DeviceArray:
    """Tensor::matmul (ops_matmul.rs:34): [.., m, k] x [k, n] or batched [b.., m, k] x [b.., k, n]."""
    if len(a.shape) < 2 or len(b.shape) < 2:
        raise ShapeError(ERR_SHAPE, "matmul: both operands need at least 2 axes")
    m, k = a.shape[-2], a.shape[-1]
    k2, n = b.shape[-2], b.shape[-1]
    if k != k2:
        raise ShapeError(ERR_SHAPE, f"matmul: inner dimensions differ: {a.shape} x {b.shape}")
    if len(b.shape) == 2:
        rows = a.size // k
        out = ctx.empty(a.shape[:-1] + (n,))
        gemm(ctx, "nn", a, b, out, rows, k, n)
        return out
    if a.shape[:-2] != b.shape[:-2]:
        raise ShapeError(ERR_SHAPE, "matmul: batched operands need the same leading axes")
    batch = int(np.prod(a.shape[:-2]))
    out = ctx.empty(a.shape[:-2] + (m, n))
    check(lib().mmh_matmul_batched(ctx.handle, a.ptr, b.ptr, out.ptr, batch, m, k, n))
    return out


def matmul_backward(ctx: Context, a, b, dc, rows: int, k: int, n: int, da=None, db=None):
    """The matmul backward closure (ops_matmul.rs:62-74): dA = dC B^T, dB = A^T dC."""
    check(lib().mmh_matmul_backward(ctx.handle, _ptr(a), _ptr(b), _ptr(dc), _ptr(da), _ptr(db),
                                    rows, k, n))


# ---- layer ops: midman-nn/src/lib.rs:45-56 --------------------------------------

def embedding(ctx: Context, table: DeviceArray, ids: np.ndarray, out: DeviceArray = None):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V, d = table.shape
    out = out or ctx.empty(ids.shape + (d,))
    check(lib().mmh_embedding(ctx.handle, table.ptr, V, d, _ip(ids), ids.size, out.ptr))
    return out


def rms_norm(ctx: Context, x: DeviceArray, w: DeviceArray, eps: float, out: DeviceArray = None):
    d = x.shape[-1]
    if w.shape != (d,):
        raise ShapeError(ERR_SHAPE, f"rms_norm: weight must have shape [{d}], got {w.shape}")
    out = out or ctx.empty(x.shape)
    check(lib().mmh_rms_norm(ctx.handle, x.ptr, w.ptr, x.size // d, d, eps, out.ptr))
    return out


class RotaryTables:
    """RotaryTables::new (rope.rs:54-85) on the device."""

    def __init__(self, ctx: Context, head_dim: int, max_seq_len: int, theta: float = 10000.0):
        self.head_dim, self.max_seq_len = head_dim, max_seq_len
        self.cos = ctx.empty((max_seq_len, head_dim // 2))
        self.sin = ctx.empty((max_seq_len, head_dim // 2))
        check(lib().mmh_rope_tables(ctx.handle, head_dim, max_seq_len, theta, self.cos.ptr,
                                    self.sin.ptr))


def apply_rope(ctx: Context, x: DeviceArray, tables: RotaryTables, out: DeviceArray = None):
    """RotaryTables::apply (rope.rs:114-128): x [.., T, hd], positions 0..T-1."""
    t, hd = x.shape[-2], x.shape[-1]
    if t > tables.max_seq_len:
        raise ShapeError(ERR_SHAPE, "rope: sequence longer than the tables")
    out = out or ctx.empty(x.shape)
    check(lib().mmh_apply_rope(ctx.handle, x.ptr, x.size // (t * hd), t, hd, tables.cos.ptr,
                               tables.sin.ptr, out.ptr))
    return out


def causal_attention(ctx: Context, q: DeviceArray, k: DeviceArray, v: DeviceArray,
                     out: DeviceArray = None):
    """attention.rs:97-101: q [B,H,T,hd], k/v [B,Hkv,T,hd] -> [B,H,T,hd]."""
    if len(q.shape) != 4 or len(k.shape) != 4 or k.shape != v.shape:
        raise ShapeError(ERR_SHAPE, "causal_attention: expected q [B,H,T,D] and k, v [B,Hkv,T,D]")
    B, H, T, hd = q.shape
    if k.shape[0] != B or k.shape[2] != T or k.shape[3] != hd:
        raise ShapeError(ERR_SHAPE, "causal_attention: q and k disagree on batch, time or head size")
    out = out or ctx.empty(q.shape)
    check(lib().mmh_causal_attention(ctx.handle, q.ptr, k.ptr, v.ptr, B, H, k.shape[1], T, hd,
                                     out.ptr))
    return out


def attention_forward(ctx: Context, x: DeviceArray, wq, wk, wv, wo, n_heads: int,
                      n_kv_heads: int, tables: RotaryTables, out: DeviceArray = None):
    """attention.rs:146-170: x [B,T,d] -> [B,T,d]."""
    B, T, d = x.shape
    out = out or ctx.empty(x.shape)
    check(lib().mmh_attention_forward(ctx.handle, x.ptr, _ptr(wq), _ptr(wk), _ptr(wv), _ptr(wo),
                                      tables.cos.ptr, tables.sin.ptr, B, T, d, n_heads,
                                      n_kv_heads, out.ptr))
    return out


def block_forward(ctx: Context, x: DeviceArray, block_weights: DeviceArray, n_heads: int,
                  n_kv_heads: int, d_ff: int, eps: float, tables: RotaryTables,
                  out: DeviceArray = None):
    """DecoderBlock::forward (block.rs:67-81): x [B,T,d] -> [B,T,d]. The
    weights are one flat array in DecoderBlock::parameters order (attn_norm,
    q, k, v, o, mlp_norm, gate, up, down)."""
    B, T, d = x.shape
    out = out or ctx.empty(x.shape)
    check(lib().mmh_block_forward(ctx.handle, x.ptr, block_weights.ptr, tables.cos.ptr,
                                  tables.sin.ptr, B, T, d, n_heads, n_kv_heads, d_ff, eps,
                                  out.ptr))
    return out


def swiglu(ctx: Context, x: DeviceArray, wg: DeviceArray, wu: DeviceArray, wd: DeviceArray,
           out: DeviceArray = None):
    """mlp.rs:20-24: (silu(x Wg) * (x Wu)) Wd."""
    d = x.shape[-1]
    ff = wg.shape[1]
    out = out or ctx.empty(x.shape)
    check(lib().mmh_swiglu(ctx.handle, x.ptr, wg.ptr, wu.ptr, wd.ptr, x.size // d, d, ff, out.ptr))
    return out


def add(ctx: Context, a: DeviceArray, b: DeviceArray, out: DeviceArray = None):
    if a.shape != b.shape:
        raise ShapeError(ERR_SHAPE, f"add: shapes {a.shape} and {b.shape} differ")
    out = out or ctx.empty(a.shape)
    check(lib().mmh_add(ctx.handle, a.ptr, b.ptr, out.ptr, a.size))
    return out


def cross_entropy(ctx: Context, logits: DeviceArray, targets: np.ndarray) -> float:
    """Tensor::cross_entropy (ops_reduce.rs:236-259): mean over rows, f64 accumulation."""
    if len(logits.shape) != 2:
        raise ShapeError(ERR_SHAPE, f"cross_entropy: logits must have shape [N, V], got {logits.shape}")
    n, v = logits.shape
    targets = np.ascontiguousarray(targets, dtype=np.int32)
    if targets.size != n:
        raise ShapeError(ERR_SHAPE, f"cross_entropy: {n} logit rows but {targets.size} targets")
    loss = ctypes.c_float()
    check(lib().mmh_cross_entropy(ctx.handle, logits.ptr, _ip(targets), n, v, ctypes.byref(loss)))
    return loss.value


# ---- backward closures of the layer seam ---------------------------------------------

def rms_norm_backward(ctx: Context, x: DeviceArray, w: DeviceArray, dy: DeviceArray, eps: float):
    """rms_norm's backward (norm.rs:36-38): (dx, dw)."""
    d = x.shape[-1]
    if w.shape != (d,) or dy.shape != x.shape:
        raise ShapeError(ERR_SHAPE, "rms_norm backward: x, w, dy do not fit")
    dx = ctx.empty(x.shape)
    dw = ctx.empty((d,))
    check(lib().mmh_rms_norm_backward(ctx.handle, x.ptr, w.ptr, dy.ptr, x.size // d, d, eps,
                                      dx.ptr, dw.ptr))
    return dx, dw


def apply_rope_backward(ctx: Context, dy: DeviceArray, tables: RotaryTables,
                        out: DeviceArray = None):
    """apply_rope's backward (rope.rs:28-32): rotation by -angle."""
    t, hd = dy.shape[-2], dy.shape[-1]
    if t > tables.max_seq_len:
        raise ShapeError(ERR_SHAPE, "rope: sequence longer than the tables")
    out = out or ctx.empty(dy.shape)
    check(lib().mmh_apply_rope_backward(ctx.handle, dy.ptr, dy.size // (t * hd), t, hd,
                                        tables.cos.ptr, tables.sin.ptr, out.ptr))
    return out


def causal_attention_backward(ctx: Context, q: DeviceArray, k: DeviceArray, v: DeviceArray,
                              dout: DeviceArray):
    """causal_attention's backward (attention.rs:79-101): (dq, dk, dv)."""
    if len(q.shape) != 4 or len(k.shape) != 4 or k.shape != v.shape or dout.shape != q.shape:
        raise ShapeError(ERR_SHAPE, "causal_attention backward: shapes do not fit")
    B, H, T, hd = q.shape
    dq, dk, dv = ctx.empty(q.shape), ctx.empty(k.shape), ctx.empty(v.shape)
    check(lib().mmh_causal_attention_backward(ctx.handle, q.ptr, k.ptr, v.ptr, dout.ptr, B, H,
                                              k.shape[1], T, hd, dq.ptr, dk.ptr, dv.ptr))
    return dq, dk, dv


def cross_entropy_backward(ctx: Context, logits: DeviceArray, targets: np.ndarray):
    """Tensor::cross_entropy backward (ops_reduce.rs:261-275): (loss, dlogits)."""
    if len(logits.shape) != 2:
        raise ShapeError(ERR_SHAPE, "cross_entropy: logits must have shape [N, V]")
    n, v = logits.shape
    targets = np.ascontiguousarray(targets, dtype=np.int32)
    if targets.size != n:
        raise ShapeError(ERR_SHAPE, f"cross_entropy: {n} logit rows but {targets.size} targets")
    out = ctx.empty(logits.shape)
    loss = ctypes.c_float()
    check(lib().mmh_cross_entropy_backward(ctx.handle, logits.ptr, _ip(targets), n, v, out.ptr,
                                           ctypes.byref(loss)))
    return loss.value, out


def swiglu_backward(ctx: Context, x: DeviceArray, wg: DeviceArray, wu: DeviceArray,
                    wd: DeviceArray, dout: DeviceArray):
    """Backward of swiglu (mlp.rs:20-24): (dx, dwg, dwu, dwd)."""
    d = x.shape[-1]
    ff = wg.shape[1]
    rows = x.size // d
    if wg.shape != (d, ff) or wu.shape != (d, ff) or wd.shape != (ff, d) or dout.size != x.size:
        raise ShapeError(ERR_SHAPE, "swiglu_backward: x [.., d], wg, wu [d, ff], wd [ff, d]")
    dx, dwg, dwu, dwd = ctx.empty(x.shape), ctx.empty((d, ff)), ctx.empty((d, ff)), ctx.empty((ff, d))
    check(lib().mmh_swiglu_backward(ctx.handle, x.ptr, wg.ptr, wu.ptr, wd.ptr, dout.ptr, rows, d,
                                    ff, dx.ptr, dwg.ptr, dwu.ptr, dwd.ptr))
    return dx, dwg, dwu, dwd


def embedding_backward(ctx: Context, ids: np.ndarray, dy: DeviceArray, vocab: int):
    """Backward of embedding (ops_shape.rs:261-269): dtable [vocab, d]."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    d = dy.shape[-1]
    if dy.size != ids.size * d:
        raise ShapeError(ERR_SHAPE, "embedding_backward: dy must be [n, d] for n ids")
    out = ctx.empty((vocab, d))
    check(lib().mmh_embedding_backward(ctx.handle, _ip(ids), ids.size, dy.ptr, vocab, d, out.ptr))
    return out


# ---- checkpoints: midman-checkpoint ----------------------------------------------------

class TensorFile:
    """midman-checkpoint's TensorFile (safetensors.rs:68-330) in the library:
    named f32 tensors plus string metadata, parsed with the reference's checks
    and serialized to the reference's exact bytes. Host-only."""

    def __init__(self, handle: Optional[int] = None):
        if handle is None:
            h = _h()
            check(lib().mmh_tensorfile_create(ctypes.byref(h)))
            handle = h.value
        self.handle = handle

    @classmethod
    def from_bytes(cls, data: bytes) -> "TensorFile":
        h = _h()
        check(lib().mmh_tensorfile_parse(data, len(data), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def load(cls, path: str) -> "TensorFile":
        with open(path, "rb") as f:
            return cls.from_bytes(f.read())

    def push(self, name: str, shape, data):
        nb = name.encode("utf-8")
        shape = [int(s) for s in shape]
        sh = (ctypes.c_uint64 * max(1, len(shape)))(*shape)
        arr = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        check(lib().mmh_tensorfile_push(self.handle, nb, len(nb), sh, len(shape), _fp(arr),
                                        arr.size))

    def set_metadata(self, key: str, value: str):
        kb, vb = key.encode("utf-8"), value.encode("utf-8")
        check(lib().mmh_tensorfile_set_metadata(self.handle, kb, len(kb), vb, len(vb)))

    def _counts(self):
        nt, nm = _i64(), _i64()
        check(lib().mmh_tensorfile_count(self.handle, ctypes.byref(nt), ctypes.byref(nm)))
        return nt.value, nm.value

    def tensors(self):
        """[(name, shape, values)] in file (or insertion) order."""
        out = []
        for i in range(self._counts()[0]):
            nl, rank, numel = ctypes.c_uint32(), ctypes.c_int32(), ctypes.c_uint64()
            check(lib().mmh_tensorfile_tensor(self.handle, i, None, 0, ctypes.byref(nl), None,
                                              None, 0, None))
            name = ctypes.create_string_buffer(max(1, nl.value))
            shape = (ctypes.c_uint64 * 16)()
            check(lib().mmh_tensorfile_tensor(self.handle, i, name, nl.value, ctypes.byref(nl),
                                              ctypes.byref(rank), shape, 16,
                                              ctypes.byref(numel)))
            vals = np.empty(numel.value, np.float32)
            check(lib().mmh_tensorfile_read(self.handle, i, _fp(vals), numel.value))
            out.append((name.raw[: nl.value].decode("utf-8"), [shape[k] for k in range(rank.value)],
                        vals))
        return out

    def metadata(self) -> dict:
        out = {}
        for i in range(self._counts()[1]):
            kl, vl = ctypes.c_uint32(), ctypes.c_uint32()
            check(lib().mmh_tensorfile_metadata(self.handle, i, None, 0, ctypes.byref(kl), None,
                                                0, ctypes.byref(vl)))
            k = ctypes.create_string_buffer(max(1, kl.value))
            v = ctypes.create_string_buffer(max(1, vl.value))
            check(lib().mmh_tensorfile_metadata(self.handle, i, k, kl.value, ctypes.byref(kl), v,
                                                vl.value, ctypes.byref(vl)))
            out[k.raw[: kl.value].decode("utf-8")] = v.raw[: vl.value].decode("utf-8")
        return out

    def to_bytes(self) -> bytes:
        n = ctypes.c_uint64()
        check(lib().mmh_tensorfile_serialize(self.handle, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(1, n.value))
        check(lib().mmh_tensorfile_serialize(self.handle, buf, n.value, ctypes.byref(n)))
        return buf.raw[: n.value]

    def close(self):
        if self.handle:
            check(lib().mmh_tensorfile_destroy(self.handle))
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


def parameter_names(config) -> list:
    """The reference's parameter names in Module order (docs/midman-model.md:20)."""
    L, tie = int(config[2]), bool(config[9])
    names = ["embed_tokens.weight"]
    for i in range(L):
        b = f"blocks.{i}."
        names += [b + "attn_norm.weight", b + "attn.q_proj.weight", b + "attn.k_proj.weight",
                  b + "attn.v_proj.weight", b + "attn.o_proj.weight", b + "mlp_norm.weight",
                  b + "mlp.gate_proj.weight", b + "mlp.up_proj.weight", b + "mlp.down_proj.weight"]
    names.append("final_norm.weight")
    if not tie:
        names.append("lm_head.weight")
    return names


# ---- training data: midman-data (hash.rs, shard.rs, batch.rs) -------------------------

def sha256(data: bytes) -> bytes:
    """midman-data's sha256 (hash.rs)."""
    out = ctypes.create_string_buffer(32)
    check(lib().mmh_sha256(data, len(data), out))
    return out.raw


def sha256_select(mode: int) -> int:
    """The compression path: 0 best available, 1 portable, 2 x86 SHA
    extensions if present. Returns the path in use (1 or 2)."""
    v = ctypes.c_int32()
    check(lib().mmh_sha256_select(mode, ctypes.byref(v)))
    return v.value


class Sha256:
    """Sha256::new / update / finalize (hash.rs)."""

    def __init__(self):
        h = _h()
        check(lib().mmh_sha256_new(ctypes.byref(h)))
        self.handle = h.value

    def update(self, data: bytes):
        check(lib().mmh_sha256_update(self.handle, data, len(data)))

    def finalize(self) -> bytes:
        out = ctypes.create_string_buffer(32)
        check(lib().mmh_sha256_finalize(self.handle, out))
        self.handle = 0
        return out.raw


class _Handle:
    _destroy = ""

    def close(self):
        if getattr(self, "handle", 0):
            check(getattr(lib(), self._destroy)(self.handle))
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


class TokenShard(_Handle):
    """TokenShard (shard.rs:53-260): token ids of one vocabulary, stored as a
    32-byte header, 2- or 4-byte little-endian ids and a SHA-256."""

    _destroy = "mmh_shard_destroy"

    def __init__(self, vocab_size: int, eos: int, tokens=(), *, _handle: Optional[int] = None):
        if _handle is None:
            t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64).astype(np.uint32))
            if np.any(np.asarray(tokens, dtype=np.int64) != t):
                raise ArgumentError(ERR_ARGUMENT, "token ids are 32-bit unsigned")
            h = _h()
            check(lib().mmh_shard_create(vocab_size, eos, t.ctypes.data_as(_u32p), t.size,
                                         ctypes.byref(h)))
            _handle = h.value
        self.handle = _handle

    @classmethod
    def from_bytes(cls, data: bytes) -> "TokenShard":
        h = _h()
        check(lib().mmh_shard_parse(data, len(data), ctypes.byref(h)))
        return cls(0, 0, _handle=h.value)

    @classmethod
    def load(cls, path: str) -> "TokenShard":
        h = _h()
        check(lib().mmh_shard_load(os.fsencode(path), ctypes.byref(h)))
        return cls(0, 0, _handle=h.value)

    def save(self, path: str):
        check(lib().mmh_shard_save(self.handle, os.fsencode(path)))

    def _info(self):
        v, e, w = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        n, fb = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mmh_shard_info(self.handle, ctypes.byref(v), ctypes.byref(e),
                                   ctypes.byref(n), ctypes.byref(w), ctypes.byref(fb)))
        return v.value, e.value, n.value, w.value, fb.value

    def vocab_size(self) -> int:
        return self._info()[0]

    def eos(self) -> int:
        return self._info()[1]

    def __len__(self) -> int:
        return self._info()[2]

    def is_empty(self) -> bool:
        return len(self) == 0

    def token_width(self) -> int:
        return self._info()[3]

    def tokens(self) -> np.ndarray:
        n = len(self)
        out = np.empty(n, np.uint32)
        check(lib().mmh_shard_tokens(self.handle, out.ctypes.data_as(_u32p), n))
        return out

    def to_bytes(self) -> bytes:
        n = ctypes.c_uint64()
        check(lib().mmh_shard_serialize(self.handle, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(1, n.value))
        check(lib().mmh_shard_serialize(self.handle, buf, n.value, ctypes.byref(n)))
        return buf.raw[: n.value]

    def __eq__(self, other):
        return (isinstance(other, TokenShard) and self._info()[:3] == other._info()[:3]
                and np.array_equal(self.tokens(), other.tokens()))

    __hash__ = None


class Sequences(_Handle):
    """Sequences (batch.rs:31-104): windows of seq_len + 1 tokens, one every
    seq_len tokens of each shard, never across shards."""

    _destroy = "mmh_sequences_destroy"

    def __init__(self, shards, seq_len: int):
        hs = (_h * max(1, len(shards)))(*[s.handle for s in shards])
        h = _h()
        check(lib().mmh_sequences_create(hs, len(shards), seq_len, ctypes.byref(h)))
        self.handle = h.value

    def _info(self):
        n, t, v = ctypes.c_uint64(), ctypes.c_uint64(), _i64()
        check(lib().mmh_sequences_info(self.handle, ctypes.byref(n), ctypes.byref(t),
                                       ctypes.byref(v)))
        return n.value, t.value, v.value

    def __len__(self) -> int:
        return self._info()[0]

    def is_empty(self) -> bool:
        return len(self) == 0

    def seq_len(self) -> int:
        return self._info()[1]

    def vocab_size(self) -> Optional[int]:
        v = self._info()[2]
        return None if v < 0 else v

    def window(self, index: int) -> Optional[np.ndarray]:
        """The seq_len + 1 ids of sequence `index`, or None."""
        if index < 0 or index >= len(self):
            return None
        out = np.empty(self.seq_len() + 1, np.uint32)
        check(lib().mmh_sequences_window(self.handle, index, out.ctypes.data_as(_u32p)))
        return out


class Batch:
    """One batch (batch.rs:107-122): inputs and targets are batch * seq ids."""

    __slots__ = ("inputs", "targets", "batch", "seq", "epoch", "index")

    def __init__(self, inputs, targets, batch, seq, epoch, index):
        self.inputs, self.targets = inputs, targets
        self.batch, self.seq, self.epoch, self.index = batch, seq, epoch, index

    def __eq__(self, other):
        return (isinstance(other, Batch)
                and (self.batch, self.seq, self.epoch, self.index)
                == (other.batch, other.seq, other.epoch, other.index)
                and np.array_equal(self.inputs, other.inputs)
                and np.array_equal(self.targets, other.targets))

    __hash__ = None


class Batcher(_Handle):
    """Batcher (batch.rs:144-240): batches of batch_size sequences, endlessly,
    each pass in the order Rng(seed).fork(epoch).shuffle(0..len)."""

    _destroy = "mmh_batcher_destroy"

    def __init__(self, data: Sequences, batch_size: int, seed: int):
        h = _h()
        check(lib().mmh_batcher_create(data.handle, batch_size, seed, ctypes.byref(h)))
        self.handle = h.value
        self.data = data

    def _info(self):
        v = [ctypes.c_uint64() for _ in range(5)]
        check(lib().mmh_batcher_info(self.handle, *[ctypes.byref(x) for x in v]))
        return [x.value for x in v]

    def batches_per_epoch(self) -> int:
        return self._info()[0]

    def epoch(self) -> int:
        return self._info()[1]

    def position(self) -> int:
        return self._info()[2]

    def seek(self, epoch: int, batches_done: int):
        check(lib().mmh_batcher_seek(self.handle, epoch, batches_done))

    def next_batch(self) -> Batch:
        _, _, _, b, t = self._info()
        x, y = np.empty(b * t, np.uint32), np.empty(b * t, np.uint32)
        e, i = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mmh_batcher_next(self.handle, x.ctypes.data_as(_u32p),
                                     y.ctypes.data_as(_u32p), ctypes.byref(e), ctypes.byref(i)))
        return Batch(x, y, b, t, e.value, i.value)


# ---- the model: midman-model/src/model.rs ------------------------------------------

# mmh_model_set_forward_path
PATH_AUTO = 0
PATH_PER_OP = 1

CONFIG_FIELDS = ("vocab_size", "d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff",
                 "max_seq_len", "rope_theta", "norm_eps", "tie_embeddings")

# presets.rs:52-83 at their default vocabularies
PRESETS = {
    "smoke": [256, 64, 2, 4, 4, 176, 128, 10000.0, 1e-5, 1],
    "tiny": [4096, 128, 4, 4, 4, 344, 256, 10000.0, 1e-5, 1],
    "small": [32000, 384, 6, 6, 6, 1024, 512, 10000.0, 1e-5, 1],
    "base": [32000, 768, 12, 12, 12, 2048, 1024, 10000.0, 1e-5, 1],
    "medium": [32000, 1024, 24, 16, 8, 2816, 2048, 10000.0, 1e-5, 1],
    "large": [32000, 2048, 20, 16, 8, 5632, 2048, 10000.0, 1e-5, 1],
}


def _config_array(config: Sequence[float]):
    if len(config) != 10:
        raise ArgumentError(ERR_ARGUMENT, "a config is 10 numbers (ffi.rs:27-32)")
    return (ctypes.c_double * 10)(*[float(v) for v in config])


class Model:
    """MidManModel on the device."""

    def __init__(self, ctx: Context, handle: int, config):
        self.ctx, self.handle, self.config = ctx, handle, list(config)
        self.vocab_size = int(config[0])

    @classmethod
    def new(cls, ctx: Context, config, seed: int, std: float = 0.02) -> "Model":
        """MidManModel::with_init_std(config, std, Rng::seed_from_u64(seed))."""
        h = _h()
        check(lib().mmh_model_create_seeded(ctx.handle, _config_array(config), seed, std,
                                            ctypes.byref(h)))
        return cls(ctx, h.value, config)

    @classmethod
    def from_weights(cls, ctx: Context, config, weights: np.ndarray) -> "Model":
        w = np.ascontiguousarray(weights, dtype=np.float32)
        h = _h()
        check(lib().mmh_model_create(ctx.handle, _config_array(config), _fp(w), w.size,
                                     ctypes.byref(h)))
        return cls(ctx, h.value, config)

    def lab_tokens(self, batch: int, seq: int):
        """Lab::new's task (lab.rs:194-203), continuing the model's Rng."""
        x = np.empty(batch * seq, np.int32)
        y = np.empty(batch * seq, np.int32)
        check(lib().mmh_model_lab_tokens(self.handle, batch, seq, _ip(x), _ip(y)))
        return x, y

    def num_parameters(self) -> int:
        n = _i64()
        check(lib().mmh_model_param_count(self.handle, ctypes.byref(n)))
        return n.value

    def weights(self) -> np.ndarray:
        n = self.num_parameters()
        out = np.empty(n, np.float32)
        check(lib().mmh_model_download_weights(self.handle, _fp(out), n))
        return out

    def forward(self, ids, batch: int, seq: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if ids.size != batch * seq:
            raise ArgumentError(ERR_ARGUMENT,
                                f"forward: {ids.size} ids do not fill {batch} sequences of {seq} tokens")
        out = np.empty((batch, seq, self.vocab_size), np.float32)
        check(lib().mmh_model_forward(self.handle, _ip(ids), batch, seq, _fp(out)))
        return out

    def loss(self, inputs, targets, batch: int, seq: int) -> float:
        x, y = self._pair(inputs, targets, batch, seq)
        loss = ctypes.c_float()
        check(lib().mmh_model_loss(self.handle, _ip(x), _ip(y), batch, seq, ctypes.byref(loss)))
        return loss.value

    def forward_loss(self, inputs, targets, batch: int, seq: int, want_logits: bool = True):
        x, y = self._pair(inputs, targets, batch, seq)
        logits = np.empty((batch, seq, self.vocab_size), np.float32) if want_logits else None
        loss = ctypes.c_float()
        check(lib().mmh_model_forward_loss(self.handle, _ip(x), _ip(y), batch, seq,
                                           _fp(logits) if want_logits else None,
                                           ctypes.byref(loss)))
        return loss.value, logits

    def _pair(self, inputs, targets, batch, seq):
        x = np.ascontiguousarray(inputs, dtype=np.int32)
        y = np.ascontiguousarray(targets, dtype=np.int32)
        if x.size != batch * seq or y.size != batch * seq:
            raise ArgumentError(ERR_ARGUMENT, "inputs/targets do not hold batch * seq ids")
        return x, y

    def stage(self, inputs, targets, batch: int, seq: int):
        """Validates and copies the ids into the model's device buffers."""
        x, y = self._pair(inputs, targets, batch, seq)
        check(lib().mmh_model_stage(self.handle, _ip(x), _ip(y), batch, seq))

    def run_staged(self, batch: int, seq: int):
        """Queues forward + loss on the staged ids; does not wait."""
        check(lib().mmh_model_run_staged(self.handle, batch, seq))

    def read_loss(self) -> float:
        loss = ctypes.c_float()
        check(lib().mmh_model_read_loss(self.handle, ctypes.byref(loss)))
        return loss.value

    def set_forward_path(self, path: int):
        """PATH_AUTO: loss-only forwards of models that fit run as one fused
        launch; PATH_PER_OP: always the per-operation kernels."""
        check(lib().mmh_model_set_forward_path(self.handle, path))

    def last_forward_fused(self) -> bool:
        """Whether the last queued forward (or the graph run_staged replays)
        was the fused launch."""
        v = ctypes.c_int32()
        check(lib().mmh_model_last_forward_fused(self.handle, ctypes.byref(v)))
        return bool(v.value)

    def fused_fallbacks(self) -> tuple:
        """(how many fused launches gave up and were redone on the
        per-operation kernels, the error word of the last one)."""
        n = ctypes.c_int64()
        e = ctypes.c_int32()
        check(lib().mmh_model_fused_fallbacks(self.handle, ctypes.byref(n), ctypes.byref(e)))
        return n.value, e.value

    def inject_fused_error(self, bits: int = 8):
        """Diagnostic: the next fused launch starts with `bits` in its error
        word, so its waits give up and the forward is redone."""
        check(lib().mmh_model_inject_fused_error(self.handle, bits))

    def fused_duration(self, batch: int, seq: int, reps: int = 200) -> tuple:
        """(median, minimum) duration in microseconds of the fused launch on
        the staged ids, from per-workgroup clock stamps over `reps` launches
        run back to back."""
        med = ctypes.c_float()
        mn = ctypes.c_float()
        check(lib().mmh_model_fused_duration(self.handle, batch, seq, reps, ctypes.byref(med),
                                             ctypes.byref(mn)))
        return med.value, mn.value

    def profile(self, batch: int, seq: int) -> dict:
        """One staged run with per-launch HIP events: {class: (ms, launches)}."""
        n = len(PROFILE_CLASSES)
        ms = (ctypes.c_float * n)()
        cnt = (ctypes.c_int32 * n)()
        check(lib().mmh_model_profile(self.handle, batch, seq, ms, cnt))
        return {name: (ms[i], cnt[i]) for i, name in enumerate(PROFILE_CLASSES)}

    # ---- checkpoints -------------------------------------------------------
    @classmethod
    def from_checkpoint(cls, ctx: Context, config, path: str) -> "Model":
        h = _h()
        check(lib().mmh_model_create_from_checkpoint(ctx.handle, _config_array(config),
                                                     path.encode(), ctypes.byref(h)))
        return cls(ctx, h.value, config)

    def save_checkpoint(self, path: str, metadata: Optional[dict] = None):
        """save_parameters (params.rs:36-80) straight from HBM."""
        items = sorted((metadata or {}).items())
        keys = (ctypes.c_char_p * max(1, len(items)))(*[k.encode() for k, _ in items])
        vals = (ctypes.c_char_p * max(1, len(items)))(*[v.encode() for _, v in items])
        check(lib().mmh_model_save_checkpoint(self.handle, path.encode(), keys, vals, len(items)))

    def load_checkpoint(self, path: str):
        """load_parameters (params.rs:82-210) straight into HBM; all or nothing."""
        check(lib().mmh_model_load_checkpoint(self.handle, path.encode()))

    # ---- training ---------------------------------------------------------
    def backward(self, inputs, targets, batch: int, seq: int) -> float:
        """loss.backward() (model.rs:174-183): returns the loss; the gradients
        stay on the device (grads(), grad_norm())."""
        x, y = self._pair(inputs, targets, batch, seq)
        loss = ctypes.c_float()
        check(lib().mmh_model_backward(self.handle, _ip(x), _ip(y), batch, seq,
                                       ctypes.byref(loss)))
        return loss.value

    def grads(self) -> np.ndarray:
        """Gradients of the last backward / step, in the reference parameter order."""
        n = self.num_parameters()
        out = np.empty(n, np.float32)
        check(lib().mmh_model_download_grads(self.handle, _fp(out), n))
        return out

    def grad_norm(self) -> float:
        out = ctypes.c_float()
        check(lib().mmh_model_grad_norm(self.handle, ctypes.byref(out)))
        return out.value

    def set_optimizer(self, beta1: float, beta2: float, eps: float, weight_decay: float,
                      clip_norm: float):
        """AdamW::new(beta1, beta2, eps, weight_decay) plus the clip limit."""
        check(lib().mmh_model_set_optimizer(self.handle, beta1, beta2, eps, weight_decay,
                                            clip_norm))

    def train_step(self, inputs, targets, batch: int, seq: int, lr: float):
        """Lab::step_once / Trainer::update: (loss, grad_norm before clipping).
        Raises Stopped, changing nothing, on a non-finite loss or norm."""
        x, y = self._pair(inputs, targets, batch, seq)
        loss, norm = ctypes.c_float(), ctypes.c_float()
        st = lib().mmh_model_train_step(self.handle, _ip(x), _ip(y), batch, seq, lr,
                                        ctypes.byref(loss), ctypes.byref(norm))
        if st == STOPPED:
            raise Stopped(st, last_error())
        check(st)
        return loss.value, norm.value

    def stage_train(self, inputs, targets, batch: int, seq: int):
        x, y = self._pair(inputs, targets, batch, seq)
        check(lib().mmh_model_stage_train(self.handle, _ip(x), _ip(y), batch, seq))

    def train_staged(self, batch: int, seq: int, lr: float):
        loss, norm = ctypes.c_float(), ctypes.c_float()
        st = lib().mmh_model_train_staged(self.handle, batch, seq, lr, ctypes.byref(loss),
                                          ctypes.byref(norm))
        if st == STOPPED:
            raise Stopped(st, last_error())
        check(st)
        return loss.value, norm.value

    def optimizer_steps(self) -> int:
        out = ctypes.c_uint64()
        check(lib().mmh_model_optimizer_steps(self.handle, ctypes.byref(out)))
        return out.value

    def train_next(self, batcher: "Batcher", lr: float):
        """Trainer::step (trainer.rs:162-183) on the batcher's next batch:
        (loss, grad_norm, epoch, index). A step that fails raises (Stopped for
        a non-finite loss or norm) and leaves the batcher where it was."""
        loss, norm = ctypes.c_float(), ctypes.c_float()
        e, i = ctypes.c_uint64(), ctypes.c_uint64()
        st = lib().mmh_model_train_next(self.handle, batcher.handle, lr, ctypes.byref(loss),
                                        ctypes.byref(norm), ctypes.byref(e), ctypes.byref(i))
        if st == STOPPED:
            raise Stopped(st, last_error())
        check(st)
        return loss.value, norm.value, e.value, i.value

    def evaluate(self, data: "Sequences", batch_size: int, max_batches: int):
        """Trainer::evaluate (trainer.rs:218-258): (loss, batches, tokens)."""
        loss, nb, nt = ctypes.c_float(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mmh_model_evaluate(self.handle, data.handle, batch_size, max_batches,
                                       ctypes.byref(loss), ctypes.byref(nb), ctypes.byref(nt)))
        return loss.value, nb.value, nt.value

    def broken_guards(self) -> int:
        """Guard words around the model's activation slots that a kernel
        overwrote (mmh_model_check_guards); 0 when every write stayed inside
        its output."""
        n = ctypes.c_uint64()
        check(lib().mmh_model_check_guards(self.handle, ctypes.byref(n)))
        return n.value

    def close(self):
        if self.handle:
            check(lib().mmh_model_destroy(self.handle))
            self.handle = 0


class Lab:
    """midman-api's Lab (lab.rs:150-310) on the device: the model from
    Rng(seed), the fixed memorization task from the same Rng, and training
    steps with WarmupCosine + global-norm clip + AdamW.

    hyper = (max_lr, min_lr, warmup_steps, total_steps, weight_decay,
    clip_norm, beta1, beta2) (lab.rs:29-46); eps is 1e-8 (lab.rs:192)."""

    def __init__(self, ctx: Context, config, hyper, seed: int, batch: int, seq: int):
        self.config, self.batch, self.seq = list(config), batch, seq
        h = [float(x) for x in hyper]
        self.max_lr, self.min_lr = h[0], h[1]
        self.warmup, self.total = int(h[2]), int(h[3])
        warmup_cosine_lr(self.max_lr, self.min_lr, self.warmup, self.total, 0)  # validates
        self.model = Model.new(ctx, config, seed)
        self.inputs, self.targets = self.model.lab_tokens(batch, seq)
        self.model.set_optimizer(h[6], h[7], 1e-8, h[4], h[5])
        self.model.stage_train(self.inputs, self.targets, batch, seq)
        self.steps = 0

    def step(self, steps: int):
        """Lab::step (lab.rs:241-258): (losses, grad_norms, lrs, stopped message or None)."""
        losses, norms, lrs = [], [], []
        stopped = None
        for _ in range(steps):
            lr = warmup_cosine_lr(self.max_lr, self.min_lr, self.warmup, self.total, self.steps)
            try:
                loss, norm = self.model.train_staged(self.batch, self.seq, lr)
            except Stopped as e:
                stopped = e.message
                break
            self.steps += 1
            losses.append(loss)
            norms.append(norm)
            lrs.append(lr)
        return losses, norms, lrs, stopped

    def eval(self):
        """Lab::eval (lab.rs:290-310): (loss, accuracy, predictions)."""
        logits = self.model.forward(self.inputs, self.batch, self.seq)
        loss = self.model.loss(self.inputs, self.targets, self.batch, self.seq)
        pred = logits.reshape(-1, logits.shape[-1]).argmax(-1).astype(np.int32)
        acc = float((pred == self.targets).mean())
        self.model.stage_train(self.inputs, self.targets, self.batch, self.seq)
        return loss, acc, pred

    def close(self):
        self.model.close()
