"""ctypes binding of oracle/liboracle.so, the CPU restatement the device is
checked against.  Test infrastructure: imported only by tests/, smoke() and
bench.py's cpu_baseline leg."""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

_lib = None


def _p(a):
    return a.ctypes.data if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, F, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        U32 = ctypes.c_uint32
        L.or_matmul.argtypes = [P, I, P, I, P, I64, I64, I64, I]
        L.or_matmul_f32acc.argtypes = [P, P, P, I64, I64, I64, I]
        L.or_eltwise.argtypes = [U32, F, F, P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64]
        L.or_reduce.argtypes = [P, I64, I64, I, I, P]
        L.or_reduce_all.argtypes = [P, I64, I]
        L.or_reduce_all.restype = F
        L.or_softmax_rows.argtypes = [P, I64, I64, P, I64, F, I, P]
        L.or_rms_norm.argtypes = [P, I64, I64, P, F, P]
        L.or_layer_norm.argtypes = [P, I64, I64, P, P, F, P]
        L.or_layer_norm_backward.argtypes = [P, I64, I64, P, P, P, F, P, P, P]
        L.or_softmax_backward.argtypes = [P, P, I64, I64, F, P]
        L.or_argmax_rows.argtypes = [P, I64, I64, P]
        L.or_select_rows.argtypes = [P, I64, I64, P, I64, P]
        L.or_pick_columns.argtypes = [P, I64, I64, P, P]
        L.or_scatter_add_columns.argtypes = [P, I64, I64, P, P, P]
        L.or_select_add_rows.argtypes = [P, I64, I64, P, I64, P, P]
        L.or_copy_strided4.argtypes = [P, ctypes.POINTER(I64), I64, ctypes.POINTER(I64), P]
        L.or_cast_to_bf16.argtypes = [P, I64, P]
        L.or_cast_from_bf16.argtypes = [P, I64, P]
        L.or_max_threads.restype = I
        L.or_bfp8_to_bf16.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
        L.or_bfp8_to_bf16.restype = ctypes.c_uint16
        L.or_bfp_round_trip.argtypes = [P, I64, I64, I, P, P]
        L.or_bfp_round_trip.restype = I
        L.or_gather.argtypes = [P, ctypes.POINTER(I64), I, P, ctypes.POINTER(I64), P]
        L.or_gather.restype = I
        _lib = L
    return _lib


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def matmul(a, b, ta=False, tb=False, threads=1):
    a, b = f32(a), f32(b)
    m = a.shape[1] if ta else a.shape[0]
    k = a.shape[0] if ta else a.shape[1]
    n = b.shape[0] if tb else b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().or_matmul(_p(a), int(ta), _p(b), int(tb), _p(c), m, n, k, threads)
    return c


def matmul_f32acc(a, b, threads=1):
    a, b = f32(a), f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().or_matmul_f32acc(_p(a), _p(b), _p(c), m, n, k, threads)
    return c


def _2d(x):
    x = f32(x)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    return x


def eltwise(kind, a, b=None, c=None, s1=0.0, s2=0.0):
    a = _2d(a)
    b = _2d(b) if b is not None else None
    c = _2d(c) if c is not None else None
    ops = [x for x in (a, b, c) if x is not None]
    R = max(x.shape[0] for x in ops)
    C = max(x.shape[1] for x in ops)
    out = np.empty((R, C), np.float32)
    dims = lambda x: (x.shape[0], x.shape[1]) if x is not None else (0, 0)
    lib().or_eltwise(kind, s1, s2, _p(a), *dims(a), _p(b), *dims(b), _p(c), *dims(c), _p(out), R, C)
    return out


def reduce(x, op, axis):
    x = _2d(x)
    R, C = x.shape
    out = np.empty((1, C) if axis == 0 else (R, 1), np.float32)
    lib().or_reduce(_p(x), R, C, op, axis, _p(out))
    return out


def reduce_all(x, op):
    x = f32(x).ravel()
    return np.float32(lib().or_reduce_all(_p(x), x.size, op))


def softmax_rows(x, mask=None, scale=1.0, log=False):
    x = _2d(x)
    R, C = x.shape
    m = np.ascontiguousarray(mask, dtype=np.uint32) if mask is not None else None
    out = np.empty_like(x)
    lib().or_softmax_rows(_p(x), R, C, _p(m), m.shape[0] if m is not None else 1, scale, int(log), _p(out))
    return out


def rms_norm(x, gamma=None, eps=1e-5):
    x = _2d(x)
    g = f32(gamma).ravel() if gamma is not None else None
    out = np.empty_like(x)
    lib().or_rms_norm(_p(x), x.shape[0], x.shape[1], _p(g), eps, _p(out))
    return out


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    x = _2d(x)
    g = f32(gamma).ravel() if gamma is not None else None
    b = f32(beta).ravel() if beta is not None else None
    out = np.empty_like(x)
    lib().or_layer_norm(_p(x), x.shape[0], x.shape[1], _p(g), _p(b), eps, _p(out))
    return out


def layer_norm_backward(x, gamma, dy, dres=None, eps=1e-5):
    x, dy = _2d(x), _2d(dy)
    R, C = x.shape
    g = f32(gamma).ravel() if gamma is not None else None
    r = _2d(dres) if dres is not None else None
    dx = np.empty_like(x)
    dg = np.empty((1, C), np.float32)
    db = np.empty((1, C), np.float32)
    lib().or_layer_norm_backward(_p(x), R, C, _p(g), _p(dy), _p(r), eps, _p(dx), _p(dg), _p(db))
    return dx, dg, db


def softmax_backward(p, dp, scale=1.0):
    p, dp = _2d(p), _2d(dp)
    out = np.empty_like(p)
    lib().or_softmax_backward(_p(p), _p(dp), p.shape[0], p.shape[1], scale, _p(out))
    return out


def argmax_rows(x):
    x = _2d(x)
    out = np.empty((x.shape[0], 1), np.int32)
    lib().or_argmax_rows(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def select_rows(table_bits, idx):
    t = np.ascontiguousarray(table_bits).view(np.uint32)
    t = t.reshape(t.shape[0], -1)
    i = np.ascontiguousarray(idx, dtype=np.int32).ravel()
    out = np.empty((i.size, t.shape[1]), np.uint32)
    st = lib().or_select_rows(_p(t), t.shape[0], t.shape[1], _p(i), i.size, _p(out))
    return out if st == 0 else None


def pick_columns(x_bits, idx):
    x = np.ascontiguousarray(x_bits).view(np.uint32)
    i = np.ascontiguousarray(idx, dtype=np.int32).ravel()
    out = np.empty((x.shape[0], 1), np.uint32)
    st = lib().or_pick_columns(_p(x), x.shape[0], x.shape[1], _p(i), _p(out))
    return out if st == 0 else None


def scatter_add_columns(x, idx, v):
    x = _2d(x)
    i = np.ascontiguousarray(idx, dtype=np.int32).ravel()
    vv = f32(v).ravel()
    out = np.empty_like(x)
    st = lib().or_scatter_add_columns(_p(x), x.shape[0], x.shape[1], _p(i), _p(vv), _p(out))
    return out if st == 0 else None


def select_add_rows(t, idx, value):
    t = _2d(t)
    i = np.ascontiguousarray(idx, dtype=np.int32).ravel()
    v = _2d(value)
    out = np.empty_like(t)
    st = lib().or_select_add_rows(_p(t), t.shape[0], t.shape[1], _p(i), i.size, _p(v), _p(out))
    return out if st == 0 else None


def copy_strided4(src_bits, dims, offset, strides):
    s = np.ascontiguousarray(src_bits).view(np.uint32).ravel()
    n = int(np.prod(dims))
    out = np.empty(n, np.uint32)
    d = (ctypes.c_int64 * 4)(*dims)
    st = (ctypes.c_int64 * 4)(*strides)
    lib().or_copy_strided4(_p(s), d, offset, st, _p(out))
    return out.reshape(dims[0] * dims[1] * dims[2], dims[3])


def to_bf16(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_cast_to_bf16(_p(x), x.size, _p(out))
    return out


def from_bf16(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_cast_from_bf16(_p(h), h.size, _p(out))
    return out


def max_threads():
    return lib().or_max_threads()


def bfp8_to_bf16(datum: int, exp: int) -> int:
    """The unpacker's decode of one BFP8 datum under its exponent byte."""
    return int(lib().or_bfp8_to_bf16(datum, exp))


def bfp_round_trip(x, width: int = 8):
    """(values held in BFP8 / BFP4 / BFP2 and read back [rows, cols], block
    exponents [rows, ceil(cols / 16)] uint8, 1 if a value was not finite)."""
    x = f32(np.atleast_2d(x))
    rows, cols = x.shape
    out = np.empty_like(x)
    exps = np.empty((rows, (cols + 15) // 16), np.uint8)
    bad = lib().or_bfp_round_trip(_p(x), rows, cols, width, _p(out), _p(exps))
    return out, exps, bad


def gather(x, dim: int, idx):
    """Burn's gather along `dim` (rank <= 4), raw 32-bit payloads: (out with
    idx's shape, 1 if an index was out of range)."""
    x = np.ascontiguousarray(x)
    assert x.dtype.itemsize == 4
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    pad = 4 - x.ndim
    dims = (ctypes.c_int64 * 4)(*([1] * pad + list(x.shape)))
    idims = (ctypes.c_int64 * 4)(*([1] * pad + list(idx.shape)))
    out = np.empty(idx.shape, np.uint32)
    bad = lib().or_gather(_p(x.view(np.uint32)), dims, dim + pad, _p(idx), idims, _p(out))
    return out.view(x.dtype), bad
