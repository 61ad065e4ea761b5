"""Python host binding of the MI355X engine (libmiburn.so, include/miburn.h).

`Engine` mirrors the reference's device-engine trait, method for method: the
`Engine` of crates/burn-tt/src/server.rs:42-788 (upload / download / free,
matmul_dram, matmul_dram_batched, eltwise_op_as, reduce, softmax_rows,
rms_norm, argmax_row, select_rows, pick_columns, select_add_rows,
random_dram, cast_float).  Buffers are row-major `[rows, cols]` matrices named
by integer ids, as the trait's `BufferId`.  Errors raise `MiError` carrying the
C status; asynchronous failures (an index out of range found by a kernel)
surface at the next `sync()` or download, as the reference defers them to its
next wait (server.rs:2951-2991).

The shared library is the only implementation: importing this module on a
machine where libmiburn.so is missing raises, and there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import weakref
import os
from typing import Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmiburn.so")

F32, I32, BOOL, BF16, BFP8 = 0, 1, 2, 3, 5
# A result form of mi_rms_norm / mi_silu_mul_halves: the F32 result as its
# BF16 parts, [rows, 2 cols] (heads, then remainders), read by linear_parts.
BF16_PARTS = 4
TILES_BF16 = 6   # an operand in the matrix cores' operand order (mi_tile)
TILES_PARTS = 7
_NP = {F32: np.float32, I32: np.int32, BOOL: np.uint32, BF16: np.uint16, BFP8: np.float32}

AXIS_ROWS, AXIS_COLS = 0, 1
MATMUL_FAST, MATMUL_ACCURATE = 0, 1
R_SUM, R_MAX, R_MEAN, R_MIN = 0, 1, 2, 3
DRAW_UNIT, DRAW_UNIFORM, DRAW_NORMAL, DRAW_BERNOULLI, DRAW_INT_RANGE = 0, 1, 2, 3, 4

# Element-wise op ids (the reference's numbering, crates/tt-kernels/src/kind.rs,
# crates/tt-kernels/src/sfpu/ops.rs:24-250).
K = dict(
    ADD=1, SUB=2, MUL=3, MUL_SCALAR=4, RELU=5, RELU_BACKWARD=6, ADD_ROW=7, ADD_SCALAR=11,
    RECIP=0x100, DIV=0x101, DIV_SCALAR=0x102, EXP=0x103, LOG=0x104,
    BOOL_NOT=0x105, BOOL_AND=0x106, BOOL_OR=0x107, BOOL_XOR=0x108,
    NEG=0x109, ABS=0x10A, SIGN=0x10B, CLAMP=0x10C, CLAMP_MIN=0x10D, CLAMP_MAX=0x10E,
    LEAKY_RELU=0x10F, HARD_SIGMOID=0x110,
    EQ=0x111, NE=0x112, GT=0x113, GE=0x114, LT=0x115, LE=0x116,
    EQ_S=0x117, NE_S=0x118, GT_S=0x119, GE_S=0x11A, LT_S=0x11B, LE_S=0x11C,
    IS_NAN=0x11D, IS_INF=0x11E, MASK_FILL=0x11F, MASK_WHERE=0x120, FILL=0x122,
    SQRT=0x123, RSQRT=0x124, LOG1P=0x125, POW=0x126, POW_S=0x127, I32_TO_F32=0x129,
    EXPM1=0x12A, SIGMOID=0x12B, SIGMOID_BACKWARD=0x12C, TANH=0x12D, ERF=0x12E,
    GELU=0x12F, GELU_BACKWARD=0x130, SIN=0x138, COS=0x139, BOOL_TO_F32=0x13F,
    ADD_RELU=0x1F0, SILU=0x1F1, SILU_MUL=0x1F2, SUB_EXP=0x1F3, MUL_ADD=0x1F4,
    SCALE_MASK_FILL=0x1F5, RSQRT_ABS_ADD=0x200,
)

STATUS = {0: "OK", -1: "ARG", -2: "ID", -3: "HIP", -4: "OOM", -5: "DOMAIN", -6: "UNSUPPORTED",
          -7: "STICKY"}


class MiError(RuntimeError):
    """A failed engine call: `status` is the C code, `kind` its name."""

    def __init__(self, status: int, msg: str):
        self.status = status
        self.kind = STATUS.get(status, str(status))
        super().__init__(f"{self.kind}: {msg}")


class Report(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "ops", "uploads", "downloads", "bytes_up", "bytes_down", "live_buffers", "device_bytes",
        "cached_bytes")]


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run `make -C metalium-rs_amd` (or "
                          "__graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    U64 = ctypes.c_uint64
    Ip = ctypes.POINTER(U64)
    c_int, c_float, c_u32 = ctypes.c_int, ctypes.c_float, ctypes.c_uint32
    sigs = {
        "mi_ctx_create": [c_int, ctypes.POINTER(P)],
        "mi_ctx_destroy": [P],
        "mi_sync": [P],
        "mi_stream": [P, ctypes.POINTER(P)],
        "mi_upload": [P, P, I64, I64, Ip],
        "mi_upload_bits": [P, P, I64, I64, c_int, Ip],
        "mi_upload_bf16": [P, P, I64, I64, Ip],
        "mi_download": [P, U64, P, I64],
        "mi_download_bits": [P, U64, P, I64],
        "mi_download_bf16": [P, U64, P, I64],
        "mi_free": [P, U64],
        "mi_metadata": [P, U64, ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(c_int)],
        "mi_fill": [P, I64, I64, c_int, c_u32, Ip],
        "mi_empty": [P, I64, I64, c_int, Ip],
        "mi_reshape": [P, U64, I64, I64],
        "mi_matmul": [P, U64, c_int, U64, c_int, c_int, Ip],
        "mi_matmul_batched": [P, U64, c_int, U64, c_int, I64, I64, I64, I64, c_int, Ip],
        "mi_linear": [P, U64, U64, c_int, U64, U64, c_int, Ip],
        "mi_linear_parts": [P, U64, U64, c_int, U64, U64, c_int, Ip],
        "mi_linear_swiglu_parts": [P, U64, U64, Ip],
        "mi_linear_swiglu": [P, U64, U64, c_int, Ip],
        "mi_linear_qkv_rope_cache": [P, U64, c_int, U64, U64, U64, I64, I64, I64, I64, U64, U64, c_int, Ip],
        "mi_matmul_slices": [P, U64, c_int, U64, c_int, Ip, ctypes.POINTER(I64)],
        "mi_matmul_items": [P, U64, c_int, ctypes.POINTER(I64), U64, c_int, ctypes.POINTER(I64), I64, I64, I64, I64,
                            I64, U64, ctypes.POINTER(I64)],
        "mi_matmul_blocks": [P, U64, c_int, U64, c_int, I64, I64, I64, I64, I64, I64, I64, I64, c_int, Ip],
        "mi_copy_into4": [P, U64, I64, ctypes.POINTER(I64), U64, I64, ctypes.POINTER(I64), ctypes.POINTER(I64)],
        "mi_rope": [P, U64, U64, U64, I64, I64, I64, Ip],
        "mi_attention_rows": [P, U64, U64, U64, I64, I64, I64, I64, I64, c_float, Ip],
        "mi_attention_rows_as": [P, U64, U64, U64, I64, I64, I64, I64, I64, c_float, c_int, Ip],
        "mi_attention_rows_into": [P, U64, U64, U64, I64, I64, I64, I64, I64, c_float, U64],
        "mi_reduce_then": [P, U64, c_int, c_int, c_u32, c_float, Ip],
        "mi_add_rms_norm": [P, U64, U64, U64, c_float, Ip, Ip],
        "mi_matmul_pairs": [P, U64, U64, I64, ctypes.POINTER(I64), ctypes.POINTER(c_int), ctypes.POINTER(I64),
                            ctypes.POINTER(c_int), I64, I64, I64, c_int, Ip],
        "mi_norm_matvec": [P, U64, U64, c_float, U64, U64, c_int, Ip],
        "mi_norm_matvec_argmax": [P, U64, U64, c_float, U64, Ip, Ip],
        "mi_norm_qkv_attention": [P, U64, U64, c_float, U64, U64, U64, I64, I64, U64, I64, I64, U64, U64, c_float,
                                  Ip],
        "mi_norm_qkv_attention_o": [P, U64, U64, c_float, U64, U64, U64, I64, I64, U64, I64, I64, U64, U64,
                                    c_float, U64, Ip],
        "mi_norm_qkv_rope": [P, U64, U64, c_float, U64, U64, U64, I64, I64, I64, U64, U64, Ip],
        "mi_norm_qkv_rope_at": [P, U64, U64, c_float, U64, U64, U64, I64, I64, U64, U64, U64, Ip],
        "mi_attention_rows_at": [P, U64, U64, U64, I64, I64, I64, I64, U64, I64, I64, c_float, Ip],
        "mi_qkv_rope_cache": [P, U64, U64, U64, I64, I64, I64, I64, U64, U64, c_int, Ip],
        "mi_silu_mul_halves": [P, U64, c_int, Ip],
        "mi_eltwise": [P, c_u32, c_float, c_float, U64, U64, U64, c_int, Ip],
        "mi_reduce": [P, U64, c_int, c_int, Ip],
        "mi_reduce_all": [P, U64, c_int, Ip],
        "mi_softmax_rows": [P, U64, U64, c_float, c_int, c_int, Ip],
        "mi_rms_norm": [P, U64, U64, c_float, c_int, Ip],
        "mi_layer_norm": [P, U64, U64, U64, c_float, Ip],
        "mi_layer_norm_backward": [P, U64, U64, U64, U64, c_float, Ip, Ip, Ip],
        "mi_softmax_backward": [P, U64, U64, c_float, Ip],
        "mi_log_softmax_ce": [P, U64, U64, c_float, Ip, Ip],
        "mi_sgd_update": [P, I64, ctypes.POINTER(U64), ctypes.POINTER(U64), c_float],
        "mi_argmax_rows": [P, U64, Ip],
        "mi_set_matmul_mode": [P, c_int],
        "mi_trace_begin": [P],
        "mi_trace_end": [P, ctypes.POINTER(U64)],
        "mi_trace_run": [P, U64, I64, ctypes.POINTER(U64), ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(I64), I64,
                         ctypes.POINTER(U64), ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(I64)],
        "mi_trace_release": [P, U64],
        "mi_copy_into": [P, U64, U64],
        "mi_cast_bfp": [P, U64, c_int, ctypes.POINTER(U64)],
        "mi_tile": [P, U64, c_int, ctypes.POINTER(U64)],
        "mi_decode_advance": [P, U64, U64, U64, U64],
        "mi_gather": [P, U64, ctypes.POINTER(I64), c_int, U64, ctypes.POINTER(I64), Ip],
        "mi_linear_add_rms_norm": [P, U64, U64, c_int, U64, U64, U64, c_float, c_int, Ip, Ip],
        "mi_get_matmul_mode": [P, ctypes.POINTER(c_int)],
        "mi_select_rows": [P, U64, U64, Ip],
        "mi_select_rows_as": [P, U64, U64, c_int, Ip],
        "mi_pick_columns": [P, U64, U64, Ip],
        "mi_scatter_add_columns": [P, U64, U64, U64, Ip],
        "mi_select_add_rows": [P, U64, U64, U64, Ip],
        "mi_copy_strided": [P, U64, I64, I64, I64, I64, I64, Ip],
        "mi_copy_strided4": [P, U64, ctypes.POINTER(I64), I64, ctypes.POINTER(I64), Ip],
        "mi_assign_block": [P, U64, U64, I64, I64],
        "mi_cast": [P, U64, c_int, Ip],
        "mi_random": [P, I64, I64, c_int, c_float, c_float, U64, Ip],
        "mi_event_record": [P, c_int],
        "mi_event_elapsed_ms": [P, c_int, c_int, ctypes.POINTER(c_float)],
        "mi_get_report": [P, ctypes.POINTER(Report)],
    }
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = c_int
    lib.mi_last_error.argtypes = [P]
    lib.mi_last_error.restype = ctypes.c_char_p
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


class Engine:
    """One device context: the reference's `KmdEngine` (server.rs:4071) for an MI355X."""

    def __init__(self, device: int = 0):
        self._children = weakref.WeakSet()  # model harnesses to close before the context
        self._lib = lib()
        ctx = ctypes.c_void_p()
        st = self._lib.mi_ctx_create(device, ctypes.byref(ctx))
        if st != 0:
            raise MiError(st, self._lib.mi_last_error(None).decode())
        self.ctx = ctx

    # -- plumbing --------------------------------------------------------
    def close(self) -> None:
        """Destroy the context; the model harnesses built on it are closed
        first (their buffers belong to the context)."""
        if self.ctx:
            for child in list(self._children):
                child.close()
            self._lib.mi_ctx_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int) -> None:
        if st != 0:
            raise MiError(st, self._lib.mi_last_error(self.ctx).decode())

    def _out(self, fn, *args) -> int:
        out = ctypes.c_uint64()
        self._check(fn(self.ctx, *args, ctypes.byref(out)))
        return out.value

    # -- storage (server.rs:91-174) ----------------------------------------
    def upload(self, x: np.ndarray) -> int:
        x = np.ascontiguousarray(x, dtype=np.float32)
        r, c = _dims(x)
        return self._out(self._lib.mi_upload, x.ctypes.data, r, c)

    def upload_bits(self, x: np.ndarray, elem: int) -> int:
        x = np.ascontiguousarray(x)
        if x.dtype.itemsize != 4:
            raise ValueError("upload_bits takes 32-bit datums")
        r, c = _dims(x)
        return self._out(self._lib.mi_upload_bits, x.ctypes.data, r, c, elem)

    def upload_i32(self, x: np.ndarray) -> int:
        return self.upload_bits(np.ascontiguousarray(x, dtype=np.int32), I32)

    def upload_bool(self, x: np.ndarray) -> int:
        return self.upload_bits(np.ascontiguousarray(x, dtype=np.uint32), BOOL)

    def upload_bf16(self, bits: np.ndarray) -> int:
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        r, c = _dims(bits)
        return self._out(self._lib.mi_upload_bf16, bits.ctypes.data, r, c)

    def metadata(self, id_: int) -> Tuple[int, int, int]:
        r, c, e = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        self._check(self._lib.mi_metadata(self.ctx, id_, ctypes.byref(r), ctypes.byref(c), ctypes.byref(e)))
        return r.value, c.value, e.value

    def download(self, id_: int) -> np.ndarray:
        r, c, e = self.metadata(id_)
        out = np.empty((r, c), dtype=_NP[e])
        if e in (F32, BFP8):  # a BFP8 buffer reads back decoded (F32)
            self._check(self._lib.mi_download(self.ctx, id_, out.ctypes.data, out.size))
        elif e == BF16:
            self._check(self._lib.mi_download_bf16(self.ctx, id_, out.ctypes.data, out.size))
        else:
            self._check(self._lib.mi_download_bits(self.ctx, id_, out.ctypes.data, out.size))
        return out

    def free(self, id_: int) -> None:
        self._check(self._lib.mi_free(self.ctx, id_))

    def reshape(self, id_: int, rows: int, cols: int) -> None:
        self._check(self._lib.mi_reshape(self.ctx, id_, rows, cols))

    def fill(self, rows: int, cols: int, elem: int, bits: int) -> int:
        return self._out(self._lib.mi_fill, rows, cols, elem, bits)

    def empty(self, rows: int, cols: int, elem: int = F32) -> int:
        """A buffer whose contents are unspecified until written."""
        return self._out(self._lib.mi_empty, rows, cols, elem)

    def sync(self) -> None:
        self._check(self._lib.mi_sync(self.ctx))

    def stream(self) -> int:
        s = ctypes.c_void_p()
        self._check(self._lib.mi_stream(self.ctx, ctypes.byref(s)))
        return s.value or 0

    # -- ops ---------------------------------------------------------------
    def matmul_dram(self, a: int, a_t: bool, b: int, b_t: bool, out_elem: int = F32) -> int:
        return self._out(self._lib.mi_matmul, a, int(a_t), b, int(b_t), out_elem)

    def matmul_slices(self, a: int, a_t: bool, b: int, b_t: bool):
        """(id, S): the product as S stacked split-K slices [S * m, n]."""
        out, sl = ctypes.c_uint64(), ctypes.c_int64()
        self._check(self._lib.mi_matmul_slices(self.ctx, a, int(a_t), b, int(b_t), ctypes.byref(out),
                                               ctypes.byref(sl)))
        return out.value, sl.value

    def linear(self, x: int, w: int, w_t: bool, bias: int = 0, residual: int = 0, out_elem: int = F32) -> int:
        """residual + (x @ op(w) + bias) in one product; 0 omits a term."""
        return self._out(self._lib.mi_linear, x, w, int(w_t), bias, residual, out_elem)

    def linear_add_rms_norm(self, x: int, w: int, w_t: bool, bias: int = 0, residual: int = 0, gamma: int = 0,
                            eps: float = 1e-5, norm_elem: int = F32):
        """mi_linear then mi_rms_norm of its result in one call: (y, y_norm)."""
        y, yn = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self._lib.mi_linear_add_rms_norm(self.ctx, x, w, int(w_t), bias, residual, gamma, eps, norm_elem,
                                                     ctypes.byref(y), ctypes.byref(yn)))
        return y.value, yn.value

    def linear_parts(self, x_parts: int, w: int, w_t: bool, bias: int = 0, residual: int = 0,
                     out_elem: int = F32) -> int:
        """linear() of an F32 operand given as its BF16 parts [m, 2k] (BF16_PARTS)."""
        return self._out(self._lib.mi_linear_parts, x_parts, w, int(w_t), bias, residual, out_elem)

    def linear_swiglu_parts(self, x_parts: int, w_pairs: int) -> int:
        """silu(x gate^T) * (x up^T) as BF16 parts, from x's parts and a gate|up
        weight whose rows interleave in 32-row groups."""
        return self._out(self._lib.mi_linear_swiglu_parts, x_parts, w_pairs)

    def linear_swiglu(self, x: int, w_pairs: int, out_elem: int = BF16) -> int:
        """silu(x gate^T) * (x up^T) from BF16 activations and the interleaved
        gate|up weight, F32 or rounded to BF16."""
        return self._out(self._lib.mi_linear_swiglu, x, w_pairs, out_elem)

    def linear_qkv_rope_cache(self, x: int, x_parts: bool, w_qkv: int, cos: int, sin: int, seq: int, heads: int,
                              kv_heads: int, pos0: int, k_cache: int, v_cache: int, grouped: bool = False) -> int:
        """The q|k|v product (BF16 activations, or an F32 operand's parts) and
        qkv_rope_cache in one launch; returns q."""
        return self._out(self._lib.mi_linear_qkv_rope_cache, x, int(x_parts), w_qkv, cos, sin, seq, heads, kv_heads,
                         pos0, k_cache, v_cache, int(grouped))

    def log_softmax_ce(self, logits: int, targets: int, grad_scale: float):
        """(picked, dlogits): logp at each row's target and the cross-entropy
        gradient exp(logp) * grad_scale - grad_scale * onehot, in one pass."""
        a, b = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self._lib.mi_log_softmax_ce(self.ctx, logits, targets, grad_scale, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def matmul_items(self, a: int, a_t: bool, a_at, b: int, b_t: bool, b_at, groups: int, per_group: int, m: int,
                     k: int, n: int, out: int, out_at) -> None:
        """Grouped strided products written in place into `out`; each `*_at`
        is (offset, group_stride, item_stride) in elements."""
        A3 = ctypes.c_int64 * 3
        self._check(self._lib.mi_matmul_items(self.ctx, a, int(a_t), A3(*a_at), b, int(b_t), A3(*b_at), groups,
                                              per_group, m, k, n, out, A3(*out_at)))

    def matmul_dram_bf16(self, a: int, a_t: bool, b: int, b_t: bool) -> int:
        return self.matmul_dram(a, a_t, b, b_t, BF16)

    def matmul_dram_batched(self, a: int, a_t: bool, b: int, b_t: bool, batch: int, m: int, k: int, n: int,
                            out_elem: int = F32) -> int:
        return self._out(self._lib.mi_matmul_batched, a, int(a_t), b, int(b_t), batch, m, k, n, out_elem)

    def matmul_blocks(self, a: int, a_t: bool, b: int, b_t: bool, batch: int, m: int, k: int, n: int,
                      a_offset: int, a_stride: int, b_offset: int, b_stride: int, out_elem: int = F32) -> int:
        return self._out(self._lib.mi_matmul_blocks, a, int(a_t), b, int(b_t), batch, m, k, n, a_offset, a_stride,
                         b_offset, b_stride, out_elem)

    def copy_into4(self, dst: int, dst_offset: int, dst_strides, src: int, src_offset: int, src_strides,
                   dims) -> None:
        A4 = ctypes.c_int64 * 4
        self._check(self._lib.mi_copy_into4(self.ctx, dst, dst_offset, A4(*dst_strides), src, src_offset,
                                            A4(*src_strides), A4(*dims)))

    def rope(self, x: int, cos: int, sin: int, heads: int, seq: int, pos0: int) -> int:
        return self._out(self._lib.mi_rope, x, cos, sin, heads, seq, pos0)

    def norm_matvec(self, x: int, gamma: int, eps: float, w: int, residual: int = 0, silu_mul: bool = False) -> int:
        """Fused decode projection: residual + rmsnorm(x) w^T, or silu(g) * u."""
        return self._out(self._lib.mi_norm_matvec, x, gamma, eps, w, residual, int(silu_mul))

    def norm_matvec_argmax(self, x: int, gamma: int, eps: float, w: int) -> Tuple[int, int]:
        """(logits, ids): rmsnorm(x) w^T and the argmax of each row, in one call."""
        lg, ids = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self._lib.mi_norm_matvec_argmax(self.ctx, x, gamma, eps, w, ctypes.byref(lg), ctypes.byref(ids)))
        return lg.value, ids.value

    def silu_mul_halves(self, gate_up: int, out_elem: int = F32) -> int:
        """silu(gate) * up over the two column halves of a fused gate|up product (F32, or rounded to BF16)."""
        return self._out(self._lib.mi_silu_mul_halves, gate_up, out_elem)

    def qkv_rope_cache(self, qkv: int, cos: int, sin: int, seq: int, heads: int, kv_heads: int, pos0: int,
                       k_cache: int, v_cache: int, grouped: bool = False) -> int:
        """Prefill q|k|v tail: RoPE on q and k, k and v into the caches; returns q."""
        return self._out(self._lib.mi_qkv_rope_cache, qkv, cos, sin, seq, heads, kv_heads, pos0, k_cache, v_cache,
                         int(grouped))

    def norm_qkv_rope(self, x: int, gamma: int, eps: float, w_qkv: int, cos: int, sin: int, heads: int,
                      kv_heads: int, pos: int, k_cache: int, v_cache: int) -> int:
        """Fused decode q|k|v projection with RoPE and the KV-cache write; returns q."""
        return self._out(self._lib.mi_norm_qkv_rope, x, gamma, eps, w_qkv, cos, sin, heads, kv_heads, pos,
                         k_cache, v_cache)

    def attention_rows(self, q: int, k_cache: int, v_cache: int, batch: int, t: int, heads: int, kv_heads: int,
                       pos0: int, scale: float) -> int:
        """Engine::attention_rows (server.rs:255-265): causal GQA of `t` new
        positions against the first pos0 + t rows of each cache item."""
        return self._out(self._lib.mi_attention_rows, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, scale)

    def attention_rows_as(self, q: int, k_cache: int, v_cache: int, batch: int, t: int, heads: int, kv_heads: int,
                          pos0: int, scale: float, out_form: int) -> int:
        """attention_rows with its result in out_form (F32, BF16, TILES_BF16, TILES_PARTS)."""
        return self._out(self._lib.mi_attention_rows_as, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, scale,
                         out_form)

    def attention_rows_at(self, q: int, k_cache: int, v_cache: int, batch: int, t: int, heads: int, kv_heads: int,
                          pos: int, pos0: int, span: int, scale: float) -> int:
        """attention_rows with the key chunks planned for `span` positions and
        pos0 read on the device from the [1, 1] I32 buffer `pos` (if nonzero)."""
        return self._out(self._lib.mi_attention_rows_at, q, k_cache, v_cache, batch, t, heads, kv_heads, pos, pos0,
                         span, scale)

    def norm_qkv_attention(self, x: int, gamma: int, eps: float, w_qkv: int, cos: int, sin: int, heads: int,
                           kv_heads: int, pos: int, pos0: int, span: int, k_cache: int, v_cache: int,
                           scale: float) -> int:
        """norm_qkv_rope(_at) then attention_rows_at (t = 1) in one call: the
        attention rows of one new position per sequence (llama.rs:380-470)."""
        return self._out(self._lib.mi_norm_qkv_attention, x, gamma, eps, w_qkv, cos, sin, heads, kv_heads, pos,
                         pos0, span, k_cache, v_cache, scale)

    def norm_qkv_attention_o(self, x: int, gamma: int, eps: float, w_qkv: int, cos: int, sin: int, heads: int,
                             kv_heads: int, pos: int, pos0: int, span: int, k_cache: int, v_cache: int,
                             scale: float, w_o: int) -> int:
        """x + norm_qkv_attention(...) w_o^T: the attention block through its
        output projection and residual (llama.rs:380-470), bit for bit the
        two calls."""
        return self._out(self._lib.mi_norm_qkv_attention_o, x, gamma, eps, w_qkv, cos, sin, heads, kv_heads, pos,
                         pos0, span, k_cache, v_cache, scale, w_o)

    def norm_qkv_rope_at(self, x: int, gamma: int, eps: float, w_qkv: int, cos: int, sin: int, heads: int,
                         kv_heads: int, pos: int, k_cache: int, v_cache: int) -> int:
        """norm_qkv_rope at the position held on the device in `pos` ([1, 1] I32)."""
        return self._out(self._lib.mi_norm_qkv_rope_at, x, gamma, eps, w_qkv, cos, sin, heads, kv_heads, pos,
                         k_cache, v_cache)

    def attention_rows_into(self, q: int, k_cache: int, v_cache: int, batch: int, t: int, heads: int,
                            kv_heads: int, pos0: int, scale: float, out: int) -> None:
        """attention_rows into the existing F32 buffer `out`, allocating
        nothing (the partials in a fixed per-GPU device array)."""
        self._check(self._lib.mi_attention_rows_into(self.ctx, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0,
                                                     scale, out))

    def eltwise_op_as(self, kind, a: int, b: int = 0, c: int = 0, scalar: float = 0.0, scalar2: float = 0.0,
                      out_elem: int = F32) -> int:
        k = K[kind] if isinstance(kind, str) else int(kind)
        return self._out(self._lib.mi_eltwise, k, scalar, scalar2, a, b, c, out_elem)

    def reduce(self, a: int, op: int, axis: int) -> int:
        return self._out(self._lib.mi_reduce, a, op, axis)

    def reduce_then(self, a: int, op: int, axis: int, then_kind=0, then_scalar: float = 0.0) -> int:
        """Engine::reduce with `then`: an exact unary kind on the result."""
        k = K[then_kind] if isinstance(then_kind, str) else int(then_kind)
        return self._out(self._lib.mi_reduce_then, a, op, axis, k, then_scalar)

    def add_rms_norm(self, a: int, b: int, gamma: int = 0, eps: float = 1e-5):
        """Engine::add_rms_norm: (a + b, rms_norm(a + b) * gamma)."""
        s, nrm = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self._lib.mi_add_rms_norm(self.ctx, a, b, gamma, eps, ctypes.byref(s), ctypes.byref(nrm)))
        return s.value, nrm.value

    def matmul_pairs(self, a: int, b: int, a_blocks, b_blocks, m: int, k: int, n: int, out_elem: int = F32) -> int:
        """Engine::matmul_dram_batched over (Block, Block) pairs: each block
        ((row, col), transposed)."""
        items = len(a_blocks)
        aat = (ctypes.c_int64 * (2 * items))(*[v for (rc, _) in a_blocks for v in rc])
        bat = (ctypes.c_int64 * (2 * items))(*[v for (rc, _) in b_blocks for v in rc])
        at_ = (ctypes.c_int * items)(*[int(t) for (_, t) in a_blocks])
        bt_ = (ctypes.c_int * items)(*[int(t) for (_, t) in b_blocks])
        return self._out(self._lib.mi_matmul_pairs, a, b, items, aat, at_, bat, bt_, m, k, n, out_elem)

    def reduce_all(self, a: int, op: int) -> int:
        return self._out(self._lib.mi_reduce_all, a, op)

    def softmax_rows(self, x: int, mask: int = 0, scale: float = 1.0, log: bool = False,
                     out_elem: int = F32) -> int:
        return self._out(self._lib.mi_softmax_rows, x, mask, scale, int(log), out_elem)

    def rms_norm(self, a: int, gamma: int = 0, eps: float = 1e-5, out_elem: int = F32) -> int:
        return self._out(self._lib.mi_rms_norm, a, gamma, eps, out_elem)

    def layer_norm(self, a: int, gamma: int = 0, beta: int = 0, eps: float = 1e-5) -> int:
        return self._out(self._lib.mi_layer_norm, a, gamma, beta, eps)

    def layer_norm_backward(self, x: int, gamma: int, dy: int, residual_grad: int = 0, eps: float = 1e-5):
        """LayerNorm's gradient, fused: (dx, dgamma, dbeta) ids."""
        outs = [ctypes.c_uint64() for _ in range(3)]
        self._check(self._lib.mi_layer_norm_backward(self.ctx, x, gamma, dy, residual_grad, eps,
                                                     *[ctypes.byref(o) for o in outs]))
        return tuple(o.value for o in outs)

    def sgd_update(self, params, grads, lr: float) -> None:
        """In place: params[i] <- params[i] - grads[i] * lr."""
        n = len(params)
        pa = (ctypes.c_uint64 * max(n, 1))(*params)
        ga = (ctypes.c_uint64 * max(n, 1))(*grads)
        self._check(self._lib.mi_sgd_update(self.ctx, n, pa, ga, lr))

    def softmax_backward(self, p: int, dp: int, scale: float = 1.0) -> int:
        return self._out(self._lib.mi_softmax_backward, p, dp, scale)

    # -- traces (server.rs:591-660) ---------------------------------------
    def begin_trace(self) -> None:
        self._check(self._lib.mi_trace_begin(self.ctx))

    def end_trace(self) -> int:
        t = ctypes.c_uint64()
        self._check(self._lib.mi_trace_end(self.ctx, ctypes.byref(t)))
        return t.value

    def run_trace(self, trace: int, inputs=None, outputs=(), out_arrays=None):
        """Overwrite each input id with its array's bytes, replay, and return
        the outputs' contents (arrays of each buffer's kind and shape, or the
        caller's `out_arrays`).  Each array's byte length goes with it (the
        library refuses an input whose length is not its buffer's size, or an
        output array with less room than its buffer)."""
        inputs = inputs or {}
        keep = [np.ascontiguousarray(v) for v in inputs.values()]
        ids_in = (ctypes.c_uint64 * max(len(keep), 1))(*inputs.keys())
        vals_in = (ctypes.c_void_p * max(len(keep), 1))(*[k.ctypes.data for k in keep])
        lens_in = (ctypes.c_int64 * max(len(keep), 1))(*[k.nbytes for k in keep])
        if out_arrays is None:
            outs = []
            for o in outputs:
                r, c, e = self.metadata(o)
                dt = {F32: np.float32, I32: np.int32, BOOL: np.uint32, BF16: np.uint16}[e]
                outs.append(np.empty((r, c), dt))
        else:
            outs = list(out_arrays)
            assert all(a.flags.c_contiguous for a in outs) and len(outs) == len(outputs)
        ids_out = (ctypes.c_uint64 * max(len(outs), 1))(*outputs)
        vals_out = (ctypes.c_void_p * max(len(outs), 1))(*[a.ctypes.data for a in outs])
        lens_out = (ctypes.c_int64 * max(len(outs), 1))(*[a.nbytes for a in outs])
        self._check(self._lib.mi_trace_run(self.ctx, trace, len(keep), ids_in, vals_in, lens_in, len(outs), ids_out,
                                           vals_out, lens_out))
        return outs

    def release_trace(self, trace: int) -> None:
        self._check(self._lib.mi_trace_release(self.ctx, trace))

    def copy_into(self, src: int, dst: int) -> None:
        self._check(self._lib.mi_copy_into(self.ctx, src, dst))

    def set_matmul_mode(self, mode: int) -> None:
        """MATMUL_FAST (F32 operands split into BF16 parts) or MATMUL_ACCURATE (F32 matrix cores)."""
        self._check(self._lib.mi_set_matmul_mode(self.ctx, mode))

    def matmul_mode(self) -> int:
        m = ctypes.c_int()
        self._check(self._lib.mi_get_matmul_mode(self.ctx, ctypes.byref(m)))
        return m.value

    def argmax_row(self, a: int) -> int:
        return self._out(self._lib.mi_argmax_rows, a)

    def select_rows(self, table: int, idx: int) -> int:
        return self._out(self._lib.mi_select_rows, table, idx)

    def select_rows_as(self, table: int, idx: int, out_elem: int) -> int:
        """select_rows then the cast to out_elem, in one launch for BF16 rows widened to F32."""
        return self._out(self._lib.mi_select_rows_as, table, idx, out_elem)

    def pick_columns(self, x: int, idx: int) -> int:
        return self._out(self._lib.mi_pick_columns, x, idx)

    def scatter_add_columns(self, x: int, idx: int, v: int) -> int:
        return self._out(self._lib.mi_scatter_add_columns, x, idx, v)

    def select_add_rows(self, t: int, idx: int, value: int) -> int:
        return self._out(self._lib.mi_select_add_rows, t, idx, value)

    def copy_strided(self, src: int, rows: int, cols: int, offset: int, row_stride: int, col_stride: int) -> int:
        return self._out(self._lib.mi_copy_strided, src, rows, cols, offset, row_stride, col_stride)

    def copy_strided4(self, src: int, dims: Sequence[int], offset: int, strides: Sequence[int]) -> int:
        d = (ctypes.c_int64 * 4)(*dims)
        s = (ctypes.c_int64 * 4)(*strides)
        return self._out(self._lib.mi_copy_strided4, src, d, offset, s)

    def assign_block(self, dst: int, src: int, row0: int, col0: int) -> None:
        self._check(self._lib.mi_assign_block(self.ctx, dst, src, row0, col0))

    def cast_float(self, a: int, out_elem: int) -> int:
        return self._out(self._lib.mi_cast, a, out_elem)

    def gather(self, x: int, dims, dim: int, idx: int, idims) -> int:
        """Burn's float_gather along `dim` of a rank <= 4 tensor (dims and the
        index tensor's dims padded with leading 1s to four)."""
        d = (ctypes.c_int64 * 4)(*dims)
        di = (ctypes.c_int64 * 4)(*idims)
        return self._out(self._lib.mi_gather, x, d, dim, idx, di)

    def decode_advance(self, next_ids: int, ids: int, pos: int, log: int) -> None:
        """A chained decode step's tail: ids <- next_ids, log[:, pos + 1] <-
        next_ids, pos <- pos + 1 (all on the device)."""
        self._check(self._lib.mi_decode_advance(self.ctx, next_ids, ids, pos, log))

    def tile(self, a: int, form: int = TILES_BF16) -> int:
        """A row-major F32/BF16 [r, c] buffer in tiles (TILES_BF16 / TILES_PARTS)."""
        return self._out(self._lib.mi_tile, a, form)

    def cast_bfp(self, a: int, fmt: int = BFP8) -> int:
        """Engine::cast_bfp: an F32 or BF16 buffer stored as BFP8 (fmt
        BFP8), or a BFP8 buffer decoded to F32 (fmt 0)."""
        return self._out(self._lib.mi_cast_bfp, a, fmt)

    def random_dram(self, rows: int, cols: int, draw: int, p1: float = 0.0, p2: float = 1.0,
                    base: int = 0) -> int:
        return self._out(self._lib.mi_random, rows, cols, draw, p1, p2, base & (2**64 - 1))

    # -- timing and report ---------------------------------------------------
    def event_record(self, slot: int) -> None:
        self._check(self._lib.mi_event_record(self.ctx, slot))

    def event_elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        self._check(self._lib.mi_event_elapsed_ms(self.ctx, a, b, ctypes.byref(ms)))
        return ms.value

    def report(self) -> dict:
        r = Report()
        self._check(self._lib.mi_get_report(self.ctx, ctypes.byref(r)))
        return {n: getattr(r, n) for n, _ in Report._fields_}


def _dims(x: np.ndarray) -> Tuple[int, int]:
    """`[rows, cols]` of an array, rank N folded to `[prod(leading), last]`
    (crates/burn-tt/src/tensor.rs:905-908)."""
    if x.ndim == 0:
        return 1, 1
    if x.ndim == 1:
        return 1, x.shape[0]
    return int(np.prod(x.shape[:-1])), x.shape[-1]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """F32 -> BF16 bits, ties to even, NaN kept a NaN (host-side conversion for uploads)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- models
class LlamaConfig(ctypes.Structure):
    """mi_llama_config (include/miburn_models.h)."""
    _fields_ = [("vocab", ctypes.c_int32), ("hidden", ctypes.c_int32), ("layers", ctypes.c_int32),
                ("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("intermediate", ctypes.c_int32), ("rope_theta", ctypes.c_float), ("eps", ctypes.c_float),
                ("max_ctx", ctypes.c_int32), ("max_batch", ctypes.c_int32), ("numerics", ctypes.c_int32)]


# Numeric contracts (include/miburn_models.h MI_NUMERICS_*; the reference's burn_tt::Numerics).
NUMERICS = {"reference": 0, "performance": 1}


# SmolLM2-135M's shape (crates/tt-models/src/llama.rs:60-71).
SMOLLM2_135M = dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, head_dim=64, intermediate=1536,
                    rope_theta=100000.0, eps=1e-5)

LLAMA_PARAMS = {"embed": 0, "final_norm": 1, "attn_norm": 2, "wq": 3, "wk": 4, "wv": 5, "wo": 6, "mlp_norm": 7,
                "wgate": 8, "wup": 9, "wdown": 10}


def _models_lib():
    L = lib()
    if getattr(L, "_models_bound", False):
        return L
    P, I32, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64
    L.mi_llama_create.argtypes = [P, ctypes.POINTER(LlamaConfig), U64, ctypes.c_float, ctypes.POINTER(P)]
    L.mi_llama_destroy.argtypes = [P]
    L.mi_llama_param.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.POINTER(U64)]
    L.mi_llama_reset.argtypes = [P]
    L.mi_llama_forward.argtypes = [P, P, I32, I32, I32, ctypes.POINTER(U64)]
    L.mi_llama_generate.argtypes = [P, P, I32, I32, I32, P, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]
    L.mi_llama_generate_traced.argtypes = L.mi_llama_generate.argtypes
    for f in (L.mi_llama_create, L.mi_llama_destroy, L.mi_llama_param, L.mi_llama_reset, L.mi_llama_forward,
              L.mi_llama_generate, L.mi_llama_generate_traced):
        f.restype = ctypes.c_int
    L.mi_models_last_error.argtypes = []
    L.mi_models_last_error.restype = ctypes.c_char_p
    L._models_bound = True
    return L


class Llama:
    """The SmolLM2-shaped decoder harness (crates/tt-models/src/llama.rs) on an Engine."""

    def __init__(self, eng: Engine, cfg: dict, max_ctx: int, max_batch: int, seed: int = 0, init_std: float = 0.02,
                 numerics: str = "reference"):
        self.eng = eng
        self.L = _models_lib()
        c = LlamaConfig(**{k: cfg[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim",
                                               "intermediate")},
                        rope_theta=cfg["rope_theta"], eps=cfg["eps"], max_ctx=max_ctx, max_batch=max_batch,
                        numerics=NUMERICS[numerics])
        self.cfg = dict(cfg, max_ctx=max_ctx, max_batch=max_batch, numerics=numerics)
        h = ctypes.c_void_p()
        self._check(self.L.mi_llama_create(eng.ctx, ctypes.byref(c), seed, init_std, ctypes.byref(h)))
        self.h = h
        eng._children.add(self)

    def _check(self, st):
        if st != 0:
            raise MiError(st, self.L.mi_models_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.mi_llama_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param(self, name: str, layer: int = 0) -> int:
        """A copy of the weight: a new id the caller frees."""
        out = ctypes.c_uint64()
        self._check(self.L.mi_llama_param(self.h, layer, LLAMA_PARAMS[name], ctypes.byref(out)))
        return out.value

    def reset(self):
        self._check(self.L.mi_llama_reset(self.h))

    def forward(self, ids: np.ndarray, all_positions: bool = False) -> int:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        b, t = ids.shape
        out = ctypes.c_uint64()
        self._check(self.L.mi_llama_forward(self.h, ids.ctypes.data, b, t, int(all_positions), ctypes.byref(out)))
        return out.value

    def generate(self, prompt: np.ndarray, n_new: int, traced: bool = False):
        """Greedy generation: ([batch, n_new] ids, prefill ms, decode ms); `traced` replays a captured
        decode step per token (mi_llama_generate_traced)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        b, t = prompt.shape
        out = np.zeros((b, n_new), np.int32)
        pf, dc = ctypes.c_double(), ctypes.c_double()
        fn = self.L.mi_llama_generate_traced if traced else self.L.mi_llama_generate
        self._check(fn(self.h, prompt.ctypes.data, b, t, n_new, out.ctypes.data, ctypes.byref(pf), ctypes.byref(dc)))
        return out, pf.value, dc.value


class Mlp:
    """The MLP training harness (crates/tt-tests/tests/step12_mnist.rs) on an Engine."""

    def __init__(self, eng: Engine, d_in: int = 784, hidden: int = 128, d_out: int = 10, lcg_seed: int = 0x3A15):
        self.eng = eng
        L = lib()
        if not getattr(L, "_mlp_bound", False):
            P, I32, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64
            L.mi_mlp_create.argtypes = [P, I32, I32, I32, U64, ctypes.POINTER(P)]
            L.mi_mlp_destroy.argtypes = [P]
            L.mi_mlp_param.argtypes = [P, ctypes.c_int, ctypes.POINTER(U64)]
            L.mi_mlp_train_step.argtypes = [P, U64, U64, ctypes.c_float, ctypes.POINTER(U64)]
            L.mi_mlp_train_synthetic.argtypes = [P, I32, I32, ctypes.c_float, U64, P, ctypes.POINTER(ctypes.c_double)]
            for f in (L.mi_mlp_create, L.mi_mlp_destroy, L.mi_mlp_param, L.mi_mlp_train_step,
                      L.mi_mlp_train_synthetic):
                f.restype = ctypes.c_int
            L.mi_mlp_last_error.restype = ctypes.c_char_p
            L._mlp_bound = True
        self.L = L
        h = ctypes.c_void_p()
        self._check(L.mi_mlp_create(eng.ctx, d_in, hidden, d_out, lcg_seed, ctypes.byref(h)))
        self.h = h
        eng._children.add(self)
        self.d_out = d_out

    def _check(self, st):
        if st != 0:
            raise MiError(st, self.L.mi_mlp_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.mi_mlp_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param(self, which: int) -> np.ndarray:
        out = ctypes.c_uint64()
        self._check(self.L.mi_mlp_param(self.h, which, ctypes.byref(out)))
        return self.eng.download(out.value)

    def train_step(self, x: np.ndarray, labels: np.ndarray, lr: float) -> float:
        xi = self.eng.upload(x)
        li = self.eng.upload_i32(np.ascontiguousarray(labels, np.int32).reshape(-1, 1))
        out = ctypes.c_uint64()
        self._check(self.L.mi_mlp_train_step(self.h, xi, li, lr, ctypes.byref(out)))
        loss = float(self.eng.download(out.value)[0, 0])
        for i in (xi, li, out.value):
            self.eng.free(i)
        return loss

    def train_step_ids(self, x: int, labels: int, lr: float) -> int:
        """One step on resident x / label ids; returns the loss id."""
        out = ctypes.c_uint64()
        self._check(self.L.mi_mlp_train_step(self.h, x, labels, lr, ctypes.byref(out)))
        return out.value

    def train_synthetic(self, batch: int, steps: int, lr: float, data_seed: int = 0):
        losses = np.zeros(steps, np.float32)
        ms = ctypes.c_double()
        self._check(self.L.mi_mlp_train_synthetic(self.h, batch, steps, lr, data_seed, losses.ctypes.data,
                                                  ctypes.byref(ms)))
        return losses, ms.value


class TransformerConfig(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_int32), ("d_model", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("d_ff", ctypes.c_int32), ("layers", ctypes.c_int32), ("eps", ctypes.c_float)]


# BASELINE config 4's shape.
TRANSFORMER_CONFIG4 = dict(vocab=8192, d_model=256, heads=4, d_ff=1024, layers=4, eps=1e-5)
TRANSFORMER_LAYER_PARAMS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b",
                            "w1", "b1", "w2", "b2")


class Transformer:
    """The transformer training harness (crates/tt-mnist/src/transformer.rs:36-166;
    step59_burn_transformer.rs) on an Engine."""

    def __init__(self, eng: Engine, cfg: dict, seed: int = 0):
        self.eng = eng
        L = lib()
        if not getattr(L, "_tf_bound", False):
            P, I32, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64
            L.mi_transformer_create.argtypes = [P, ctypes.POINTER(TransformerConfig), U64, ctypes.POINTER(P)]
            L.mi_transformer_destroy.argtypes = [P]
            L.mi_transformer_param.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.POINTER(U64)]
            L.mi_transformer_train_step.argtypes = [P, U64, U64, I32, I32, ctypes.c_float, ctypes.POINTER(U64)]
            L.mi_transformer_train_synthetic.argtypes = [P, I32, I32, I32, ctypes.c_float, U64, P,
                                                         ctypes.POINTER(ctypes.c_double)]
            for f in (L.mi_transformer_create, L.mi_transformer_destroy, L.mi_transformer_param,
                      L.mi_transformer_train_step, L.mi_transformer_train_synthetic):
                f.restype = ctypes.c_int
            L.mi_transformer_last_error.restype = ctypes.c_char_p
            L._tf_bound = True
        self.L = L
        self.cfg = dict(cfg)
        c = TransformerConfig(vocab=cfg["vocab"], d_model=cfg["d_model"], heads=cfg["heads"], d_ff=cfg["d_ff"],
                              layers=cfg["layers"], eps=cfg.get("eps", 1e-5))
        h = ctypes.c_void_p()
        self._check(L.mi_transformer_create(eng.ctx, ctypes.byref(c), seed, ctypes.byref(h)))
        self.h = h
        eng._children.add(self)

    def _check(self, st):
        if st != 0:
            raise MiError(st, self.L.mi_transformer_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.mi_transformer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param(self, name: str, layer: int = -1) -> np.ndarray:
        which = ("embed", "head_w", "head_b").index(name) if layer < 0 else TRANSFORMER_LAYER_PARAMS.index(name)
        out = ctypes.c_uint64()
        self._check(self.L.mi_transformer_param(self.h, layer, which, ctypes.byref(out)))
        try:
            return self.eng.download(out.value)
        finally:
            self.eng.free(out.value)

    def train_step(self, tokens: np.ndarray, targets: np.ndarray, lr: float) -> float:
        """One step on host tokens / targets [batch, seq]."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        b, s = tokens.shape
        ti = self.eng.upload_i32(tokens.reshape(-1, 1))
        yi = self.eng.upload_i32(np.ascontiguousarray(targets, np.int32).reshape(-1, 1))
        out = ctypes.c_uint64()
        self._check(self.L.mi_transformer_train_step(self.h, ti, yi, b, s, lr, ctypes.byref(out)))
        loss = float(self.eng.download(out.value)[0, 0])
        for i in (ti, yi, out.value):
            self.eng.free(i)
        return loss

    def train_step_ids(self, tokens: int, targets: int, batch: int, seq: int, lr: float) -> int:
        """One step on resident token / target ids; returns the loss id (the
        form a captured trace records)."""
        out = ctypes.c_uint64()
        self._check(self.L.mi_transformer_train_step(self.h, tokens, targets, batch, seq, lr, ctypes.byref(out)))
        return out.value

    def train_synthetic(self, batch: int, seq: int, steps: int, lr: float, data_seed: int = 0):
        losses = np.zeros(steps, np.float32)
        ms = ctypes.c_double()
        self._check(self.L.mi_transformer_train_synthetic(self.h, batch, seq, steps, lr, data_seed,
                                                          losses.ctypes.data, ctypes.byref(ms)))
        return losses, ms.value
