"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible slip in the oracle fails it: golden
vectors computed independently in float64 numpy/scipy (tests/golden/
make_golden.py), exact answers from small-integer products (the reference's
step11 trick), the reference's portable known answers (signed zero through a
transpose, crates/burn-tt/tests/essentials.rs:33-56; gather of +-0/inf/NaN
payloads, crates/tt-tests/tests/step61_burn_gather.rs:1-13; argmax's first
maximum and NaN rule, crates/tt-models/src/generate.rs:176-183), closed forms
and invariants (softmax rows sum to one and ignore a shift; mean = sum / n),
and brute-force loops on tiny inputs.  No GPU is needed.
"""
import os

import math

import numpy as np
import pytest

import oracle_lib as orc
from miburn import AXIS_COLS, AXIS_ROWS, K, R_MAX, R_MEAN, R_MIN, R_SUM

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v1.npz"))
ULP = 2.0 ** -23


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def assert_bits(a, b):
    a, b = bits(a).ravel(), bits(b).ravel()
    assert a.size == b.size, (a.size, b.size)
    assert np.array_equal(a, b), np.flatnonzero(a != b)[:5]


def assert_ulps(got, want, n_ulp):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape
    tol = n_ulp * ULP * np.abs(want) + 1e-38
    bad = np.abs(got - want) > tol
    assert not bad.any(), (np.flatnonzero(bad)[:5], got.ravel()[bad.ravel()][:3], want.ravel()[bad.ravel()][:3])


# ------------------------------------------------------------ element-wise
@pytest.mark.parametrize("kind,key,src,n_ulp", [
    ("EXP", "ew_exp", "ew_x", 1), ("TANH", "ew_tanh", "ew_x", 1), ("ERF", "ew_erf", "ew_x", 1),
    ("GELU", "ew_gelu", "ew_x", 1), ("GELU", "ew_gelu_tail", "ew_gelu_tail_x", 1), ("SIGMOID", "ew_sigmoid", "ew_x", 1), ("SILU", "ew_silu", "ew_x", 2),
    ("LOG", "ew_log", "ew_pos", 1), ("SQRT", "ew_sqrt", "ew_pos", 0), ("RSQRT", "ew_rsqrt", "ew_pos", 1),
])
def test_unary_against_float64_golden(kind, key, src, n_ulp):
    got = orc.eltwise(K[kind], G[src]).ravel()
    if n_ulp == 0:
        assert_bits(got, G[key])
    else:
        assert_ulps(got, G[key], n_ulp)


@pytest.mark.parametrize("kind,key,src,s1,n_ulp", [
    ("LOG1P", "ew_log1p", "ew_log1p_x", 0.0, 1), ("EXPM1", "ew_expm1", "ew_x", 0.0, 1),
    ("SIN", "ew_sin", "ew_trig_x", 0.0, 1), ("COS", "ew_cos", "ew_trig_x", 0.0, 1),
    ("POW_S", "ew_pow_s25", "ew_pos", 2.5, 1), ("POW_S", "ew_pow_sm05", "ew_pos", -0.5, 1),
    ("RECIP", "ew_recip", "ew_x", 0.0, 0), ("DIV_SCALAR", "ew_div_s3", "ew_x", 3.0, 0),
    ("RSQRT_ABS_ADD", "ew_rsqrt_abs_add", "ew_rsq_x", 1e-6, 1),
])
def test_more_unary_against_float64_golden(kind, key, src, s1, n_ulp):
    got = orc.eltwise(K[kind], G[src], s1=s1).ravel()
    if n_ulp == 0:
        assert_bits(got, G[key])
    else:
        assert_ulps(got, G[key], n_ulp)


def test_pow_against_float64_golden():
    assert_ulps(orc.eltwise(K["POW"], G["ew_pos"], G["ew_g"]).ravel(), G["ew_pow"], 1)


def test_sigmoid_backward_golden():
    s, g = G["ew_sig_s"], G["ew_g"]
    got = orc.eltwise(K["SIGMOID_BACKWARD"], s, g).ravel()
    # Flex's order, (g s)(1 - s), bit for bit; and within 2 ulps of the exact value.
    assert_bits(got, G["ew_sig_bwd"])
    assert_ulps(got, G["ew_sig_bwd64"], 2)


@pytest.mark.parametrize("kind,key,s1,s2", [
    ("NEG", "sp_neg", 0.0, 0.0), ("ABS", "sp_abs", 0.0, 0.0), ("SIGN", "sp_sign", 0.0, 0.0),
    ("LEAKY_RELU", "sp_leaky", 0.01, 0.0), ("HARD_SIGMOID", "sp_hard_sigmoid", 0.2, 0.5),
    ("DIV_SCALAR", "sp_div_s0", 0.0, 0.0),
])
def test_exact_unary_with_special_values(kind, key, s1, s2):
    assert_bits(orc.eltwise(K[kind], G["sp_a"], s1=s1, s2=s2).ravel(), G[key])


def test_scale_mask_fill_golden():
    got = orc.eltwise(K["SCALE_MASK_FILL"], G["sp_a"], G["sp_mask"], s1=0.125, s2=-np.inf).ravel()
    assert_bits(got, G["sp_scale_mask_fill"])


def test_gelu_backward_golden():
    got = orc.eltwise(K["GELU_BACKWARD"], G["ew_x"], G["ew_g"]).ravel()
    want = G["ew_gelu_bwd"].astype(np.float64)
    # Cancellation near x = -0.75 makes the value small: bound by the terms' size.
    scale = np.abs(G["ew_g"]).astype(np.float64) * 1.5
    assert np.all(np.abs(got - want) <= 4 * ULP * (np.abs(want) + scale))


@pytest.mark.parametrize("kind,key", [("ADD", "sp_add"), ("SUB", "sp_sub"), ("MUL", "sp_mul"), ("DIV", "sp_div"),
                                      ("RELU_BACKWARD", "sp_relu_bwd"), ("GT", "sp_gt"), ("EQ", "sp_eq")])
def test_exact_binary_with_special_values(kind, key):
    assert_bits(orc.eltwise(K[kind], G["sp_a"], G["sp_b"]).ravel(), G[key])


def test_relu_special_values():
    # kind.rs:19-22: a positive datum passes; zeros, negatives and NaN give +0.
    assert_bits(orc.eltwise(K["RELU"], G["sp_a"]).ravel(), G["sp_relu"])
    x = np.array([-0.0, np.nan, -np.inf, 1e-45], np.float32)
    assert_bits(orc.eltwise(K["RELU"], x).ravel(), np.array([0.0, 0.0, 0.0, 1e-45], np.float32))


def test_broadcast_row_column_value():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    row = np.array([[10, 20, 30, 40]], np.float32)
    col = np.array([[100], [200], [300]], np.float32)
    assert_bits(orc.eltwise(K["ADD"], a, row), a + row)
    assert_bits(orc.eltwise(K["ADD"], a, col), a + col)
    assert_bits(orc.eltwise(K["SUB"], a, np.float32([[1.5]])), a - np.float32(1.5))
    # The broadcast operand may be the first.
    assert_bits(orc.eltwise(K["SUB"], row, a), row - a)


def test_fused_kinds_equal_their_compositions():
    x, y, z = G["ew_x"][:512], G["ew_g"][:512], G["ew_x"][512:1024]
    sig = orc.eltwise(K["SIGMOID"], x)
    assert_bits(orc.eltwise(K["SILU"], x), orc.eltwise(K["MUL"], x, sig))
    assert_bits(orc.eltwise(K["SILU_MUL"], x, y), orc.eltwise(K["MUL"], orc.eltwise(K["SILU"], x), y))
    assert_bits(orc.eltwise(K["ADD_RELU"], x, y), orc.eltwise(K["RELU"], orc.eltwise(K["ADD"], x, y)))
    assert_bits(orc.eltwise(K["MUL_ADD"], x, y, z), orc.eltwise(K["ADD"], z, orc.eltwise(K["MUL"], x, y)))
    assert_bits(orc.eltwise(K["SUB_EXP"], x, y), orc.eltwise(K["EXP"], orc.eltwise(K["SUB"], x, y)))


def test_scalar_forms_and_clamps():
    x = np.array([-2.0, -0.0, 0.0, 0.5, 3.0, np.nan], np.float32)
    assert_bits(orc.eltwise(K["ADD_SCALAR"], x, s1=-1.25), x + np.float32(-1.25))
    assert_bits(orc.eltwise(K["MUL_SCALAR"], x, s1=3.0), x * np.float32(3.0))
    # Flex's clamp_min is f32::max: a NaN datum gives the scalar, equal values the scalar.
    assert_bits(orc.eltwise(K["CLAMP_MIN"], x, s1=0.0), np.array([0, 0, 0, 0.5, 3, 0], np.float32))
    assert_bits(orc.eltwise(K["CLAMP_MAX"], x, s1=0.0), np.array([-2, 0, 0, 0, 0, 0], np.float32))
    c = orc.eltwise(K["CLAMP"], x, s1=-1.0, s2=1.0).ravel()
    assert_bits(c[:5], np.array([-1, -0.0, 0, 0.5, 1], np.float32))
    assert np.isnan(c[5])
    # FILL (sfpu/ops.rs:90-91): the scalar everywhere, whatever the datum.
    assert_bits(orc.eltwise(K["FILL"], x, s1=1.5), np.full((1, 6), 1.5, np.float32))


def test_mask_fill_and_where():
    a = np.array([[1, 2, 3, 4]], np.float32)
    m = np.array([[0, 1, 0, 1]], np.float32)
    assert_bits(orc.eltwise(K["MASK_FILL"], a, m, s1=-np.inf), np.array([[1, -np.inf, 3, -np.inf]], np.float32))
    c = np.array([[9, 8, 7, 6]], np.float32)
    assert_bits(orc.eltwise(K["MASK_WHERE"], a, m, c), np.array([[1, 8, 3, 6]], np.float32))


# ---------------------------------------------------------------- products
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_integer_product_exact_every_orientation(ta, tb):
    a, b = G["mm_ai"], G["mm_bi"]
    got = orc.matmul(a.T.copy() if ta else a, b.T.copy() if tb else b, ta, tb)
    assert_bits(got, G["mm_ci"])


def test_float_product_against_float64():
    got = orc.matmul(G["mm_a"], G["mm_b"])
    assert_bits(got, G["mm_c"])  # double accumulation rounded once == float64 numpy


def test_product_brute_force_tiny():
    a = np.array([[1.5, -2.0, 0.25], [3.0, 0.5, -1.0]], np.float32)
    b = np.array([[2.0, 1.0], [0.5, -4.0], [8.0, 0.0]], np.float32)
    want = np.array([[sum(float(a[i, k]) * float(b[k, j]) for k in range(3)) for j in range(2)] for i in range(2)],
                    np.float32)
    assert_bits(orc.matmul(a, b), want)
    # A non-square, non-symmetric pair catches a transposed operand.
    assert orc.matmul(a, b).shape == (2, 2)
    assert_bits(orc.matmul(b.T.copy(), a.T.copy()), want.T.copy())


def test_f32acc_product_is_the_k_ascending_sum():
    a, b = G["mm_a"], G["mm_b"]
    got = orc.matmul_f32acc(a, b)
    want = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for k in range(a.shape[1]):
        want = (want + a[:, k:k + 1] * b[k:k + 1, :]).astype(np.float32)
    assert_bits(got, want)


def test_bf16_casts():
    x = np.array([1.0, 1.00390625, 1.005859375, -0.0, np.inf, np.nan, 3.0e38, 1e-40], np.float32)
    h = orc.to_bf16(x)
    # ties to even: 1 + 2^-8 (a tie) -> 1.0; 1 + 1.5 * 2^-8 -> 1 + 2^-7
    assert h[0] == 0x3F80 and h[1] == 0x3F80 and h[2] == 0x3F81
    assert h[3] == 0x8000 and h[4] == 0x7F80 and (h[5] & 0x7F80) == 0x7F80 and (h[5] & 0x7F) != 0
    assert_bits(orc.from_bf16(h)[:5], np.array([1.0, 1.0, 1.0078125, -0.0, np.inf], np.float32))


# -------------------------------------------------------------- reductions
def test_reductions_against_float64():
    x = G["red_x"]
    assert_bits(orc.reduce(x, R_SUM, AXIS_ROWS), G["red_sum0"])
    assert_bits(orc.reduce(x, R_SUM, AXIS_COLS), G["red_sum1"])
    assert_bits(orc.reduce(x, R_MAX, AXIS_ROWS), G["red_max0"])
    assert_bits(orc.reduce(x, R_MAX, AXIS_COLS), G["red_max1"])
    assert_bits(orc.reduce(x, R_MIN, AXIS_ROWS), G["red_min0"])
    assert_bits(orc.reduce(x, R_MIN, AXIS_COLS), G["red_min1"])
    assert_bits(np.array([orc.reduce_all(x, R_MEAN)]), G["red_mean_all"])


def test_mean_is_sum_over_count():
    x = G["red_x"]
    s = orc.reduce(x, R_SUM, AXIS_COLS)
    assert_bits(orc.reduce(x, R_MEAN, AXIS_COLS), (s / np.float32(x.shape[1])).astype(np.float32))


def test_max_propagates_nan_and_sum_keeps_exact_values():
    x = np.array([[1.0, np.nan, 3.0], [-1.0, -2.0, -0.5]], np.float32)
    m = orc.reduce(x, R_MAX, AXIS_COLS).ravel()
    assert np.isnan(m[0]) and m[1] == -0.5
    m = orc.reduce(x, R_MIN, AXIS_COLS).ravel()
    assert np.isnan(m[0]) and m[1] == -2.0
    y = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    assert orc.reduce(y, R_SUM, AXIS_COLS)[0, 0] == 10.0


# ------------------------------------------------------------------ softmax
def test_softmax_against_float64():
    assert_ulps(orc.softmax_rows(G["sm_x"]), G["sm_softmax"], 1)
    assert_bits(orc.softmax_rows(G["sm_x"], log=True), G["sm_log_softmax"])


def test_softmax_invariants():
    x = G["sm_x"]
    p = orc.softmax_rows(x)
    assert np.allclose(p.sum(axis=1), 1.0, atol=x.shape[1] * ULP * 2)
    # A row shift leaves softmax unchanged (to rounding) -- a missing max
    # shift overflows on row 0, whose entries exceed 80.
    assert np.all(np.isfinite(p))
    assert np.allclose(orc.softmax_rows(x - np.float32(7.0)), p, rtol=1e-5, atol=1e-30)


def test_attention_softmax_clamps():
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    mask = np.array([[0, 1, 0], [1, 1, 1]], np.uint32)
    p = orc.softmax_rows(x, mask=mask)
    assert p[0, 1] == 0.0 and np.isclose(p[0, 0] + p[0, 2], 1.0)
    assert np.all(p[1] == 0.0)  # fully masked: zeros, not NaN
    q = orc.softmax_rows(x, scale=0.5)
    assert_ulps(q, orc.softmax_rows(x * np.float32(0.5)), 0)


# -------------------------------------------------------------------- norms
def test_norms_against_float64():
    assert_ulps(orc.rms_norm(G["nm_x"], G["nm_gamma"], 1e-5), G["nm_rms"], 1)
    assert_ulps(orc.layer_norm(G["nm_x"], G["nm_gamma"], G["nm_beta"], 1e-5), G["nm_ln"], 1)


# ----------------------------------------------------------------- indexing
def test_select_and_pick_move_raw_bits():
    t = G["ix_table"]
    assert_bits(orc.select_rows(t, G["ix_idx"]).view(np.float32), G["ix_select"])
    assert_bits(orc.pick_columns(t, G["ix_cols"]).view(np.float32), G["ix_pick"])
    # step61: a NaN payload survives the copy.
    tb = t.view(np.uint32).copy()
    tb[0, 0] = 0x7FC0BEEF
    assert orc.select_rows(tb, np.array([0], np.int32))[0, 0] == 0x7FC0BEEF


def test_index_out_of_range_is_an_error():
    t = G["ix_table"]
    assert orc.select_rows(t, np.array([0, 50], np.int32)) is None
    assert orc.select_rows(t, np.array([-1], np.int32)) is None
    assert orc.pick_columns(t, np.full(50, 12, np.int32)) is None


def test_argmax_first_maximum_and_nan():
    assert np.array_equal(orc.argmax_rows(G["am_x"]), G["am_idx"])


def test_scatter_add_columns_brute_force():
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    idx = np.array([3, 0, 3], np.int32)
    v = np.array([0.5, -1.0, 10.0], np.float32)
    want = x.copy()
    for r in range(3):
        want[r, idx[r]] += v[r]
    assert_bits(orc.scatter_add_columns(x, idx, v), want)


def test_select_add_rows_folds_duplicates_in_index_order():
    t = G["red_x"][:10, :8].copy()
    idx = np.array([3, 1, 3, 3, 9, 1], np.int32)
    val = G["red_x"][10:16, :8].copy()
    want = t.copy()
    for i, r in enumerate(idx):  # sequential f32 adds, in index order
        want[r] = (want[r] + val[i]).astype(np.float32)
    assert_bits(orc.select_add_rows(t, idx, val), want)


def test_copy_strided_transpose_keeps_negative_zero():
    # essentials.rs:33-45: [[-0.0, 2.5], [3.0, 4.0]].transpose().reshape([4, 1]) == [-0.0, 3.0, 2.5, 4.0]
    x = np.array([[-0.0, 2.5], [3.0, 4.0]], np.float32)
    got = orc.copy_strided4(x, (1, 1, 2, 2), 0, (0, 0, 1, 2)).view(np.float32).reshape(4)
    assert_bits(got, np.array([-0.0, 3.0, 2.5, 4.0], np.float32))


# ----------------------------------------------------------- backward rows
# The fused backward restatements are pinned by central differences of the
# oracle's own forward functions (a derivative fixed by the forward, not a
# retyped formula): a dropped mean term, a wrong sign or a missing 1/den fails.
def _fd(f, x, h=1e-2):
    g = np.zeros(x.size)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += h
        xm.flat[i] -= h
        g[i] = (f(xp) - f(xm)) / (2 * h)
    return g.reshape(x.shape)


def test_layer_norm_backward_matches_finite_differences():
    rng = np.random.default_rng(41)
    R, C = 3, 7
    x = (rng.standard_normal((R, C)) * 2 + 0.5).astype(np.float32)
    gam = (rng.standard_normal((1, C)) + 1).astype(np.float32)
    bet = rng.standard_normal((1, C)).astype(np.float32)
    dy = rng.standard_normal((R, C)).astype(np.float32)
    dres = rng.standard_normal((R, C)).astype(np.float32)

    def loss(xv, g=gam, b=bet):
        return float(np.sum(dy.astype(np.float64) * orc.layer_norm(xv.astype(np.float32), g, b)))

    dx, dg, db = orc.layer_norm_backward(x, gam, dy, dres)
    fx = _fd(lambda v: loss(v), x.astype(np.float64))
    fg = _fd(lambda v: loss(x, g=v.astype(np.float32)), gam.astype(np.float64))
    fb = _fd(lambda v: loss(x, b=v.astype(np.float32)), bet.astype(np.float64))
    assert np.allclose(dx - dres, fx, atol=2e-3, rtol=2e-3)
    assert np.allclose(dg, fg, atol=2e-3, rtol=2e-3)
    assert np.allclose(db, fb, atol=2e-3, rtol=2e-3)
    # Without gamma: the unit gain.
    dx1, _, _ = orc.layer_norm_backward(x, None, dy)
    dx2, _, _ = orc.layer_norm_backward(x, np.ones((1, C), np.float32), dy)
    assert np.array_equal(dx1, dx2)


def test_softmax_backward_matches_finite_differences():
    rng = np.random.default_rng(42)
    x = rng.standard_normal((4, 9)).astype(np.float32)
    dp = rng.standard_normal((4, 9)).astype(np.float32)
    scale = 0.37
    p = orc.softmax_rows(x, scale=scale)
    ds = orc.softmax_backward(p, dp, scale)
    f = _fd(lambda v: float(np.sum(dp.astype(np.float64) * orc.softmax_rows(v.astype(np.float32), scale=scale))),
            x.astype(np.float64))
    assert np.allclose(ds, f, atol=1e-3, rtol=1e-3)
    # Rows of the gradient sum to zero (softmax is shift-invariant).
    assert np.abs(ds.astype(np.float64).sum(1)).max() < 1e-6


# ------------------------------------------------------------------- guard
# Where each element-wise kind and reduction the device tests grade against
# the oracle is pinned in this file (a golden vector, a known answer or a
# composition of pinned kinds).
PINNED = {
    "ADD": "sp_add", "SUB": "sp_sub", "MUL": "sp_mul", "DIV": "sp_div", "RELU": "sp_relu",
    "RELU_BACKWARD": "sp_relu_bwd", "GT": "sp_gt", "EQ": "sp_eq", "NEG": "sp_neg", "ABS": "sp_abs",
    "SIGN": "sp_sign", "LEAKY_RELU": "sp_leaky", "HARD_SIGMOID": "sp_hard_sigmoid",
    "SCALE_MASK_FILL": "sp_scale_mask_fill", "EXP": "ew_exp", "TANH": "ew_tanh", "ERF": "ew_erf",
    "GELU": "ew_gelu", "SIGMOID": "ew_sigmoid", "SILU": "ew_silu", "LOG": "ew_log", "SQRT": "ew_sqrt",
    "RSQRT": "ew_rsqrt", "LOG1P": "ew_log1p", "EXPM1": "ew_expm1", "SIN": "ew_sin", "COS": "ew_cos",
    "POW": "ew_pow", "POW_S": "ew_pow_s25", "RECIP": "ew_recip", "DIV_SCALAR": "ew_div_s3",
    "RSQRT_ABS_ADD": "ew_rsqrt_abs_add", "SIGMOID_BACKWARD": "ew_sig_bwd", "GELU_BACKWARD": "ew_gelu_bwd",
    # known answers and compositions above
    "SILU_MUL": "test_fused_kinds_equal_their_compositions", "ADD_RELU": "test_fused_kinds_equal_their_compositions",
    "MUL_ADD": "test_fused_kinds_equal_their_compositions", "SUB_EXP": "test_fused_kinds_equal_their_compositions",
    "ADD_SCALAR": "test_scalar_forms_and_clamps", "MUL_SCALAR": "test_scalar_forms_and_clamps",
    "CLAMP": "test_scalar_forms_and_clamps", "CLAMP_MIN": "test_scalar_forms_and_clamps",
    "CLAMP_MAX": "test_scalar_forms_and_clamps", "FILL": "test_scalar_forms_and_clamps", "MASK_FILL": "test_mask_fill_and_where",
    "MASK_WHERE": "test_mask_fill_and_where", "NE": "test_comparisons_known_answers",
    "GE": "test_comparisons_known_answers", "LT": "test_comparisons_known_answers",
    "LE": "test_comparisons_known_answers",
    "R_SUM": "red_sum0", "R_MAX": "red_max0", "R_MIN": "red_min0", "R_MEAN": "red_mean_all",
}


def test_comparisons_known_answers():
    # IEEE comparisons (sfpu/ops.rs:66-72): -0 == +0, a NaN unordered (only NE true).
    a = np.array([1.0, -0.0, np.nan, 2.0, -np.inf], np.float32)
    b = np.array([1.0, 0.0, np.nan, 3.0, -np.inf], np.float32)
    want = {"EQ": [1, 1, 0, 0, 1], "NE": [0, 0, 1, 1, 0], "GT": [0, 0, 0, 0, 0], "GE": [1, 1, 0, 0, 1],
            "LT": [0, 0, 0, 1, 0], "LE": [1, 1, 0, 1, 1]}
    for kind, w in want.items():
        assert_bits(orc.eltwise(K[kind], a, b).ravel(), np.array(w, np.float32))


def test_every_kind_the_device_is_graded_on_is_pinned():
    """Fails when a device test grades against an oracle function that no
    check in this file pins."""
    import glob
    import re
    here = os.path.dirname(os.path.abspath(__file__))
    used = set()
    for path in glob.glob(os.path.join(here, "test_gpu_*.py")):
        text = open(path).read()
        used |= {m for m in re.findall(r'"([A-Z][A-Z0-9_]*)"', text) if m in K}
        used |= set(re.findall(r"\b(R_(?:SUM|MAX|MIN|MEAN))\b", text))
    missing = sorted(used - set(PINNED))
    assert not missing, missing
    me = open(os.path.abspath(__file__)).read()
    for kind, where in PINNED.items():
        assert where in G.files or f"def {where}(" in me, (kind, where)


# ------------------------------------------------------------ BFP8 / BFP4
# oracle/oracle.c's restatement of crates/tt-isa/src/tile.rs:619 (the
# unpacker's BFP8 decode) and crates/tt-models/src/quant.rs:185-235
# (bfp_round_trip), pinned by the mathematics rather than by its procedure.

def _bf16_value(h):
    return float(orc.from_bf16(np.array([h], np.uint16))[0])


def test_bfp8_decode_every_datum_and_exponent():
    """All 65536 (datum, exponent) pairs.  Where the normalised exponent
    stays in 1..254 the BF16 value is the closed form +-mag * 2^(exp - 133);
    a zero magnitude is +0, or -inf with the sign set (tile.rs:1158-1167's
    known answers); past the range the exponent field wraps modulo 256 with
    the significand still the normalised magnitude."""
    for datum in range(256):
        sign, mag = datum >> 7, datum & 0x7F
        for exp in range(256):
            h = orc.bfp8_to_bf16(datum, exp)
            if mag == 0:
                assert h == (0xFF80 if sign else 0), (datum, exp)
                continue
            nb = mag.bit_length()
            dexp = exp - (7 - nb)  # leading zeros of the magnitude's 8-bit form
            assert (h >> 15) == sign
            if 1 <= dexp <= 254:
                assert _bf16_value(h) == (-1) ** sign * math.ldexp(mag, exp - 133), (datum, exp)
            else:
                assert (h >> 7) & 0xFF == dexp % 256, (datum, exp)
                assert 1 + (h & 0x7F) / 128 == mag / 2 ** (nb - 1), (datum, exp)


def test_bfp_round_trip_hand_worked_block():
    # Block exponent 127 (from 1.0): quantum 2^-6.
    v = np.zeros(16, np.float32)
    v[:10] = [1.0, 0.3, -0.3, 0.5, 2.0 ** -7, 1.5 * 2.0 ** -8, 0.0, -0.0, 1.9921875, -3 * 2.0 ** -7]
    out, exps, bad = orc.bfp_round_trip(v.reshape(1, 16))
    assert bad == 0 and exps[0, 0] == 127
    # 0.3 truncates to BF16 0.298828125 = 19.125 quanta -> 19; 2^-7 is half a
    # quantum -> 1 (half away from zero); 1.5 * 2^-8 is 0.375 quanta -> 0;
    # 1.9921875 is 127.5 quanta -> 128, clamped to 127; -3 * 2^-7 is -1.5
    # quanta -> -2.  -0.0 comes back +0.0 (datum 0).
    want = [1.0, 19 / 64, -19 / 64, 0.5, 1 / 64, 0.0, 0.0, 0.0, 127 / 64, -2 / 64] + [0.0] * 6
    assert out[0].tolist() == want
    assert not np.signbit(out[0, 7])
    # BFP4 keeps the top 3 magnitude bits: 19 -> 16 quanta (0.25), 64 -> 1.0,
    # 32 -> 0.5, 127 -> 112 quanta (1.75), 1 and 2 -> 0.
    out4, _, _ = orc.bfp_round_trip(v.reshape(1, 16), width=4)
    assert out4[0, :10].tolist() == [1.0, 0.25, -0.25, 0.5, 0.0, 0.0, 0.0, 0.0, 1.75, 0.0]


def test_bfp_round_trip_is_the_nearest_block_value():
    """Each value is the nearest of the 255 values k * 2^(E - 133), |k| <=
    127, to its BF16 truncation (ties away from zero; beyond 127 quanta the
    largest), E the block's largest biased exponent: a brute-force search,
    not the rounding the oracle does.  Rows of mixed scales, a partial last
    block, the reference's own step92 pattern."""
    rng = np.random.default_rng(41)
    scale = 2.0 ** rng.integers(-30, 30, (24, 1))
    x = (rng.standard_normal((24, 40)) * scale).astype(np.float32)
    x[3, 5] = 0.0
    x[4, 17:19] = [-0.0, 1e-39]  # a signed zero and a subnormal: zero magnitude
    i = np.arange(1024)
    step92 = (((i % 16) - 8 + np.where(i % 3 == 0, 65 / 1024, 0)) * 2.0 ** ((i // 16 % 9) - 4)).astype(np.float32)
    for data in (x, step92.reshape(16, 64)):
        out, exps, bad = orc.bfp_round_trip(data)
        assert bad == 0
        rows, cols = data.shape
        t = (data.view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
        k = np.arange(-127, 128, dtype=np.float64)
        for r in range(rows):
            for b in range((cols + 15) // 16):
                blk = slice(16 * b, min(16 * b + 16, cols))
                E = int(np.max(data[r, blk].view(np.uint32) >> 23 & 0xFF))
                assert exps[r, b] == E
                cand = k * math.ldexp(1.0, E - 133)
                for c in range(blk.start, blk.stop):
                    tv = t[r, c] if (data[r, c].view(np.uint32) >> 23) & 0xFF else 0.0
                    d = np.abs(cand - tv)
                    best = np.flatnonzero(d == d.min())
                    j = best[np.argmax(np.abs(k[best]))]  # a tie goes away from zero
                    assert out[r, c] == cand[j], (r, c, data[r, c], out[r, c], cand[j])


def test_bfp_round_trip_invariants():
    rng = np.random.default_rng(43)
    x = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    out, exps, _ = orc.bfp_round_trip(x)
    again, exps2, _ = orc.bfp_round_trip(out)
    assert np.array_equal(again, out)  # held values are held exactly
    neg, _, _ = orc.bfp_round_trip(-x)
    assert np.array_equal(neg, -out)  # odd (zeros aside: +0 either way)
    # Every held value is a BF16 value (at most 7 significant bits), within
    # half a quantum of the BF16 truncation, and exact in BFP8's 1 + 1/16
    # bytes a value: sign, 7 magnitude bits, the block's exponent byte.
    assert np.array_equal(orc.from_bf16(orc.to_bf16(out)), out)
    q = np.ldexp(1.0, exps.astype(np.int64) - 133).repeat(16, 1)[:, :96]
    m = out.astype(np.float64) / q
    assert np.array_equal(m, np.round(m)) and np.abs(m).max() <= 127
    t = (x.view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    assert np.all(np.abs(out - t) <= 0.5 * q)
    # A non-finite value is refused (the reference asserts finite values).
    y = x.copy()
    y[2, 3] = np.inf
    _, _, bad = orc.bfp_round_trip(y)
    assert bad == 1



def test_gather_along_any_dim_matches_take_along_axis():
    """or_gather (ops.rs:1102-1160) against numpy's take_along_axis, ranks 1
    to 4 and every dim, with NaN / -0.0 / infinity payloads kept bit for bit;
    an index out of range is reported and gives zero bits."""
    rng = np.random.default_rng(51)
    for shape in [(7,), (5, 9), (3, 4, 6), (2, 3, 4, 5)]:
        x = rng.standard_normal(shape).astype(np.float32)
        flat = x.reshape(-1)
        flat[::7] = np.nan
        flat[1::11] = -0.0
        flat[2::13] = np.inf
        for dim in range(len(shape)):
            ishape = list(shape)
            ishape[dim] = 3 + dim
            idx = rng.integers(0, shape[dim], ishape).astype(np.int32)
            got, bad = orc.gather(x, dim, idx)
            assert bad == 0
            want = np.take_along_axis(x, idx.astype(np.int64), dim)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    x = rng.standard_normal((4, 5)).astype(np.float32)
    idx = np.zeros((4, 2), np.int32)
    idx[2, 1] = 5
    got, bad = orc.gather(x, 1, idx)
    assert bad == 1 and got.view(np.uint32)[2, 1] == 0
