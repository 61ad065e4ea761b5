"""Device parity: every engine op through the C ABI against the CPU oracle on
the same seeded inputs.

Bars: indexing, gather, argmax, casts and copies
bit-exact; F32 element-wise ops and reductions within rel 1e-5; BF16-input
products within rel 2e-2 of the F32 oracle and, against the oracle fed the
same BF16 values, within the F32 accumulation bound.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc
from miburn import AXIS_COLS, AXIS_ROWS, BF16, BOOL, F32, I32, K, R_MAX, R_MEAN, R_MIN, R_SUM

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20240611)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def same_bits(a, b):
    a = np.ascontiguousarray(a).view(np.uint32)
    b = np.ascontiguousarray(b).view(np.uint32)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{bad.size} datums differ, first at {bad[0]}: {a.ravel()[bad[0]]:#x} vs {b.ravel()[bad[0]]:#x}"


def close(got, want, rtol=1e-5, atol=0.0):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN positions differ: {np.flatnonzero(gn != wn)[:5]}"
    g, w = got[~gn], want[~wn]
    inf = np.isinf(w)
    assert np.array_equal(g[inf], w[inf]), "infinities differ"
    g, w = g[~inf].astype(np.float64), w[~inf].astype(np.float64)
    err = np.abs(g - w)
    lim = rtol * np.abs(w) + atol
    worst = np.argmax(err - lim) if err.size else 0
    assert np.all(err <= lim), f"max excess at {worst}: got {g[worst]!r} want {w[worst]!r} (tol {lim[worst]:.3g})"


# --------------------------------------------------------------- element-wise
EXACT_UNARY = ["NEG", "ABS", "RELU", "SIGN", "SQRT"]
APPROX_UNARY = ["EXP", "LOG", "RECIP", "RSQRT", "SIGMOID", "TANH", "ERF", "GELU", "SILU", "LOG1P", "EXPM1",
                "SIN", "COS"]


def unary_input(kind, shape):
    x = rnd(*shape)
    if kind in ("LOG", "RSQRT", "SQRT"):
        x = np.abs(x) + np.float32(1e-3)
    if kind == "LOG1P":
        x = np.abs(x)
    return x


@pytest.mark.parametrize("kind", EXACT_UNARY + APPROX_UNARY)
@pytest.mark.parametrize("shape", [(64, 256), (37, 13)])
def test_unary(engine, kind, shape):
    x = unary_input(kind, shape)
    a = engine.upload(x)
    y = engine.eltwise_op_as(kind, a)
    got = engine.download(y)
    want = orc.eltwise(K[kind], x)
    if kind in EXACT_UNARY:
        same_bits(got, want)
    else:
        close(got, want, rtol=1e-5, atol=1e-7)
    engine.free(a)
    engine.free(y)


@pytest.mark.parametrize("kind", ["ADD", "SUB", "MUL", "DIV", "RELU_BACKWARD", "ADD_RELU"])
@pytest.mark.parametrize("bshape", ["full", "row", "col", "one"])
def test_binary_broadcast_exact(engine, kind, bshape):
    R, C = 48, 96
    x = rnd(R, C)
    y = {"full": rnd(R, C), "row": rnd(1, C), "col": rnd(R, 1), "one": rnd(1, 1)}[bshape]
    if kind == "DIV":
        y = np.where(np.abs(y) < 0.1, np.float32(0.5), y).astype(np.float32)
    a, b = engine.upload(x), engine.upload(y)
    got = engine.download(engine.eltwise_op_as(kind, a, b))
    same_bits(got, orc.eltwise(K[kind], x, y))


def test_sigmoid_within_its_bound(engine):
    """The logistic function (hardware 2^y of y = -|x| log2 e, hardware
    reciprocal) against float64 over |x| < 87: relative error within
    (6 + 1.25 |x|) 2^-24 (y's rounding and the F32 log2 e's 0.22 2^-24 scale
    with |x|); beyond, the tails' limits; and the special values."""
    x = np.concatenate([np.linspace(-86.9, 86.9, 200001), rnd(1, 4096).ravel() * np.float32(8)]).astype(np.float32)
    got = engine.download(engine.eltwise_op_as("SIGMOID", engine.upload(x.reshape(1, -1)))).ravel()
    xd = x.astype(np.float64)
    want = np.where(xd >= 0, 1.0 / (1.0 + np.exp(-xd)), np.exp(xd) / (1.0 + np.exp(xd)))
    rel = np.abs(got - want) / want
    bound = (6 + 1.25 * np.abs(xd)) * 2.0 ** -24
    assert np.all(rel <= bound), float(np.max(rel / bound))
    sp = np.array([[0.0, -0.0, np.inf, -np.inf, np.nan, 100.0, -100.0, 88.0]], np.float32)
    g = engine.download(engine.eltwise_op_as("SIGMOID", engine.upload(sp))).ravel()
    assert g[0] == 0.5 and g[1] == 0.5 and g[2] == 1.0 and g[3] == 0.0 and np.isnan(g[4])
    assert g[5] == 1.0 and 0.0 <= g[6] < 1e-40 and g[7] == 1.0


@pytest.mark.parametrize("kind", ["SIGMOID_BACKWARD", "GELU_BACKWARD", "SILU_MUL", "SUB_EXP", "POW"])
def test_binary_approx(engine, kind):
    R, C = 40, 200
    x, y = rnd(R, C), rnd(R, C)
    if kind == "POW":
        x = np.abs(x) + np.float32(0.1)
    if kind == "SIGMOID_BACKWARD":
        x = 1.0 / (1.0 + np.exp(-x)).astype(np.float32)
    a, b = engine.upload(x), engine.upload(y)
    got = engine.download(engine.eltwise_op_as(kind, a, b))
    close(got, orc.eltwise(K[kind], x, y), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind,s1,s2", [("MUL_SCALAR", -1.75, 0.0), ("ADD_SCALAR", 2.7, 0.0),
                                        ("ADD_SCALAR", -0.0, 0.0), ("DIV_SCALAR", 3.0, 0.0),
                                        ("CLAMP", -0.5, 0.75), ("CLAMP_MIN", 0.25, 0.0), ("CLAMP_MAX", -0.1, 0.0),
                                        ("LEAKY_RELU", 0.01, 0.0), ("HARD_SIGMOID", 0.2, 0.5), ("FILL", 1.5, 0.0),
                                        ("POW_S", 2.0, 0.0)])
def test_scalar_ops_exact(engine, kind, s1, s2):
    x = rnd(33, 64)
    a = engine.upload(x)
    got = engine.download(engine.eltwise_op_as(kind, a, scalar=s1, scalar2=s2))
    want = orc.eltwise(K[kind], x, s1=s1, s2=s2)
    if kind == "POW_S":
        close(got, want, rtol=1e-6)
    else:
        same_bits(got, want)


def test_gelu_negative_tail(engine):
    """Below a = -5.3, 1 + erf(a / sqrt 2) cancels to zero in F32; GELU stays
    within rel 1e-5 down to a = -13 (the erfc form)."""
    x = np.linspace(-13.0, -4.0, 4099, dtype=np.float32).reshape(1, -1)
    close(engine.download(engine.eltwise_op_as("GELU", engine.upload(x))), orc.eltwise(K["GELU"], x), rtol=1e-5)
    # Special values: +inf stays, -inf and NaN give NaN (inf * 0), signed
    # zeros keep their sign; below -13 the value is under F32's normal range.
    sp = np.array([[np.inf, -np.inf, np.nan, 0.0, -0.0, -14.0, -40.0, 13.2, 20.0, 1e30]], np.float32)
    got = engine.download(engine.eltwise_op_as("GELU", engine.upload(sp)))
    close(got, orc.eltwise(K["GELU"], sp), rtol=1e-5, atol=1e-37)
    assert np.signbit(got[0, 4]) and not np.signbit(got[0, 3])


def test_rsqrt_abs_add_fused(engine):
    x = rnd(128, 128)
    a = engine.upload(x)
    got = engine.download(engine.eltwise_op_as("RSQRT_ABS_ADD", a, scalar=1e-6))
    close(got, orc.eltwise(K["RSQRT_ABS_ADD"], x, s1=1e-6), rtol=1e-5)


@pytest.mark.parametrize("kind", ["EQ", "NE", "GT", "GE", "LT", "LE"])
def test_compare(engine, kind):
    x = rnd(16, 40)
    y = x.copy()
    y[::2] = rnd(8, 40)
    y[0, 0], x[0, 0] = np.nan, 1.0
    x[1, 1], y[1, 1] = -0.0, 0.0
    a, b = engine.upload(x), engine.upload(y)
    out = engine.eltwise_op_as(kind, a, b)
    assert engine.metadata(out)[2] == BOOL
    got = engine.download(out)
    same_bits(got, orc.eltwise(K[kind], x, y).astype(np.uint32))


def test_mask_fill_and_where(engine):
    x, z = rnd(24, 80), rnd(24, 80)
    m = (RNG.random((24, 80)) < 0.3).astype(np.uint32)
    mrow = (RNG.random((1, 80)) < 0.5).astype(np.uint32)
    a, c = engine.upload(x), engine.upload(z)
    mb, mr = engine.upload_bool(m), engine.upload_bool(mrow)
    same_bits(engine.download(engine.eltwise_op_as("MASK_FILL", a, mb, scalar=-np.inf)),
              orc.eltwise(K["MASK_FILL"], x, m, s1=-np.inf))
    same_bits(engine.download(engine.eltwise_op_as("MASK_FILL", a, mr, scalar=7.0)),
              orc.eltwise(K["MASK_FILL"], x, mrow, s1=7.0))
    same_bits(engine.download(engine.eltwise_op_as("MASK_WHERE", a, mb, c)),
              orc.eltwise(K["MASK_WHERE"], x, m, z))
    same_bits(engine.download(engine.eltwise_op_as("SCALE_MASK_FILL", a, mr, scalar=0.125, scalar2=-np.inf)),
              orc.eltwise(K["SCALE_MASK_FILL"], x, mrow, s1=0.125, s2=-np.inf))


def test_mul_add_ternary(engine):
    x, y, z = rnd(30, 64), rnd(30, 64), rnd(30, 64)
    a, b, c = engine.upload(x), engine.upload(y), engine.upload(z)
    same_bits(engine.download(engine.eltwise_op_as("MUL_ADD", a, b, c)), orc.eltwise(K["MUL_ADD"], x, y, z))


def test_special_values_relu_and_neg(engine):
    x = np.array([[0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.0]], np.float32)
    a = engine.upload(x)
    same_bits(engine.download(engine.eltwise_op_as("RELU", a)), orc.eltwise(K["RELU"], x))
    same_bits(engine.download(engine.eltwise_op_as("NEG", a)), orc.eltwise(K["NEG"], x))
    same_bits(engine.download(engine.eltwise_op_as("ABS", a)), orc.eltwise(K["ABS"], x))


def test_bf16_narrowing_over_every_head(engine):
    """F32 -> BF16 on the device (gfx950's conversion instruction) against the
    oracle's integer rounding: every sign/exponent/7-bit-mantissa head with
    low halves at the rounding boundaries (exact, just below and at the tie,
    past it, the largest) and random ones -- NaN payloads, infinities,
    subnormals, overflow to infinity and ties to even included."""
    heads = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    u = (heads[:, None] | lows[None, :]).ravel()
    u = np.concatenate([u, heads | RNG.integers(0, 1 << 16, heads.size, dtype=np.uint32)])
    x = u.view(np.float32).reshape(-1, 1024)
    got = engine.download(engine.cast_float(engine.upload_bits(u.reshape(-1, 1024), F32), BF16))
    assert np.array_equal(got, orc.to_bf16(x))


def test_bf16_in_and_out(engine):
    x = rnd(64, 128)
    xb = orc.to_bf16(x)
    a = engine.upload_bf16(xb)
    y = engine.eltwise_op_as("GELU", a, out_elem=BF16)
    assert engine.metadata(y)[2] == BF16
    got = miburn.bf16_to_f32(engine.download(y))
    want = orc.from_bf16(orc.to_bf16(orc.eltwise(K["GELU"], orc.from_bf16(xb))))
    # One rounding to BF16 of values within 1e-5 of each other: at most one BF16 ulp apart.
    close(got, want, rtol=2 ** -7, atol=1e-30)


def test_large_vector_path(engine):
    x, y = rnd(1024, 4096), rnd(1, 4096)
    a, b = engine.upload(x), engine.upload(y)
    same_bits(engine.download(engine.eltwise_op_as("ADD", a, b)), x + y)
    close(engine.download(engine.eltwise_op_as("EXP", a)), orc.eltwise(K["EXP"], x), rtol=1e-5)


@pytest.mark.parametrize("n", [5 * (8 << 20) + 123, 3 * (8 << 20), 1000])
def test_transfer_round_trip_chunks(engine, n):
    # More 32 MiB staging chunks than slots (downloads keep four in flight),
    # sizes that are not a chunk multiple, F32, BF16 and raw 32-bit datums.
    x = RNG.standard_normal(n).astype(np.float32).reshape(1, n)
    ix = engine.upload(x)
    same_bits(engine.download(ix), x)
    b = (x.view(np.uint32) >> 16).astype(np.uint16)
    ib = engine.upload_bf16(b)
    assert np.array_equal(engine.download(ib), b)
    bits = x.view(np.uint32)
    iu = engine.upload_bits(bits, I32)
    assert np.array_equal(engine.download(iu).view(np.uint32), bits)
    same_bits(engine.download(ix), x)  # again, after the slots were reused by the uploads
    for i in (ix, ib, iu):
        engine.free(i)


# ------------------------------------------------------------------ reductions
def reduce_tol(x, axis):
    # Normwise: rel 1e-5 of the sum of magnitudes along the reduced axis.
    return 1e-5 * np.abs(x.astype(np.float64)).sum(axis=1 - axis if axis in (0, 1) else None, keepdims=True)


@pytest.mark.parametrize("shape", [(1, 1), (7, 3), (64, 10), (130, 1000), (1000, 130), (2048, 512), (5, 9000),
                                   (1024, 8192), (1500, 8224), (4096, 8192)])
@pytest.mark.parametrize("axis", [AXIS_ROWS, AXIS_COLS])
def test_sum_mean(engine, shape, axis):
    x = rnd(*shape)
    a = engine.upload(x)
    n = shape[0] if axis == AXIS_ROWS else shape[1]
    absx = np.abs(x.astype(np.float64)).sum(axis=0 if axis == AXIS_ROWS else 1)
    absx = absx.reshape((1, -1) if axis == AXIS_ROWS else (-1, 1))
    for op in (R_SUM, R_MEAN):
        got = engine.download(engine.reduce(a, op, axis))
        want = orc.reduce(x, op, axis)
        scale = absx if op == R_SUM else absx / n
        assert got.shape == want.shape
        assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * scale + 1e-30)


@pytest.mark.parametrize("shape", [(4096, 8192), (1500, 8224), (100, 3000), (70, 1024)])
def test_column_sum_repeatable(engine, shape):
    # The one-launch column reduction resets its arrival counters: calls in a
    # row, and interleaved with other shapes, give the same bits.
    x = rnd(*shape)
    a = engine.upload(x)
    other = engine.upload(rnd(300, 2048))
    first = engine.download(engine.reduce(a, R_SUM, AXIS_ROWS))
    for _ in range(3):
        engine.free(engine.reduce(other, R_MEAN, AXIS_ROWS))
        same_bits(engine.download(engine.reduce(a, R_SUM, AXIS_ROWS)), first)
    absx = np.abs(x.astype(np.float64)).sum(axis=0, keepdims=True)
    assert np.all(np.abs(first.astype(np.float64) - orc.reduce(x, R_SUM, AXIS_ROWS)) <= 1e-5 * absx + 1e-30)


@pytest.mark.parametrize("shape", [(3, 5), (64, 10), (300, 700), (1500, 8224)])
@pytest.mark.parametrize("axis", [AXIS_ROWS, AXIS_COLS])
def test_max_min_exact(engine, shape, axis):
    x = rnd(*shape)
    x[0, 0] = np.nan
    x[-1, -1] = np.nan  # the last row of a column
    a = engine.upload(x)
    for op in (R_MAX, R_MIN):
        same_bits(engine.download(engine.reduce(a, op, axis)), orc.reduce(x, op, axis))


def test_reduce_then_is_reduce_then_op(engine):
    """Engine::reduce's `then`: the exact unary kind on the reduction, bit for
    bit the two ops (a softmax's clamp_min of its row max)."""
    x = rnd(37, 300)
    x[5] = -np.inf
    ix = engine.upload(x)
    for op, axis, kind, sc in [(R_MAX, AXIS_COLS, "CLAMP_MIN", -3.4028235e38), (R_SUM, AXIS_ROWS, "MUL_SCALAR", 0.5),
                               (R_MEAN, AXIS_COLS, 0, 0.0)]:
        got = engine.download(engine.reduce_then(ix, op, axis, kind, sc))
        r = engine.reduce(ix, op, axis)
        want = engine.download(engine.eltwise_op_as(kind, r, scalar=sc)) if kind else engine.download(r)
        same_bits(got, want)
        if kind:
            same_bits(got, orc.eltwise(K[kind], orc.reduce(x, op, axis), s1=sc))


def test_add_rms_norm(engine):
    a, b, g = rnd(9, 576), rnd(9, 576), rnd(1, 576) + np.float32(1.0)
    s, n = engine.add_rms_norm(engine.upload(a), engine.upload(b), engine.upload(g), 1e-5)
    same_bits(engine.download(s), a + b)
    close(engine.download(n), orc.rms_norm(a + b, g, 1e-5), rtol=1e-5, atol=1e-30)


def test_matmul_pairs_arbitrary_blocks(engine):
    """matmul_dram_batched over (Block, Block) items: a constant-stride run,
    then items in any order, transposed blocks among them."""
    A, B = rnd(96, 80), rnd(120, 64)
    m, k, n = 16, 24, 32
    a_blocks = [((0, 0), False), ((16, 0), False), ((32, 0), False), ((8, 40), False), ((40, 8), True), ((0, 56), True)]
    b_blocks = [((0, 0), False), ((24, 0), False), ((48, 0), False), ((96, 32), False), ((3, 5), True), ((60, 30), True)]
    got = engine.download(engine.matmul_pairs(engine.upload(A), engine.upload(B), a_blocks, b_blocks, m, k, n))
    assert got.shape == (6 * m, n)
    for i, (((ar, ac), at), ((br, bc), bt)) in enumerate(zip(a_blocks, b_blocks)):
        ab = A[ar:ar + (k if at else m), ac:ac + (m if at else k)]
        bb = B[br:br + (n if bt else k), bc:bc + (k if bt else n)]
        want = orc.matmul(ab.copy(), bb.copy(), at, bt)
        assert np.all(np.abs(got[i * m:(i + 1) * m] - want) <= mm_tol(ab, bb, at, bt, 1e-5) + 1e-30), i
    with pytest.raises(miburn.MiError) as e:
        engine.matmul_pairs(engine.upload(A), engine.upload(B), [((90, 0), False)], [((0, 0), False)], m, k, n)
    assert e.value.kind == "ARG"  # the A block leaves its buffer


def test_reduce_all(engine):
    x = rnd(333, 777)
    a = engine.upload(x)
    tol = 1e-5 * np.abs(x.astype(np.float64)).sum()
    got = engine.download(engine.reduce_all(a, R_SUM))[0, 0]
    assert abs(float(got) - float(orc.reduce_all(x, R_SUM))) <= tol
    got = engine.download(engine.reduce_all(a, R_MEAN))[0, 0]
    assert abs(float(got) - float(orc.reduce_all(x, R_MEAN))) <= tol / x.size
    same_bits(engine.download(engine.reduce_all(a, R_MAX)).ravel(), np.array([orc.reduce_all(x, R_MAX)]))


def test_bf16_reduce(engine):
    x = orc.to_bf16(rnd(100, 300))
    a = engine.upload_bf16(x)
    xf = orc.from_bf16(x)
    got = engine.download(engine.reduce(a, R_SUM, AXIS_COLS))
    tol = 1e-5 * np.abs(xf.astype(np.float64)).sum(axis=1, keepdims=True)
    assert np.all(np.abs(got - orc.reduce(xf, R_SUM, AXIS_COLS)) <= tol)


# --------------------------------------------------------------------- softmax
@pytest.mark.parametrize("cols", [1, 10, 64, 128, 640, 1000, 1030, 8192, 9000, 20000])
@pytest.mark.parametrize("log", [False, True])
def test_softmax(engine, cols, log):
    x = rnd(17, cols, scale=3.0)
    a = engine.upload(x)
    got = engine.download(engine.softmax_rows(a, log=log))
    want = orc.softmax_rows(x, log=log)
    close(got, want, rtol=1e-5, atol=1e-6 if log else 1e-12)
    if not log:
        assert np.allclose(got.sum(axis=1), 1.0, atol=cols * 6e-8 + 1e-6)


@pytest.mark.parametrize("rows,cols", [(2600, 8192), (4100, 4096), (8200, 2048)])
@pytest.mark.parametrize("log,scale", [(False, 1.0), (True, 1.0), (False, 0.125)])
def test_softmax_streamed_rows(engine, rows, cols, log, scale):
    # Inputs past the streaming threshold (2 x 4 x rows x cols >= 128 MiB):
    # nontemporal accesses.  Rows are independent and fold alike at any size,
    # so a subset of rows (cached accesses) has the same bits.
    x = rnd(rows, cols, scale=3.0)
    x[1, 5] = np.nan      # a NaN makes its whole row NaN
    x[2, 7] = np.inf      # so does +inf (inf - inf)
    x[3, :] = -np.inf     # and a row of -inf
    full = engine.download(engine.softmax_rows(engine.upload(x), log=log, scale=scale))
    sel = np.r_[0:40, rows // 2:rows // 2 + 40, rows - 40:rows]
    part = engine.download(engine.softmax_rows(engine.upload(np.ascontiguousarray(x[sel])), log=log, scale=scale))
    finite = np.isfinite(x[sel]).all(axis=1)
    same_bits(full[sel][finite], part[finite])
    assert np.isnan(full[1:4]).all()
    want = orc.softmax_rows(x[sel], log=log, scale=scale)
    close(full[sel], want, rtol=1e-5, atol=1e-6 if log else 1e-12)


def test_softmax_masked_scaled(engine):
    R, C = 36, 200
    x = rnd(R, C)
    mask = (RNG.random((12, C)) < 0.4).astype(np.uint32)
    mask[3, :] = 1  # a fully masked row gives zeros
    a, m = engine.upload(x), engine.upload_bool(mask)
    got = engine.download(engine.softmax_rows(a, m, scale=0.125))
    want = orc.softmax_rows(x, mask=mask, scale=0.125)
    close(got, want, rtol=1e-5, atol=1e-12)
    assert np.all(got[3] == 0.0) and np.all(got[15] == 0.0)


@pytest.mark.parametrize("cols", [4, 36, 512, 1000, 1024])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_masked_vector_rows(engine, cols, log):
    # F32 rows of a multiple of 4 up to 1024 columns with a mask: float4 loads.
    R = 24
    x = rnd(R, cols, scale=2.0)
    mask = (RNG.random((8, cols)) < 0.3).astype(np.uint32)
    mask[5, :] = 1            # rows 5, 13, 21 fully masked
    x[2, 1] = np.nan          # row 2: NaN unless masked
    mask[2, 1] = 0
    got = engine.download(engine.softmax_rows(engine.upload(x), engine.upload_bool(mask), scale=0.25, log=log))
    want = orc.softmax_rows(x, mask=mask, scale=0.25, log=log)
    close(got, want, rtol=1e-5, atol=1e-6 if log else 1e-12)
    assert np.isnan(got[2]).all()


def test_softmax_shift_invariance(engine):
    x = rnd(8, 512)
    a, b = engine.upload(x), engine.upload(x + np.float32(4.0))
    close(engine.download(engine.softmax_rows(a)), engine.download(engine.softmax_rows(b)), rtol=5e-6, atol=1e-12)


# ----------------------------------------------------------------------- norms
@pytest.mark.parametrize("rows,cols", [(50, 64), (50, 576), (50, 1000), (8193, 576)])  # 8193: two rows a wavefront
def test_rms_norm(engine, rows, cols):
    x, g = rnd(rows, cols), rnd(1, cols)
    a, gb = engine.upload(x), engine.upload(g)
    close(engine.download(engine.rms_norm(a, gb, 1e-5)), orc.rms_norm(x, g, 1e-5), rtol=1e-5, atol=1e-7)
    close(engine.download(engine.rms_norm(a, 0, 1e-5)), orc.rms_norm(x, None, 1e-5), rtol=1e-5, atol=1e-7)


def test_layer_norm(engine):
    x, g, b = rnd(64, 256), rnd(1, 256), rnd(1, 256)
    ids = [engine.upload(v) for v in (x, g, b)]
    close(engine.download(engine.layer_norm(*ids, eps=1e-5)), orc.layer_norm(x, g, b, 1e-5), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,cols", [(2048, 256), (37, 1000), (5, 64)])
@pytest.mark.parametrize("res", [False, True])
def test_layer_norm_backward(engine, rows, cols, res):
    x = rnd(rows, cols, scale=2.0) + np.float32(0.3)
    g, dy = rnd(1, cols) + np.float32(1.0), rnd(rows, cols)
    dres = rnd(rows, cols) if res else None
    ids = engine.layer_norm_backward(engine.upload(x), engine.upload(g), engine.upload(dy),
                                     engine.upload(dres) if res else 0, 1e-5)
    dx, dg, db = (engine.download(i) for i in ids)
    wx, wg, wb = orc.layer_norm_backward(x, g, dy, dres, 1e-5)
    # Cancellation inside dx and sums over all rows for dgamma / dbeta: bound
    # the error by the magnitudes of the terms.
    den = np.sqrt(x.astype(np.float64).var(1, keepdims=True) + 1e-5)
    close(dx, wx, rtol=1e-5, atol=2e-6 * np.abs(dy * g / den).max())
    xh = (x - x.astype(np.float64).mean(1, keepdims=True)) / den
    close(dg, wg, rtol=1e-5, atol=2e-7 * np.abs(dy * xh).sum(0).max())
    close(db, wb, rtol=1e-5, atol=2e-7 * np.abs(dy).sum(0).max())


def test_softmax_backward(engine):
    x, dp = rnd(512, 128, scale=2.0), rnd(512, 128)
    p = orc.softmax_rows(x, scale=0.125)
    got = engine.download(engine.softmax_backward(engine.upload(p), engine.upload(dp), 0.125))
    want = orc.softmax_backward(p, dp, 0.125)
    close(got, want, rtol=1e-5, atol=1e-6 * 0.125 * np.abs(p * dp).sum(1, keepdims=True).max())


def test_sgd_update_in_place_bits(engine):
    sizes = [(256, 256), (1, 256), (1, 7), (33, 5), (1024, 1024)] * 11  # 55 parameters: two launches
    ps = [rnd(*s) for s in sizes]
    gs = [rnd(*s) for s in sizes]
    pid = [engine.upload(p) for p in ps]
    gid = [engine.upload(g.reshape(-1, 1) if i % 3 == 0 else g) for i, g in enumerate(gs)]  # any folding
    lr = np.float32(0.05)
    engine.sgd_update(pid, gid, float(lr))
    for i, (p, g) in enumerate(zip(ps, gs)):
        same_bits(engine.download(pid[i]), (p - g * lr).astype(np.float32))
    with pytest.raises(miburn.MiError):
        engine.sgd_update([pid[0]], [pid[0]], 0.1)
    with pytest.raises(miburn.MiError):
        engine.sgd_update([pid[0]], [gid[1]], 0.1)  # 65536 parameters, 256 gradients


# ------------------------------------------------------------------ products
def mm_tol(a, b, ta, tb, rel):
    aa = np.abs(a.T if ta else a).astype(np.float64)
    bb = np.abs(b.T if tb else b).astype(np.float64)
    return rel * (aa @ bb)


@pytest.fixture(params=["fast", "accurate"])
def mode(request, engine):
    """Run the test in each matmul mode, restoring the default after."""
    engine.set_matmul_mode(miburn.MATMUL_FAST if request.param == "fast" else miburn.MATMUL_ACCURATE)
    yield request.param
    engine.set_matmul_mode(miburn.MATMUL_FAST)


def test_matmul_mode_api(engine):
    assert engine.matmul_mode() == miburn.MATMUL_FAST  # the reference's default is its fast mode
    engine.set_matmul_mode(miburn.MATMUL_ACCURATE)
    assert engine.matmul_mode() == miburn.MATMUL_ACCURATE
    with pytest.raises(miburn.MiError) as e:
        engine.set_matmul_mode(2)  # an exact (k-ordered) mode is not offered
    assert e.value.kind == "UNSUPPORTED"
    engine.set_matmul_mode(miburn.MATMUL_FAST)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("mnk", [(64, 128, 784), (64, 10, 128), (100, 70, 33), (256, 256, 256), (1, 576, 1536),
                                 (513, 129, 77), (2048, 256, 256), (1024, 1024, 64), (2048, 2048, 2048),
                                 (2000, 2100, 2050)])
def test_matmul_f32(engine, mode, ta, tb, mnk):
    m, n, k = mnk
    a = rnd(k, m) if ta else rnd(m, k)
    b = rnd(n, k) if tb else rnd(k, n)
    ia, ib = engine.upload(a), engine.upload(b)
    got = engine.download(engine.matmul_dram(ia, ta, ib, tb))
    want = orc.matmul(a, b, ta, tb, threads=16)
    assert got.shape == (m, n)
    assert np.all(np.abs(got - want) <= mm_tol(a, b, ta, tb, 1e-5) + 1e-30)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("mnk", [(512, 512, 512), (256, 512, 192), (128, 64, 64), (100, 70, 33), (1, 576, 1536),
                                 (2048, 256, 1024), (1024, 1024, 1024), (768, 768, 2048), (384, 1024, 2048),
                                 (512, 512, 4096)])
def test_matmul_bf16(engine, ta, tb, mnk):
    m, n, k = mnk
    a = rnd(k, m) if ta else rnd(m, k)
    b = rnd(n, k) if tb else rnd(k, n)
    ab, bb = orc.to_bf16(a), orc.to_bf16(b)
    ia, ib = engine.upload_bf16(ab), engine.upload_bf16(bb)
    got = engine.download(engine.matmul_dram(ia, ta, ib, tb))
    af, bf = orc.from_bf16(ab), orc.from_bf16(bb)
    # Against the oracle fed the same BF16 values: exact products, F32 accumulation.
    assert np.all(np.abs(got - orc.matmul(af, bf, ta, tb)) <= mm_tol(af, bf, ta, tb, 1e-5) + 1e-30)
    # Against the unrounded F32 product: the north star's rel 2e-2 (normwise).
    assert np.all(np.abs(got - orc.matmul(a, b, ta, tb)) <= mm_tol(a, b, ta, tb, 2e-2))


def test_matmul_bf16_out(engine):
    a, b = rnd(256, 128), rnd(128, 384)
    ab, bb = orc.to_bf16(a), orc.to_bf16(b)
    out = engine.matmul_dram(engine.upload_bf16(ab), False, engine.upload_bf16(bb), False, BF16)
    got = miburn.bf16_to_f32(engine.download(out))
    af, bf = orc.from_bf16(ab), orc.from_bf16(bb)
    want = orc.matmul(af, bf)
    # One BF16 rounding (half an ulp, 2^-9 relative) of an F32 sum within the normwise bound.
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + mm_tol(af, bf, False, False, 1e-5))


@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("mnk", [(64, 48, 96), (512, 576, 576), (300, 200, 136), (2048, 2048, 2048), (512, 192, 576),
                                 (256, 1536, 576), (512, 576, 1536)])
def test_matmul_mixed_f32_bf16(engine, mode, tb, mnk):
    m, n, k = mnk
    a, b = rnd(m, k), orc.to_bf16(rnd(n, k) if tb else rnd(k, n))
    got = engine.download(engine.matmul_dram(engine.upload(a), False, engine.upload_bf16(b), tb))
    bf = orc.from_bf16(b)
    assert np.all(np.abs(got - orc.matmul(a, bf, False, tb, threads=16)) <= mm_tol(a, bf, False, tb, 1e-5) + 1e-30)


@pytest.mark.parametrize("mnk", [(4096, 2048, 576), (8192, 960, 576), (16384, 576, 576), (4096, 3072, 1536)])
def test_matmul_mixed_stacked_split(engine, mode, mnk):
    """F32 activations x BF16 weights [n, k] at the prefill's sizes: in the
    fast mode the activations are split once into BF16 hi | lo parts and the
    product runs on the direct BF16 kernel with the weight's k wrapping (width
    960 takes its edge tiles, 576 at 16384 rows its 256 x 192 tiles).  Random operands within the F32 bound;
    small integers bit for bit; a linear layer's bias and residual too."""
    m, n, k = mnk
    a, b = rnd(m, k), orc.to_bf16(rnd(n, k))
    bf = orc.from_bf16(b)
    ib = engine.upload_bf16(b)
    got = engine.download(engine.matmul_dram(engine.upload(a), False, ib, True))
    assert np.all(np.abs(got - orc.matmul(a, bf, False, True, threads=16)) <= mm_tol(a, bf, False, True, 1e-5) + 1e-30)
    ai = RNG.integers(-8, 9, (m, k)).astype(np.float32)
    bi = orc.to_bf16(RNG.integers(-8, 9, (n, k)).astype(np.float32))
    got = engine.download(engine.matmul_dram(engine.upload(ai), False, engine.upload_bf16(bi), True))
    same_bits(got, (ai.astype(np.float64) @ orc.from_bf16(bi).astype(np.float64).T).astype(np.float32))
    bias, res = rnd(1, n), rnd(m, n)
    got = engine.download(engine.linear(engine.upload(ai), engine.upload_bf16(bi), True, engine.upload(bias),
                                        engine.upload(res)))
    want = (ai.astype(np.float64) @ orc.from_bf16(bi).astype(np.float64).T).astype(np.float32)
    same_bits(got, (res + (want + bias)).astype(np.float32))


@pytest.mark.parametrize("mnk", [(4096, 576, 1536), (16384, 960, 576), (16384, 576, 576)])
def test_matmul_bf16_edge_tiles(engine, mnk):
    """BF16 x BF16 [n, k] products whose width the tiles do not divide (the
    performance contract's prefill products): the direct kernel's edge tiles
    (128 x 128 at 4096 rows, 256 x 256 at 16384; 576 wide there, 256 x 192
    tiles that divide it), small integers bit for bit
    against float64, random operands within the F32 bound of the oracle fed
    the same BF16 values, and a linear layer's residual bit for bit."""
    m, n, k = mnk
    ai = orc.to_bf16(RNG.integers(-8, 9, (m, k)).astype(np.float32))
    bi = orc.to_bf16(RNG.integers(-8, 9, (n, k)).astype(np.float32))
    got = engine.download(engine.matmul_dram(engine.upload_bf16(ai), False, engine.upload_bf16(bi), True))
    want = (orc.from_bf16(ai).astype(np.float64) @ orc.from_bf16(bi).astype(np.float64).T).astype(np.float32)
    same_bits(got, want)
    res = rnd(m, n)
    got = engine.download(engine.linear(engine.upload_bf16(ai), engine.upload_bf16(bi), True, 0, engine.upload(res)))
    same_bits(got, (res + want).astype(np.float32))
    a, b = orc.to_bf16(rnd(m, k)), orc.to_bf16(rnd(n, k))
    af, bf = orc.from_bf16(a), orc.from_bf16(b)
    got = engine.download(engine.matmul_dram(engine.upload_bf16(a), False, engine.upload_bf16(b), True))
    assert np.all(np.abs(got - orc.matmul(af, bf, False, True, threads=16)) <= mm_tol(af, bf, False, True, 1e-5) + 1e-30)


def test_matmul_fast_split_keeps_large_finite_values(engine, mode):
    """Values near FLT_MAX stay finite through the split (the BF16 head of a
    value above the largest BF16 would round to infinity, so it is truncated).
    Its remainder is then up to 2^-8 |a|: the split's error reaches 2^-17 |a|
    and the dropped lo x lo term 2^-17 |a||b|, hence the looser bound for this
    case (measured 2.4e-5).  2048^3 takes the split."""
    a = rnd(2048, 2048)
    a[3, 5] = np.float32(3.4e38)
    a[7, 1] = np.float32(-3.39e38)
    b = (rnd(2048, 2048) * np.float32(1e-3)).astype(np.float32)
    got = engine.download(engine.matmul_dram(engine.upload(a), False, engine.upload(b), False))
    want = orc.matmul(a, b, threads=16)
    assert np.all(np.isfinite(got))
    ratio = np.abs(got - want) / (mm_tol(a, b, False, False, 1.0) + 1e-30)
    worst = np.unravel_index(np.argmax(ratio), ratio.shape)
    assert ratio.max() <= 5e-5, (ratio.max(), worst, got[worst], want[worst])


@pytest.mark.parametrize("dtype,n", [("f32", 1024), ("f32", 2048), ("bf16", 1024), ("bf16", 2048), ("bf16", 4096)])
def test_matmul_integer_exact_big(engine, mode, dtype, n):
    """The reference's step11 trick: small-integer operands make every
    summation order exact, so the device must equal the float64 product bit
    for bit -- for each kernel the shape selects (bf16: 64x64 tiles at 1024,
    128x128 direct-to-LDS at 2048, 256x256 direct-to-LDS at 4096)."""
    a = RNG.integers(-4, 5, (n, n)).astype(np.float32)
    b = RNG.integers(-4, 5, (n, n)).astype(np.float32)
    if dtype == "bf16":
        ia, ib = engine.upload_bf16(orc.to_bf16(a)), engine.upload_bf16(orc.to_bf16(b))
    else:
        ia, ib = engine.upload(a), engine.upload(b)
    for ta, tb in ((False, False), (False, True), (True, False), (True, True)):
        got = engine.download(engine.matmul_dram(ia, ta, ib, tb))
        want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
        same_bits(got, want.astype(np.float32))


@pytest.mark.parametrize("bcast", ["none", "a", "b"])
def test_matmul_batched(engine, bcast):
    batch, m, k, n = 6, 64, 48, 80
    a = rnd(1 if bcast == "a" else batch, m, k)
    b = rnd(1 if bcast == "b" else batch, k, n)
    ia, ib = engine.upload(a.reshape(-1, k)), engine.upload(b.reshape(-1, n))
    got = engine.download(engine.matmul_dram_batched(ia, False, ib, False, batch, m, k, n)).reshape(batch, m, n)
    for z in range(batch):
        az, bz = a[0 if bcast == "a" else z], b[0 if bcast == "b" else z]
        assert np.all(np.abs(got[z] - orc.matmul(az, bz)) <= mm_tol(az, bz, False, False, 1e-5) + 1e-30)


def test_matmul_batched_bf16_transposed(engine):
    batch, m, k, n = 16, 128, 64, 128
    a = orc.to_bf16(rnd(batch, m, k))
    b = orc.to_bf16(rnd(batch, n, k))  # B transposed: items [n, k]
    got = engine.download(engine.matmul_dram_batched(engine.upload_bf16(a.reshape(-1, k)), False,
                                                     engine.upload_bf16(b.reshape(-1, k)), True, batch, m, k, n))
    got = got.reshape(batch, m, n)
    af, bf = orc.from_bf16(a), orc.from_bf16(b)
    for z in range(batch):
        want = orc.matmul(af[z], bf[z], False, True)
        assert np.all(np.abs(got[z] - want) <= mm_tol(af[z], bf[z], False, True, 1e-5) + 1e-30)


@pytest.mark.parametrize("tb", [False, True])
def test_matmul_batched_bf16_integer_exact_256_tiles(engine, tb):
    """12 items of 1024^2 give 192 tiles of 256x256: the direct kernel's
    batched path, exact with small-integer operands."""
    batch, m, k, n = 12, 1024, 1024, 1024
    a = RNG.integers(-3, 4, (batch, m, k)).astype(np.float32)
    b = RNG.integers(-3, 4, (batch, n, k) if tb else (batch, k, n)).astype(np.float32)
    ia = engine.upload_bf16(orc.to_bf16(a.reshape(-1, k)))
    ib = engine.upload_bf16(orc.to_bf16(b.reshape(-1, b.shape[-1])))
    got = engine.download(engine.matmul_dram_batched(ia, False, ib, tb, batch, m, k, n)).reshape(batch, m, n)
    bb = b.transpose(0, 2, 1) if tb else b
    want = np.matmul(a.astype(np.float64), bb.astype(np.float64)).astype(np.float32)
    same_bits(got, want)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)])
@pytest.mark.parametrize("mnk", [(512, 512, 512), (768, 768, 2048), (384, 1024, 2048)])
def test_matmul_bf16_integer_exact_few_tiles(engine, ta, tb, mnk):
    """16 to 36 tiles of 128 x 128: the pipelined kernel over the whole k
    loop (no split), exact with small-integer operands."""
    m, n, k = mnk
    a = RNG.integers(-3, 4, (k, m) if ta else (m, k)).astype(np.float32)
    b = RNG.integers(-3, 4, (n, k) if tb else (k, n)).astype(np.float32)
    got = engine.download(engine.matmul_dram(engine.upload_bf16(orc.to_bf16(a)), ta,
                                             engine.upload_bf16(orc.to_bf16(b)), tb))
    aa, bb = (a.T if ta else a), (b.T if tb else b)
    same_bits(got, (aa.astype(np.float64) @ bb.astype(np.float64)).astype(np.float32))


def test_matmul_bf16_out_direct_kernel(engine):
    a, b = rnd(4096, 512), rnd(512, 4096)
    ab, bb = orc.to_bf16(a), orc.to_bf16(b)
    out = engine.matmul_dram(engine.upload_bf16(ab), False, engine.upload_bf16(bb), False, BF16)
    got = miburn.bf16_to_f32(engine.download(out))
    af, bf = orc.from_bf16(ab), orc.from_bf16(bb)
    want = af.astype(np.float64) @ bf.astype(np.float64)
    tol = 2.0 ** -8 * np.abs(want) + 1e-5 * (np.abs(af).astype(np.float64) @ np.abs(bf).astype(np.float64))
    assert np.all(np.abs(got - want) <= tol)


def test_matmul_shape_error(engine):
    ia, ib = engine.upload(rnd(4, 5)), engine.upload(rnd(6, 7))
    with pytest.raises(miburn.MiError) as e:
        engine.matmul_dram(ia, False, ib, False)
    assert e.value.kind == "ARG"


# -------------------------------------------------------------------- indexing
def special_table(rows, cols):
    t = rnd(rows, cols)
    flat = t.ravel()
    flat[:6] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40]
    bits = t.view(np.uint32).copy()
    bits.ravel()[6] = 0x7FC0BEEF  # a NaN payload
    return bits


def test_select_rows_bits(engine):
    V, D = 1000, 576
    bits = special_table(V, D)
    idx = RNG.integers(0, V, (3, 700)).astype(np.int32)
    idx[0, 0] = 0
    t = engine.upload_bits(bits, F32)
    out = engine.select_rows(t, engine.upload_i32(idx))
    same_bits(engine.download(out).view(np.uint32), orc.select_rows(bits, idx))


@pytest.mark.parametrize("D", [576, 13, 2])
def test_select_rows_widths(engine, D):
    bits = RNG.integers(0, 2**32, (77, D), dtype=np.uint64).astype(np.uint32)
    idx = RNG.integers(0, 77, 300).astype(np.int32)
    got = engine.download(engine.select_rows(engine.upload_bits(bits, I32), engine.upload_i32(idx)))
    same_bits(got.view(np.uint32), orc.select_rows(bits, idx))


def test_select_rows_bf16(engine):
    bits = RNG.integers(0, 2**16, (50, 64), dtype=np.uint32).astype(np.uint16)
    idx = RNG.integers(0, 50, 99).astype(np.int32)
    got = engine.download(engine.select_rows(engine.upload_bf16(bits), engine.upload_i32(idx)))
    assert np.array_equal(got, bits[idx])


def test_select_rows_out_of_range_is_domain(engine):
    engine.sync()
    t = engine.upload(rnd(10, 8))
    idx = engine.upload_i32(np.array([1, 2, 10], np.int32))
    engine.select_rows(t, idx)  # submitted: the failure is deferred
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    engine.sync()  # reported once, then cleared


def test_pick_and_scatter_add_columns(engine):
    R, C = 2048, 8192 // 8
    bits = special_table(R, C)
    idx = RNG.integers(0, C, R).astype(np.int32)
    x = engine.upload_bits(bits, F32)
    ix = engine.upload_i32(idx.reshape(R, 1))
    same_bits(engine.download(engine.pick_columns(x, ix)).view(np.uint32), orc.pick_columns(bits, idx))
    xf = rnd(R, C)
    v = rnd(R, 1)
    got = engine.download(engine.scatter_add_columns(engine.upload(xf), ix, engine.upload(v)))
    same_bits(got, orc.scatter_add_columns(xf, idx, v))


@pytest.mark.parametrize("V,D,n,hot", [(300, 64, 2048, 40),  # one-block sort
                                       (49152, 64, 20000, 49152),  # chunk sorts and merge passes above 8192 ids
                                       (1000, 576, 9000, 30),
                                       (49152, 16, 70001, 700)])   # four merge passes, a partial last run
def test_select_add_rows_duplicates_in_order(engine, V, D, n, hot):
    t = rnd(V, D)
    idx = RNG.integers(0, hot, n).astype(np.int32)  # duplicates (many when hot is small)
    val = rnd(n, D)
    got = engine.download(engine.select_add_rows(engine.upload(t), engine.upload_i32(idx), engine.upload(val)))
    same_bits(got, orc.select_add_rows(t, idx, val))


@pytest.mark.parametrize("cols", [3072, 1000])  # block-per-row and wave-per-row kernels
def test_argmax_first_and_nan(engine, cols):
    x = rnd(40, cols)
    x[1, 5] = x[1, 9] = 100.0  # tie: the first wins
    x[2, 7] = np.nan  # NaN above every number
    x[2, 3] = np.inf
    x[3, :] = 0.0
    x[3, 4] = -0.0
    got = engine.download(engine.argmax_row(engine.upload(x)))
    assert np.array_equal(got, orc.argmax_rows(x))
    assert got[1, 0] == 5 and got[2, 0] == 7 and got[3, 0] == 0


@pytest.mark.parametrize("rows", [32, 100])  # column chunks and their fold
def test_argmax_vocab_rows(engine, rows):
    x = rnd(rows, 49152)
    x[rows - 1, 30000] = x[rows - 1, 20000] = 60.0  # a tie across chunks: the first wins
    x[0, 45000] = np.nan
    got = engine.download(engine.argmax_row(engine.upload(x)))
    assert np.array_equal(got, orc.argmax_rows(x))
    assert got[rows - 1, 0] == 20000 and got[0, 0] == 45000


@pytest.mark.parametrize("n,cols", [(1, 576), (32, 576), (5, 12)])
def test_select_rows_as_equals_gather_then_cast(engine, n, cols):
    """The gather with its cast: BF16 rows widened in one launch (widths of
    8s), other pairs through the two ops -- bit for bit select_rows then
    cast either way."""
    tb = orc.to_bf16(rnd(300, cols))
    idx = RNG.integers(0, 300, n).astype(np.int32)
    it, ii = engine.upload_bf16(tb), engine.upload_i32(idx)
    want = engine.download(engine.cast_float(engine.select_rows(it, ii), miburn.F32))
    got = engine.download(engine.select_rows_as(it, ii, miburn.F32))
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got, orc.from_bf16(tb[idx]))
    tf = rnd(300, cols)
    got = engine.download(engine.select_rows_as(engine.upload(tf), ii, miburn.BF16))
    assert np.array_equal(got, orc.to_bf16(tf[idx]))


def test_select_rows_as_out_of_range_is_domain(engine):
    engine.sync()
    it = engine.upload_bf16(orc.to_bf16(rnd(10, 64)))
    engine.select_rows_as(it, engine.upload_i32(np.array([3, 10], np.int32)), miburn.F32)  # deferred
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    engine.sync()


def test_argmax_bf16_long_rows(engine):
    x = rnd(8, 49152)
    x[2, 40000] = x[2, 40001] = 50.0
    xb = orc.to_bf16(x)  # ties from the rounding: the first wins
    got = engine.download(engine.argmax_row(engine.upload_bf16(xb)))
    assert np.array_equal(got, orc.argmax_rows(orc.from_bf16(xb)))
    assert got[2, 0] == 40000


# ------------------------------------------------------------------ attention
def attention_ref(q, kc, vc, batch, t, heads, kvh, pos0, scale):
    """float64 causal GQA over the cache (crates/burn-tt/src/ops.rs:4520-4595)."""
    D = kc.shape[1]
    G = heads // kvh
    maxc = kc.shape[0] // (batch * kvh)
    K = kc.reshape(batch, kvh, maxc, D).astype(np.float64)
    V = vc.reshape(batch, kvh, maxc, D).astype(np.float64)
    Q = q.reshape(batch, t, heads, D).astype(np.float64)
    out = np.zeros((batch, t, heads, D))
    for b in range(batch):
        for p in range(t):
            n = pos0 + p + 1
            for h in range(heads):
                s = K[b, h // G, :n] @ Q[b, p, h] * scale
                w = np.exp(s - s.max())
                out[b, p, h] = (w / w.sum()) @ V[b, h // G, :n]
    return out.reshape(batch * t, heads * D)


@pytest.mark.parametrize("batch,t,heads,kvh,D,pos0,maxc", [
    (1, 1, 9, 3, 64, 639, 640),      # SmolLM2 decode at a long context: many key chunks
    (1, 1, 9, 3, 64, 0, 640),        # first position: one key
    (32, 1, 9, 3, 64, 200, 640),     # batch 32 decode
    (2, 5, 4, 2, 16, 7, 64),         # several new positions, causal inside the chunk
    (3, 16, 8, 1, 128, 30, 64),      # 8 query heads per kv head
    (2, 3, 4, 4, 32, 2000, 2304),    # no grouping, context over one chunk's limit
    (1, 2, 6, 2, 64, 0, 8),          # whole cache, one chunk, direct write
    (1, 512, 9, 3, 64, 0, 640),      # a 512-token prompt at batch 1 (prefill takes the fused kernel)
    (4, 100, 9, 3, 64, 28, 160),     # prompts of 4 sequences after 28 cached positions
    (1, 300, 2, 1, 64, 0, 300),      # two key chunks: early positions' second chunk is empty
    (1, 1100, 9, 3, 64, 0, 1100),    # a prompt past one chunk at SmolLM2's heads: empty chunks too
    (1, 63, 9, 3, 64, 0, 64),        # just below the matrix-core kernel: the chunk kernel
    (32, 96, 9, 3, 64, 32, 160),     # 64+ positions filling the chip: the matrix-core (flash) kernel
    (48, 70, 8, 1, 64, 5, 80),       # flash: 8 heads a group, a partial last query block
    (64, 64, 2, 2, 64, 0, 64),       # flash: no grouping, the whole cache
])
def test_attention_rows(engine, batch, t, heads, kvh, D, pos0, maxc):
    q = rnd(batch * t, heads * D)
    kc = rnd(batch * kvh * maxc, D)
    vc = rnd(batch * kvh * maxc, D)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    got = engine.download(engine.attention_rows(engine.upload(q), engine.upload(kc), engine.upload(vc), batch, t,
                                                heads, kvh, pos0, scale))
    want = attention_ref(q, kc, vc, batch, t, heads, kvh, pos0, scale)
    assert got.shape == want.shape
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max()), np.abs(got - want).max()


@pytest.mark.parametrize("batch,t,heads,kvh,D,pos0,maxc", [
    (1, 1, 9, 3, 64, 639, 640),      # decode, many key chunks
    (32, 1, 9, 3, 64, 200, 640),     # batch 32 decode
    (2, 5, 4, 2, 16, 7, 64),         # 16-wide heads
    (3, 16, 8, 1, 128, 30, 64),      # 128-wide heads, 8 a group
    (1, 512, 9, 3, 64, 0, 640),      # a 512-token prompt at batch 1
    (32, 96, 9, 3, 64, 32, 160),     # the matrix-core (flash) kernel
    (48, 70, 8, 1, 64, 5, 80),       # flash, a partial last query block
])
def test_attention_rows_bf16_caches(engine, batch, t, heads, kvh, D, pos0, maxc):
    # The performance contract's BF16 caches: widened exactly as loaded, so
    # the float64 reference on the BF16 values holds to the F32 bound.
    q = rnd(batch * t, heads * D)
    kb = orc.to_bf16(rnd(batch * kvh * maxc, D))
    vb = orc.to_bf16(rnd(batch * kvh * maxc, D))
    scale = float(np.float32(1.0 / np.sqrt(D)))
    got = engine.download(engine.attention_rows(engine.upload(q), engine.upload_bf16(kb), engine.upload_bf16(vb),
                                                batch, t, heads, kvh, pos0, scale))
    want = attention_ref(q, orc.from_bf16(kb), orc.from_bf16(vb), batch, t, heads, kvh, pos0, scale)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max()), np.abs(got - want).max()


@pytest.mark.parametrize("batch,t,heads,kvh,D,pos0,span,maxc", [
    (1, 1, 9, 3, 64, 575, 576, 640),    # decode: span = the attended length
    (1, 1, 9, 3, 64, 513, 576, 640),    # span past the context: trailing chunks empty
    (32, 1, 9, 3, 64, 100, 128, 640),   # batch 32
    (2, 5, 4, 2, 16, 7, 64, 64),        # several new positions
    (1, 1, 9, 3, 64, 0, 64, 64),        # the first position
])
def test_attention_rows_at_device_position(engine, batch, t, heads, kvh, D, pos0, span, maxc):
    # Planned for `span`: within the F32 bound of the float64 reference; the
    # device-held position gives the immediate one's bits.
    q = rnd(batch * t, heads * D)
    kc = rnd(batch * kvh * maxc, D)
    vc = rnd(batch * kvh * maxc, D)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    iq, ik, iv = engine.upload(q), engine.upload(kc), engine.upload(vc)
    imm = engine.download(engine.attention_rows_at(iq, ik, iv, batch, t, heads, kvh, 0, pos0, span, scale))
    pos = engine.upload_bits(np.array([[pos0]], np.int32), I32)
    dev = engine.download(engine.attention_rows_at(iq, ik, iv, batch, t, heads, kvh, pos, 0, span, scale))
    same_bits(dev, imm)
    want = attention_ref(q, kc, vc, batch, t, heads, kvh, pos0, scale)
    assert np.abs(imm - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    if span == pos0 + t:  # the plain call's plan
        same_bits(imm, engine.download(engine.attention_rows(iq, ik, iv, batch, t, heads, kvh, pos0, scale)))


def test_attention_rows_at_errors(engine):
    q = engine.upload(rnd(1, 2 * 64))
    k = engine.upload(rnd(64, 64))
    with pytest.raises(miburn.MiError) as e:
        engine.attention_rows_at(q, k, k, 1, 1, 2, 1, 0, 60, 32, 0.125)  # span below pos0 + t
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:
        engine.attention_rows_at(q, k, k, 1, 1, 2, 1, 0, 0, 65, 0.125)  # span beyond the cache
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:  # a position buffer that is not [1, 1] I32
        engine.attention_rows_at(q, k, k, 1, 1, 2, 1, engine.upload(rnd(1, 1)), 0, 32, 0.125)
    assert e.value.kind == "ARG"
    # A device position past the span: attended from 0 (in bounds), reported at the next wait.
    bad = engine.upload_bits(np.array([[40]], np.int32), I32)
    engine.attention_rows_at(q, k, k, 1, 1, 2, 1, bad, 0, 32, 0.125)
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    engine.sync()


def test_attention_rows_mixed_caches_refused(engine):
    q = engine.upload(rnd(1, 2 * 64))
    kf = engine.upload(rnd(8, 64))
    kb = engine.upload_bf16(orc.to_bf16(rnd(8, 64)))
    with pytest.raises(miburn.MiError) as e:
        engine.attention_rows(q, kf, kb, 1, 1, 2, 1, 0, 0.125)
    assert e.value.kind == "ARG"


# ------------------------------------------------------ fused decode projections
def decode_inputs(M, K, N):
    x = rnd(M, K)
    g = rnd(1, K) + np.float32(1.0)
    w = orc.to_bf16(rnd(N, K, scale=0.05))
    return x, g, w


def rms_ref(x, g, eps):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + eps) * g.astype(np.float64)


@pytest.mark.parametrize("M", [1, 2, 3, 8, 9, 17, 32])  # one GEMV wavefront per row pair up to 6 rows; matrix cores above
@pytest.mark.parametrize("N,K", [(576, 576), (577, 576), (576, 1536), (100, 2056), (16400, 576)])
def test_norm_matvec_residual(engine, M, N, K):
    # k 2056 is not a multiple of 16: the GEMV up to 8 rows, the LDS-staged form above.
    eps = 1e-5
    x, g, wb = decode_inputs(M, K, N)
    res = rnd(M, N)
    w = orc.from_bf16(wb).astype(np.float64)
    got = engine.download(engine.norm_matvec(engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb),
                                             engine.upload(res)))
    xn = rms_ref(x, g, eps)
    want = res + xn @ w.T
    assert np.abs(got - want).max() <= 1e-5 * (np.abs(xn) @ np.abs(w).T).max() + 1e-6 * np.abs(res).max()
    # Without a gain: the plain product.
    got = engine.download(engine.norm_matvec(engine.upload(x), 0, 0.0, engine.upload_bf16(wb)))
    assert np.abs(got - x @ w.T).max() <= 1e-5 * (np.abs(x) @ np.abs(w).T).max()


@pytest.mark.parametrize("N,K", [(30001, 576), (30000, 1024), (29200, 600)])
def test_norm_matvec_streamed_head(engine, N, K):
    # A weight of 32 MiB or more is streamed; one row takes the head kernel (4
    # pairs a wavefront, the row and gain read once for them), two rows the
    # plain streamed kernel: row 0's products are the same bits either way,
    # with and without a gain and a residual; odd N leaves a lone last row.
    eps = 1e-5
    x, g, wb = decode_inputs(2, K, N)
    res = rnd(2, N)
    w = engine.upload_bf16(wb)
    for gamma, r in ((engine.upload(g), 0), (0, engine.upload(res))):
        one = engine.download(engine.norm_matvec(engine.upload(x[:1]), gamma, eps, w,
                                                 engine.upload(res[:1]) if r else 0))
        two = engine.download(engine.norm_matvec(engine.upload(x), gamma, eps, w, r))
        same_bits(one[0], two[0])
    xn = rms_ref(x[:1], g, eps)
    w64 = orc.from_bf16(wb).astype(np.float64)
    got = engine.download(engine.norm_matvec(engine.upload(x[:1]), engine.upload(g), eps, w))
    assert np.abs(got - xn @ w64.T).max() <= 1e-5 * (np.abs(xn) @ np.abs(w64).T).max()


@pytest.mark.parametrize("N,K,M", [(30001, 576, 1), (30000, 1024, 1), (30001, 576, 2)])
def test_norm_matvec_argmax(engine, N, K, M):
    # The head and the greedy pick in one call: the logits are norm_matvec's
    # bits and the ids argmax_rows' pick of them -- a planted tie of two equal
    # largest rows picks the first, NaN rows the first NaN.  One row takes the
    # fused launch (the head's blocks fold their logits), two the two calls.
    eps = 1e-5
    x, g, wb = decode_inputs(M, K, N)
    xd, gd = engine.upload(x), engine.upload(g)
    y = rms_ref(x, g, eps) @ orc.from_bf16(wb).astype(np.float64).T
    top = int(np.argmax(y[0]))
    tie = wb.copy()
    tie[[17, N - 2]] = orc.to_bf16(orc.from_bf16(wb[top]) * np.float32(4.0))
    nan = wb.copy()
    nan[[20000, 25000]] = 0x7FC0
    for w, want_id in ((wb, None), (tie, 17), (nan, 20000)):
        wd = engine.upload_bf16(w)
        lg, ids = engine.norm_matvec_argmax(xd, gd, eps, wd)
        ref = engine.norm_matvec(xd, gd, eps, wd)
        same_bits(engine.download(lg), engine.download(ref))
        got = engine.download(ids)
        assert got.shape == (M, 1)
        assert np.array_equal(got, engine.download(engine.argmax_row(ref)))
        if want_id is not None:
            assert got[0, 0] == want_id
        else:
            assert got[0, 0] == top


@pytest.mark.parametrize("M,K", [(4, 1536), (20, 1536), (9, 576), (20, 576), (32, 576), (32, 64)])
def test_norm_matvec_silu_mul(engine, M, K):
    # Above 2 rows and up to k 768 with a gain: the matrix-core form.
    I, eps = 1536, 1e-5
    x, g, wb = decode_inputs(M, K, 2 * I)
    w = orc.from_bf16(wb).astype(np.float64)
    got = engine.download(engine.norm_matvec(engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb),
                                             silu_mul=True))
    y = rms_ref(x, g, eps) @ w.T
    gate, up = y[:, :I], y[:, I:]
    want = gate / (1 + np.exp(-gate)) * up
    assert got.shape == (M, I)
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("M", [1, 5, 32])
def test_norm_qkv_rope_writes_cache(engine, M):
    H, KVH, D, K, maxc, pos, eps = 9, 3, 64, 576, 40, 17, 1e-5
    x, g, wb = decode_inputs(M, K, (H + 2 * KVH) * D)
    w = orc.from_bf16(wb).astype(np.float64)
    ang = pos * (1e5 ** (-2.0 * np.arange(D // 2) / D))
    cos = np.tile(np.concatenate([np.cos(ang), np.cos(ang)]), (maxc, 1)).astype(np.float32)
    sin = np.tile(np.concatenate([-np.sin(ang), np.sin(ang)]), (maxc, 1)).astype(np.float32)
    kc0 = rnd(M * KVH * maxc, D)
    vc0 = rnd(M * KVH * maxc, D)
    kc, vc = engine.upload(kc0), engine.upload(vc0)
    q = engine.download(engine.norm_qkv_rope(engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb),
                                             engine.upload(cos), engine.upload(sin), H, KVH, pos, kc, vc))
    y = rms_ref(x, g, eps) @ w.T  # [M, (H + 2 KVH) D]

    def rope(h):  # h [M, heads, D]
        rot = np.concatenate([h[..., D // 2:], h[..., :D // 2]], -1)
        return h * cos[pos] + rot * sin[pos]
    scale = (np.abs(rms_ref(x, g, eps)) @ np.abs(w).T).max()
    want_q = rope(y[:, :H * D].reshape(M, H, D)).reshape(M, H * D)
    assert np.abs(q - want_q).max() <= 2e-5 * scale
    kc1 = engine.download(kc).reshape(M, KVH, maxc, D)
    vc1 = engine.download(vc).reshape(M, KVH, maxc, D)
    want_k = rope(y[:, H * D:(H + KVH) * D].reshape(M, KVH, D))
    want_v = y[:, (H + KVH) * D:].reshape(M, KVH, D)
    assert np.abs(kc1[:, :, pos] - want_k).max() <= 2e-5 * scale
    assert np.abs(vc1[:, :, pos] - want_v).max() <= 2e-5 * scale
    # Every other cache row is untouched.
    keep = np.ones(maxc, bool)
    keep[pos] = False
    assert np.array_equal(kc1[:, :, keep], kc0.reshape(M, KVH, maxc, D)[:, :, keep])
    assert np.array_equal(vc1[:, :, keep], vc0.reshape(M, KVH, maxc, D)[:, :, keep])


def qkv_attention_case(engine, M, kv16, pos0, maxc, seed=0, H=9, KVH=3):
    rng = np.random.default_rng(seed)
    D, K, eps = 64, 576, 1e-5
    x = rng.standard_normal((M, K)).astype(np.float32)
    g = (rng.standard_normal((1, K)) * 0.1 + 1.0).astype(np.float32)
    wb = orc.to_bf16((rng.standard_normal(((H + 2 * KVH) * D, K)) * 0.05).astype(np.float32))
    ang = np.arange(maxc)[:, None] * (1e5 ** (-2.0 * np.arange(D // 2) / D))[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32)
    sin = np.concatenate([-np.sin(ang), np.sin(ang)], 1).astype(np.float32)
    kc0 = rng.standard_normal((M * KVH * maxc, D)).astype(np.float32)
    vc0 = rng.standard_normal((M * KVH * maxc, D)).astype(np.float32)
    if kv16:
        kc0, vc0 = orc.to_bf16(kc0), orc.to_bf16(vc0)
    up = engine.upload_bf16 if kv16 else engine.upload
    args = (engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb), engine.upload(cos), engine.upload(sin),
            H, KVH)
    return dict(H=H, KVH=KVH, D=D, K=K, eps=eps, x=x, g=g, wb=wb, cos=cos, sin=sin, kc0=kc0, vc0=vc0, up=up,
                args=args, scale=float(np.float32(1.0 / np.sqrt(D))))


@pytest.mark.parametrize("M", [1, 2, 6, 8])  # one launch and a combine up to 6 sequences, the two calls above
@pytest.mark.parametrize("kv16", [False, True])
@pytest.mark.parametrize("pos0,span,maxc", [(575, 576, 640), (100, 192, 640), (40, 64, 64), (0, 64, 64)])
def test_norm_qkv_attention(engine, M, kv16, pos0, span, maxc):
    # Against the two calls it fuses, on the same inputs: the attention rows
    # within the F32 bound, the new cache row within the projection's bound
    # (exact in BF16 up to one rounding), every other row untouched; and
    # against float64 over the caches as written.  The device position gives
    # the immediate one's bits.
    c = qkv_attention_case(engine, M, kv16, pos0, maxc)
    H, KVH, D = c["H"], c["KVH"], c["D"]
    k1, v1 = c["up"](c["kc0"]), c["up"](c["vc0"])
    got = engine.download(engine.norm_qkv_attention(*c["args"], 0, pos0, span, k1, v1, c["scale"]))
    k2, v2 = c["up"](c["kc0"]), c["up"](c["vc0"])
    q = engine.norm_qkv_rope(*c["args"], pos0, k2, v2)
    want = engine.download(engine.attention_rows_at(q, k2, v2, M, 1, H, KVH, 0, pos0, span, c["scale"]))
    dl = (lambda b: orc.from_bf16(engine.download(b))) if kv16 else engine.download
    kc1, vc1, kc2, vc2 = (dl(b).reshape(M, KVH, maxc, D) for b in (k1, v1, k2, v2))
    x64 = rms_ref(c["x"], c["g"], c["eps"])
    w = orc.from_bf16(c["wb"]).astype(np.float64)
    bound = (np.abs(x64) @ np.abs(w).T).max()
    tol_row = 2e-5 * bound + (2.0 ** -8 * np.abs(kc2[:, :, pos0]).max() if kv16 else 0.0)
    assert np.abs(kc1[:, :, pos0] - kc2[:, :, pos0]).max() <= tol_row
    assert np.abs(vc1[:, :, pos0] - vc2[:, :, pos0]).max() <= tol_row
    keep = np.ones(maxc, bool)
    keep[pos0] = False
    assert np.array_equal(kc1[:, :, keep], kc2[:, :, keep])
    assert np.array_equal(vc1[:, :, keep], vc2[:, :, keep])
    # float64 attention over this call's caches and queries, the queries from float64 too.
    y = x64 @ w.T
    qh = y[:, :H * D].reshape(M, H, D)
    rot = np.concatenate([qh[..., D // 2:], qh[..., :D // 2]], -1)
    q64 = (qh * c["cos"][pos0] + rot * c["sin"][pos0]).reshape(M, H * D)
    a64 = attention_ref(q64.astype(np.float32), kc1.reshape(-1, D), vc1.reshape(-1, D), M, 1, H, KVH, pos0,
                        c["scale"])
    vmax = np.abs(vc1).max()
    assert np.abs(got - a64).max() <= 1e-4 * vmax * max(1.0, bound * c["scale"] * np.abs(kc1).max())
    assert np.abs(got - want).max() <= 1e-4 * vmax * max(1.0, bound * c["scale"] * np.abs(kc1).max())
    if M > 6:  # the two calls themselves
        same_bits(got, want)
    ipos = engine.upload_bits(np.array([[pos0]], np.int32), I32)
    k3, v3 = c["up"](c["kc0"]), c["up"](c["vc0"])
    same_bits(engine.download(engine.norm_qkv_attention(*c["args"], ipos, 0, span, k3, v3, c["scale"])), got)
    same_bits(engine.download(k3), engine.download(k1))
    same_bits(engine.download(v3), engine.download(v1))


@pytest.mark.parametrize("M,kv16", [(1, False), (2, True)])
def test_norm_qkv_attention_refuses_bad_positions(engine, M, kv16):
    c = qkv_attention_case(engine, M, kv16, 10, 64)
    H, KVH, D = c["H"], c["KVH"], c["D"]
    k1, v1 = c["up"](c["kc0"]), c["up"](c["vc0"])
    with pytest.raises(miburn.MiError) as e:  # immediate position past the span
        engine.norm_qkv_attention(*c["args"], 0, 64, 64, k1, v1, c["scale"])
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:  # span beyond the cache
        engine.norm_qkv_attention(*c["args"], 0, 10, 65, k1, v1, c["scale"])
    assert e.value.kind == "ARG"
    # A device position past the span: no cache row written, reported at the next wait.
    # The step then attends from position 0: its only key is the cache's
    # position-0 row as stored, weight 1, so every query head's output is its
    # kv head's position-0 value row exactly -- the same on every call.
    bad = engine.upload_bits(np.array([[64]], np.int32), I32)
    v0 = (orc.from_bf16(c["vc0"]) if kv16 else c["vc0"]).reshape(M, KVH, 64, D)[:, :, 0]
    want = np.repeat(v0, H // KVH, axis=1).reshape(M * H, D)
    for _ in range(2):
        out = engine.norm_qkv_attention(*c["args"], bad, 0, 64, k1, v1, c["scale"])
        with pytest.raises(miburn.MiError) as e:
            engine.sync()
        assert e.value.kind == "DOMAIN"
        engine.sync()
        got = engine.download(out).reshape(M * H, D)
        assert np.all(np.isfinite(got))
        same_bits(got, want)
        same_bits(engine.download(k1), c["kc0"])
        same_bits(engine.download(v1), c["vc0"])


@pytest.mark.parametrize("M", [1, 2])  # the combine inside the projection's launch for one sequence; the two calls
@pytest.mark.parametrize("kv16", [False, True])
@pytest.mark.parametrize("bfp", [False, True])
@pytest.mark.parametrize("pos0,span,maxc", [(575, 576, 640), (40, 64, 64), (0, 64, 64), (2000, 2048, 2048)])
def test_norm_qkv_attention_o(engine, M, kv16, bfp, pos0, span, maxc):
    # The attention block through its o projection and residual: bit for bit
    # norm_qkv_attention then norm_matvec(o, w_o, residual x) on copies of the
    # caches, the caches written the same, at the immediate and the device
    # position.  2048 keys: 32 chunks, past the 16 a thread holds in registers.
    c = qkv_attention_case(engine, M, kv16, pos0, maxc)
    H, KVH, D, K = c["H"], c["KVH"], c["D"], c["K"]
    rng = np.random.default_rng(7)
    wo32 = (rng.standard_normal((K, H * D)) * 0.05).astype(np.float32)
    wo = engine.cast_bfp(engine.upload(wo32)) if bfp else engine.upload_bf16(orc.to_bf16(wo32))
    x = c["args"][0]
    k1, v1 = c["up"](c["kc0"]), c["up"](c["vc0"])
    got = engine.download(engine.norm_qkv_attention_o(*c["args"], 0, pos0, span, k1, v1, c["scale"], wo))
    k2, v2 = c["up"](c["kc0"]), c["up"](c["vc0"])
    o = engine.norm_qkv_attention(*c["args"], 0, pos0, span, k2, v2, c["scale"])
    want = engine.download(engine.norm_matvec(o, 0, 0.0, wo, x))
    assert got.shape == (M, K)
    same_bits(got, want)
    same_bits(engine.download(k1), engine.download(k2))
    same_bits(engine.download(v1), engine.download(v2))
    # Within the F32 bound of float64 x + o w_o^T over the two calls' attention rows.
    wo64 = (engine.download(wo) if bfp else orc.from_bf16(orc.to_bf16(wo32))).astype(np.float64)  # BFP8 reads decoded
    o64 = engine.download(o).astype(np.float64)
    ref = c["x"].astype(np.float64) + o64 @ wo64.T
    assert np.abs(got - ref).max() <= 1e-5 * (np.abs(c["x"]).max() + (np.abs(o64) @ np.abs(wo64).T).max())
    ipos = engine.upload_bits(np.array([[pos0]], np.int32), I32)
    k3, v3 = c["up"](c["kc0"]), c["up"](c["vc0"])
    same_bits(engine.download(engine.norm_qkv_attention_o(*c["args"], ipos, 0, span, k3, v3, c["scale"], wo)), got)
    same_bits(engine.download(k3), engine.download(k1))


@pytest.mark.parametrize("H,KVH", [(16, 4), (8, 1), (4, 4), (6, 2)])
@pytest.mark.parametrize("M", [1, 2])
def test_norm_qkv_attention_o_head_shapes(engine, H, KVH, M):
    # Other head counts and groups (1 to 8 query heads a kv head, 4 to 16
    # heads): the combine's rows past the last head, the 128-thread combine
    # above 4 heads a group, o weights of 256 to 1024 columns -- still bit
    # for bit the two calls, and near float64.
    pos0, span, maxc = 300, 320, 384
    c = qkv_attention_case(engine, M, False, pos0, maxc, seed=3, H=H, KVH=KVH)
    D, K = c["D"], c["K"]
    rng = np.random.default_rng(11)
    wo32 = (rng.standard_normal((K, H * D)) * 0.05).astype(np.float32)
    wo = engine.upload_bf16(orc.to_bf16(wo32))
    k1, v1 = c["up"](c["kc0"]), c["up"](c["vc0"])
    got = engine.download(engine.norm_qkv_attention_o(*c["args"], 0, pos0, span, k1, v1, c["scale"], wo))
    k2, v2 = c["up"](c["kc0"]), c["up"](c["vc0"])
    o = engine.norm_qkv_attention(*c["args"], 0, pos0, span, k2, v2, c["scale"])
    same_bits(got, engine.download(engine.norm_matvec(o, 0, 0.0, wo, c["args"][0])))
    same_bits(engine.download(k1), engine.download(k2))
    x64 = rms_ref(c["x"], c["g"], c["eps"])
    w = orc.from_bf16(c["wb"]).astype(np.float64)
    y = x64 @ w.T
    qh = y[:, :H * D].reshape(M, H, D)
    rot = np.concatenate([qh[..., D // 2:], qh[..., :D // 2]], -1)
    q64 = (qh * c["cos"][pos0] + rot * c["sin"][pos0]).reshape(M, H * D)
    kc1 = engine.download(k1).reshape(-1, D)
    vc1 = engine.download(v1).reshape(-1, D)
    a64 = attention_ref(q64.astype(np.float32), kc1, vc1, M, 1, H, KVH, pos0, c["scale"]).astype(np.float64)
    wo64 = orc.from_bf16(orc.to_bf16(wo32)).astype(np.float64)
    ref = c["x"].astype(np.float64) + a64 @ wo64.T
    bound = (np.abs(a64) @ np.abs(wo64).T).max() + np.abs(c["x"]).max()
    assert np.abs(got - ref).max() <= 1e-4 * bound


def test_norm_qkv_attention_o_refuses(engine):
    # A missing or mis-shaped o weight is refused before any cache row is written.
    c = qkv_attention_case(engine, 1, False, 10, 64)
    H, D, K = c["H"], c["D"], c["K"]
    k1, v1 = c["up"](c["kc0"]), c["up"](c["vc0"])
    for wo in (engine.upload_bf16(orc.to_bf16(np.zeros((K, H * D - 64), np.float32))),
               engine.upload(np.zeros((K, H * D), np.float32)), 0):
        with pytest.raises(miburn.MiError) as e:
            engine.norm_qkv_attention_o(*c["args"], 0, 10, 64, k1, v1, c["scale"], wo)
        assert e.value.kind == "ARG"
    same_bits(engine.download(k1), c["kc0"])
    same_bits(engine.download(v1), c["vc0"])
    # A device position past the span: the same refusal and the same output as the two calls.
    bad = engine.upload_bits(np.array([[64]], np.int32), I32)
    wo = engine.upload_bf16(orc.to_bf16(np.full((K, H * D), 0.01, np.float32)))
    outs = []
    for fused in (True, False):
        if fused:
            out = engine.norm_qkv_attention_o(*c["args"], bad, 0, 64, k1, v1, c["scale"], wo)
        else:
            out = engine.norm_matvec(engine.norm_qkv_attention(*c["args"], bad, 0, 64, k1, v1, c["scale"]), 0, 0.0,
                                     wo, c["args"][0])
        with pytest.raises(miburn.MiError) as e:
            engine.sync()
        assert e.value.kind == "DOMAIN"
        engine.sync()
        outs.append(engine.download(out))
    same_bits(outs[0], outs[1])
    same_bits(engine.download(k1), c["kc0"])


@pytest.mark.parametrize("M", [1, 5, 32])
def test_norm_qkv_rope_bf16_caches(engine, M):
    # The same kernel into BF16 caches: q unchanged, the new cache row the F32
    # form's rounded to nearest even, every other row untouched.
    H, KVH, D, K, maxc, pos, eps = 9, 3, 64, 576, 40, 17, 1e-5
    x, g, wb = decode_inputs(M, K, (H + 2 * KVH) * D)
    cos, sin = rnd(maxc, D), rnd(maxc, D)
    kc0 = orc.to_bf16(rnd(M * KVH * maxc, D))
    vc0 = orc.to_bf16(rnd(M * KVH * maxc, D))
    args = (engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb), engine.upload(cos), engine.upload(sin),
            H, KVH, pos)
    kf, vf = engine.upload(orc.from_bf16(kc0)), engine.upload(orc.from_bf16(vc0))
    kb, vb = engine.upload_bf16(kc0), engine.upload_bf16(vc0)
    qf = engine.download(engine.norm_qkv_rope(*args, kf, vf))
    qb = engine.download(engine.norm_qkv_rope(*args, kb, vb))
    same_bits(qb, qf)
    assert np.array_equal(engine.download(kb), orc.to_bf16(engine.download(kf)))
    assert np.array_equal(engine.download(vb), orc.to_bf16(engine.download(vf)))
    with pytest.raises(miburn.MiError) as e:
        engine.norm_qkv_rope(*args, kb, vf)
    assert e.value.kind == "ARG"


@pytest.mark.parametrize("M", [1, 5, 32])
def test_norm_qkv_rope_at_device_position(engine, M):
    # The position read on the device: the immediate call's q and cache bits.
    H, KVH, D, K, maxc, pos, eps = 9, 3, 64, 576, 40, 23, 1e-5
    x, g, wb = decode_inputs(M, K, (H + 2 * KVH) * D)
    cos, sin = rnd(maxc, D), rnd(maxc, D)
    kc0, vc0 = rnd(M * KVH * maxc, D), rnd(M * KVH * maxc, D)
    args = (engine.upload(x), engine.upload(g), eps, engine.upload_bf16(wb), engine.upload(cos), engine.upload(sin),
            H, KVH)
    k1, v1 = engine.upload(kc0), engine.upload(vc0)
    k2, v2 = engine.upload(kc0), engine.upload(vc0)
    q1 = engine.download(engine.norm_qkv_rope(*args, pos, k1, v1))
    ipos = engine.upload_bits(np.array([[pos]], np.int32), I32)
    q2 = engine.download(engine.norm_qkv_rope_at(*args, ipos, k2, v2))
    same_bits(q2, q1)
    same_bits(engine.download(k2), engine.download(k1))
    same_bits(engine.download(v2), engine.download(v1))
    # Outside the cache: nothing written, reported at the next wait.
    bad = engine.upload_bits(np.array([[maxc]], np.int32), I32)
    engine.norm_qkv_rope_at(*args, bad, k2, v2)
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    engine.sync()
    same_bits(engine.download(k2), engine.download(k1))
    with pytest.raises(miburn.MiError) as e:  # tables shorter than the cache
        engine.norm_qkv_rope_at(*args[:4], engine.upload(cos[:30]), engine.upload(sin[:30]), H, KVH, ipos, k2, v2)
    assert e.value.kind == "ARG"


def test_decode_projection_errors(engine):
    w = engine.upload_bf16(orc.to_bf16(rnd(64, 576)))
    with pytest.raises(miburn.MiError) as e:
        engine.norm_matvec(engine.upload(rnd(33, 576)), 0, 0.0, w)  # 33 rows
    assert e.value.kind == "UNSUPPORTED"
    with pytest.raises(miburn.MiError) as e:
        engine.norm_matvec(engine.upload(rnd(2, 576)), 0, 0.0, engine.upload(rnd(64, 576)))  # F32 weight
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:
        engine.norm_matvec(engine.upload(rnd(2, 572)), 0, 0.0, engine.upload_bf16(orc.to_bf16(rnd(64, 572))))
    assert e.value.kind == "UNSUPPORTED"  # width not a multiple of 8
    with pytest.raises(miburn.MiError) as e:
        engine.norm_matvec(engine.upload(rnd(2, 576)), 0, 0.0, engine.upload_bf16(orc.to_bf16(rnd(63, 576))),
                           silu_mul=True)  # odd gate|up rows
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:
        engine.norm_matvec(engine.empty(2, 0), 0, 0.0, engine.empty(64, 0, BF16))  # no columns
    assert e.value.kind == "UNSUPPORTED"


def test_attention_rows_errors(engine):
    q = engine.upload(rnd(2, 10 * 64))
    k = engine.upload(rnd(2 * 1 * 16, 64))
    for args, kind in [((2, 1, 10, 1, 0), "UNSUPPORTED"),  # 10 query heads per kv head
                       ((2, 1, 10, 2, 16), "ARG"),          # cache holds 8 positions per item, not 17
                       ((2, 1, 10, 3, 0), "ARG")]:          # heads not a multiple of kv heads
        with pytest.raises(miburn.MiError) as e:
            engine.attention_rows(q, k, k, *args[:4], args[4], 0.125)
        assert e.value.kind == kind, (args, e.value)
    q48 = engine.upload(rnd(1, 2 * 48))
    k48 = engine.upload(rnd(4, 48))
    with pytest.raises(miburn.MiError) as e:
        engine.attention_rows(q48, k48, k48, 1, 1, 2, 1, 0, 0.125)
    assert e.value.kind == "UNSUPPORTED"


# ------------------------------------------------------------- casts, copies
def test_cast_roundtrip_bits(engine):
    x = rnd(64, 100)
    x.ravel()[:5] = [np.nan, np.inf, -0.0, 1e-40, 3.0000002]
    a = engine.upload(x)
    h = engine.cast_float(a, BF16)
    assert np.array_equal(engine.download(h), orc.to_bf16(x))
    same_bits(engine.download(engine.cast_float(h, F32)), orc.from_bf16(orc.to_bf16(x)))


def test_cast_i32_to_f32(engine):
    v = np.array([[0, -1, 2**24 + 1, -(2**31), 2**31 - 1]], np.int32)
    got = engine.download(engine.cast_float(engine.upload_i32(v), F32))
    same_bits(got, v.astype(np.float32))


def test_copy_strided_transpose_keeps_negative_zero(engine):
    # essentials.rs:33-56: owned storage keeps -0.0 through transpose + reshape.
    x = rnd(12, 20)
    x[3, 4] = -0.0
    a = engine.upload(x)
    t = engine.copy_strided(a, 20, 12, 0, 1, 20)
    same_bits(engine.download(t), np.ascontiguousarray(x.T))


def test_copy_strided4_head_split(engine):
    B, T, H, Dh = 4, 16, 4, 8
    x = rnd(B * T, H * Dh)
    a = engine.upload(x)
    # [B, T, H, Dh] -> [B, H, T, Dh]
    dims, strides = (B, H, T, Dh), (T * H * Dh, Dh, H * Dh, 1)
    got = engine.download(engine.copy_strided4(a, dims, 0, strides))
    same_bits(got, orc.copy_strided4(x, dims, 0, strides).view(np.float32))
    same_bits(got, x.reshape(B, T, H, Dh).transpose(0, 2, 1, 3).reshape(-1, Dh))


def test_assign_block(engine):
    cache = np.zeros((64, 32), np.float32)
    blk = rnd(5, 32)
    c = engine.upload(cache)
    engine.assign_block(c, engine.upload(blk), 10, 0)
    cache[10:15] = blk
    same_bits(engine.download(c), cache)


# --------------------------------------------------------------------- random
def test_random_is_seeded_and_distributed(engine):
    a = engine.download(engine.random_dram(512, 512, miburn.DRAW_UNIT, base=7))
    b = engine.download(engine.random_dram(512, 512, miburn.DRAW_UNIT, base=7))
    c = engine.download(engine.random_dram(512, 512, miburn.DRAW_UNIT, base=8))
    same_bits(a, b)
    assert not np.array_equal(a, c)
    assert a.min() >= 0.0 and a.max() < 1.0 and abs(a.mean() - 0.5) < 0.01
    n = engine.download(engine.random_dram(1024, 1024, miburn.DRAW_NORMAL, 0.0, 0.02, base=3))
    assert abs(n.mean()) < 1e-3 and abs(n.std() - 0.02) < 5e-4
    u = engine.download(engine.random_dram(256, 256, miburn.DRAW_UNIFORM, -0.125, 0.125, base=5))
    assert u.min() >= -0.125 and u.max() < 0.125
    i = engine.download(engine.random_dram(100, 1000, miburn.DRAW_INT_RANGE, 0, 10, base=9))
    assert i.dtype == np.int32 and i.min() == 0 and i.max() == 9


# --------------------------------------------------------------------- errors
def test_stale_id_and_report(engine):
    a = engine.upload(rnd(4, 4))
    engine.free(a)
    with pytest.raises(miburn.MiError) as e:
        engine.download(a)
    assert e.value.kind == "ID"
    with pytest.raises(miburn.MiError):
        engine.eltwise_op_as("EXP", a)
    r = engine.report()
    assert r["uploads"] > 0 and r["ops"] > 0


def test_decode_advance_chains_on_the_device(engine):
    """mi_decode_advance: ids <- next, log[:, pos + 1] <- next, pos <- pos + 1;
    a position whose log column is past the log writes no entry, keeps the
    position and raises MI_E_DOMAIN at the next wait."""
    B, cols = 5, 12
    nxt = engine.upload_bits(np.arange(100, 100 + B, dtype=np.int32).reshape(B, 1), I32)
    ids = engine.upload_bits(np.zeros((B, 1), np.int32), I32)
    pos = engine.upload_bits(np.array([[3]], np.int32), I32)
    log = engine.upload_bits(np.full((B, cols), -1, np.int32), I32)
    engine.decode_advance(nxt, ids, pos, log)
    engine.decode_advance(ids, ids, pos, log)  # next is this step's input: logged again one further
    assert engine.download(pos)[0, 0] == 5
    want = np.full((B, cols), -1, np.int32)
    want[:, 4] = want[:, 5] = np.arange(100, 100 + B)
    assert np.array_equal(engine.download(log), want)
    assert np.array_equal(engine.download(ids).ravel(), np.arange(100, 100 + B))
    end = engine.upload_bits(np.array([[cols - 1]], np.int32), I32)
    engine.decode_advance(nxt, ids, end, log)
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    assert engine.download(end)[0, 0] == cols - 1
    assert np.array_equal(engine.download(log), want)
    with pytest.raises(miburn.MiError) as e:  # mismatched rows are refused at the call
        engine.decode_advance(nxt, ids, pos, engine.upload_bits(np.zeros((B + 1, cols), np.int32), I32))
    assert e.value.kind == "ARG"


@pytest.mark.parametrize("shape", [(7,), (5, 9), (3, 4, 6), (2, 3, 4, 5), (64, 3, 128)])
def test_gather_along_any_dim(engine, shape):
    """mi_gather (Burn's float_gather, ops.rs:1102-1160) along every dim
    against the oracle, bit for bit, NaN / -0.0 / infinity payloads kept;
    BF16 payloads gathered as they lie."""
    rng = np.random.default_rng(len(shape) * 10 + shape[0])
    x = rng.standard_normal(shape).astype(np.float32)
    flat = x.reshape(-1)
    flat[::7] = np.nan
    flat[1::11] = -0.0
    flat[2::13] = np.inf
    pad = 4 - len(shape)
    dims = [1] * pad + list(shape)
    xid = engine.upload(x.reshape(-1, shape[-1]))
    xb = engine.upload_bf16(orc.to_bf16(x.reshape(-1, shape[-1])))
    for dim in range(len(shape)):
        ishape = list(shape)
        ishape[dim] = 3 + 2 * dim
        idx = rng.integers(0, shape[dim], ishape).astype(np.int32)
        iid = engine.upload_bits(idx.reshape(-1, ishape[-1]), I32)
        idims = [1] * pad + ishape
        got = engine.download(engine.gather(xid, dims, dim + pad, iid, idims))
        want, bad = orc.gather(x, dim, idx)
        assert bad == 0
        assert np.array_equal(got.reshape(ishape).view(np.uint32), want.view(np.uint32)), dim
        gb = engine.download(engine.gather(xb, dims, dim + pad, iid, idims))
        wb = np.take_along_axis(orc.to_bf16(x), idx.astype(np.int64), dim)
        assert np.array_equal(gb.reshape(ishape), wb), dim
    engine.sync()


def test_gather_errors(engine):
    x = engine.upload(rnd(4, 5))
    idx = np.zeros((4, 2), np.int32)
    idx[2, 1] = 5
    out = engine.gather(x, [1, 1, 4, 5], 3, engine.upload_bits(idx, I32), [1, 1, 4, 2])
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    assert engine.download(out).view(np.uint32)[2, 1] == 0
    for dims, dim, idims in (([1, 1, 4, 5], 4, [1, 1, 4, 2]), ([1, 1, 4, 5], 3, [1, 1, 3, 2]),
                             ([1, 1, 4, 6], 3, [1, 1, 4, 2])):
        with pytest.raises(miburn.MiError) as e:
            engine.gather(x, dims, dim, engine.upload_bits(np.zeros((4, 2), np.int32), I32), idims)
        assert e.value.kind == "ARG"
