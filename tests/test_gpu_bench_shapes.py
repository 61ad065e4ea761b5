"""Parity at the sizes the bench times, so the kernels behind the reported
figures are the kernels under test.

BASELINE config 3 on [8192, 8192] F32 (256 MiB an operand: element-wise
operations moving 128 MiB or more take the streaming-access instantiations),
the embedding gather of 65,536 ids from a [49152, 576] table (the streaming
row copy), row softmax and the row / column sums and means; config 2's ends:
the 8192^3 products in BF16 and F32 (both matmul modes) and the batched
[16, 512, 512] x [16, 512, 512] product in F32 and BF16.

Bars: bit-exact for the exact element-wise ops,
the gather and small-integer products (every summation order is exact when
all partial sums are integers below 2^24); rel 1e-5 against the oracle for
the F32 transcendental ops, softmax and reductions; the F32 accumulation
bound 1e-5 * sum |a||b| for random batched products against the oracle fed
the same values.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc
from miburn import AXIS_COLS, AXIS_ROWS, BF16, F32, K, R_MEAN, R_SUM
from test_gpu_ops import close, mm_tol, mode, same_bits  # noqa: F401 (mode: a fixture)

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(8192)
N = 8192


@pytest.fixture(scope="module")
def big(engine):
    x = RNG.standard_normal((N, N), dtype=np.float32)
    y = RNG.standard_normal((N, N), dtype=np.float32)
    ix, iy = engine.upload(x), engine.upload(y)
    yield x, y, ix, iy
    engine.free(ix)
    engine.free(iy)


@pytest.mark.parametrize("kind", ["ADD", "MUL"])
def test_streaming_binary_exact(engine, big, kind):
    x, y, ix, iy = big
    out = engine.eltwise_op_as(kind, ix, iy)
    got = engine.download(out)
    engine.free(out)
    same_bits(got, x + y if kind == "ADD" else x * y)


@pytest.mark.parametrize("kind,s1", [("EXP", 0.0), ("GELU", 0.0), ("SILU", 0.0), ("RSQRT_ABS_ADD", 1e-6)])
def test_streaming_unary(engine, big, kind, s1):
    x, _, ix, _ = big
    out = engine.eltwise_op_as(kind, ix, scalar=s1)
    got = engine.download(out)
    engine.free(out)
    close(got, orc.eltwise(K[kind], x, s1=s1), rtol=1e-5, atol=1e-37)


def test_row_softmax_full_size(engine, big):
    x, _, ix, _ = big
    out = engine.softmax_rows(ix)
    got = engine.download(out)
    engine.free(out)
    close(got, orc.softmax_rows(x), rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("op", [R_SUM, R_MEAN])
@pytest.mark.parametrize("axis", [AXIS_ROWS, AXIS_COLS])
def test_sums_and_means_full_size(engine, big, op, axis):
    x, _, ix, _ = big
    out = engine.reduce(ix, op, axis)
    got = engine.download(out)
    engine.free(out)
    want = orc.reduce(x, op, axis)
    # A sum of N(0, 1) values can land near zero: bound against the sum of
    # magnitudes (the F32 summation bound) as well as relatively.
    mag = np.abs(x).sum(axis=0 if axis == AXIS_ROWS else 1, dtype=np.float64).reshape(want.shape)
    if op == R_MEAN:
        mag /= N
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * mag), np.abs(got - want).max()


def test_embedding_gather_full_size(engine):
    """65,536 ids into a [49152, 576] table with special payloads (signed
    zeros, infinities, NaNs with payload, a subnormal) copied bit for bit."""
    V, D = 49152, 576
    bits = RNG.standard_normal((V, D), dtype=np.float32).view(np.uint32).copy()
    bits.ravel()[:7] = [0x0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x7FC0BEEF]
    idx = RNG.integers(0, V, (1, 65536)).astype(np.int32)
    idx[0, :3] = [0, V - 1, 0]
    t, i = engine.upload_bits(bits, F32), engine.upload_i32(idx)
    out = engine.select_rows(t, i)
    got = engine.download(out).view(np.uint32)
    for h in (t, i, out):
        engine.free(h)
    same_bits(got, orc.select_rows(bits, idx))


@pytest.fixture(scope="module")
def int_cube():
    a = RNG.integers(-4, 5, (N, N)).astype(np.float32)
    b = RNG.integers(-4, 5, (N, N)).astype(np.float32)
    # Every partial sum is an integer of magnitude <= 16 * 8192 < 2^24, so
    # any F32 summation order (this BLAS call's included) is exact.
    return a, b, a @ b


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_matmul_8192_integer_exact(engine, mode, int_cube, dtype):
    a, b, want = int_cube
    if dtype == "bf16":
        ia, ib = engine.upload_bf16(orc.to_bf16(a)), engine.upload_bf16(orc.to_bf16(b))
    else:
        ia, ib = engine.upload(a), engine.upload(b)
    out = engine.matmul_dram(ia, False, ib, False)
    got = engine.download(out)
    for h in (ia, ib, out):
        engine.free(h)
    same_bits(got, want)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_batched_16x512_cubed(engine, mode, dtype):
    batch, m = 16, 512
    a = RNG.standard_normal((batch, m, m), dtype=np.float32)
    b = RNG.standard_normal((batch, m, m), dtype=np.float32)
    if dtype == "bf16":
        ab, bb = orc.to_bf16(a.reshape(-1, m)), orc.to_bf16(b.reshape(-1, m))
        ia, ib = engine.upload_bf16(ab), engine.upload_bf16(bb)
        a, b = orc.from_bf16(ab).reshape(batch, m, m), orc.from_bf16(bb).reshape(batch, m, m)
    else:
        ia, ib = engine.upload(a.reshape(-1, m)), engine.upload(b.reshape(-1, m))
    out = engine.matmul_dram_batched(ia, False, ib, False, batch, m, m, m)
    got = engine.download(out).reshape(batch, m, m)
    for h in (ia, ib, out):
        engine.free(h)
    for z in range(batch):
        want = orc.matmul(a[z], b[z], threads=16)
        assert np.all(np.abs(got[z] - want) <= mm_tol(a[z], b[z], False, False, 1e-5) + 1e-30), z
