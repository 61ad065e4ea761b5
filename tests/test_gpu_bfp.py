"""BFP8 weight storage on the device (the reference's performance-contract
weight format: Engine::cast_bfp, crates/burn-tt/src/server.rs:141-147; the
packer rule crates/tt-models/src/quant.rs:185-235; the unpacker's decode
crates/tt-isa/src/tile.rs:619-636).

* mi_cast_bfp against the oracle's bfp_round_trip (oracle/oracle.c, pinned in
  tests/test_oracle.py): the decoded values bit for bit, over mixed scales,
  signed zeros, subnormals, blocks of tiny values, partial blocks and the
  reference's own step92 input pattern, from F32 and BF16 sources.
* Every kernel that reads BFP8 weights itself -- the decode GEMVs, the
  matrix-core decode projections (whole and split over k), the fused decode
  attention -- gives, bit for bit, what the same kernel gives on the BF16
  weight holding the decoded values (a BFP8 value is a BF16 value, and the
  kernels form each weight before the same products in the same order); so
  does every product that decodes its BFP8 operand first.
* Non-finite values are refused (MI_E_DOMAIN at the next wait), and ops that
  read datums as plain slots refuse a BFP8 buffer.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc
from miburn import BF16, BFP8, F32, I32

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(777)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def same_bits(a, b):
    a = np.ascontiguousarray(a).view(np.uint32)
    b = np.ascontiguousarray(b).view(np.uint32)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{bad.size} datums differ, first at {bad[0]}: {a.ravel()[bad[0]]:#x} vs {b.ravel()[bad[0]]:#x}"


def mixed(rows, cols):
    """Rows at scales 2^-40 .. 2^40, with zeros, -0.0, subnormals and blocks
    of values just above the smallest normal (block exponents 1 .. 6)."""
    x = rnd(rows, cols) * (2.0 ** RNG.integers(-40, 40, (rows, 1))).astype(np.float32)
    flat = x.reshape(-1)
    flat[RNG.integers(0, flat.size, 7)] = 0.0
    flat[RNG.integers(0, flat.size, 5)] = -0.0
    flat[RNG.integers(0, flat.size, 5)] = np.float32(3e-39)  # subnormal
    if rows > 2:
        x[2] = (rnd(cols) * np.float32(2.0 ** -124)).astype(np.float32)  # tiny normals
    return x


@pytest.mark.parametrize("rows,cols", [(64, 576), (3, 37), (33, 1536), (1, 16), (5, 8)])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_cast_bfp_matches_the_oracle(engine, rows, cols, src):
    x = mixed(rows, cols)
    if src == "bf16":
        bits = orc.to_bf16(x)
        x = orc.from_bf16(bits)
        a = engine.upload_bf16(bits)
    else:
        a = engine.upload(x)
    q = engine.cast_bfp(a)
    assert engine.metadata(q) == (rows, cols, BFP8)
    want, _, bad = orc.bfp_round_trip(x)
    assert bad == 0
    same_bits(engine.download(q), want)  # the decoded values (mi_download)
    same_bits(engine.download(engine.cast_bfp(q, 0)), want)  # mi_cast_bfp to F32
    assert np.array_equal(engine.download(engine.cast_float(q, BF16)), orc.to_bf16(want))  # exact in BF16
    # Held values are held exactly: packing them again changes nothing.
    same_bits(engine.download(engine.cast_bfp(engine.upload(want))), want)


def test_cast_bfp_step92_pattern(engine):
    # The reference's own packer input (crates/tt-tests/tests/step92_bfp_formats.rs:52-57).
    i = np.arange(1024)
    v = (((i % 16) - 8 + np.where(i % 3 == 0, 65 / 1024, 0)) * 2.0 ** ((i // 16 % 9) - 4)).astype(np.float32)
    v = v.reshape(32, 32)
    want, _, _ = orc.bfp_round_trip(v)
    same_bits(engine.download(engine.cast_bfp(engine.upload(v))), want)


def test_cast_bfp_refuses_non_finite(engine):
    x = rnd(4, 64)
    x[1, 20] = np.inf
    x[3, 0] = np.nan
    q = engine.cast_bfp(engine.upload(x))
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    got = engine.download(q)
    want, _, _ = orc.bfp_round_trip(np.where(np.isfinite(x), x, 0).astype(np.float32))
    # The two blocks holding them are zeros; every other block is packed.
    assert np.all(got[1, 16:32] == 0) and np.all(got[3, 0:16] == 0)
    keep = np.ones_like(got, bool)
    keep[1, 16:32] = False
    keep[3, 0:16] = False
    same_bits(got[keep], want[keep])


def test_bfp8_refused_where_datums_are_plain_slots(engine):
    q = engine.cast_bfp(engine.upload(rnd(8, 32)))
    idx = engine.upload_i32(np.array([1, 2], np.int32))
    for call in (lambda: engine.copy_strided(q, 2, 2, 0, 32, 1), lambda: engine.select_rows(q, idx),
                 lambda: engine.fill(2, 16, BFP8, 0), lambda: engine.empty(2, 16, BFP8),
                 lambda: engine.eltwise_op_as("EXP", q), lambda: engine.reshape(q, 16, 16),
                 lambda: engine.upload_bits(np.zeros((2, 16), np.uint32), BFP8)):
        with pytest.raises(miburn.MiError) as e:
            call()
        assert e.value.kind == "ARG"
    engine.sync()


def pair(engine, n, k, scale=0.05):
    """A BFP8 weight [n, k] and the BF16 weight holding its decoded values."""
    w = engine.cast_bfp(engine.upload(rnd(n, k, scale=scale)))
    return w, engine.cast_float(w, BF16)


# (M, K, N): the GEMV up to 6 rows (two chunks a lane to k 1024, four above,
# the loop form past 2048), the matrix-core form from 7 (split over k where
# its grid is small), and shapes only the LDS-staged kernel takes (decoded).
MATVEC = [(1, 576, 576), (2, 576, 3072), (5, 1536, 576), (6, 2048, 256), (3, 4096, 64), (7, 576, 576),
          (8, 1536, 576), (17, 576, 3072), (32, 1536, 576), (32, 576, 3072), (12, 3072, 64)]


@pytest.mark.parametrize("M,Kd,N", MATVEC)
@pytest.mark.parametrize("mode", ["plain", "residual", "silu", "norm"])
def test_norm_matvec_bfp8_equals_bf16(engine, M, Kd, N, mode):
    x = engine.upload(rnd(M, Kd))
    g = engine.upload(rnd(1, Kd) + np.float32(1.0))
    w, wb = pair(engine, N, Kd)
    if mode == "silu":
        args = (g, 1e-5, None, 0, True)
    elif mode == "residual":
        r = engine.upload(rnd(M, N))
        args = (0, 0.0, None, r, False)
    elif mode == "norm":
        args = (g, 1e-5, None, 0, False)
    else:
        args = (0, 0.0, None, 0, False)
    gam, eps, _, res, silu = args
    a = engine.download(engine.norm_matvec(x, gam, eps, w, res, silu))
    b = engine.download(engine.norm_matvec(x, gam, eps, wb, res, silu))
    same_bits(a, b)


@pytest.mark.parametrize("M", [1, 5, 8, 32])
@pytest.mark.parametrize("kv16", [False, True])
def test_norm_qkv_rope_bfp8_equals_bf16(engine, M, kv16):
    H, KVH, D, Kd, maxc, pos = 9, 3, 64, 576, 40, 17
    x, g = engine.upload(rnd(M, Kd)), engine.upload(rnd(1, Kd) + np.float32(1.0))
    w, wb = pair(engine, (H + 2 * KVH) * D, Kd)
    cos, sin = engine.upload(rnd(maxc, D)), engine.upload(rnd(maxc, D))
    c0 = rnd(M * KVH * maxc, D)

    def caches():
        if kv16:
            return engine.upload_bf16(orc.to_bf16(c0)), engine.upload_bf16(orc.to_bf16(c0))
        return engine.upload(c0), engine.upload(c0)
    k1, v1 = caches()
    k2, v2 = caches()
    q1 = engine.download(engine.norm_qkv_rope(x, g, 1e-5, w, cos, sin, H, KVH, pos, k1, v1))
    q2 = engine.download(engine.norm_qkv_rope(x, g, 1e-5, wb, cos, sin, H, KVH, pos, k2, v2))
    same_bits(q1, q2)
    for a, b in ((k1, k2), (v1, v2)):
        assert np.array_equal(engine.download(a), engine.download(b))


@pytest.mark.parametrize("M", [1, 2, 6, 9])  # the fused launch up to 6 sequences, the two calls above
@pytest.mark.parametrize("kv16", [False, True])
def test_norm_qkv_attention_bfp8_equals_bf16(engine, M, kv16):
    H, KVH, D, Kd, maxc, pos0, span = 9, 3, 64, 576, 640, 575, 576
    x, g = engine.upload(rnd(M, Kd)), engine.upload(rnd(1, Kd) + np.float32(1.0))
    w, wb = pair(engine, (H + 2 * KVH) * D, Kd)
    ang = np.arange(maxc)[:, None] * (1e5 ** (-2.0 * np.arange(D // 2) / D))[None, :]
    cos = engine.upload(np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32))
    sin = engine.upload(np.concatenate([-np.sin(ang), np.sin(ang)], 1).astype(np.float32))
    c0, v0 = rnd(M * KVH * maxc, D), rnd(M * KVH * maxc, D)

    def caches():
        if kv16:
            return engine.upload_bf16(orc.to_bf16(c0)), engine.upload_bf16(orc.to_bf16(v0))
        return engine.upload(c0), engine.upload(v0)
    k1, v1 = caches()
    k2, v2 = caches()
    scale = float(np.float32(1.0 / np.sqrt(D)))
    a = engine.download(engine.norm_qkv_attention(x, g, 1e-5, w, cos, sin, H, KVH, 0, pos0, span, k1, v1, scale))
    b = engine.download(engine.norm_qkv_attention(x, g, 1e-5, wb, cos, sin, H, KVH, 0, pos0, span, k2, v2, scale))
    same_bits(a, b)
    for p, q in ((k1, k2), (v1, v2)):
        assert np.array_equal(engine.download(p), engine.download(q))


@pytest.mark.parametrize("m,k,n", [(4, 576, 1536), (512, 576, 3072), (64, 1536, 576)])
def test_products_take_a_bfp8_operand(engine, m, k, n):
    """mi_matmul and mi_linear decode a BFP8 operand first: the BF16 product's bits."""
    x = engine.upload(rnd(m, k))
    w, wb = pair(engine, n, k)
    same_bits(engine.download(engine.matmul_dram(x, False, w, True)), engine.download(engine.matmul_dram(x, False, wb, True)))
    r = engine.upload(rnd(m, n))
    same_bits(engine.download(engine.linear(x, w, True, residual=r)), engine.download(engine.linear(x, wb, True, residual=r)))
    xb = engine.cast_float(x, BF16)
    same_bits(engine.download(engine.matmul_dram(xb, False, w, True)), engine.download(engine.matmul_dram(xb, False, wb, True)))
