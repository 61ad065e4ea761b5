"""Device parity of the short-row product path: operands in the matrix cores'
operand order ("tiles", MI_TILES_BF16 / MI_TILES_PARTS).

* mi_tile, mi_rms_norm and mi_linear_swiglu's tiled results hold exactly the
  row-major values (or the F32 values' parts) at the offsets the layout
  formula gives, restated here in numpy.
* mi_linear against a tiled weight: with small-integer operands every
  summation order is exact, so each activation form (F32 rows split in
  registers, BF16 rows, parts tiles, BF16 tiles) equals float64 bit for bit
  with bias and residual; with random operands it stays within the F32
  accumulation bound of float64 fed the same BF16 parts; an F32 operand's
  parts from mi_tile give the bits of the F32 rows (the same split), and BF16
  tiles the bits of BF16 rows.
* mi_linear_swiglu, mi_linear_qkv_rope_cache and mi_linear_add_rms_norm on a
  tiled weight: bit for bit mi_linear against the same tiled weight followed
  by mi_silu_mul_halves / mi_qkv_rope_cache / mi_rms_norm.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc
from miburn import BF16, F32, TILES_BF16, TILES_PARTS
from test_gpu_fused_products import pairs_of, split_parts

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20_261_202)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def ints(*shape, lo=-4, hi=4):
    return RNG.integers(lo, hi + 1, shape).astype(np.float32)


def same_bits(a, b, view=np.uint32):
    a = np.ascontiguousarray(a).view(view)
    b = np.ascontiguousarray(b).view(view)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{bad.size} datums differ, first at {bad[0]}: {a.ravel()[bad[0]]:#x} vs {b.ravel()[bad[0]]:#x}"


def tiled(v):
    """Row-major [r, c] -> the tile order, flat: block (r / 32, c / 16) of 64
    lanes x 8, lane r % 32 + 32 ((c / 8) % 2), value c % 8."""
    r, c = v.shape
    t = v.reshape(r // 32, 32, c // 16, 2, 8)          # [tm, row, ks, half, e]
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(-1)  # [tm, ks, half, row, e]


def tiled_parts(y):
    p = split_parts(y)
    c = y.shape[1]
    return np.concatenate([tiled(p[:, :c]), tiled(p[:, c:])])


def untile(flat, r, c):
    return np.ascontiguousarray(flat.reshape(r // 32, c // 16, 2, 32, 8).transpose(0, 3, 1, 2, 4)).reshape(r, c)


def test_tile_offsets_match_the_formula():
    # The numpy restatement against the header's formula, element by element.
    r, c = 64, 48
    v = np.arange(r * c).reshape(r, c)
    t = tiled(v)
    for row in (0, 5, 31, 32, 63):
        for col in (0, 7, 8, 15, 16, 47):
            off = (((row // 32) * (c // 16) + col // 16) * 64 + row % 32 + 32 * ((col // 8) % 2)) * 8 + col % 8
            assert t[off] == v[row, col]
    assert np.array_equal(untile(t, r, c), v)


@pytest.mark.parametrize("r,c", [(32, 16), (512, 576), (96, 1536)])
def test_tile_holds_the_values(engine, r, c):
    x = rnd(r, c)
    x[0, :3] = [3.4e38, np.inf, np.nan]
    ix = engine.upload(x)
    tb = engine.tile(ix, TILES_BF16)
    assert engine.metadata(tb) == (r, c, BF16)
    same_bits(engine.download(tb).reshape(-1), tiled(orc.to_bf16(x)), np.uint16)
    tp = engine.tile(ix, TILES_PARTS)
    assert engine.metadata(tp) == (r, 2 * c, BF16)
    same_bits(engine.download(tp).reshape(-1), tiled_parts(x), np.uint16)
    xb = orc.to_bf16(x)
    same_bits(engine.download(engine.tile(engine.upload_bf16(xb), TILES_BF16)).reshape(-1), tiled(xb), np.uint16)


@pytest.mark.parametrize("form", [TILES_BF16, TILES_PARTS])
def test_rms_norm_tiles(engine, form):
    x, g = rnd(512, 576), rnd(1, 576)
    ix, ig = engine.upload(x), engine.upload(g)
    y = engine.download(engine.rms_norm(ix, ig, 1e-5))
    got = engine.download(engine.rms_norm(ix, ig, 1e-5, form)).reshape(-1)
    same_bits(got, tiled(orc.to_bf16(y)) if form == TILES_BF16 else tiled_parts(y), np.uint16)


# (m, n, k): a batch-1 prefill's four products, one k step, the longest k.
SHAPES = [(512, 960, 576), (512, 576, 576), (512, 3072, 576), (512, 576, 1536), (32, 32, 16), (64, 96, 1536)]


def operand(engine, x, form):
    """x (F32 values) in one of the activation forms the tiled path reads."""
    if form == "f32":
        return engine.upload(x)
    if form == "bf16":
        return engine.upload_bf16(orc.to_bf16(x))
    return engine.tile(engine.upload(x), TILES_PARTS if form == "parts" else TILES_BF16)


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("form", ["f32", "bf16", "parts", "tiles_bf16"])
def test_linear_tiles_integer_exact(engine, m, n, k, form):
    x, w = ints(m, k), ints(n, k)
    bias, res = ints(1, n), ints(m, n, lo=-100, hi=100)
    iw = engine.tile(engine.upload_bf16(orc.to_bf16(w)), TILES_BF16)
    got = engine.download(engine.linear(operand(engine, x, form), iw, True, engine.upload(bias), engine.upload(res)))
    want = (x.astype(np.float64) @ w.T.astype(np.float64) + bias + res).astype(np.float32)
    same_bits(got, want)


@pytest.mark.parametrize("m,n,k", SHAPES[:4])
def test_linear_tiles_random_within_the_bound(engine, m, n, k):
    x, w = rnd(m, k), orc.to_bf16(rnd(n, k, scale=0.05))
    iw = engine.tile(engine.upload_bf16(w), TILES_BF16)
    wf = orc.from_bf16(w).astype(np.float64)
    got = engine.download(engine.linear(engine.upload(x), iw, True))
    p = split_parts(x)
    a = orc.from_bf16(p[:, :k]).astype(np.float64) + orc.from_bf16(p[:, k:]).astype(np.float64)
    want = a @ wf.T
    bound = 1e-5 * (np.abs(a) @ np.abs(wf).T) + 1e-30
    assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) / bound))
    # The same split made beforehand (mi_tile's parts): the same bits.
    same_bits(engine.download(engine.linear(engine.tile(engine.upload(x), TILES_PARTS), iw, True)), got)
    # BF16 rows and BF16 tiles: the same MFMA steps, the same bits.
    xb = engine.upload_bf16(orc.to_bf16(x))
    same_bits(engine.download(engine.linear(engine.tile(xb, TILES_BF16), iw, True)),
              engine.download(engine.linear(xb, iw, True)))


@pytest.mark.parametrize("form", ["f32", "parts", "tiles_bf16"])
@pytest.mark.parametrize("out", [F32, BF16, miburn.BF16_PARTS, TILES_BF16, TILES_PARTS])
def test_linear_swiglu_tiles_equals_composition(engine, form, out):
    m, k, inter = 512, 576, 1536
    x = rnd(m, k)
    gu = orc.to_bf16(rnd(2 * inter, k, scale=0.05))
    iw = engine.tile(engine.upload_bf16(pairs_of(gu, inter)), TILES_BF16)
    ix = operand(engine, x, form)
    prod = engine.download(engine.linear(ix, iw, True))  # interleaved columns: 32 gate, 32 up, ...
    halves = prod.reshape(m, inter // 32, 2, 32).transpose(0, 2, 1, 3).reshape(m, 2 * inter)
    y = engine.download(engine.silu_mul_halves(engine.upload(halves)))  # F32
    got = engine.download(engine.linear_swiglu(ix, iw, out))
    if out == F32:
        same_bits(got, y)
    elif out == BF16:
        same_bits(got, orc.to_bf16(y), np.uint16)
    elif out == miburn.BF16_PARTS:
        same_bits(got, split_parts(y), np.uint16)
    elif out == TILES_BF16:
        same_bits(got.reshape(-1), tiled(orc.to_bf16(y)), np.uint16)
    else:
        same_bits(got.reshape(-1), tiled_parts(y), np.uint16)


@pytest.mark.parametrize("batch,seq,heads,kvh,hidden,pos0,grouped,cache,form", [
    (1, 512, 9, 3, 576, 0, False, "f32", "parts"),   # the SmolLM2 batch-1 prompt
    (1, 512, 9, 3, 576, 0, True, "bf16", "tiles_bf16"),
    (2, 96, 4, 2, 256, 40, False, "f32", "f32"),     # positions after cached ones
    (2, 48, 4, 1, 128, 8, True, "bf16", "bf16"),     # 32-row tiles straddling sequences
])
def test_linear_qkv_rope_cache_tiles_equals_composition(engine, batch, seq, heads, kvh, hidden, pos0, grouped, cache,
                                                        form):
    D, maxc = 64, pos0 + seq + 16
    rows = batch * seq
    n = (heads + 2 * kvh) * D
    x = rnd(rows, hidden)
    iw = engine.tile(engine.upload_bf16(orc.to_bf16(rnd(n, hidden, scale=0.05))), TILES_BF16)
    ang = np.arange(maxc)[:, None] * (1e5 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    ic = engine.upload(np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32))
    is_ = engine.upload(np.concatenate([-np.sin(ang), np.sin(ang)], 1).astype(np.float32))
    ix = operand(engine, x, form)
    init = rnd(batch * kvh * maxc, D)

    def caches():
        if cache == "bf16":
            return engine.upload_bf16(orc.to_bf16(init)), engine.upload_bf16(orc.to_bf16(init))
        return engine.upload(init), engine.upload(init)
    k1, v1 = caches()
    q1 = engine.download(engine.qkv_rope_cache(engine.linear(ix, iw, True), ic, is_, seq, heads, kvh, pos0, k1, v1,
                                               grouped))
    k2, v2 = caches()
    q2 = engine.download(engine.linear_qkv_rope_cache(ix, False, iw, ic, is_, seq, heads, kvh, pos0, k2, v2, grouped))
    same_bits(q2, q1)
    view = np.uint16 if cache == "bf16" else np.uint32
    same_bits(engine.download(k2), engine.download(k1), view)
    same_bits(engine.download(v2), engine.download(v1), view)


@pytest.mark.parametrize("k,form", [(576, "f32"), (1536, "parts")])
@pytest.mark.parametrize("norm", [F32, miburn.BF16_PARTS, TILES_PARTS, TILES_BF16])
def test_linear_add_rms_norm_tiles_equals_composition(engine, k, form, norm):
    m, n = 512, 576
    x, r, g = rnd(m, k), rnd(m, n), rnd(1, n)
    iw = engine.tile(engine.upload_bf16(orc.to_bf16(rnd(n, k, scale=0.05))), TILES_BF16)
    ix, ir, ig = operand(engine, x, form), engine.upload(r), engine.upload(g)
    y1 = engine.linear(ix, iw, True, 0, ir)
    n1 = engine.download(engine.rms_norm(y1, ig, 1e-5, norm))
    y2, n2 = engine.linear_add_rms_norm(ix, iw, True, 0, ir, ig, 1e-5, norm)
    same_bits(engine.download(y2), engine.download(y1))
    same_bits(engine.download(n2), n1, np.uint32 if norm == F32 else np.uint16)


def test_tiles_refusals(engine):
    w = engine.upload_bf16(orc.to_bf16(rnd(64, 64)))
    iw = engine.tile(w, TILES_BF16)
    x = engine.upload(rnd(64, 64))

    def kind(call):
        with pytest.raises(miburn.MiError) as e:
            call()
        return e.value.kind
    assert kind(lambda: engine.matmul_dram(x, False, iw, True)) == "ARG"        # tiles through a plain product
    assert kind(lambda: engine.linear(x, iw, False)) == "ARG"                   # a tiled weight is [n, k]
    assert kind(lambda: engine.tile(iw, TILES_BF16)) == "ARG"                   # already tiles
    assert kind(lambda: engine.tile(w, TILES_PARTS)) == "ARG"                   # parts of BF16 values
    assert kind(lambda: engine.tile(engine.upload(rnd(40, 64)), TILES_BF16)) == "ARG"  # rows not in 32s
    assert kind(lambda: engine.reshape(iw, 32, 128)) == "ARG"
    assert kind(lambda: engine.rms_norm(iw)) == "ARG"
    assert kind(lambda: engine.rms_norm(engine.upload(rnd(40, 64)), 0, 1e-5, TILES_PARTS)) == "ARG"
    assert kind(lambda: engine.linear_parts(engine.upload_bf16(orc.to_bf16(rnd(64, 128))), iw, True)) == "ARG"
    assert kind(lambda: engine.linear(engine.upload(rnd(48, 64)), iw, True)) == "UNSUPPORTED"  # rows not in 32s
    big = engine.tile(engine.upload_bf16(orc.to_bf16(rnd(32, 1552))), TILES_BF16)
    assert kind(lambda: engine.linear(engine.upload(rnd(32, 1552)), big, True)) == "UNSUPPORTED"  # k past 1536
    engine.set_matmul_mode(miburn.MATMUL_ACCURATE)
    try:
        assert kind(lambda: engine.linear(x, iw, True)) == "UNSUPPORTED"  # F32 rows need the fast mode's split
        engine.download(engine.linear(engine.tile(x, TILES_PARTS), iw, True))  # parts made beforehand: any mode
    finally:
        engine.set_matmul_mode(miburn.MATMUL_FAST)
    engine.sync()


# (1, 512): the matrix-core kernel split over keys, then the combine; (32,
# 256): unsplit, item-major, each form stored by the kernel itself; (2, 16):
# the key-chunk kernels.
@pytest.mark.parametrize("batch,t,pos0,kv16", [(1, 512, 0, False), (1, 512, 0, True), (2, 128, 64, False),
                                               (32, 256, 0, False), (32, 256, 0, True), (2, 16, 8, False)])
@pytest.mark.parametrize("form", [BF16, miburn.BF16_PARTS, TILES_BF16, TILES_PARTS])
def test_attention_rows_as_equals_rows_then_form(engine, batch, t, pos0, kv16, form):
    H, KVH, D = 9, 3, 64
    maxc = pos0 + t + 8
    q = engine.upload(rnd(batch * t, H * D))
    kc, vc = rnd(batch * KVH * maxc, D), rnd(batch * KVH * maxc, D)
    if kv16:
        k, v = engine.upload_bf16(orc.to_bf16(kc)), engine.upload_bf16(orc.to_bf16(vc))
    else:
        k, v = engine.upload(kc), engine.upload(vc)
    scale = float(np.float32(1 / 8))
    y = engine.download(engine.attention_rows(q, k, v, batch, t, H, KVH, pos0, scale))
    got = engine.download(engine.attention_rows_as(q, k, v, batch, t, H, KVH, pos0, scale, form))
    if form == BF16:
        same_bits(got, orc.to_bf16(y), np.uint16)
    elif form == miburn.BF16_PARTS:
        same_bits(got, split_parts(y), np.uint16)
        # mi_cast's parts of the F32 rows: the same bits.
        same_bits(engine.download(engine.cast_float(engine.upload(y), miburn.BF16_PARTS)), split_parts(y), np.uint16)
    elif form == TILES_BF16:
        same_bits(got.reshape(-1), tiled(orc.to_bf16(y)), np.uint16)
    else:
        same_bits(got.reshape(-1), tiled_parts(y), np.uint16)
