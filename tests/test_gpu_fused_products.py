"""Device parity of the fused product entry points.

mi_linear (residual + (x op(w) + bias), the adds in the product's epilogue):
bit-identical to the engine's own product followed by the two F32 adds (the
product itself is pinned against the oracle by the matmul tests), for every
kernel a shape selects -- the GEMV, split-K, the 64x64 tiles guarded and
exact, the fast mode's split kernel, both direct-to-LDS BF16 kernels -- and
within the matmul bound of the oracle.

mi_linear_parts (an F32 operand given as its BF16 parts, MI_BF16_PARTS): bit
for bit the fast mode's own linear where that splits the operand itself,
and within the F32 bound of float64 on the other shapes; the parts that
mi_rms_norm and mi_silu_mul_halves produce are bit for bit the split of
their F32 results (the split restated here in numpy and checked on
hand-worked values); mi_linear_swiglu_parts is bit for bit that product
against [gate; up] followed by the SiLU-mul to parts, mi_linear_qkv_rope_cache
the q|k|v product followed by mi_qkv_rope_cache (q and both caches).

mi_matmul_items (grouped strided items written in place): each item within
the F32 accumulation bound of the oracle's product of the same blocks, the
rest of the result buffer untouched, on the transformer's head layout and on
single strided items that take the GEMV and split-K paths.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc
from miburn import BF16, F32

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(7_2024)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def same_bits(a, b, view=np.uint32):
    a = np.ascontiguousarray(a).view(view)
    b = np.ascontiguousarray(b).view(view)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{bad.size} datums differ, first at {bad[0]}: {a.ravel()[bad[0]]:#x} vs {b.ravel()[bad[0]]:#x}"


def mm_tol(a, b, rel):
    return rel * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))


@pytest.fixture(params=["fast", "accurate"])
def mode(request, engine):
    engine.set_matmul_mode(miburn.MATMUL_FAST if request.param == "fast" else miburn.MATMUL_ACCURATE)
    yield request.param
    engine.set_matmul_mode(miburn.MATMUL_FAST)


# (m, n, k, w transposed, operand kind, the kernel it selects)
LINEAR_SHAPES = [
    (4, 576, 1536, True, "f32", "gemv"),
    (3, 576, 1536, True, "w_bf16", "gemv bf16 weight"),
    (64, 256, 2048, False, "f32", "split-K"),
    (2048, 256, 256, False, "f32", "64x64 exact"),
    (100, 70, 33, False, "f32", "64x64 guarded"),
    (2048, 2048, 2048, False, "f32", "fast: split kernel"),
    (2048, 2048, 512, True, "bf16", "direct 128x128"),
    (4096, 4096, 256, False, "bf16", "direct 256x256"),
    (16384, 960, 576, True, "w_bf16", "fast: split kernel, 128-aligned columns + edge"),
    (5, 7, 0, False, "f32", "empty sums"),
]


@pytest.mark.parametrize("m,n,k,tw,kind,path", LINEAR_SHAPES, ids=[s[-1] for s in LINEAR_SHAPES])
@pytest.mark.parametrize("terms", ["bias", "residual", "both", "none"])
def test_linear_equals_product_then_adds(engine, mode, m, n, k, tw, kind, path, terms):
    x = rnd(m, k)
    w = rnd(n, k) if tw else rnd(k, n)
    if kind == "bf16":
        ix, iw = engine.upload_bf16(orc.to_bf16(x)), engine.upload_bf16(orc.to_bf16(w))
    elif kind == "w_bf16":
        ix, iw = engine.upload(x), engine.upload_bf16(orc.to_bf16(w))
    else:
        ix, iw = engine.upload(x), engine.upload(w)
    bias = rnd(1, n)
    resid = rnd(m, n)
    ib = engine.upload(bias) if terms in ("bias", "both") else 0
    ir = engine.upload(resid) if terms in ("residual", "both") else 0
    got = engine.download(engine.linear(ix, iw, tw, ib, ir))
    mm = engine.download(engine.matmul_dram(ix, False, iw, tw)) if k else np.zeros((m, n), np.float32)
    want = mm
    if ib:
        want = want + bias
    if ir:
        want = resid + want
    same_bits(got, want.astype(np.float32))
    if k and kind == "f32":
        wf = w.T if tw else w
        ref = orc.matmul(x, wf, threads=16).astype(np.float64)
        if ib:
            ref = ref + bias
        if ir:
            ref = resid + ref
        assert np.all(np.abs(got - ref) <= mm_tol(x, wf, 1e-5) + 1e-6 * (np.abs(ref) + 1e-30))


@pytest.mark.parametrize("m,n,k", [(16384, 960, 576), (16384, 576, 1536)])
def test_split_kernel_column_blocks_against_oracle(engine, m, n, k):
    """Widths that are not a multiple of 128 on the fast mode's split kernel:
    the 128-aligned columns and the rest run as two launches.  Rows sampled
    against float64 within the normwise F32 bound."""
    x = rnd(m, k)
    wb = orc.to_bf16(rnd(n, k))
    got = engine.download(engine.matmul_dram(engine.upload(x), False, engine.upload_bf16(wb), True))
    w = orc.from_bf16(wb).astype(np.float64)
    sel = np.r_[0:64, m // 2:m // 2 + 64, m - 64:m]
    xs = x[sel].astype(np.float64)
    ref = xs @ w.T
    assert np.all(np.abs(got[sel] - ref) <= 1e-5 * (np.abs(xs) @ np.abs(w).T) + 1e-30)


def test_linear_bf16_result_rounds_once_after_the_adds(engine):
    x, w, bias, resid = rnd(300, 200), rnd(200, 136), rnd(1, 136), rnd(300, 136)
    ix, iw, ib, ir = engine.upload(x), engine.upload(w), engine.upload(bias), engine.upload(resid)
    f32 = engine.download(engine.linear(ix, iw, False, ib, ir))
    bf = engine.download(engine.linear(ix, iw, False, ib, ir, BF16))
    same_bits(bf, orc.to_bf16(f32), np.uint16)


def test_linear_argument_errors(engine):
    ix, iw = engine.upload(rnd(8, 16)), engine.upload(rnd(16, 32))
    for bad in (engine.upload(rnd(1, 31)), engine.upload_bf16(orc.to_bf16(rnd(1, 32)))):
        with pytest.raises(miburn.MiError) as e:
            engine.linear(ix, iw, False, bad, 0)
        assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:
        engine.linear(ix, iw, False, 0, engine.upload(rnd(8, 31)))
    assert e.value.kind == "ARG"


# ------------------------------------------------ F32 operands as BF16 parts
def split_parts(y):
    """[rows, cols] F32 -> [rows, 2 cols] BF16 bits: each row's heads (round to
    nearest even through the oracle's cast; a finite value that would round to
    infinity keeps its truncated head), then the BF16 of the exact remainders
    (0 where the remainder is NaN: an infinite value)."""
    y = np.ascontiguousarray(y, np.float32)
    u = y.view(np.uint32)
    hi = orc.to_bf16(y)
    ovf = ((hi & 0x7FFF) == 0x7F80) & ((u & 0x7F800000) != 0x7F800000)
    hi = np.where(ovf, (u >> 16).astype(np.uint16), hi)
    with np.errstate(invalid="ignore"):
        r = (y.astype(np.float64) - orc.from_bf16(hi).astype(np.float64)).astype(np.float32)
    lo = np.where(np.isnan(r), np.uint16(0), orc.to_bf16(np.nan_to_num(r)))
    return np.concatenate([hi, lo], axis=1)


def test_split_parts_reference_cases():
    """The test's own split against hand-worked values: an exact BF16 value
    has no remainder; 1 + 2^-9 rounds its head to 1 (ties to even) and keeps
    2^-9; the largest F32 keeps its truncated head 0x7f7f, its remainder
    (2^16 - 1) 2^104 rounding up to 2^120; infinity is its head alone."""
    y = np.array([[1.5, 1 + 2.0 ** -9, np.finfo(np.float32).max, np.inf]], np.float32)
    p = split_parts(y)
    assert list(p[0, :4]) == [0x3FC0, 0x3F80, 0x7F7F, 0x7F80]
    lo = orc.from_bf16(p[:, 4:])[0]
    assert lo[0] == 0 and lo[1] == 2.0 ** -9 and lo[3] == 0
    assert lo[2] == 2.0 ** 120


@pytest.mark.parametrize("rows,cols", [(64, 576), (300, 1000), (5, 8192), (8195, 576)])
def test_rms_norm_parts_split_its_f32_result(engine, rows, cols):
    x = rnd(rows, cols)
    gamma = rnd(1, cols)
    gamma[0, :3] = [3.4e38, -3.39e38, 1e38]  # heads past the largest BF16, infinities
    ix, ig = engine.upload(x), engine.upload(gamma)
    f32 = engine.download(engine.rms_norm(ix, ig, 1e-5))
    parts = engine.download(engine.rms_norm(ix, ig, 1e-5, miburn.BF16_PARTS))
    same_bits(parts, split_parts(f32), np.uint16)


@pytest.mark.parametrize("rows,inner", [(64, 1536), (33, 7), (4, 4)])
def test_silu_mul_halves_parts_split_its_f32_result(engine, rows, inner):
    gu = rnd(rows, 2 * inner, scale=4.0)
    ig = engine.upload(gu)
    f32 = engine.download(engine.silu_mul_halves(ig))
    parts = engine.download(engine.silu_mul_halves(ig, miburn.BF16_PARTS))
    same_bits(parts, split_parts(f32), np.uint16)


# (m, n, k): shapes the fast mode splits into stacked parts for F32 x.
@pytest.mark.parametrize("m,n,k,terms", [(16384, 960, 576, "none"), (16384, 576, 1536, "residual"),
                                         (16384, 3072, 576, "both")])
def test_linear_parts_equals_the_fast_linear(engine, m, n, k, terms):
    """Where the fast mode's mi_linear splits F32 activations itself, the
    product from parts made elsewhere is the same, bit for bit."""
    x = rnd(m, k)
    w = orc.to_bf16(rnd(n, k))
    ix, iw = engine.upload(x), engine.upload_bf16(w)
    ip = engine.upload_bf16(split_parts(x))
    ib = engine.upload(rnd(1, n)) if terms == "both" else 0
    ir = engine.upload(rnd(m, n)) if terms != "none" else 0
    want = engine.download(engine.linear(ix, iw, True, ib, ir))
    got = engine.download(engine.linear_parts(ip, iw, True, ib, ir))
    same_bits(got, want)
    engine.set_matmul_mode(miburn.MATMUL_ACCURATE)
    try:
        again = engine.download(engine.linear_parts(ip, iw, True, ib, ir))
    finally:
        engine.set_matmul_mode(miburn.MATMUL_FAST)
    same_bits(again, want)


@pytest.mark.parametrize("m,n,k,tw", [(100, 70, 48, True), (512, 256, 64, False), (256, 300, 32, False),
                                      (512, 512, 40, True), (3, 576, 1536, True), (7, 5, 0, True),
                                      (384, 960, 576, True), (4096, 576, 1536, True), (2048, 3072, 576, True)])
def test_linear_parts_other_shapes(engine, m, n, k, tw):
    """The direct kernel's 128 x 128 tiles (edge tiles for widths of 16s) and
    shapes outside its tiling (the weight repeated along k): the sums head . w
    + remainder . w within the F32 accumulation bound of float64."""
    x = rnd(m, k)
    wb = orc.to_bf16(rnd(n, k) if tw else rnd(k, n))
    p = split_parts(x)
    bias, resid = rnd(1, n), rnd(m, n)
    got = engine.download(engine.linear_parts(engine.upload_bf16(p), engine.upload_bf16(wb), tw,
                                              engine.upload(bias), engine.upload(resid)))
    w = orc.from_bf16(wb).astype(np.float64)
    w = w.T if tw else w
    a = orc.from_bf16(p).astype(np.float64)
    xs = a[:, :k] + a[:, k:]
    ref = resid + (xs @ w + bias)
    tol = 1e-5 * (np.abs(xs) @ np.abs(w)) + 1e-6 * (np.abs(ref) + np.abs(bias) + np.abs(resid)) + 1e-30
    assert got.shape == (m, n)
    assert np.all(np.abs(got - ref) <= tol)


def pairs_of(gu, inter):
    """[gate; up] rows [2 i, k] -> rows interleaved in 32-row groups."""
    k = gu.shape[1]
    return np.ascontiguousarray(gu.reshape(2, inter // 32, 32, k).transpose(1, 0, 2, 3).reshape(2 * inter, k))


@pytest.mark.parametrize("m,k,inter", [(16384, 576, 1536), (4096, 576, 1536), (512, 576, 1536), (256, 64, 128)])
def test_linear_swiglu_parts_equals_composition(engine, m, k, inter):
    """The fused SwiGLU half from interleaved weights: bit for bit the
    product from parts against [gate; up] then the SiLU-mul to parts (256 x
    256 tiles at 4096+ rows, 128 x 128 below)."""
    x = rnd(m, k)
    gu = orc.to_bf16(rnd(2 * inter, k, scale=0.05))
    ip = engine.upload_bf16(split_parts(x))
    want = engine.download(engine.silu_mul_halves(engine.linear_parts(ip, engine.upload_bf16(gu), True),
                                                  miburn.BF16_PARTS))
    got = engine.download(engine.linear_swiglu_parts(ip, engine.upload_bf16(pairs_of(gu, inter))))
    assert got.shape == (m, 2 * inter)
    same_bits(got, want, np.uint16)


@pytest.mark.parametrize("m,k,inter", [(16384, 576, 1536), (512, 576, 1536), (256, 64, 128)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_linear_swiglu_equals_composition(engine, m, k, inter, out):
    """BF16 activations: bit for bit the BF16 product against [gate; up]
    (the direct kernel at these shapes) then the SiLU-mul, F32 or rounded to
    BF16."""
    oe = BF16 if out == "bf16" else F32
    ix = engine.upload_bf16(orc.to_bf16(rnd(m, k)))
    gu = orc.to_bf16(rnd(2 * inter, k, scale=0.05))
    want = engine.download(engine.silu_mul_halves(engine.matmul_dram(ix, False, engine.upload_bf16(gu), True), oe))
    got = engine.download(engine.linear_swiglu(ix, engine.upload_bf16(pairs_of(gu, inter)), oe))
    assert got.shape == (m, inter)
    same_bits(got, want, np.uint16 if oe == BF16 else np.uint32)


QKV_CASES = [  # (batch, seq, heads, kv heads, hidden, pos0, grouped, cache)
    (32, 512, 9, 3, 576, 0, False, "f32"),   # the SmolLM2 batch-32 prompt: 256 x 256 tiles, an edge tile column
    (8, 512, 9, 3, 576, 0, True, "bf16"),    # 4096 rows, grouped queries, a BF16 cache
    (2, 256, 4, 2, 256, 64, False, "f32"),   # 512 rows on 128 x 128 tiles, positions after cached ones
    # 4608 rows of 144-token sequences: 32-row fragments straddle two
    # sequences, so the epilogue finds each row's sequence and position itself
    (32, 144, 9, 3, 576, 8, True, "bf16"),
]


@pytest.mark.parametrize("batch,seq,heads,kvh,hidden,pos0,grouped,cache", QKV_CASES)
@pytest.mark.parametrize("parts", [True, False])
def test_linear_qkv_rope_cache_equals_composition(engine, batch, seq, heads, kvh, hidden, pos0, grouped, cache, parts):
    """The q|k|v product with RoPE, cache writes and q's layout in its
    epilogue: q and both caches (every row, the untouched ones included) bit
    for bit the product followed by mi_qkv_rope_cache."""
    D, maxc = 64, pos0 + seq + 32
    rows = batch * seq
    n = (heads + 2 * kvh) * D
    x = rnd(rows, hidden)
    w = engine.upload_bf16(orc.to_bf16(rnd(n, hidden, scale=0.05)))
    ang = np.arange(maxc)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32)
    sin = np.concatenate([-np.sin(ang), np.sin(ang)], 1).astype(np.float32)
    ic, is_ = engine.upload(cos), engine.upload(sin)
    if parts:
        ix = engine.upload_bf16(split_parts(x))
        qkv = engine.linear_parts(ix, w, True)
    else:
        ix = engine.upload_bf16(orc.to_bf16(x))
        qkv = engine.matmul_dram(ix, False, w, True)
    init = rnd(batch * kvh * maxc, D)
    def caches():
        if cache == "bf16":
            return engine.upload_bf16(orc.to_bf16(init)), engine.upload_bf16(orc.to_bf16(init))
        return engine.upload(init), engine.upload(init)
    k1, v1 = caches()
    q1 = engine.download(engine.qkv_rope_cache(qkv, ic, is_, seq, heads, kvh, pos0, k1, v1, grouped))
    k2, v2 = caches()
    q2 = engine.download(engine.linear_qkv_rope_cache(ix, parts, w, ic, is_, seq, heads, kvh, pos0, k2, v2, grouped))
    same_bits(q2, q1)
    view = np.uint16 if cache == "bf16" else np.uint32
    same_bits(engine.download(k2), engine.download(k1), view)
    same_bits(engine.download(v2), engine.download(v1), view)


def test_linear_qkv_rope_cache_refuses(engine):
    w = engine.upload_bf16(orc.to_bf16(rnd(8 * 64, 128)))
    ic = engine.upload(rnd(64, 64))
    k, v = engine.upload(rnd(2 * 2 * 64, 64)), engine.upload(rnd(2 * 2 * 64, 64))
    with pytest.raises(miburn.MiError) as e:  # 100 rows: not whole 128-row tiles
        engine.linear_qkv_rope_cache(engine.upload_bf16(orc.to_bf16(rnd(100, 128))), False, w, ic, ic, 50, 4, 2, 0, k, v)
    assert e.value.kind == "UNSUPPORTED"
    with pytest.raises(miburn.MiError) as e:  # the weight's rows are not (heads + 2 kv heads) x 64
        engine.linear_qkv_rope_cache(engine.upload_bf16(orc.to_bf16(rnd(128, 128))), False, w, ic, ic, 64, 2, 1, 0,
                                     k, v)
    assert e.value.kind == "ARG"


def test_linear_swiglu_parts_refuses_partial_tiles(engine):
    w = engine.upload_bf16(orc.to_bf16(rnd(256, 64)))
    for rows, cols, kind in ((200, 128, "UNSUPPORTED"), (256, 127, "ARG")):
        with pytest.raises(miburn.MiError) as e:
            engine.linear_swiglu_parts(engine.upload_bf16(orc.to_bf16(rnd(rows, cols))), w)
        assert e.value.kind == kind
    with pytest.raises(miburn.MiError) as e:  # 192 weight rows: 96 outputs, not a whole tile column
        engine.linear_swiglu_parts(engine.upload_bf16(orc.to_bf16(rnd(256, 128))),
                                   engine.upload_bf16(orc.to_bf16(rnd(192, 64))))
    assert e.value.kind == "UNSUPPORTED"
    for x, kind in ((engine.upload_bf16(orc.to_bf16(rnd(200, 64))), "UNSUPPORTED"), (engine.upload(rnd(256, 64)), "ARG")):
        with pytest.raises(miburn.MiError) as e:
            engine.linear_swiglu(x, w)
        assert e.value.kind == kind


def test_linear_parts_argument_errors(engine):
    iw = engine.upload_bf16(orc.to_bf16(rnd(32, 16)))
    for bad in (engine.upload_bf16(orc.to_bf16(rnd(8, 31))),   # odd width
                engine.upload(rnd(8, 32)),                      # F32, not parts
                engine.upload_bf16(orc.to_bf16(rnd(8, 48)))):   # k 24 against the weight's 16
        with pytest.raises(miburn.MiError) as e:
            engine.linear_parts(bad, iw, True)
        assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:  # an F32 weight
        engine.linear_parts(engine.upload_bf16(orc.to_bf16(rnd(8, 32))), engine.upload(rnd(32, 16)), True)
    assert e.value.kind == "ARG"


# ------------------------------------------------------------ strided items
SENTINEL = np.float32(-1234.5)


def head_layout(B, H, S, dk):
    """The transformer's placements: q | k | v inside [B*S, 3d], the heads'
    outputs inside [B*S, d], scores stored item after item."""
    d, W = H * dk, 3 * H * dk
    return dict(q=(0, S * W, dk), k=(d, S * W, dk), v=(2 * d, S * W, dk), o=(0, S * d, dk),
                s=(0, H * S * S, S * S))


def block(buf, at, g, i, rows, cols):
    flat = buf.ravel()
    ld = buf.shape[1]
    start = at[0] + g * at[1] + i * at[2]
    return np.stack([flat[start + r * ld:start + r * ld + cols] for r in range(rows)])


def check_items(got, before, at, groups, per_group, want_fn, m, n, tol_fn):
    """Each result item against want_fn(g, i); everything else unchanged."""
    touched = np.zeros(got.size, bool)
    ld = got.shape[1]
    for g in range(groups):
        for i in range(per_group):
            start = at[0] + g * at[1] + i * at[2]
            for r in range(m):
                touched[start + r * ld:start + r * ld + n] = True
            want = want_fn(g, i)
            item = block(got, at, g, i, m, n)
            assert np.all(np.abs(item - want) <= tol_fn(g, i) + 1e-30), (g, i)
    same_bits(got.ravel()[~touched], before.ravel()[~touched])


@pytest.mark.parametrize("B,H,S,dk", [(3, 4, 40, 16), (2, 4, 128, 64)])
def test_matmul_items_attention_products(engine, mode, B, H, S, dk):
    """The four attention products of the transformer's forward and backward
    straight out of the fused projection, results written into place."""
    d, W = H * dk, 3 * H * dk
    R = B * S
    at = head_layout(B, H, S, dk)
    qkv, dom, p = rnd(R, W), rnd(R, d), rnd(B * H * S, S)
    iqkv, idom, ip = engine.upload(qkv), engine.upload(dom), engine.upload(p)

    def run(a, ta, a_at, b, tb, b_at, m, k, n, out_shape, out_at, A, Bm):
        before = np.full(out_shape, SENTINEL, np.float32)
        before.ravel()[::7] = rnd(before.size // 7 + 1)[: before.ravel()[::7].size]
        io = engine.upload(before)
        engine.matmul_items(a, ta, a_at, b, tb, b_at, B, H, m, k, n, io, out_at)
        got = engine.download(io)

        def operand(buf, at_, g, i, trans, rows, cols):
            blk = block(buf, at_, g, i, cols if trans else rows, rows if trans else cols)
            return blk.T if trans else blk

        def want(g, i):
            return orc.matmul(operand(A, a_at, g, i, ta, m, k), operand(Bm, b_at, g, i, tb, k, n))

        def tol(g, i):
            return mm_tol(operand(A, a_at, g, i, ta, m, k), operand(Bm, b_at, g, i, tb, k, n), 1e-5)

        check_items(got, before, out_at, B, H, want, m, n, tol)

    # scores = q k^T
    run(iqkv, False, at["q"], iqkv, True, at["k"], S, dk, S, (B * H * S, S), at["s"], qkv, qkv)
    # o = p v, merged into [R, d]
    run(ip, False, at["s"], iqkv, False, at["v"], S, S, dk, (R, d), at["o"], p, qkv)
    # dv = p^T do, into the v columns of [R, 3d]
    run(ip, True, at["s"], idom, False, at["o"], S, S, dk, (R, W), at["v"], p, dom)
    # dp = do v^T
    run(idom, False, at["o"], iqkv, True, at["v"], S, dk, S, (B * H * S, S), at["s"], dom, qkv)


def test_matmul_items_bf16_operands_into_bf16(engine):
    B, H, S, dk = 2, 2, 64, 64
    at = head_layout(B, H, S, dk)
    qkv = orc.to_bf16(rnd(B * S, 3 * H * dk))
    iq = engine.upload_bf16(qkv)
    io = engine.fill(B * H * S, S, BF16, 0)
    engine.matmul_items(iq, False, at["q"], iq, True, at["k"], B, H, S, dk, S, io, at["s"])
    got = miburn.bf16_to_f32(engine.download(io))
    qf = orc.from_bf16(qkv)
    for g in range(B):
        for i in range(H):
            q = block(qf, at["q"], g, i, S, dk)
            k = block(qf, at["k"], g, i, S, dk)
            want = q.astype(np.float64) @ k.T.astype(np.float64)
            item = block(got, at["s"], g, i, S, S)
            tol = 2.0 ** -8 * np.abs(want) + mm_tol(q, k.T, 1e-5)
            assert np.all(np.abs(item - want) <= tol), (g, i)


@pytest.mark.parametrize("m,k,n,tb,path", [(4, 1536, 96, True, "gemv"), (64, 2048, 128, False, "split-K"),
                                           (96, 80, 72, False, "tiled")])
def test_matmul_items_single_strided_item(engine, m, k, n, tb, path):
    """One item (groups = per_group = 1) written at an offset inside a wider
    buffer: the result pitch is the buffer's, on every path."""
    a = rnd(m, k)
    b = rnd(n, k) if tb else rnd(k, n)
    out_shape = (m + 3, n + 40)
    before = rnd(*out_shape)
    io = engine.upload(before)
    at = (2 * out_shape[1] + 17, 0, 0)
    engine.matmul_items(engine.upload(a), False, (0, 0, 0), engine.upload(b), tb, (0, 0, 0), 1, 1, m, k, n, io, at)
    got = engine.download(io)
    bb = b.T if tb else b
    check_items(got, before, at, 1, 1, lambda g, i: orc.matmul(a, bb, threads=16), m, n,
                lambda g, i: mm_tol(a, bb, 1e-5))


def test_matmul_items_argument_errors(engine):
    a = engine.upload(rnd(64, 64))
    out = engine.empty(64, 64)
    z = (0, 0, 0)
    cases = [
        lambda: engine.matmul_items(a, False, z, a, False, z, 1, 1, 64, 64, 64, a, z),          # result is an operand
        lambda: engine.matmul_items(a, False, (1, 0, 0), a, False, z, 1, 1, 64, 64, 64, out, z),  # A past the end
        lambda: engine.matmul_items(a, False, z, a, False, z, 2, 1, 64, 64, 64, out, (0, 4096, 0)),  # result past
        lambda: engine.matmul_items(a, False, z, a, False, z, 1, 1, 64, 0, 64, out, z),          # k = 0
        lambda: engine.matmul_items(a, False, z, a, False, z, 1, 1, 65, 64, 64, out, z),         # m > rows
        lambda: engine.matmul_items(a, False, (0, -1, 0), a, False, z, 2, 1, 8, 8, 8, out, z),   # negative stride
    ]
    for c in cases:
        with pytest.raises(miburn.MiError) as e:
            c()
        assert e.value.kind == "ARG"


def test_empty_has_shape_and_kind(engine):
    i = engine.empty(7, 9, BF16)
    assert engine.metadata(i) == (7, 9, BF16)
    engine.free(i)


# ------------------------------------------------------ fused cross-entropy
def ce_composition(engine, iz, it, rows, cols, inv):
    """The composition the fused kernel replaces, op by op on the engine:
    log-softmax, gather at the target, exp, one-hot scattered, MUL_ADD."""
    logp = engine.softmax_rows(iz, 0, 1.0, True)
    picked = engine.download(engine.pick_columns(logp, it))
    minus = np.full((rows, 1), -inv, np.float32)
    onehot = engine.scatter_add_columns(engine.fill(rows, cols, F32, 0), it, engine.upload(minus))
    scale = engine.upload(np.full((1, 1), inv, np.float32))
    dz = engine.download(engine.eltwise_op_as("MUL_ADD", engine.eltwise_op_as("EXP", logp), scale, onehot))
    return picked, dz


@pytest.mark.parametrize("rows,cols", [(2048, 8192), (300, 8192), (4100, 4096), (8200, 2048), (64, 10), (37, 1001),
                                       (16, 16384), (5, 1024), (7, 3000)])
def test_log_softmax_ce_equals_composition(engine, rows, cols):
    z = rnd(rows, cols, scale=3.0)
    tgt = RNG.integers(0, cols, (rows, 1)).astype(np.int32)
    iz, it = engine.upload(z), engine.upload_i32(tgt)
    inv = np.float32(1.0 / rows)
    ip, idz = engine.log_softmax_ce(iz, it, float(inv))
    got_p, got_dz = engine.download(ip), engine.download(idz)
    want_p, want_dz = ce_composition(engine, iz, it, rows, cols, float(inv))
    same_bits(got_p, want_p)
    same_bits(got_dz, want_dz)
    # And against float64: logp at the target, softmax / rows minus the one-hot.
    z64 = z.astype(np.float64)
    lse = np.log(np.exp(z64 - z64.max(1, keepdims=True)).sum(1, keepdims=True)) + z64.max(1, keepdims=True)
    logp = z64 - lse
    assert np.allclose(got_p[:, 0], logp[np.arange(rows), tgt[:, 0]], rtol=1e-5, atol=1e-5)
    ref = np.exp(logp) / rows
    ref[np.arange(rows), tgt[:, 0]] -= 1.0 / rows
    assert np.all(np.abs(got_dz - ref) <= 1e-5 * np.abs(ref) + 1e-6 / rows)


@pytest.mark.parametrize("rows,cols", [(2048, 8192), (16, 16384)])
def test_log_softmax_ce_nan_rows(engine, rows, cols):
    # A NaN or +inf logit makes its row's loss and gradient NaN, as in the
    # composition; the other rows keep their bits.
    z = rnd(rows, cols, scale=3.0)
    z[1, 3], z[2, 9] = np.nan, np.inf
    tgt = RNG.integers(0, cols, (rows, 1)).astype(np.int32)
    iz, it = engine.upload(z), engine.upload_i32(tgt)
    inv = float(np.float32(1.0 / rows))
    ip, idz = engine.log_softmax_ce(iz, it, inv)
    got_p, got_dz = engine.download(ip), engine.download(idz)
    want_p, want_dz = ce_composition(engine, iz, it, rows, cols, inv)
    bad = np.zeros(rows, bool)
    bad[1:3] = True
    assert np.isnan(got_p[bad]).all() and np.isnan(got_dz[bad]).all()
    assert np.isnan(want_p[bad]).all() and np.isnan(want_dz[bad]).all()
    same_bits(got_p[~bad], want_p[~bad])
    same_bits(got_dz[~bad], want_dz[~bad])


def test_log_softmax_ce_target_out_of_range_is_domain(engine):
    engine.sync()
    iz = engine.upload(rnd(4, 64))
    it = engine.upload_i32(np.array([[1], [64], [3], [-1]], np.int32))
    ip, idz = engine.log_softmax_ce(iz, it, 0.25)
    with pytest.raises(miburn.MiError) as e:
        engine.sync()
    assert e.value.kind == "DOMAIN"
    engine.sync()
    p = engine.download(ip)
    assert p[1, 0] == 0.0 and p[3, 0] == 0.0


# --------------------------------------------- split-K slices folded by SGD
@pytest.mark.parametrize("m,n,k,ta,sliced", [(256, 256, 2048, True, True), (1024, 256, 2048, True, True),
                                             (256, 768, 2048, True, True), (64, 128, 784, False, True),
                                             (2048, 1024, 256, False, False)])
def test_matmul_slices_sum_to_the_product(engine, m, n, k, ta, sliced):
    a = rnd(k, m) if ta else rnd(m, k)
    b = rnd(k, n)
    ia, ib = engine.upload(a), engine.upload(b)
    sid, S = engine.matmul_slices(ia, ta, ib, False)
    parts = engine.download(sid)
    assert parts.shape == (S * m, n)
    total = parts[:m].copy()
    for z in range(1, S):  # slice order, F32 adds: split-K's own reduce
        total = (total + parts[z * m:(z + 1) * m]).astype(np.float32)
    same_bits(total, engine.download(engine.matmul_dram(ia, ta, ib, False)))
    # Long-k weight-gradient shapes are sliced; a full wave of tiles is one slice.
    assert (S > 1) == sliced


def test_sgd_folds_stacked_slices(engine):
    lr = np.float32(0.05)
    # A weight gradient from slices, against the same update from the reduced product.
    x, dy = rnd(2048, 256), rnd(2048, 256)
    ix, idy = engine.upload(x), engine.upload(dy)
    sid, S = engine.matmul_slices(ix, True, idy, False)
    assert S > 1
    p = rnd(256, 256)
    p1, p2 = engine.upload(p), engine.upload(p)
    engine.sgd_update([p1], [sid], float(lr))
    engine.sgd_update([p2], [engine.matmul_dram(ix, True, idy, False)], float(lr))
    same_bits(engine.download(p1), engine.download(p2))
    # Widths that are not a multiple of 4 take the scalar path.
    q = rnd(1, 7)
    g = rnd(3, 7)
    iq = engine.upload(q)
    engine.sgd_update([iq], [engine.upload(g)], float(lr))
    gsum = ((g[0] + g[1]).astype(np.float32) + g[2]).astype(np.float32)
    same_bits(engine.download(iq), (q - gsum * lr).astype(np.float32))
    with pytest.raises(miburn.MiError):
        engine.sgd_update([iq], [engine.upload(rnd(1, 10))], 0.1)  # 10 gradients for 7 parameters


# (m, k, n, x kind): a short prompt's o and down projections (the product
# splits over k, so the reduce forms the norm), and shapes that do not split.
LIN_NORM_CASES = [(512, 576, 576, "f32"), (512, 1536, 576, "f32"), (512, 1536, 576, "bf16"), (64, 512, 1000, "f32"),
                  (4096, 576, 576, "f32"), (4096, 1536, 576, "bf16"), (3, 576, 576, "f32")]


@pytest.mark.parametrize("m,k,n,xk", LIN_NORM_CASES)
@pytest.mark.parametrize("norm_elem", ["f32", "bf16", "parts"])
def test_linear_add_rms_norm_equals_linear_then_norm(engine, m, k, n, xk, norm_elem):
    """mi_linear_add_rms_norm: y and its RMSNorm bit for bit mi_linear then
    mi_rms_norm, with and without bias and gain."""
    ne = {"f32": miburn.F32, "bf16": miburn.BF16, "parts": miburn.BF16_PARTS}[norm_elem]
    x32 = rnd(m, k)
    x = engine.upload(x32) if xk == "f32" else engine.upload_bf16(orc.to_bf16(x32))
    w = engine.upload_bf16(orc.to_bf16(rnd(n, k, scale=0.05)))
    r = engine.upload(rnd(m, n))
    g = engine.upload(rnd(1, n) + np.float32(1.0))
    b = engine.upload(rnd(1, n, scale=0.1))
    for bias, gamma in ((0, g), (b, 0)):
        y, yn = engine.linear_add_rms_norm(x, w, True, bias=bias, residual=r, gamma=gamma, eps=1e-5, norm_elem=ne)
        y2 = engine.linear(x, w, True, bias=bias, residual=r)
        yn2 = engine.rms_norm(y2, gamma, 1e-5, ne)
        same_bits(engine.download(y), engine.download(y2))
        assert np.array_equal(engine.download(yn).view(np.uint32) if ne == miburn.F32 else engine.download(yn),
                              engine.download(yn2).view(np.uint32) if ne == miburn.F32 else engine.download(yn2))
        for t in (y, yn, y2, yn2):
            engine.free(t)
