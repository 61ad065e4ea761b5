"""Device parity of the prefill's fused tails.

mi_rope and mi_copy_into4 on their own, against numpy: RoPE bit for bit
against the reference's composition `x cos + rotate_half(x) sin` in F32
(crates/tt-models/src/rope.rs:6-60, 128-135; two products and a sum, each
rounded) and within 1e-6 of the float64 rotation of each pair (i, i + d/2)
by the angle pos * theta^(-2i/d); the strided 4-D copy bit for bit against a
numpy strided assignment, the rest of the destination untouched.

mi_qkv_rope_cache (RoPE on the q and k heads of the fused q|k|v rows, the
cache writes, q in either layout; float4 rows for head widths of a multiple
of 8, the element-wise form otherwise): bit-identical to the engine's own
composition -- mi_rope on the q and k blocks, mi_copy_into4 of k and v into
the caches, mi_copy_strided4 for the regrouped queries (mi_rope and
mi_copy_into4 checked against numpy above, mi_copy_strided4 against the
oracle in test_gpu_ops.py) -- with every cache row outside the written
positions left as it was.

mi_silu_mul_halves: bit-identical to MI_K_SILU_MUL of the two halves, on the
vector and the scalar paths.

BF16 storage (the performance numeric contract's KV cache and activation
operands): mi_qkv_rope_cache into BF16 caches writes exactly the F32 form's
values rounded to nearest even (the oracle's pinned cast) and the same q;
mi_silu_mul_halves to BF16 is its F32 result so rounded.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(31_2024)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, f"{bad.size} datums differ, first at {bad[0]}"


@pytest.fixture(scope="module")
def engine():
    e = miburn.Engine(0)
    yield e
    e.close()


def rope_tables(n, d, theta=1e5):
    inv = theta ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(n)[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32)
    sin = np.concatenate([-np.sin(ang), np.sin(ang)], 1).astype(np.float32)
    return cos, sin


@pytest.mark.parametrize("heads,seq,d,pos0", [(9, 40, 64, 0), (3, 7, 64, 25), (4, 5, 16, 3), (2, 3, 12, 1)])
def test_rope_against_numpy(engine, heads, seq, d, pos0):
    batch, theta = 2, 1e5
    maxc = pos0 + seq
    x = rnd(batch * seq * heads, d)  # rows (sequence, position, head)
    # The tables as the reference builds them: F32 angles pos * freq, then
    # cos and sin, sin's first half negated.
    freq = (theta ** (-np.arange(0, d, 2, dtype=np.float64) / d)).astype(np.float32)
    ang = (np.arange(maxc, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32)
    cos = np.concatenate([np.cos(ang.astype(np.float64))] * 2, 1).astype(np.float32)
    s_ = np.sin(ang.astype(np.float64)).astype(np.float32)
    sin = np.concatenate([-s_, s_], 1)
    got = engine.download(engine.rope(engine.upload(x), engine.upload(cos), engine.upload(sin), heads, seq, pos0))
    pos = pos0 + (np.arange(x.shape[0]) // heads) % seq
    rot = np.concatenate([x[:, d // 2:], x[:, :d // 2]], 1)
    want = ((x * cos[pos]).astype(np.float32) + (rot * sin[pos]).astype(np.float32)).astype(np.float32)
    same_bits(got, want)
    # The rotation it stands for, in float64: pair (i, i + d/2) turned by the angle.
    a = ang[pos].astype(np.float64)
    x1, x2 = x[:, :d // 2].astype(np.float64), x[:, d // 2:].astype(np.float64)
    exact = np.concatenate([x1 * np.cos(a) - x2 * np.sin(a), x2 * np.cos(a) + x1 * np.sin(a)], 1)
    assert np.abs(got - exact).max() <= 1e-6 * np.abs(x).max() * 4


@pytest.mark.parametrize("dims,dst_off,dst_st,src_off,src_st", [
    ((2, 3, 5, 64), 7 * 64, (3 * 20 * 64, 20 * 64, 64, 1), 0, (5 * 3 * 64, 64, 3 * 64, 1)),  # KV-cache append
    ((1, 4, 6, 3), 5, (0, 40, 2, 7), 11, (0, 1, 4, 24)),                                     # arbitrary strides
])
def test_copy_into4_against_numpy(engine, dims, dst_off, dst_st, src_off, src_st):
    def span(off, st):
        return off + sum((n - 1) * s for n, s in zip(dims, st)) + 1
    dst0 = rnd(span(dst_off, dst_st) + 9)
    src = rnd(span(src_off, src_st) + 3)
    idst = engine.upload(dst0.reshape(1, -1))
    engine.copy_into4(idst, dst_off, dst_st, engine.upload(src.reshape(1, -1)), src_off, src_st, dims)
    want = dst0.copy()
    it = np.stack(np.meshgrid(*[np.arange(n) for n in dims], indexing="ij"), -1).reshape(-1, 4)
    want[dst_off + it @ np.array(dst_st)] = src[src_off + it @ np.array(src_st)]
    same_bits(engine.download(idst).reshape(-1), want)
    # A destination range past the buffer is refused and writes nothing.
    with pytest.raises(miburn.MiError) as e:
        engine.copy_into4(idst, dst0.size, dst_st, engine.upload(src.reshape(1, -1)), src_off, src_st, dims)
    assert e.value.kind == "ARG"
    same_bits(engine.download(idst).reshape(-1), want)


# (3, 7, 32, 8, 64): rows of 3072 columns, wider than one pass of a wavefront's loads.
@pytest.mark.parametrize("batch,seq,heads,kv,d,pos0,maxc", [(2, 5, 9, 3, 64, 3, 16), (1, 33, 4, 4, 32, 0, 40),
                                                           (3, 7, 8, 2, 16, 9, 20), (2, 3, 2, 1, 12, 1, 8),
                                                           (3, 7, 32, 8, 64, 2, 12)])
def test_qkv_rope_cache_equals_composition(engine, batch, seq, heads, kv, d, pos0, maxc):
    rows, w = batch * seq, (heads + 2 * kv) * d
    qkv = rnd(rows, w)
    cos, sin = rope_tables(maxc, d)
    ic, isn = engine.upload(cos), engine.upload(sin)
    kc0, vc0 = rnd(batch * kv * maxc, d), rnd(batch * kv * maxc, d)
    iq = engine.upload(qkv)
    # The fused tail, both layouts (the second call rewrites the same cache rows).
    k1, v1 = engine.upload(kc0), engine.upload(vc0)
    q_nat = engine.download(engine.qkv_rope_cache(iq, ic, isn, seq, heads, kv, pos0, k1, v1, grouped=False))
    q_grp = engine.download(engine.qkv_rope_cache(iq, ic, isn, seq, heads, kv, pos0, k1, v1, grouped=True))
    # The composition.
    qd, kvd = heads * d, kv * d
    q = engine.rope(engine.upload(np.ascontiguousarray(qkv[:, :qd]).reshape(rows * heads, d)), ic, isn, heads, seq, pos0)
    k = engine.rope(engine.upload(np.ascontiguousarray(qkv[:, qd:qd + kvd]).reshape(rows * kv, d)), ic, isn, kv, seq,
                    pos0)
    v = engine.upload(np.ascontiguousarray(qkv[:, qd + kvd:]).reshape(rows * kv, d))
    k2, v2 = engine.upload(kc0), engine.upload(vc0)
    dims, dst, src = (batch, kv, seq, d), (kv * maxc * d, maxc * d, d, 1), (seq * kv * d, d, kv * d, 1)
    engine.copy_into4(k2, pos0 * d, dst, k, 0, src, dims)
    engine.copy_into4(v2, pos0 * d, dst, v, 0, src, dims)
    G = heads // kv
    qg = engine.copy_strided4(q, (batch, kv, seq, G * d), 0, (seq * heads * d, G * d, heads * d, 1))
    same_bits(q_nat, engine.download(q))
    same_bits(q_grp, engine.download(qg).reshape(rows * heads, d))
    same_bits(engine.download(k1), engine.download(k2))
    same_bits(engine.download(v1), engine.download(v2))
    # Rows outside positions pos0 .. pos0 + seq - 1 are untouched.
    kk = engine.download(k1).reshape(batch * kv, maxc, d)
    keep = np.ones(maxc, bool)
    keep[pos0:pos0 + seq] = False
    same_bits(kk[:, keep], kc0.reshape(batch * kv, maxc, d)[:, keep])


@pytest.mark.parametrize("batch,seq,heads,kv,d,pos0,maxc", [(2, 5, 9, 3, 64, 3, 16), (1, 70, 9, 3, 64, 0, 80),
                                                           (2, 3, 2, 1, 12, 1, 8)])
def test_qkv_rope_cache_bf16_caches(engine, batch, seq, heads, kv, d, pos0, maxc):
    rows, w = batch * seq, (heads + 2 * kv) * d
    iq = engine.upload(rnd(rows, w))
    cos, sin = rope_tables(maxc, d)
    ic, isn = engine.upload(cos), engine.upload(sin)
    kc0, vc0 = orc.to_bf16(rnd(batch * kv * maxc, d)), orc.to_bf16(rnd(batch * kv * maxc, d))
    kf, vf = engine.upload(orc.from_bf16(kc0)), engine.upload(orc.from_bf16(vc0))
    kb, vb = engine.upload_bf16(kc0), engine.upload_bf16(vc0)
    for grouped in (False, True):
        qf = engine.download(engine.qkv_rope_cache(iq, ic, isn, seq, heads, kv, pos0, kf, vf, grouped=grouped))
        qb = engine.download(engine.qkv_rope_cache(iq, ic, isn, seq, heads, kv, pos0, kb, vb, grouped=grouped))
        same_bits(qb, qf)
    assert np.array_equal(engine.download(kb), orc.to_bf16(engine.download(kf)))
    assert np.array_equal(engine.download(vb), orc.to_bf16(engine.download(vf)))
    with pytest.raises(miburn.MiError) as e:  # one cache of each kind
        engine.qkv_rope_cache(iq, ic, isn, seq, heads, kv, pos0, kf, vb)
    assert e.value.kind == "ARG"


def test_qkv_rope_cache_argument_errors(engine):
    cos, sin = rope_tables(8, 16)
    ic, isn = engine.upload(cos), engine.upload(sin)
    kc, vc = engine.upload(rnd(2 * 8, 16)), engine.upload(rnd(2 * 8, 16))
    good = engine.upload(rnd(4, 4 * 16))  # 2 heads + 2 x 1 kv head
    engine.qkv_rope_cache(good, ic, isn, 4, 2, 1, 0, kc, vc)  # 1 sequence, 2 x 1 x 8 cache rows: max_ctx 16
    for args in [(engine.upload(rnd(4, 3 * 16)), 4, 2, 1, 0),  # width is not (heads + 2 kv) d
                 (good, 3, 2, 1, 0),                            # 4 rows are not sequences of 3
                 (good, 4, 3, 2, 0),                            # heads not a multiple of kv heads
                 (good, 4, 2, 1, 6)]:                           # positions beyond the rope table
        with pytest.raises(miburn.MiError) as e:
            engine.qkv_rope_cache(args[0], ic, isn, args[1], args[2], args[3], args[4], kc, vc)
        assert e.value.kind == "ARG"


@pytest.mark.parametrize("rows,inner", [(512, 1536), (7, 13), (3, 4)])
def test_silu_mul_halves_equals_silu_mul(engine, rows, inner):
    gu = rnd(rows, 2 * inner, scale=3.0)
    got = engine.download(engine.silu_mul_halves(engine.upload(gu)))
    g, u = engine.upload(np.ascontiguousarray(gu[:, :inner])), engine.upload(np.ascontiguousarray(gu[:, inner:]))
    same_bits(got, engine.download(engine.eltwise_op_as("SILU_MUL", g, u)))
    got16 = engine.download(engine.silu_mul_halves(engine.upload(gu), miburn.BF16))
    assert got16.dtype == np.uint16 and np.array_equal(got16, orc.to_bf16(got))
    with pytest.raises(miburn.MiError):
        engine.silu_mul_halves(engine.upload(rnd(2, 5)))  # odd width
    with pytest.raises(miburn.MiError):
        engine.silu_mul_halves(engine.upload(gu), miburn.I32)
