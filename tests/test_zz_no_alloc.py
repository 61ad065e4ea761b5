"""mi_attention_rows_into, the entry point that allocates nothing, against
mi_attention_rows (the same kernels and key chunks): bit-identical outputs on
two calls in a row, the second with a smaller input, and neither call adding
a buffer, device bytes or cached bytes to the engine's report.  A call whose
key-chunk partials exceed the fixed 4 MiB per-GPU array is refused and leaves
the output as it was.  Runs through the C ABI on the device."""
import numpy as np
import pytest

import miburn

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(7_0707)


def rnd(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


@pytest.fixture(scope="module")
def eng():
    e = miburn.Engine(0)
    yield e
    e.close()


def inputs(eng, batch, t, heads, kvh, D, maxc):
    q = eng.upload(rnd(batch * t, heads * D))
    k = eng.upload(rnd(batch * kvh * maxc, D))
    v = eng.upload(rnd(batch * kvh * maxc, D))
    return q, k, v


def footprint(eng):
    r = eng.report()
    return r["live_buffers"], r["device_bytes"], r["cached_bytes"]


# SmolLM2 decode at batch 32 (96 key-chunk items of several chunks each),
# then batch 1 at a shorter context (fewer, smaller partials): the second call
# reads an array the first one left full; then a prompt long enough for the
# matrix-core kernel (no partials).
CASES = [(32, 1, 9, 3, 64, 600, 640), (1, 1, 9, 3, 64, 300, 320), (32, 96, 9, 3, 64, 0, 96)]


def test_into_equals_allocating_entry_twice(eng):
    outs = []
    for batch, t, heads, kvh, D, pos0, maxc in CASES:
        q, k, v = inputs(eng, batch, t, heads, kvh, D, maxc)
        scale = float(np.float32(1.0 / np.sqrt(D)))
        out = eng.fill(batch * t, heads * D, miburn.F32, 0x7FC00000)  # NaN-filled destination
        eng.sync()
        before = footprint(eng)
        eng.attention_rows_into(q, k, v, batch, t, heads, kvh, pos0, scale, out)
        eng.sync()
        assert footprint(eng) == before, "the no-allocation entry point changed the engine's memory"
        got = eng.download(out)
        want = eng.download(eng.attention_rows(q, k, v, batch, t, heads, kvh, pos0, scale))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (batch, pos0)
        outs.append(got)
    assert outs[1].shape == (1, 9 * 64) and outs[2].shape == (3072, 9 * 64)


def test_into_refuses_partials_beyond_its_array_and_bad_outputs(eng):
    # 16 sequences x 3 kv heads x 48 new positions after 4000 cached ones:
    # 2304 items x 4 key chunks x 3 heads x (64 + 2) floats is 7 MiB.
    batch, t, heads, kvh, D, pos0, maxc = 16, 48, 9, 3, 64, 4000, 4048
    q, k, v = inputs(eng, batch, t, heads, kvh, D, maxc)
    out = eng.fill(batch * t, heads * D, miburn.F32, 0x3F800000)
    with pytest.raises(miburn.MiError) as e:
        eng.attention_rows_into(q, k, v, batch, t, heads, kvh, pos0, 0.125, out)
    assert e.value.kind == "UNSUPPORTED"
    assert np.all(eng.download(out) == 1.0)
    # The same call through the allocating entry point runs.
    assert eng.download(eng.attention_rows(q, k, v, batch, t, heads, kvh, pos0, 0.125)).shape == (768, 576)
    small = eng.fill(batch * t, heads * D - 64, miburn.F32, 0)
    with pytest.raises(miburn.MiError) as e:
        eng.attention_rows_into(q, k, v, batch, t, heads, kvh, 0, 0.125, small)  # wrong output shape
    assert e.value.kind == "ARG"
    with pytest.raises(miburn.MiError) as e:
        eng.attention_rows_into(q, k, v, batch, t, heads, kvh, 0, 0.125, q)  # output is an input
    assert e.value.kind == "ARG"
