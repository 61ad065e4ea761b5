"""Traces (the reference's Engine::begin_trace / end_trace / run_trace,
crates/burn-tt/src/server.rs:591-660, and TracedTrainingStep,
crates/burn-tt/src/trace.rs:989-1010) as HIP graphs: every replay equals the
eager result bit for bit (same kernels, same order), with eager work and
waits between replays; memory the trace uses is never handed to other work;
host transfers and waits are refused while capturing.
"""
import numpy as np
import pytest

import miburn
import oracle_lib as orc

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(99)


def rnd(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def ops(eng, x, b):
    y = eng.eltwise_op_as("EXP", x)
    z = eng.eltwise_op_as("ADD", y, x)
    w = eng.matmul_dram(z, False, b, False)
    s = eng.softmax_rows(w)
    for i in (y, z, w):
        eng.free(i)
    return s


def test_trace_replays_equal_eager(engine):
    b = engine.upload(rnd(128, 96))
    x = engine.upload(rnd(64, 128))
    engine.begin_trace()
    out = ops(engine, x, b)
    trace = engine.end_trace()
    for rep in range(4):
        xv = rnd(64, 128)
        got, = engine.run_trace(trace, {x: xv}, [out])
        # Eager reference, with its own allocations and a wait between replays.
        xe = engine.upload(xv)
        want = ops(engine, xe, b)
        engine.sync()
        assert np.array_equal(bits(got), bits(engine.download(want))), rep
        engine.free(xe)
        engine.free(want)
    engine.release_trace(trace)
    for i in (b, x, out):
        engine.free(i)


def test_trace_run_checks_host_lengths(engine):
    """An input whose host bytes are not its buffer's size, or an output
    array with less room than its buffer, is refused (MI_E_ARG) before
    anything is written or replayed: the input buffer, the output buffer and
    the caller's array keep their contents."""
    b = engine.upload(rnd(128, 96))
    x = engine.upload(rnd(64, 128))
    engine.begin_trace()
    out = ops(engine, x, b)
    trace = engine.end_trace()
    x0 = rnd(64, 128)
    first, = engine.run_trace(trace, {x: x0}, [out])
    for bad in (rnd(64, 100), rnd(65, 128), np.zeros(0, np.float32)):  # short, long, empty
        with pytest.raises(miburn.MiError) as e:
            engine.run_trace(trace, {x: bad}, [out])
        assert e.value.kind == "ARG"
    small = np.full((10, 10), 7.0, np.float32)
    with pytest.raises(miburn.MiError) as e:  # a fresh input with an undersized output
        engine.run_trace(trace, {x: rnd(64, 128)}, [out], out_arrays=[small])
    assert e.value.kind == "ARG"
    assert np.all(small == 7.0)
    assert np.array_equal(bits(engine.download(x)), bits(x0))
    assert np.array_equal(bits(engine.download(out)), bits(first))
    # Room to spare is accepted; the buffer's bytes land at the front.
    roomy = np.full(64 * 96 + 5, 3.0, np.float32)
    engine.run_trace(trace, {x: x0}, [out], out_arrays=[roomy])
    assert np.array_equal(bits(roomy[:64 * 96].reshape(64, 96)), bits(first)) and np.all(roomy[-5:] == 3.0)
    engine.release_trace(trace)
    for i in (b, x, out):
        engine.free(i)


def test_trace_memory_is_reserved(engine):
    """A buffer the capture freed keeps its memory: an allocation after the
    capture never receives it, so a replay cannot overwrite eager data."""
    x = engine.upload(rnd(256, 256))
    engine.begin_trace()
    t = engine.eltwise_op_as("EXP", x)  # written by every replay
    u = engine.eltwise_op_as("NEG", t)
    engine.free(t)
    trace = engine.end_trace()
    keep = [engine.upload(np.full((256, 256), float(i), np.float32)) for i in range(4)]
    for _ in range(3):
        engine.run_trace(trace, {x: rnd(256, 256)})
    engine.sync()
    for i, k in enumerate(keep):
        assert np.all(engine.download(k) == float(i))
    engine.release_trace(trace)
    for i in keep + [x, u]:
        engine.free(i)


def test_capture_refuses_transfers_and_waits(engine):
    x = engine.upload(rnd(8, 8))
    with pytest.raises(miburn.MiError) as e:
        engine.end_trace()
    assert e.value.kind == "ARG"
    engine.begin_trace()
    with pytest.raises(miburn.MiError) as e:
        engine.begin_trace()
    assert e.value.kind == "ARG"
    for call in (lambda: engine.upload(rnd(2, 2)), lambda: engine.download(x), engine.sync):
        with pytest.raises(miburn.MiError) as e:
            call()
        assert e.value.kind == "UNSUPPORTED"
    y = engine.eltwise_op_as("ABS", x)
    trace = engine.end_trace()
    got, = engine.run_trace(trace, {}, [y])
    assert np.array_equal(got, np.abs(engine.download(x)))
    engine.release_trace(trace)
    with pytest.raises(miburn.MiError) as e:
        engine.run_trace(trace)
    assert e.value.kind == "ID"
    engine.free(x)
    engine.free(y)


def progressions(step, batch, seq, vocab):
    x = np.zeros((batch, seq), np.int32)
    y = np.zeros((batch, seq), np.int32)
    for b in range(batch):
        stride = 1 + (b + step) % 3
        start = (7 * b + 3 * step) % vocab
        x[b] = (start + stride * np.arange(seq)) % vocab
        y[b] = (start + stride * (np.arange(seq) + 1)) % vocab
    return x, y


def test_transformer_training_step_trace(engine):
    """The captured training step (forward, loss, backward, in-place SGD,
    embedding backward) replayed on new batches gives the eager model's
    losses and parameters bit for bit."""
    cfg = dict(vocab=96, d_model=64, heads=2, d_ff=128, layers=2, eps=1e-5)
    eager = miburn.Transformer(engine, cfg, seed=11)
    traced = miburn.Transformer(engine, cfg, seed=11)
    B, S, lr = 4, 16, 0.05
    tok = engine.upload_i32(np.zeros((B * S, 1), np.int32))
    tgt = engine.upload_i32(np.zeros((B * S, 1), np.int32))
    engine.begin_trace()
    loss_id = traced.train_step_ids(tok, tgt, B, S, lr)
    trace = engine.end_trace()
    for step in range(4):
        x, y = progressions(step, B, S, cfg["vocab"])
        want = eager.train_step(x, y, lr)
        got, = engine.run_trace(trace, {tok: x.reshape(-1, 1), tgt: y.reshape(-1, 1)}, [loss_id])
        assert np.float32(want).view(np.uint32) == got.reshape(-1)[0:1].view(np.uint32)[0], (step, want, got)
    for name in ("embed", "head_w", "head_b"):
        assert np.array_equal(bits(eager.param(name)), bits(traced.param(name))), name
    for l in range(cfg["layers"]):
        for name in miburn.TRANSFORMER_LAYER_PARAMS:
            assert np.array_equal(bits(eager.param(name, l)), bits(traced.param(name, l))), (l, name)
    engine.release_trace(trace)
    for i in (tok, tgt, loss_id):
        engine.free(i)
    eager.close()
    traced.close()


def test_mlp_training_step_trace(engine):
    eager = miburn.Mlp(engine)
    traced = miburn.Mlp(engine)
    x = engine.upload(np.zeros((64, 784), np.float32))
    lab = engine.upload_i32(np.zeros((64, 1), np.int32))
    engine.begin_trace()
    loss_id = traced.train_step_ids(x, lab, 0.01)
    trace = engine.end_trace()
    for step in range(3):
        xv = RNG.random((64, 784)).astype(np.float32)
        yv = RNG.integers(0, 10, (64, 1)).astype(np.int32)
        want = eager.train_step(xv, yv, 0.01)
        got, = engine.run_trace(trace, {x: xv, lab: yv}, [loss_id])
        assert np.float32(want).view(np.uint32) == got.reshape(-1)[0:1].view(np.uint32)[0], step
    for i in range(4):
        assert np.array_equal(bits(eager.param(i)), bits(traced.param(i))), i
    engine.release_trace(trace)
    for i in (x, lab, loss_id):
        engine.free(i)
    eager.close()
    traced.close()


def test_mlp_trace_replays_back_to_back(engine):
    """Replays on fresh host batches with nothing read back between them (each
    batch staged ahead on the transfer stream, an input's two device copies
    used in turn): the parameters after eight replays equal eight eager
    steps' bit for bit."""
    eager = miburn.Mlp(engine)
    traced = miburn.Mlp(engine)
    x = engine.upload(np.zeros((64, 784), np.float32))
    lab = engine.upload_i32(np.zeros((64, 1), np.int32))
    engine.begin_trace()
    loss_id = traced.train_step_ids(x, lab, 0.01)
    trace = engine.end_trace()
    batches = [(RNG.random((64, 784)).astype(np.float32), RNG.integers(0, 10, (64, 1)).astype(np.int32))
               for _ in range(8)]
    for xv, yv in batches:
        eager.train_step(xv, yv, 0.01)
    for xv, yv in batches:
        engine.run_trace(trace, {x: xv, lab: yv})
    engine.sync()
    for i in range(4):
        assert np.array_equal(bits(eager.param(i)), bits(traced.param(i))), i
    engine.release_trace(trace)
    for i in (x, lab, loss_id):
        engine.free(i)
    eager.close()
    traced.close()

