"""The MLP training harness on the device against a float32 CPU autograd run
of the same model (crates/tt-tests/tests/step12_mnist.rs:57-114: Burn
`Linear` layers, LCG init, ReLU, CrossEntropyLoss, SGD) on the same data.

Bar: the first loss within rel 1e-3 of the CPU model's (the reference's own
criterion, step59_burn_transformer.rs:18-22), three steps of losses and
parameters within F32 accumulation tolerances, and the loss falling over
BASELINE config 1's 100 steps.
"""
import numpy as np
import pytest
import torch

import miburn

pytestmark = pytest.mark.gpu


def lcg_init(d_in, hidden, d_out, seed=0x3A15):
    s = seed
    M = (1 << 64) - 1

    def unit():
        nonlocal s
        s = (s * 6364136223846793005 + 1442695040888963407) & M
        return np.float32((s >> 33) / float(1 << 30) - 1.0)

    out = []
    for din, dout in ((d_in, hidden), (hidden, d_out)):
        k = np.float32(1.0) / np.sqrt(np.float32(din))
        w = np.array([unit() * k for _ in range(din * dout)], np.float32).reshape(din, dout)
        b = np.array([unit() * k for _ in range(dout)], np.float32).reshape(1, dout)
        out += [w, b]
    return out


def test_init_is_step12s(engine):
    m = miburn.Mlp(engine, 20, 8, 4)
    want = lcg_init(20, 8, 4)
    for i in range(4):
        assert np.array_equal(m.param(i), want[i])


def test_three_steps_match_cpu_autograd(engine):
    d_in, hid, d_out, B, lr = 784, 128, 10, 64, 0.01
    m = miburn.Mlp(engine, d_in, hid, d_out)
    params = [torch.tensor(p, requires_grad=True) for p in lcg_init(d_in, hid, d_out)]
    rng = np.random.default_rng(11)
    for step in range(3):
        x = rng.random((B, d_in), dtype=np.float32)
        y = rng.integers(0, d_out, B).astype(np.int32)
        got = m.train_step(x, y, lr)
        w1, b1, w2, b2 = params
        z = torch.relu(torch.from_numpy(x) @ w1 + b1) @ w2 + b2
        loss = torch.nn.functional.cross_entropy(z, torch.from_numpy(y.astype(np.int64)))
        loss.backward()
        with torch.no_grad():
            for p in params:
                p -= lr * p.grad
                p.grad = None
        assert abs(got - loss.item()) <= 1e-3 * abs(loss.item()), (step, got, loss.item())
        for i, p in enumerate(params):
            dev = m.param(i)
            ref = p.detach().numpy()
            assert np.abs(dev - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-7, (step, i)


def test_config1_loss_falls(engine):
    m = miburn.Mlp(engine)
    losses, ms = m.train_synthetic(64, 100, 0.01, data_seed=1)
    assert np.all(np.isfinite(losses))
    # Random labels: the loss can only fall to the label entropy, ln 10;
    # SGD from the init must move it down from where it started.
    assert losses[:10].mean() > losses[-10:].mean()
    assert ms > 0
