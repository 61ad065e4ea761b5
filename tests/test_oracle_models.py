"""Pins the torch CPU restatements of the three model workloads
(oracle/models_cpu.py) before they are trusted as the device harnesses'
checker and timed as the CPU baseline.  Invariants the models fix, so a
dropped term, a wrong index or a transposed operand fails one of them:
incremental decoding through the KV cache equals the full-sequence forward;
causality; RoPE's rotation (pair norms kept, the score of two rotated vectors
a function of their distance only); the first-maximum / NaN rule of greedy
argmax; and the training losses' gradients against central differences in
float64.  CPU only."""
import math

import numpy as np
import pytest
import torch

import models_cpu as mc

TINY_LLAMA = dict(vocab=97, hidden=32, layers=2, heads=4, kv_heads=2, head_dim=8, intermediate=48,
                  rope_theta=10000.0, eps=1e-5)


def tiny_weights():
    W = mc.llama_random_weights(TINY_LLAMA, seed=3, std=0.3)
    g = torch.Generator().manual_seed(4)
    for L in W["layers"]:  # non-trivial gains, so a dropped gain shows
        L["attn_norm"] = 1 + 0.3 * torch.randn(TINY_LLAMA["hidden"], generator=g)
        L["mlp_norm"] = 1 + 0.3 * torch.randn(TINY_LLAMA["hidden"], generator=g)
    return W


def test_kv_cache_decoding_equals_the_full_forward():
    W = tiny_weights()
    ids = np.random.default_rng(1).integers(0, 97, (3, 9))
    full = mc.llama_hidden(W, TINY_LLAMA, ids)
    cache = mc.LlamaCache(TINY_LLAMA, 3, 16)
    got = [mc.llama_step(W, TINY_LLAMA, cache, ids[:, :5])]
    for p in range(5, 9):
        got.append(mc.llama_step(W, TINY_LLAMA, cache, ids[:, p:p + 1]))
    got = torch.cat(got, 1)
    assert torch.allclose(got, full, atol=1e-5, rtol=1e-5)
    # Two tokens at once after the cache equals them one by one.
    cache2 = mc.LlamaCache(TINY_LLAMA, 3, 16)
    mc.llama_step(W, TINY_LLAMA, cache2, ids[:, :7])
    assert torch.allclose(mc.llama_step(W, TINY_LLAMA, cache2, ids[:, 7:9]), full[:, 7:9], atol=1e-5, rtol=1e-5)


def test_causality():
    W = tiny_weights()
    ids = np.random.default_rng(2).integers(0, 97, (2, 8))
    a = mc.llama_hidden(W, TINY_LLAMA, ids)
    ids2 = ids.copy()
    ids2[:, 6] = (ids2[:, 6] + 1) % 97
    b = mc.llama_hidden(W, TINY_LLAMA, ids2)
    assert torch.equal(a[:, :6], b[:, :6])
    assert not torch.allclose(a[:, 6:], b[:, 6:])


def test_rope_rotates_pairs_by_distance():
    cfg = dict(TINY_LLAMA, head_dim=16)
    cos, sin = mc.rope_tables(cfg, 40)
    D = 16
    g = torch.Generator().manual_seed(5)
    q, k = torch.randn(1, 1, 1, D, generator=g), torch.randn(1, 1, 1, D, generator=g)

    def at(x, p):
        return mc._rope(x, cos[p:p + 1], sin[p:p + 1], D).reshape(D).double()
    # Pair norms kept.
    r = at(q, 17)
    qq = q.reshape(D).double()
    assert torch.allclose(r[:8] ** 2 + r[8:] ** 2, qq[:8] ** 2 + qq[8:] ** 2, rtol=1e-5)
    # <rope(q, p1), rope(k, p2)> depends on p1 - p2 only.
    s1 = torch.dot(at(q, 9), at(k, 4))
    s2 = torch.dot(at(q, 35), at(k, 30))
    assert abs(float(s1 - s2)) < 1e-4 * float(qq.norm() * k.norm())
    # Position 0 is the identity; the angle of pair i at position p is p theta^(-2i/d).
    assert torch.allclose(at(q, 0), qq)
    e = torch.zeros(1, 1, 1, D)
    e[..., 3] = 1.0
    ang = 7 * 10000.0 ** (-2 * 3 / D)
    r = at(e, 7)
    assert abs(float(r[3]) - math.cos(ang)) < 1e-6 and abs(float(r[3 + 8]) - math.sin(ang)) < 1e-6


def test_argmax_first_maximum_and_nan():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [1.0, float("inf"), float("nan"), float("nan")],
                      [0.0, -0.0, -1.0, 0.0], [float("-inf")] * 4])
    assert mc.argmax_first(x).tolist() == [1, 2, 0, 0]


def test_greedy_generation_follows_the_logits():
    W = tiny_weights()
    prompt = np.random.default_rng(6).integers(0, 97, (2, 5))
    out, _, _ = mc.llama_generate(W, TINY_LLAMA, prompt, 4)
    seq = np.concatenate([prompt, out], 1)
    logits = mc.llama_logits(W, TINY_LLAMA, seq)
    assert np.array_equal(out, torch.argmax(logits[:, 4:8], -1).numpy())


def _fd_check(loss_fn, params, picks, h=1e-6):
    loss = loss_fn()
    loss.backward()
    for t, idx in picks:
        g = t.grad.reshape(-1)[idx].item()
        with torch.no_grad():
            flat = t.reshape(-1)
            old = flat[idx].item()
            flat[idx] = old + h
            lp = loss_fn().item()
            flat[idx] = old - h
            lm = loss_fn().item()
            flat[idx] = old
        assert abs(g - (lp - lm) / (2 * h)) <= 1e-6 + 1e-5 * abs(g), (g, (lp - lm) / (2 * h))


def test_mlp_gradient_matches_central_differences():
    g = torch.Generator().manual_seed(7)
    params = [torch.randn(12, 8, dtype=torch.float64, generator=g).requires_grad_(),
              torch.randn(8, dtype=torch.float64, generator=g).requires_grad_(),
              torch.randn(8, 5, dtype=torch.float64, generator=g).requires_grad_(),
              torch.randn(5, dtype=torch.float64, generator=g).requires_grad_()]
    x = torch.rand(6, 12, dtype=torch.float64, generator=g)
    y = torch.tensor([0, 4, 2, 2, 1, 3])
    _fd_check(lambda: mc.mlp_loss(params, x, y), params, [(params[0], 17), (params[1], 3), (params[2], 9),
                                                          (params[3], 4)])


def test_transformer_gradient_matches_central_differences():
    cfg = dict(vocab=11, d_model=8, heads=2, d_ff=12, layers=1, eps=1e-5)
    P, layers = mc.transformer_init(cfg, seed=1)
    P = {k: v.detach().double().requires_grad_() for k, v in P.items()}
    layers = [{k: v.detach().double().requires_grad_() for k, v in L.items()} for L in layers]
    rng = np.random.default_rng(8)
    x, y = rng.integers(0, 11, (2, 5)), rng.integers(0, 11, (2, 5))
    L = layers[0]
    _fd_check(lambda: mc.transformer_loss(P, layers, cfg, x, y), None,
              [(P["embed"], 3), (P["head_w"], 20), (L["wq"], 5), (L["wk"], 11), (L["wv"], 30), (L["ln1_g"], 2),
               (L["w1"], 40), (L["b2"], 1)])
    # Loss at init near ln(vocab) for a head of small logits.
    assert abs(mc.transformer_loss(P, layers, cfg, x, y).item() - math.log(11)) < 3.0
