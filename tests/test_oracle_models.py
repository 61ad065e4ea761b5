"""Pins the torch CPU restatements of the three model workloads
(oracle/models_cpu.py) before they are trusted as the device harnesses'
checker and timed as the CPU baseline.

* Against independent implementations of the same architectures, weights
  copied in: the Llama decoder's logits (full sequence and through the KV
  cache) and greedy tokens against Hugging Face transformers'
  LlamaForCausalLM; the transformer's loss and gradients against
  torch.nn.TransformerEncoderLayer(norm_first, GELU, no dropout) in float64;
  the MLP's losses and SGD updates against torch.nn and torch.optim.SGD.
  Mistakes planted in the oracle (scale 1/d or none, gate and up swapped, ReLU
  for GELU, a dropped gain or bias) are each shown to fail these checks.
* Invariants the models fix, so a dropped term, a wrong index or a transposed
  operand fails one of them: incremental decoding through the KV cache equals
  the full-sequence forward; causality; RoPE's rotation (pair norms kept, the
  score of two rotated vectors a function of their distance only); the
  first-maximum / NaN rule of greedy argmax; and the training losses'
  gradients against central differences in float64.

CPU only."""
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


# ---------------------------------------------------------------------------
# The forwards against independent implementations of the same architectures
# (the Llama decoder against Hugging Face transformers' LlamaForCausalLM, as
# the reference checks its own host model, crates/tt-tests/tests/
# step167_smollm2.rs:4-7; the transformer against torch.nn's pre-norm
# TransformerEncoderLayer, burn-nn's TransformerEncoderConfig
# .with_norm_first(true).with_dropout(0.0), crates/tt-mnist/src/
# transformer.rs:44-52; the MLP against torch.nn), with the weights copied
# in.  Each check is then shown to catch a mistake planted in the oracle.

PIN_LLAMA = dict(vocab=101, hidden=48, layers=2, heads=6, kv_heads=2, head_dim=8, intermediate=40,
                 rope_theta=100000.0, eps=1e-5)


def pin_llama_weights():
    W = mc.llama_random_weights(PIN_LLAMA, seed=11, std=0.25)
    g = torch.Generator().manual_seed(12)
    for L in W["layers"]:
        L["attn_norm"] = 1 + 0.3 * torch.randn(PIN_LLAMA["hidden"], generator=g)
        L["mlp_norm"] = 1 + 0.3 * torch.randn(PIN_LLAMA["hidden"], generator=g)
    W["final_norm"] = 1 + 0.3 * torch.randn(PIN_LLAMA["hidden"], generator=g)
    return W


def hf_llama(W, cfg):
    from transformers import LlamaConfig, LlamaForCausalLM
    c = LlamaConfig(vocab_size=cfg["vocab"], hidden_size=cfg["hidden"], intermediate_size=cfg["intermediate"],
                    num_hidden_layers=cfg["layers"], num_attention_heads=cfg["heads"],
                    num_key_value_heads=cfg["kv_heads"], head_dim=cfg["head_dim"], rms_norm_eps=cfg["eps"],
                    rope_theta=cfg["rope_theta"], tie_word_embeddings=True, max_position_embeddings=128,
                    attention_bias=False, mlp_bias=False, hidden_act="silu")
    c._attn_implementation = "eager"
    m = LlamaForCausalLM(c).eval()
    assert m.lm_head.weight is m.model.embed_tokens.weight
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(W["embed"])
        m.model.norm.weight.copy_(W["final_norm"])
        for L, hl in zip(W["layers"], m.model.layers):
            a, f = hl.self_attn, hl.mlp
            for mod, key in ((a.q_proj, "wq"), (a.k_proj, "wk"), (a.v_proj, "wv"), (a.o_proj, "wo"),
                             (f.gate_proj, "wgate"), (f.up_proj, "wup"), (f.down_proj, "wdown")):
                assert mod.weight.shape == L[key].shape
                mod.weight.copy_(L[key])
            hl.input_layernorm.weight.copy_(L["attn_norm"])
            hl.post_attention_layernorm.weight.copy_(L["mlp_norm"])
    return m


def llama_matches_hf(W, hf, ids):
    """Full-sequence logits and incremental (KV cache) logits against HF's."""
    with torch.no_grad():
        want = hf(torch.as_tensor(ids, dtype=torch.int64)).logits
        got = mc.llama_logits(W, PIN_LLAMA, ids)
        cache = mc.LlamaCache(PIN_LLAMA, ids.shape[0], ids.shape[1])
        inc = [mc.llama_step(W, PIN_LLAMA, cache, ids[:, :7])]
        for p in range(7, ids.shape[1]):
            inc.append(mc.llama_step(W, PIN_LLAMA, cache, ids[:, p:p + 1]))
        inc = torch.cat(inc, 1) @ W["embed"].T
    tol = 2e-5 * float(want.abs().max())
    return float((got - want).abs().max()) <= tol and float((inc - want).abs().max()) <= tol


def test_llama_forward_matches_transformers():
    W = pin_llama_weights()
    hf = hf_llama(W, PIN_LLAMA)
    ids = np.random.default_rng(13).integers(0, PIN_LLAMA["vocab"], (2, 40))
    assert llama_matches_hf(W, hf, ids)
    # Greedy decoding gives HF's greedy tokens.
    prompt = ids[:, :6]
    out, _, _ = mc.llama_generate(W, PIN_LLAMA, prompt, 8)
    seq = torch.as_tensor(prompt, dtype=torch.int64)
    with torch.no_grad():
        for _ in range(8):
            nxt = hf(seq).logits[:, -1].argmax(-1)
            seq = torch.cat([seq, nxt[:, None]], 1)
    assert np.array_equal(out, seq[:, 6:].numpy())


@pytest.mark.parametrize("mistake", ["scale 1/d", "gate and up swapped", "no final norm gain"])
def test_llama_pin_catches_a_planted_mistake(monkeypatch, mistake):
    W = pin_llama_weights()
    hf = hf_llama(W, PIN_LLAMA)
    ids = np.random.default_rng(13).integers(0, PIN_LLAMA["vocab"], (2, 40))
    if mistake == "scale 1/d":
        monkeypatch.setattr(mc, "score_divisor", lambda d: float(d))
    elif mistake == "gate and up swapped":
        monkeypatch.setattr(mc, "swiglu", lambda hn, L: torch.nn.functional.silu(hn @ L["wup"].T)
                            * (hn @ L["wgate"].T))
    else:
        W = dict(W, final_norm=torch.ones(PIN_LLAMA["hidden"]))
    assert not llama_matches_hf(W, hf, ids)


PIN_TF = dict(vocab=37, d_model=16, heads=4, d_ff=24, layers=2, eps=1e-5)


def pin_transformer_params():
    P, layers = mc.transformer_init(PIN_TF, seed=21)
    g = torch.Generator().manual_seed(22)
    P = {k: v.detach().double().requires_grad_() for k, v in P.items()}
    out = []
    for L in layers:
        L = {k: v.detach().double() for k, v in L.items()}
        for k in ("ln1_g", "ln2_g"):  # non-trivial LayerNorm gains and biases
            L[k] = 1 + 0.3 * torch.randn(PIN_TF["d_model"], generator=g, dtype=torch.float64)
        for k in ("ln1_b", "ln2_b"):
            L[k] = 0.2 * torch.randn(PIN_TF["d_model"], generator=g, dtype=torch.float64)
        out.append({k: v.requires_grad_() for k, v in L.items()})
    return P, out


def torch_transformer_loss(P, layers, cfg, tokens, targets):
    nn = torch.nn
    d, V = cfg["d_model"], cfg["vocab"]
    x = P["embed"][torch.as_tensor(tokens, dtype=torch.int64)]
    for L in layers:
        e = nn.TransformerEncoderLayer(d, cfg["heads"], cfg["d_ff"], dropout=0.0, activation="gelu",
                                       layer_norm_eps=cfg["eps"], batch_first=True, norm_first=True,
                                       dtype=torch.float64)
        e.train()  # the composed (not the fused inference) path
        # Burn's Linear weight is [d_in, d_out]; torch's is [d_out, d_in].  The
        # layer runs on these tensors (functional_call), so gradients reach them.
        params = {"self_attn.in_proj_weight": torch.cat([L["wq"].T, L["wk"].T, L["wv"].T], 0),
                  "self_attn.in_proj_bias": torch.cat([L["bq"], L["bk"], L["bv"]]),
                  "self_attn.out_proj.weight": L["wo"].T, "self_attn.out_proj.bias": L["bo"],
                  "linear1.weight": L["w1"].T, "linear1.bias": L["b1"],
                  "linear2.weight": L["w2"].T, "linear2.bias": L["b2"],
                  "norm1.weight": L["ln1_g"], "norm1.bias": L["ln1_b"],
                  "norm2.weight": L["ln2_g"], "norm2.bias": L["ln2_b"]}
        assert set(params) == {n for n, _ in e.named_parameters()}
        x = torch.func.functional_call(e, params, (x,))
    z = x.reshape(-1, d) @ P["head_w"] + P["head_b"]
    return nn.functional.cross_entropy(z.reshape(-1, V), torch.as_tensor(targets, dtype=torch.int64).reshape(-1))


def transformer_matches_torch(P, layers, tokens, targets):
    mine = mc.transformer_loss(P, layers, PIN_TF, tokens, targets)
    theirs = torch_transformer_loss(P, layers, PIN_TF, tokens, targets)
    if abs(mine.item() - theirs.item()) > 1e-12 * abs(theirs.item()):
        return False
    picks = [P["embed"], P["head_w"], layers[0]["wq"], layers[0]["wk"], layers[1]["wv"], layers[1]["ln2_g"],
             layers[0]["ln1_b"], layers[1]["w1"], layers[0]["b2"]]
    g1 = torch.autograd.grad(mine, picks)
    g2 = torch.autograd.grad(theirs, picks)
    return all(torch.allclose(a, b, rtol=1e-10, atol=1e-13) for a, b in zip(g1, g2))


def test_transformer_forward_and_gradients_match_torch_encoder_layer():
    P, layers = pin_transformer_params()
    rng = np.random.default_rng(23)
    x, y = rng.integers(0, PIN_TF["vocab"], (3, 9)), rng.integers(0, PIN_TF["vocab"], (3, 9))
    assert transformer_matches_torch(P, layers, x, y)


@pytest.mark.parametrize("mistake", ["no 1/sqrt(d_k)", "ReLU for GELU", "LayerNorm bias dropped"])
def test_transformer_pin_catches_a_planted_mistake(monkeypatch, mistake):
    P, layers = pin_transformer_params()
    rng = np.random.default_rng(23)
    x, y = rng.integers(0, PIN_TF["vocab"], (3, 9)), rng.integers(0, PIN_TF["vocab"], (3, 9))
    if mistake == "no 1/sqrt(d_k)":
        monkeypatch.setattr(mc, "score_divisor", lambda d: 1.0)
        assert not transformer_matches_torch(P, layers, x, y)
    elif mistake == "ReLU for GELU":
        monkeypatch.setattr(mc, "ffn_activation", torch.relu)
        assert not transformer_matches_torch(P, layers, x, y)
    else:
        # The oracle run without the first LayerNorm's bias, the reference with it.
        mine = mc.transformer_loss(P, [dict(layers[0], ln1_b=torch.zeros_like(layers[0]["ln1_b"])), layers[1]],
                                   PIN_TF, x, y)
        theirs = torch_transformer_loss(P, layers, PIN_TF, x, y)
        assert abs(mine.item() - theirs.item()) > 1e-12 * abs(theirs.item())


def test_mlp_step_matches_torch_nn_and_sgd():
    nn = torch.nn
    g = torch.Generator().manual_seed(31)
    w1, b1 = torch.randn(20, 12, generator=g) * 0.2, torch.randn(12, generator=g) * 0.2
    w2, b2 = torch.randn(12, 7, generator=g) * 0.2, torch.randn(7, generator=g) * 0.2
    x, y = torch.rand(9, 20, generator=g), torch.randint(0, 7, (9,), generator=g)
    mine = [t.clone().requires_grad_() for t in (w1, b1, w2, b2)]
    net = nn.Sequential(nn.Linear(20, 12), nn.ReLU(), nn.Linear(12, 7))
    with torch.no_grad():
        net[0].weight.copy_(w1.T); net[0].bias.copy_(b1)
        net[2].weight.copy_(w2.T); net[2].bias.copy_(b2)
    opt = torch.optim.SGD(net.parameters(), lr=0.01)
    for _ in range(3):
        l1 = mc.mlp_loss(mine, x, y)
        l1.backward()
        mc.sgd(mine, 0.01)
        l2 = nn.CrossEntropyLoss()(net(x), y)
        opt.zero_grad()
        l2.backward()
        opt.step()
        assert abs(l1.item() - l2.item()) <= 1e-6 * abs(l2.item())
    for a, b in ((mine[0], net[0].weight.T), (mine[1], net[0].bias), (mine[2], net[2].weight.T),
                 (mine[3], net[2].bias)):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-7)
