"""CPU restatements of the reference's three model workloads in float32 torch.

TEST INFRASTRUCTURE ONLY.  Only tests/ (as the checker the device harnesses
are compared against) and bench.py's cpu_baseline leg (as the CPU figure timed
beside the device) import this module; the product never does.  The
reference's CPU path is burn-flex 0.21.0, which cannot be built here (a
crates.io Rust dependency, no toolchain); these functions restate what the
reference's models compute, op by op, with torch's float32 CPU kernels:

* the MLP of crates/tt-tests/tests/step12_mnist.rs:57-114 (Burn Linear
  layers, ReLU, CrossEntropyLoss, SGD) -- `mlp_loss`, `sgd`;
* the pre-norm transformer encoder of crates/tt-mnist/src/transformer.rs:
  36-166 (Embedding, LayerNorm, multi-head self-attention without a mask,
  Linear-GELU-Linear, Linear head, CrossEntropyLoss) -- `transformer_loss`;
* the Llama decoder of crates/tt-models/src/llama.rs:140-520, 1030-1178 with
  RoPE in the rotate-half layout (crates/tt-models/src/rope.rs:6-60): RMSNorm,
  grouped-query attention with a KV cache, SwiGLU, the tied head, greedy
  decoding -- `llama_hidden` (full sequence from position 0), `LlamaCache` /
  `llama_step` (incremental, with a KV cache), `llama_generate`.

How they are pinned (tests/test_oracle_models.py, CPU): every op is a torch
library routine, and each model's forward is checked against an independent
implementation of the same architecture with the same weights copied in --
the Llama decoder against Hugging Face `transformers`' LlamaForCausalLM (the
implementation the reference pins its own host model against,
crates/tt-tests/tests/step167_smollm2.rs:4-7, crates/tt-models/tests/
llama_host.rs:1-3), the transformer against torch.nn.TransformerEncoderLayer
(norm_first, GELU, no dropout: burn-nn's TransformerEncoderConfig
.with_norm_first(true).with_dropout(0.0), transformer.rs:44-52), the MLP
against torch.nn.Linear / ReLU / CrossEntropyLoss and torch.optim.SGD.  The
attention scale, the feed-forward activation and SwiGLU are module-level
functions (`score_divisor`, `ffn_activation`, `swiglu`), so the tests plant a
wrong scale, ReLU for GELU or gate and up swapped and show each caught.  On
top of that, invariants the models fix: incremental decoding through the KV
cache equals the full-sequence forward position by position, causality,
RoPE turning each (i, i + d/2) pair by the angle pos * theta^(-2i/d), the
first-maximum / NaN rule of greedy argmax, and the training losses'
gradients against central differences in float64.
"""
from __future__ import annotations

import math
import time

import numpy as np
import torch

# ------------------------------------------------ shared model pieces


def score_divisor(head_dim):
    """Attention scores are q.k / sqrt(d_head): Burn's default scale
    1/sqrt(d_head) (crates/burn-tt/src/ops.rs:4481), the one burn-nn's
    MultiHeadAttention and the Llama attention use."""
    return math.sqrt(head_dim)


def ffn_activation(x):
    """burn-nn's PositionWiseFeedForward activation in the transformer:
    erf GELU 0.5 x (1 + erf(x / sqrt 2)) (crates/burn-tt/src/ops.rs:5297-5301)."""
    return torch.nn.functional.gelu(x)


def swiglu(hn, L):
    """Llama MLP's SwiGLU: silu(x Wgate^T) * (x Wup^T), the gate through SiLU
    (crates/tt-models/src/llama.rs:482-500)."""
    return torch.nn.functional.silu(hn @ L["wgate"].T) * (hn @ L["wup"].T)


# ----------------------------------------------------------------- MLP


def mlp_loss(params, x, y):
    """step12_mnist.rs:57-114: relu(x W1 + b1) W2 + b2, cross-entropy mean."""
    w1, b1, w2, b2 = params
    z = torch.relu(x @ w1 + b1) @ w2 + b2
    return torch.nn.functional.cross_entropy(z, y)


def sgd(tensors, lr):
    """burn-optim Sgd without momentum or decay: p <- p - lr * grad."""
    with torch.no_grad():
        for t in tensors:
            t -= lr * t.grad
            t.grad = None


# --------------------------------------------------------- transformer

TRANSFORMER_LAYER_PARAMS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b",
                            "w1", "b1", "w2", "b2")


def transformer_loss(P, layers, cfg, tokens, targets):
    """transformer.rs:36-166: pre-norm encoder layers (no mask), Linear head,
    cross-entropy mean over every position.  tokens / targets int [B, S]."""
    B, S = tokens.shape
    d, H = cfg["d_model"], cfg["heads"]
    dk = d // H
    eps = cfg["eps"]

    def ln(x, g, b):
        mu = x.mean(-1, keepdim=True)
        var = ((x - mu) ** 2).mean(-1, keepdim=True)
        return (x - mu) / torch.sqrt(var + eps) * g + b

    def heads(t):
        return t.reshape(B, S, H, dk).transpose(1, 2)

    x = P["embed"][torch.as_tensor(np.asarray(tokens).reshape(-1), dtype=torch.int64)]
    for L in layers:
        n1 = ln(x, L["ln1_g"], L["ln1_b"])
        q, k, v = (heads(n1 @ L[w] + L[b]) for w, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
        s = (q @ k.transpose(-1, -2).contiguous()) / score_divisor(dk)
        o = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B * S, d)
        x = x + o @ L["wo"] + L["bo"]
        n2 = ln(x, L["ln2_g"], L["ln2_b"])
        x = x + ffn_activation(n2 @ L["w1"] + L["b1"]) @ L["w2"] + L["b2"]
    z = x @ P["head_w"] + P["head_b"]
    return torch.nn.functional.cross_entropy(z, torch.as_tensor(np.asarray(targets).reshape(-1), dtype=torch.int64))


def transformer_init(cfg, seed=0):
    """Burn's default init drawn on the host (embedding N(0, 1), Linear
    U(+-1/sqrt(d_in)), LayerNorm 1 / 0): for the CPU baseline, whose timing
    does not depend on the draw."""
    g = torch.Generator().manual_seed(seed)
    d, F, V = cfg["d_model"], cfg["d_ff"], cfg["vocab"]

    def lin(i, o):
        k = 1.0 / math.sqrt(i)
        return ((torch.rand(i, o, generator=g) * 2 - 1) * k).requires_grad_(), \
            ((torch.rand(o, generator=g) * 2 - 1) * k).requires_grad_()
    P = {"embed": torch.randn(V, d, generator=g).requires_grad_()}
    P["head_w"], P["head_b"] = lin(d, V)
    layers = []
    for _ in range(cfg["layers"]):
        L = {"ln1_g": torch.ones(d, requires_grad=True), "ln1_b": torch.zeros(d, requires_grad=True),
             "ln2_g": torch.ones(d, requires_grad=True), "ln2_b": torch.zeros(d, requires_grad=True)}
        for w, b, i, o in (("wq", "bq", d, d), ("wk", "bk", d, d), ("wv", "bv", d, d), ("wo", "bo", d, d),
                           ("w1", "b1", d, F), ("w2", "b2", F, d)):
            L[w], L[b] = lin(i, o)
        layers.append(L)
    return P, layers


# -------------------------------------------------------------- Llama


def rope_tables(cfg, n):
    """rope.rs:6-60: angle = pos * theta^(-2i/d) in F32, cos of the angles
    repeated over both halves, sin with its first half negated: [n, d]."""
    D = cfg["head_dim"]
    half = D // 2
    freq = np.array([np.float32(cfg["rope_theta"] ** (-2.0 * i / D)) for i in range(half)], np.float32)
    ang = (np.arange(n, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32)
    cos = np.cos(ang.astype(np.float64)).astype(np.float32)
    sin = np.sin(ang.astype(np.float64)).astype(np.float32)
    return torch.from_numpy(np.concatenate([cos, cos], 1)), torch.from_numpy(np.concatenate([-sin, sin], 1))


def _rms(x, g, eps):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g.reshape(-1)


def _rope(x, cos, sin, D):
    """x [B, T, heads, D] at the positions of cos / sin [T, D]."""
    rot = torch.cat([x[..., D // 2:], x[..., : D // 2]], -1)
    return x * cos[None, :, None, :] + rot * sin[None, :, None, :]


def llama_hidden(W, cfg, ids):
    """The final RMSNorm's output of the full-sequence forward from position
    0 (llama.rs:371-520: pre-norm, GQA via repeat_kv, causal attention,
    SwiGLU, residuals): [B, T, hidden].  ids int [B, T]."""
    B, T = ids.shape
    H, KVH, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    G = H // KVH
    eps = cfg["eps"]
    cos, sin = rope_tables(cfg, T)
    x = W["embed"][torch.as_tensor(np.asarray(ids), dtype=torch.int64)]
    causal = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    for L in W["layers"]:
        xn = _rms(x, L["attn_norm"], eps)
        q = _rope((xn @ L["wq"].T).reshape(B, T, H, D), cos, sin, D)
        k = _rope((xn @ L["wk"].T).reshape(B, T, KVH, D), cos, sin, D).repeat_interleave(G, dim=2)
        v = (xn @ L["wv"].T).reshape(B, T, KVH, D).repeat_interleave(G, dim=2)
        s = torch.einsum("bthd,bshd->bhts", q, k) / score_divisor(D)
        p = torch.softmax(s.masked_fill(causal, float("-inf")), -1)
        o = torch.einsum("bhts,bshd->bthd", p, v).reshape(B, T, H * D)
        x = x + o @ L["wo"].T
        hn = _rms(x, L["mlp_norm"], eps)
        x = x + swiglu(hn, L) @ L["wdown"].T
    return _rms(x, W["final_norm"], eps)


def llama_logits(W, cfg, ids):
    """Tied head over every position: [B, T, vocab] (llama.rs:1055-1090)."""
    return llama_hidden(W, cfg, ids) @ W["embed"].T


class LlamaCache:
    """Per-layer key / value caches [B, KVH, max_ctx, D] and the filled length
    (llama.rs:415-435's slice_assign into the cache)."""

    def __init__(self, cfg, batch, max_ctx):
        shape = (batch, cfg["kv_heads"], max_ctx, cfg["head_dim"])
        self.k = [torch.zeros(shape) for _ in range(cfg["layers"])]
        self.v = [torch.zeros(shape) for _ in range(cfg["layers"])]
        self.len = 0
        self.cos, self.sin = rope_tables(cfg, max_ctx)


def llama_step(W, cfg, cache, ids):
    """Forward of t new tokens per sequence after `cache.len` cached ones,
    writing their keys and values into the cache; returns the final-norm
    hidden rows [B, t, hidden]."""
    B, t = ids.shape
    H, KVH, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    G = H // KVH
    eps = cfg["eps"]
    p0 = cache.len
    n = p0 + t
    cos, sin = cache.cos[p0:n], cache.sin[p0:n]
    x = W["embed"][torch.as_tensor(np.asarray(ids), dtype=torch.int64)]
    # Query position p0 + i sees cache positions 0 .. p0 + i.
    mask = torch.arange(n)[None, :] > (p0 + torch.arange(t))[:, None]
    for li, L in enumerate(W["layers"]):
        xn = _rms(x, L["attn_norm"], eps)
        q = _rope((xn @ L["wq"].T).reshape(B, t, H, D), cos, sin, D)
        cache.k[li][:, :, p0:n] = _rope((xn @ L["wk"].T).reshape(B, t, KVH, D), cos, sin, D).transpose(1, 2)
        cache.v[li][:, :, p0:n] = (xn @ L["wv"].T).reshape(B, t, KVH, D).transpose(1, 2)
        # Head h reads kv head h // G (repeat_kv), taken as the G query heads
        # of a kv head stacked over its rows: [B, KVH, G t, D] against the
        # cache's [B, KVH, n, D], no copy of the cache.
        qg = q.reshape(B, t, KVH, G, D).permute(0, 2, 3, 1, 4).reshape(B, KVH, G * t, D)
        s = (qg @ cache.k[li][:, :, :n].transpose(-1, -2)) / score_divisor(D)  # [B, KVH, G t, n]
        pr = torch.softmax(s.masked_fill(mask.repeat(G, 1), float("-inf")), -1)
        o = (pr @ cache.v[li][:, :, :n]).reshape(B, KVH, G, t, D).permute(0, 3, 1, 2, 4).reshape(B, t, H * D)
        x = x + o @ L["wo"].T
        hn = _rms(x, L["mlp_norm"], eps)
        x = x + swiglu(hn, L) @ L["wdown"].T
    cache.len = n
    return _rms(x, W["final_norm"], eps)


def argmax_first(logits):
    """The first maximum, a NaN above every number (generate.rs:176-183):
    the first NaN of a row that has one, else the first of its maxima."""
    nan = torch.isnan(logits)
    first_max = torch.argmax(torch.where(nan, torch.full_like(logits, float("-inf")), logits), -1)
    first_nan = torch.argmax(nan.to(torch.int8), -1)
    return torch.where(nan.any(-1), first_nan, first_max)


def llama_generate(W, cfg, prompt, n_new, max_ctx=None):
    """Greedy decoding (llama.rs:1147-1178): prefill the prompt, then one
    token a step through the KV cache.  Returns (tokens [B, n_new],
    prefill_ms, decode_ms)."""
    B, T = prompt.shape
    cache = LlamaCache(cfg, B, max_ctx or T + n_new)
    with torch.no_grad():
        t0 = time.perf_counter()
        h = llama_step(W, cfg, cache, prompt)
        nxt = argmax_first(h[:, -1] @ W["embed"].T)
        t1 = time.perf_counter()
        out = [nxt]
        for _ in range(n_new - 1):
            h = llama_step(W, cfg, cache, nxt[:, None].numpy())
            nxt = argmax_first(h[:, -1] @ W["embed"].T)
            out.append(nxt)
        t2 = time.perf_counter()
    return torch.stack(out, 1).numpy().astype(np.int32), (t1 - t0) * 1e3, (t2 - t1) * 1e3


def llama_random_weights(cfg, seed=0, std=0.02):
    """N(0, std) weights rounded to BF16 and held as F32 (the device model's
    BF16 weights widened), norms' gains 1; [out, in] projections."""
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16).to(torch.float32)
    h, I, D = cfg["hidden"], cfg["intermediate"], cfg["head_dim"]
    W = {"embed": w(cfg["vocab"], h), "final_norm": torch.ones(h), "layers": []}
    for _ in range(cfg["layers"]):
        W["layers"].append({"attn_norm": torch.ones(h), "wq": w(cfg["heads"] * D, h),
                            "wk": w(cfg["kv_heads"] * D, h), "wv": w(cfg["kv_heads"] * D, h),
                            "wo": w(h, cfg["heads"] * D), "mlp_norm": torch.ones(h), "wgate": w(I, h),
                            "wup": w(I, h), "wdown": w(h, I)})
    return W
