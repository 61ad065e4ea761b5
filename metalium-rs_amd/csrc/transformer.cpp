// The transformer training harness over the engine (4
// layers, d_model 256, 4 heads, FFN 1024 GELU, LayerNorm, vocab 8192, seq
// 128, batch 16, fp32, SGD).
//
// Reference: crates/tt-mnist/src/transformer.rs:36-166 -- Burn's `Embedding`,
// a pre-norm `TransformerEncoder` (norm_first, dropout 0, no attention mask)
// and a `Linear` head, `CrossEntropyLoss`, `Sgd`; the gate that trains it,
// crates/tt-tests/tests/step59_burn_transformer.rs.  A layer (burn-nn's
// TransformerEncoderLayer, norm_first):
//   x = x + Wo(MHA(LN1(x))),  x = x + W2(GELU(W1(LN2(x)))),
// MHA with q/k/v/o Linears (bias), heads split from d_model, softmax(q k^T /
// sqrt(d_head)) v (crates/burn-tt/src/ops.rs:4447-4600 for the attention op).
// Initialisation follows Burn's defaults, drawn on the device: Embedding
// N(0, 1); Linear weight [d_in, d_out] and bias U(-1/sqrt(d_in), 1/sqrt(d_in))
// (Kaiming-uniform, gain 1/sqrt(3)); LayerNorm gamma 1, beta 0.
//
// The backward restates burn-autodiff's rules per op (the same as the MLP
// harness for Linear, cross-entropy and SGD), with two fused engine kernels:
// LayerNorm's gradient and softmax's.  Attention's products run per
// (sequence, head) item over the head-split activations; the split and merge
// are strided copies (swap_dims materialised).
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/miburn_models.h"
#include "burn.hpp"

namespace {
thread_local std::string g_tf_error;
using burn::Tensor;

struct TLayer {
  Tensor ln1_g, ln1_b, wq, bq, wk, bk, wv, bv, wo, bo, ln2_g, ln2_b, w1, b1, w2, b2;
  // Parameter `which` in the order of the members above.
  Tensor *at(int which) {
    Tensor *p[] = {&ln1_g, &ln1_b, &wq, &bq, &wk, &bk, &wv, &bv, &wo, &bo, &ln2_g, &ln2_b, &w1, &b1, &w2, &b2};
    return p[which];
  }
};
constexpr int kLayerParams = 16;
}  // namespace

struct mi_transformer {
  mi_ctx *ctx;
  mi_transformer_config cfg;
  Tensor embed, head_w, head_b;
  std::vector<TLayer> layers;
};

namespace {

int fail_tf(const std::exception &e) {
  g_tf_error = e.what();
  if (auto *be = dynamic_cast<const burn::Error *>(&e)) return be->status;
  return MI_E_ARG;
}

// A [1, 1] F32 value (broadcast by the element-wise ops).
Tensor scalar(mi_ctx *ctx, float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  return burn::fill(ctx, {1, 1}, MI_F32, bits);
}

// [B * S, H * dk] rows (sequence, position), heads along the row ->
// [B * H * S, dk] items (sequence, head).
Tensor split_heads(const Tensor &x, int64_t B, int64_t S, int64_t H, int64_t dk) {
  const int64_t dims[4] = {B, H, S, dk};
  const int64_t st[4] = {S * H * dk, dk, H * dk, 1};
  return burn::copy4(x, dims, 0, st);
}

Tensor merge_heads(const Tensor &x, int64_t B, int64_t S, int64_t H, int64_t dk) {
  const int64_t dims[4] = {B, S, H, dk};
  const int64_t st[4] = {H * S * dk, dk, S * dk, 1};
  return burn::copy4(x, dims, 0, st).reshape({B * S, H * dk});
}

// Linear forward: x W + b (Burn's `Linear`, weight [d_in, d_out]).
Tensor linear(const Tensor &x, const Tensor &w, const Tensor &b) {
  return burn::float_add(burn::float_matmul(x, false, w, false), b);
}

struct Saved {
  Tensor x_in, n1, qh, kh, vh, p, om, x_mid, n2, h1, g;
};

// One training step on tokens / targets [B * S] I32; returns the loss [1, 1].
Tensor step(mi_transformer *m, const Tensor &tokens, const Tensor &targets, int64_t B, int64_t S, float lr) {
  mi_ctx *ctx = m->ctx;
  const mi_transformer_config &c = m->cfg;
  const int64_t R = B * S, d = c.d_model, H = c.heads, dk = d / H, V = c.vocab;
  const float scale = 1.0f / std::sqrt(static_cast<float>(dk));
  const float eps = c.eps;
  const int64_t items = B * H;

  // Forward.
  Tensor x = burn::select_rows(m->embed, tokens).reshape({R, d});
  std::vector<Saved> saved(m->layers.size());
  for (size_t l = 0; l < m->layers.size(); ++l) {
    TLayer &L = m->layers[l];
    Saved &sv = saved[l];
    sv.x_in = x;
    sv.n1 = burn::layer_norm(x, L.ln1_g, L.ln1_b, eps);
    sv.qh = split_heads(linear(sv.n1, L.wq, L.bq), B, S, H, dk);
    sv.kh = split_heads(linear(sv.n1, L.wk, L.bk), B, S, H, dk);
    sv.vh = split_heads(linear(sv.n1, L.wv, L.bv), B, S, H, dk);
    Tensor sc = burn::matmul_blocks(sv.qh, false, sv.kh, true, items, S, dk, S, 0, S * dk, 0, S * dk);
    sv.p = burn::softmax_rows(sc, nullptr, scale, false);
    Tensor oh = burn::matmul_blocks(sv.p, false, sv.vh, false, items, S, S, dk, 0, S * S, 0, S * dk);
    sv.om = merge_heads(oh, B, S, H, dk);
    x = burn::float_add(x, linear(sv.om, L.wo, L.bo));
    sv.x_mid = x;
    sv.n2 = burn::layer_norm(x, L.ln2_g, L.ln2_b, eps);
    sv.h1 = linear(sv.n2, L.w1, L.b1);
    sv.g = burn::gelu(sv.h1);
    x = burn::float_add(x, linear(sv.g, L.w2, L.b2));
  }
  Tensor z = linear(x, m->head_w, m->head_b);                       // [R, V]
  Tensor logp = burn::softmax_rows(z, nullptr, 1.0f, true);
  Tensor loss = burn::float_neg(burn::reduce_all(burn::pick_columns(logp, targets), MI_R_MEAN));

  // Backward.  Cross-entropy through log_softmax: d logp = -1/R at each
  // row's target (negation, mean and gather); dz = d logp - exp(logp) *
  // rowsum(d logp), the row sum being -1/R exactly.
  const float inv = 1.0f / static_cast<float>(R);
  uint32_t minus_inv;
  const float mi = -inv;
  std::memcpy(&minus_inv, &mi, 4);
  Tensor onehot =
      burn::scatter_add_columns(burn::fill(ctx, {R, V}, MI_F32, 0), targets, burn::fill(ctx, {R, 1}, MI_F32, minus_inv));
  Tensor inv_t = scalar(ctx, inv);  // dz = onehot + exp(logp) * (1/R)
  Tensor dz = burn::eltwise(MI_K_MUL_ADD, burn::float_exp(logp), &inv_t, &onehot);
  // SGD (p <- p - grad * lr) runs once, in place, after the backward: the
  // gradients are collected here.
  std::vector<const Tensor *> upd_p;
  std::vector<Tensor> upd_g;
  auto sgd = [&](const Tensor &p, const Tensor &grad) {
    upd_p.push_back(&p);
    upd_g.push_back(grad);
  };
  // Linear's backward (ops.rs:5006-5029): dW = x^T dy, db = sum_rows(dy),
  // dx = dy W^T.
  auto linear_back = [&](const Tensor &xin, const Tensor &dy, const Tensor &w, const Tensor &b) {
    Tensor dw = burn::float_matmul(xin, true, dy, false);
    Tensor db = burn::reduce(dy, MI_R_SUM, MI_AXIS_ROWS);
    Tensor dx = burn::float_matmul(dy, false, w, true);
    sgd(w, dw);
    sgd(b, db);
    return dx;
  };
  Tensor dx = linear_back(x, dz, m->head_w, m->head_b);
  for (size_t li = m->layers.size(); li-- > 0;) {
    TLayer &L = m->layers[li];
    Saved &sv = saved[li];
    // Feed-forward block.
    Tensor dg = linear_back(sv.g, dx, L.w2, L.b2);
    Tensor dh1 = burn::gelu_backward(sv.h1, dg);
    Tensor dn2 = linear_back(sv.n2, dh1, L.w1, L.b1);
    burn::NormGrads n2g = burn::layer_norm_backward(sv.x_mid, L.ln2_g, dn2, dx, eps);
    sgd(L.ln2_g, n2g.dgamma);
    sgd(L.ln2_b, n2g.dbeta);
    Tensor dx2 = n2g.dx;
    // Attention block.
    Tensor dom = linear_back(sv.om, dx2, L.wo, L.bo);
    Tensor doh = split_heads(dom, B, S, H, dk);
    Tensor dp = burn::matmul_blocks(doh, false, sv.vh, true, items, S, dk, S, 0, S * dk, 0, S * dk);
    Tensor dvh = burn::matmul_blocks(sv.p, true, doh, false, items, S, S, dk, 0, S * S, 0, S * dk);
    Tensor ds = burn::softmax_backward(sv.p, dp, scale);
    Tensor dqh = burn::matmul_blocks(ds, false, sv.kh, false, items, S, S, dk, 0, S * S, 0, S * dk);
    Tensor dkh = burn::matmul_blocks(ds, true, sv.qh, false, items, S, S, dk, 0, S * S, 0, S * dk);
    Tensor dn1 = linear_back(sv.n1, merge_heads(dqh, B, S, H, dk), L.wq, L.bq);
    dn1 = burn::float_add(dn1, linear_back(sv.n1, merge_heads(dkh, B, S, H, dk), L.wk, L.bk));
    dn1 = burn::float_add(dn1, linear_back(sv.n1, merge_heads(dvh, B, S, H, dk), L.wv, L.bv));
    burn::NormGrads n1g = burn::layer_norm_backward(sv.x_in, L.ln1_g, dn1, dx2, eps);
    sgd(L.ln1_g, n1g.dgamma);
    sgd(L.ln1_b, n1g.dbeta);
    dx = n1g.dx;
  }
  // Embedding's backward (ops.rs:4976-5000): rows added at their ids, in order.
  Tensor de = burn::select_add_rows(burn::fill(ctx, {V, d}, MI_F32, 0), tokens, dx);
  sgd(m->embed, de);
  burn::sgd_update(ctx, upd_p, upd_g, lr);
  return loss;
}

// Burn's Linear init: weight [din, dout] and bias [1, dout], each
// U(-1/sqrt(din), 1/sqrt(din)).
Tensor kaiming(mi_ctx *ctx, int64_t din, int64_t dout, uint64_t base) {
  const float k = 1.0f / std::sqrt(static_cast<float>(din));
  return burn::random(ctx, {din, dout}, MI_DRAW_UNIFORM, -k, k, base);
}
Tensor bias(mi_ctx *ctx, int64_t din, int64_t dout, uint64_t base) {
  const float k = 1.0f / std::sqrt(static_cast<float>(din));
  return burn::random(ctx, {1, dout}, MI_DRAW_UNIFORM, -k, k, base);
}

}  // namespace

extern "C" {

const char *mi_transformer_last_error(void) { return g_tf_error.c_str(); }

int mi_transformer_create(mi_ctx *ctx, const mi_transformer_config *cfg, uint64_t seed, mi_transformer **out) {
  if (!ctx || !cfg || !out) return MI_E_ARG;
  const mi_transformer_config &c = *cfg;
  if (c.vocab <= 0 || c.d_model <= 0 || c.heads <= 0 || c.d_model % c.heads || c.d_ff <= 0 || c.layers < 0) {
    g_tf_error = "invalid transformer config";
    return MI_E_ARG;
  }
  mi_transformer *m = new mi_transformer();
  try {
    m->ctx = ctx;
    m->cfg = c;
    uint64_t base = seed * 0x9e3779b97f4a7c15ull + 17;
    auto next = [&]() { return base++; };
    const int64_t d = c.d_model, F = c.d_ff, V = c.vocab;
    m->embed = burn::random(ctx, {V, d}, MI_DRAW_NORMAL, 0.0f, 1.0f, next());
    m->layers.resize(c.layers);
    const uint32_t one = 0x3f800000u;
    for (TLayer &L : m->layers) {
      L.ln1_g = burn::fill(ctx, {1, d}, MI_F32, one);
      L.ln1_b = burn::fill(ctx, {1, d}, MI_F32, 0);
      L.wq = kaiming(ctx, d, d, next());
      L.bq = bias(ctx, d, d, next());
      L.wk = kaiming(ctx, d, d, next());
      L.bk = bias(ctx, d, d, next());
      L.wv = kaiming(ctx, d, d, next());
      L.bv = bias(ctx, d, d, next());
      L.wo = kaiming(ctx, d, d, next());
      L.bo = bias(ctx, d, d, next());
      L.ln2_g = burn::fill(ctx, {1, d}, MI_F32, one);
      L.ln2_b = burn::fill(ctx, {1, d}, MI_F32, 0);
      L.w1 = kaiming(ctx, d, F, next());
      L.b1 = bias(ctx, d, F, next());
      L.w2 = kaiming(ctx, F, d, next());
      L.b2 = bias(ctx, F, d, next());
    }
    m->head_w = kaiming(ctx, d, V, next());
    m->head_b = bias(ctx, d, V, next());
  } catch (const std::exception &e) {
    delete m;
    return fail_tf(e);
  }
  *out = m;
  return MI_OK;
}

int mi_transformer_destroy(mi_transformer *m) {
  delete m;
  return MI_OK;
}

int mi_transformer_param(mi_transformer *m, int layer, int which, mi_id *out) {
  if (!m || !out) return MI_E_ARG;
  const Tensor *t = nullptr;
  if (layer < 0) {
    const Tensor *g[] = {&m->embed, &m->head_w, &m->head_b};
    if (which >= 0 && which < 3) t = g[which];
  } else if (layer < static_cast<int>(m->layers.size()) && which >= 0 && which < kLayerParams) {
    t = m->layers[layer].at(which);
  }
  if (!t) {
    g_tf_error = "no such parameter";
    return MI_E_ARG;
  }
  try {
    t->use();
  } catch (const std::exception &e) {
    return fail_tf(e);
  }
  *out = t->id();
  return MI_OK;
}

int mi_transformer_train_step(mi_transformer *m, mi_id tokens, mi_id targets, int32_t batch, int32_t seq, float lr,
                              mi_id *loss) {
  if (!m || !loss || batch <= 0 || seq <= 0) return MI_E_ARG;
  try {
    const int64_t R = static_cast<int64_t>(batch) * seq;
    int64_t r, cc;
    int e;
    for (mi_id id : {tokens, targets}) {
      burn::check(m->ctx, mi_metadata(m->ctx, id, &r, &cc, &e), "ids");
      if (e != MI_I32 || r * cc != R) throw burn::Error(MI_E_ARG, "tokens and targets must be batch * seq I32");
    }
    mi_id ti, yi;
    burn::check(m->ctx, mi_cast(m->ctx, tokens, MI_I32, &ti), "tokens");
    burn::check(m->ctx, mi_cast(m->ctx, targets, MI_I32, &yi), "targets");
    Tensor tt(m->ctx, ti, {R}), yt(m->ctx, yi, {R, 1});
    Tensor l = step(m, tt, yt, batch, seq, lr);
    mi_id id;
    burn::check(m->ctx, mi_cast(m->ctx, l.use(), MI_F32, &id), "loss");
    *loss = id;
  } catch (const std::exception &e) {
    return fail_tf(e);
  }
  return MI_OK;
}

int mi_transformer_train_synthetic(mi_transformer *m, int32_t batch, int32_t seq, int32_t steps, float lr,
                                   uint64_t data_seed, float *losses, double *ms) {
  if (!m || batch <= 0 || seq <= 0 || steps < 0) return MI_E_ARG;
  using clock = std::chrono::steady_clock;
  try {
    const int64_t R = static_cast<int64_t>(batch) * seq;
    const float V = static_cast<float>(m->cfg.vocab);
    std::vector<Tensor> ls;
    ls.reserve(static_cast<size_t>(steps));
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    auto t0 = clock::now();
    for (int32_t s = 0; s < steps; ++s) {
      const uint64_t base = data_seed * 0x100000001b3ull + static_cast<uint64_t>(s) * 2;
      Tensor x = burn::random(m->ctx, {R}, MI_DRAW_INT_RANGE, 0.0f, V, base);
      Tensor y = burn::random(m->ctx, {R, 1}, MI_DRAW_INT_RANGE, 0.0f, V, base + 1);
      ls.push_back(step(m, x, y, batch, seq, lr));
    }
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    auto t1 = clock::now();
    if (ms) *ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (losses)
      for (int32_t s = 0; s < steps; ++s) losses[s] = burn::float_into_data(ls[s])[0];
  } catch (const std::exception &e) {
    return fail_tf(e);
  }
  return MI_OK;
}

}  // extern "C"
