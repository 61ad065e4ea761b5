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
// LayerNorm's gradient and softmax's.  The q, k and v Linears are one product
// against a [d, 3d] weight (columns q | k | v); attention's products run per
// (sequence, head) item straight out of that [rows, 3d] projection and write
// their results into place (the head split and merge, swap_dims in Burn, are
// item strides, never copies).  Linear biases and the residual adds ride in
// the products' epilogues.
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
  Tensor ln1_g, ln1_b;
  Tensor wqkv, bqkv;  // [d, 3d] and [1, 3d]: columns q | k | v
  Tensor wo, bo, ln2_g, ln2_b, w1, b1, w2, b2;
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

// Linear forward, x W + b (Burn's `Linear`, weight [d_in, d_out]), plus an
// optional residual: residual + (x W + b), as Burn's float_add(residual,
// linear(x)) rounds it.
Tensor linear(const Tensor &x, const Tensor &w, const Tensor &b, const Tensor *residual = nullptr) {
  return burn::linear(x, w, false, &b, residual);
}

struct Saved {
  Tensor x_in, n1, qkv, p, om, x_mid, n2, h1, g;
};

// One training step on tokens / targets [B * S] I32; returns the loss [1, 1].
Tensor step(mi_transformer *m, const Tensor &tokens, const Tensor &targets, int64_t B, int64_t S, float lr) {
  mi_ctx *ctx = m->ctx;
  const mi_transformer_config &c = m->cfg;
  const int64_t R = B * S, d = c.d_model, H = c.heads, dk = d / H, V = c.vocab;
  const float scale = 1.0f / std::sqrt(static_cast<float>(dk));
  const float eps = c.eps;
  const int64_t items = B * H, W = 3 * d;
  // Item (sequence b, head h) of each operand: q, k, v inside the [R, 3d]
  // projection, the head's output columns inside [R, d], and the [S, S]
  // scores, stored item after item.
  const burn::Items q_at{0, S * W, dk}, k_at{d, S * W, dk}, v_at{2 * d, S * W, dk};
  const burn::Items o_at{0, S * d, dk}, s_at{0, H * S * S, S * S};

  // Forward.
  Tensor x = burn::select_rows(m->embed, tokens).reshape({R, d});
  std::vector<Saved> saved(m->layers.size());
  for (size_t l = 0; l < m->layers.size(); ++l) {
    TLayer &L = m->layers[l];
    Saved &sv = saved[l];
    sv.x_in = x;
    sv.n1 = burn::layer_norm(x, L.ln1_g, L.ln1_b, eps);
    sv.qkv = linear(sv.n1, L.wqkv, L.bqkv);  // [R, 3d]
    Tensor sc = burn::empty(ctx, {items * S, S});
    burn::matmul_items(sv.qkv, false, q_at, sv.qkv, true, k_at, B, H, S, dk, S, sc, s_at);
    sv.p = burn::softmax_rows(sc, nullptr, scale, false);
    sv.om = burn::empty(ctx, {R, d});
    burn::matmul_items(sv.p, false, s_at, sv.qkv, false, v_at, B, H, S, S, dk, sv.om, o_at);
    x = linear(sv.om, L.wo, L.bo, &x);
    sv.x_mid = x;
    sv.n2 = burn::layer_norm(x, L.ln2_g, L.ln2_b, eps);
    sv.h1 = linear(sv.n2, L.w1, L.b1);
    sv.g = burn::gelu(sv.h1);
    x = linear(sv.g, L.w2, L.b2, &x);
  }
  Tensor z = linear(x, m->head_w, m->head_b);                       // [R, V]
  // Cross-entropy through log_softmax: the loss is -mean(logp[target]); its
  // gradient d logp = -1/R at each row's target (negation, mean and gather)
  // gives dz = d logp - exp(logp) * rowsum(d logp) = exp(logp) / R - onehot / R,
  // formed in the same pass over the logits.
  const float inv = 1.0f / static_cast<float>(R);
  burn::CrossEntropy ce = burn::log_softmax_ce(z, targets, inv);
  Tensor loss = burn::float_neg(burn::reduce_all(ce.picked, MI_R_MEAN));

  // Backward.
  Tensor dz = ce.dlogits;
  // SGD (p <- p - grad * lr) runs once, in place, after the backward: the
  // gradients are collected here.
  std::vector<const Tensor *> upd_p;
  std::vector<Tensor> upd_g;
  auto sgd = [&](const Tensor &p, const Tensor &grad) {
    upd_p.push_back(&p);
    upd_g.push_back(grad);
  };
  // Linear's backward (ops.rs:5006-5029): dW = x^T dy, db = sum_rows(dy),
  // dx = dy W^T.  dW is left as its split-K slices: the SGD step folds them.
  auto linear_back = [&](const Tensor &xin, const Tensor &dy, const Tensor &w, const Tensor &b) {
    Tensor dw = burn::matmul_slices(xin, true, dy, false);
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
    // Attention block: d scores = d o v^T, dv = p^T d o, then through the
    // softmax, dq = ds k and dk = ds^T q, each written into its columns of
    // the [R, 3d] gradient of the fused projection.
    Tensor dom = linear_back(sv.om, dx2, L.wo, L.bo);
    Tensor dp = burn::empty(ctx, {items * S, S});
    burn::matmul_items(dom, false, o_at, sv.qkv, true, v_at, B, H, S, dk, S, dp, s_at);
    Tensor dqkv = burn::empty(ctx, {R, W});
    burn::matmul_items(sv.p, true, s_at, dom, false, o_at, B, H, S, S, dk, dqkv, v_at);
    Tensor ds = burn::softmax_backward(sv.p, dp, scale);
    burn::matmul_items(ds, false, s_at, sv.qkv, false, k_at, B, H, S, S, dk, dqkv, q_at);
    burn::matmul_items(ds, true, s_at, sv.qkv, false, q_at, B, H, S, S, dk, dqkv, k_at);
    Tensor dn1 = linear_back(sv.n1, dqkv, L.wqkv, L.bqkv);
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
      // q, k and v drawn one after another, as three Linears, then placed
      // side by side.
      L.wqkv = burn::empty(ctx, {d, 3 * d});
      L.bqkv = burn::empty(ctx, {1, 3 * d});
      for (int64_t part = 0; part < 3; ++part) {
        const Tensor w = kaiming(ctx, d, d, next());
        const Tensor b = bias(ctx, d, d, next());
        const int64_t dst_st[4] = {0, 0, 3 * d, 1}, src_st[4] = {0, 0, d, 1};
        const int64_t wdims[4] = {1, 1, d, d}, bdims[4] = {1, 1, 1, d};
        burn::copy_into4(L.wqkv, part * d, dst_st, w, 0, src_st, wdims);
        burn::copy_into4(L.bqkv, part * d, dst_st, b, 0, src_st, bdims);
      }
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
  int64_t col0 = 0, ncols = -1;  // a column block of the fused q | k | v
  if (layer < 0) {
    const Tensor *g[] = {&m->embed, &m->head_w, &m->head_b};
    if (which >= 0 && which < 3) t = g[which];
  } else if (layer < static_cast<int>(m->layers.size()) && which >= 0 && which < kLayerParams) {
    TLayer &L = m->layers[layer];
    const Tensor *p[] = {&L.ln1_g, &L.ln1_b, &L.wqkv, &L.bqkv, &L.wqkv, &L.bqkv, &L.wqkv, &L.bqkv,
                         &L.wo,    &L.bo,    &L.ln2_g, &L.ln2_b, &L.w1,  &L.b1,   &L.w2,   &L.b2};
    t = p[which];
    if (which >= 2 && which < 8) {
      ncols = m->cfg.d_model;
      col0 = (which - 2) / 2 * ncols;
    }
  }
  if (!t) {
    g_tf_error = "no such parameter";
    return MI_E_ARG;
  }
  try {
    // A copy (of the whole parameter or of its column block) the caller frees.
    const int64_t rows = t->rows(), cols = t->cols();
    const int64_t n = ncols < 0 ? cols : ncols;
    const int64_t dims[4] = {1, 1, rows, n};
    const int64_t st[4] = {0, 0, cols, 1};
    mi_id id;
    burn::check(m->ctx, mi_copy_strided4(m->ctx, t->use(), dims, col0, st, &id), "param");
    *out = id;
  } catch (const std::exception &e) {
    return fail_tf(e);
  }
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
