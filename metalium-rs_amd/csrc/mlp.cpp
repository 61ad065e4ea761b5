// The MLP training harness over the engine (784 -> 128 ->
// 10, ReLU, softmax cross-entropy, SGD).
//
// Reference: the MNIST gate crates/tt-tests/tests/step12_mnist.rs -- Burn's
// `Linear` (weight [d_in, d_out], y = x W + b) initialised U(-k, k),
// k = 1 / sqrt(d_in), from the 64-bit LCG seeded 0x3a15 (57-103), forward
// l2(relu(l1(x))) (112-114), `CrossEntropyLoss` and `Sgd`.  The loss is Burn's
// composition -- log_softmax, gather of each row's target, mean, negation
// (crates/burn-tt/src/ops.rs:5057, 1001, 3255) -- and the backward restates
// burn-autodiff's rules for each op: negation and mean give -1/B at every
// element the gather picked (scatter_add_columns, ops.rs:1043); log_softmax's
// backward is g - exp(y) * sum_row(g); Linear's is dW = x^T dY, db = the row
// sum of dY, dX = dY W^T (ops.rs:5006-5029); ReLU's passes dY where the
// output is positive (ops.rs:5174).  SGD: p <- p - lr * grad.
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/miburn_models.h"
#include "burn.hpp"

namespace {
thread_local std::string g_mlp_error;
using burn::Tensor;
}  // namespace

struct mi_mlp {
  mi_ctx *ctx;
  int64_t d_in, hidden, d_out;
  Tensor w1, b1, w2, b2;
};

namespace {

int fail_mlp(const std::exception &e) {
  g_mlp_error = e.what();
  if (auto *be = dynamic_cast<const burn::Error *>(&e)) return be->status;
  return MI_E_ARG;
}

// step12's generator: x <- 6364136223846793005 x + 1442695040888963407,
// value (x >> 33) / 2^30 - 1 in [-1, 1).
struct Lcg {
  uint64_t s;
  float unit() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return static_cast<float>(static_cast<double>(s >> 33) / static_cast<double>(1ull << 30) - 1.0);
  }
};

// One training step on resident x [B, d_in] and labels [B, 1] I32; returns the
// loss [1, 1] and updates the parameters in place (new buffers).
Tensor step(mi_mlp *m, const Tensor &x, const Tensor &labels, float lr) {
  const int64_t B = x.rows();
  // Forward.
  Tensor a1 = burn::float_add(burn::float_matmul(x, false, m->w1, false), m->b1);
  Tensor h = burn::relu(a1);
  Tensor z = burn::float_add(burn::float_matmul(h, false, m->w2, false), m->b2);
  Tensor logp = burn::softmax_rows(z, nullptr, 1.0f, true);
  Tensor picked = burn::pick_columns(logp, labels);                 // [B, 1]
  Tensor loss = burn::float_neg(burn::reduce_all(picked, MI_R_MEAN));  // [1, 1]
  // Backward.  d(picked) = -1/B at each row's target column of d(logp).
  Tensor zeros = burn::fill(m->ctx, {B, m->d_out}, MI_F32, 0);
  const float inv = -1.0f / static_cast<float>(B);
  uint32_t inv_bits;
  std::memcpy(&inv_bits, &inv, 4);
  Tensor gv = burn::fill(m->ctx, {B, 1}, MI_F32, inv_bits);
  Tensor g = burn::scatter_add_columns(zeros, labels, gv);          // d logp
  Tensor gs = burn::reduce(g, MI_R_SUM, MI_AXIS_COLS);              // [B, 1]
  Tensor dz = burn::float_sub(g, burn::float_mul(burn::float_exp(logp), gs));
  Tensor dw2 = burn::float_matmul(h, true, dz, false);              // h^T dz
  Tensor db2 = burn::reduce(dz, MI_R_SUM, MI_AXIS_ROWS);
  Tensor dh = burn::float_matmul(dz, false, m->w2, true);           // dz W2^T
  Tensor da1 = burn::relu_backward(h, dh);
  Tensor dw1 = burn::float_matmul(x, true, da1, false);
  Tensor db1 = burn::reduce(da1, MI_R_SUM, MI_AXIS_ROWS);
  // SGD, in place, one launch.
  burn::sgd_update(m->ctx, {&m->w1, &m->b1, &m->w2, &m->b2}, {dw1, db1, dw2, db2}, lr);
  return loss;
}

}  // namespace

extern "C" {

const char *mi_mlp_last_error(void) { return g_mlp_error.c_str(); }

int mi_mlp_create(mi_ctx *ctx, int32_t d_in, int32_t hidden, int32_t d_out, uint64_t lcg_seed, mi_mlp **out) {
  if (!ctx || !out || d_in <= 0 || hidden <= 0 || d_out <= 0) return MI_E_ARG;
  mi_mlp *m = new mi_mlp();
  try {
    m->ctx = ctx;
    m->d_in = d_in;
    m->hidden = hidden;
    m->d_out = d_out;
    Lcg rng{lcg_seed};
    auto layer = [&](int64_t din, int64_t dout, Tensor &w, Tensor &b) {
      const float k = 1.0f / std::sqrt(static_cast<float>(din));
      std::vector<float> wv(static_cast<size_t>(din * dout)), bv(static_cast<size_t>(dout));
      for (float &v : wv) v = rng.unit() * k;
      for (float &v : bv) v = rng.unit() * k;
      w = burn::float_from_data(ctx, wv.data(), {din, dout});
      b = burn::float_from_data(ctx, bv.data(), {1, dout});
    };
    layer(d_in, hidden, m->w1, m->b1);
    layer(hidden, d_out, m->w2, m->b2);
  } catch (const std::exception &e) {
    delete m;
    return fail_mlp(e);
  }
  *out = m;
  return MI_OK;
}

int mi_mlp_destroy(mi_mlp *m) {
  delete m;
  return MI_OK;
}

int mi_mlp_param(mi_mlp *m, int which, mi_id *out) {
  if (!m || !out || which < 0 || which > 3) return MI_E_ARG;
  const Tensor *t[] = {&m->w1, &m->b1, &m->w2, &m->b2};
  try {
    t[which]->use();
  } catch (const std::exception &e) {
    return fail_mlp(e);
  }
  *out = t[which]->id();
  return MI_OK;
}

int mi_mlp_train_step(mi_mlp *m, mi_id x, mi_id labels, float lr, mi_id *loss) {
  if (!m || !loss) return MI_E_ARG;
  try {
    int64_t xr, xc, lr_, lc;
    int xe, le;
    burn::check(m->ctx, mi_metadata(m->ctx, x, &xr, &xc, &xe), "x");
    burn::check(m->ctx, mi_metadata(m->ctx, labels, &lr_, &lc, &le), "labels");
    if (xc != m->d_in || xe != MI_F32 || le != MI_I32 || lr_ * lc != xr)
      throw burn::Error(MI_E_ARG, "mlp step: x must be [B, d_in] F32 and labels B I32");
    // Borrow the caller's buffers without taking ownership: copy the ids into
    // fresh tensors (the engine copies are device-to-device).
    mi_id xi, li;
    burn::check(m->ctx, mi_cast(m->ctx, x, MI_F32, &xi), "x");
    burn::check(m->ctx, mi_cast(m->ctx, labels, MI_I32, &li), "labels");
    Tensor xt(m->ctx, xi, {xr, xc}), lt(m->ctx, li, {xr, 1});
    Tensor l = step(m, xt, lt, lr);
    mi_id id;
    burn::check(m->ctx, mi_cast(m->ctx, l.use(), MI_F32, &id), "loss");
    *loss = id;
  } catch (const std::exception &e) {
    return fail_mlp(e);
  }
  return MI_OK;
}

int mi_mlp_train_synthetic(mi_mlp *m, int32_t batch, int32_t steps, float lr, uint64_t data_seed, float *losses,
                           double *ms) {
  if (!m || batch <= 0 || steps < 0) return MI_E_ARG;
  using clock = std::chrono::steady_clock;
  try {
    std::vector<Tensor> ls;
    ls.reserve(static_cast<size_t>(steps));
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    auto t0 = clock::now();
    for (int32_t s = 0; s < steps; ++s) {
      const uint64_t base = data_seed * 0x100000001b3ull + static_cast<uint64_t>(s) * 2;
      Tensor x = burn::random(m->ctx, {batch, m->d_in}, MI_DRAW_UNIT, 0.0f, 1.0f, base);
      Tensor y = burn::random(m->ctx, {batch, 1}, MI_DRAW_INT_RANGE, 0.0f, static_cast<float>(m->d_out), base + 1);
      ls.push_back(step(m, x, y, lr));
    }
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    auto t1 = clock::now();
    if (ms) *ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (losses)
      for (int32_t s = 0; s < steps; ++s) losses[s] = burn::float_into_data(ls[s])[0];
  } catch (const std::exception &e) {
    return fail_mlp(e);
  }
  return MI_OK;
}

}  // extern "C"
