// Host-side tensor layer over the engine's C ABI: the shape of the
// reference's Burn backend surface (`FloatTensorOps` / `IntTensorOps`,
// crates/burn-tt/src/generated/ops.rs:78, 2423) for the model harnesses.
//
// A Tensor is a shared handle on one engine buffer plus its logical shape;
// dropping the last handle frees the buffer (crates/burn-tt/src/tensor.rs:
// 188-192).  Rank-N shapes fold to `[prod(leading), last]`
// (tensor.rs:905-908).  A failed engine call throws `burn::Error` carrying the
// engine's status and message; model entry points catch it at the C boundary.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/miburn.h"

namespace burn {

struct Error : std::runtime_error {
  int status;
  Error(int st, const std::string &m) : std::runtime_error(m), status(st) {}
};

inline void check(mi_ctx *ctx, int st, const char *what) {
  if (st != MI_OK) throw Error(st, std::string(what) + ": " + mi_last_error(ctx));
}

struct Buf {
  mi_ctx *ctx;
  mi_id id;
  Buf(mi_ctx *c, mi_id i) : ctx(c), id(i) {}
  ~Buf() { mi_free(ctx, id); }
  Buf(const Buf &) = delete;
  Buf &operator=(const Buf &) = delete;
};

class Tensor {
 public:
  Tensor() = default;
  Tensor(mi_ctx *ctx, mi_id id, std::vector<int64_t> shape) : buf_(std::make_shared<Buf>(ctx, id)), shape_(std::move(shape)) {}

  mi_id id() const { return buf_ ? buf_->id : 0; }
  // The id with the engine buffer's [rows, cols] set to this tensor's folded
  // shape (handles sharing storage may fold it differently): pass this to
  // every op.
  mi_id use() const {
    check(ctx(), mi_reshape(ctx(), id(), rows(), cols()), "shape");
    return id();
  }
  mi_ctx *ctx() const { return buf_->ctx; }
  const std::vector<int64_t> &shape() const { return shape_; }
  int64_t dim(int i) const { return shape_[i < 0 ? shape_.size() + i : i]; }
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape_) n *= d;
    return n;
  }
  int64_t cols() const { return shape_.empty() ? 1 : shape_.back(); }
  int64_t rows() const { return cols() == 0 ? 0 : numel() / cols(); }
  bool defined() const { return static_cast<bool>(buf_); }

  // float_reshape: a new logical shape over the same storage (free).  The
  // engine buffer takes the folded [rows, cols] of the new shape.
  Tensor reshape(std::vector<int64_t> shape) const {
    Tensor t = *this;
    t.shape_ = std::move(shape);
    check(ctx(), mi_reshape(ctx(), id(), t.rows(), t.cols()), "reshape");
    return t;
  }

 private:
  std::shared_ptr<Buf> buf_;
  std::vector<int64_t> shape_;
};

// Wrap a fresh engine id with a logical shape.
inline Tensor wrap(mi_ctx *ctx, mi_id id, std::vector<int64_t> shape) {
  Tensor t(ctx, id, std::move(shape));
  check(ctx, mi_reshape(ctx, id, t.rows(), t.cols()), "shape");
  return t;
}

// ------------------------------------------------------------------ ops
// Names follow Burn's trait methods; each is one engine call.

inline Tensor float_from_data(mi_ctx *ctx, const float *v, std::vector<int64_t> shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_upload(ctx, v, cols ? n / cols : 0, cols, &id), "float_from_data");
  return Tensor(ctx, id, std::move(shape));
}

inline Tensor int_from_data(mi_ctx *ctx, const int32_t *v, std::vector<int64_t> shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_upload_bits(ctx, reinterpret_cast<const uint32_t *>(v), cols ? n / cols : 0, cols, MI_I32, &id),
        "int_from_data");
  return Tensor(ctx, id, std::move(shape));
}

inline Tensor bool_from_data(mi_ctx *ctx, const uint32_t *v, std::vector<int64_t> shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_upload_bits(ctx, v, cols ? n / cols : 0, cols, MI_BOOL, &id), "bool_from_data");
  return Tensor(ctx, id, std::move(shape));
}

inline std::vector<float> float_into_data(const Tensor &t) {
  std::vector<float> v(static_cast<size_t>(t.numel()));
  check(t.ctx(), mi_download(t.ctx(), t.use(), v.data(), t.numel()), "float_into_data");
  return v;
}

inline std::vector<int32_t> int_into_data(const Tensor &t) {
  std::vector<int32_t> v(static_cast<size_t>(t.numel()));
  check(t.ctx(), mi_download_bits(t.ctx(), t.use(), reinterpret_cast<uint32_t *>(v.data()), t.numel()),
        "int_into_data");
  return v;
}

inline Tensor random(mi_ctx *ctx, std::vector<int64_t> shape, int draw, float p1, float p2, uint64_t base) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_random(ctx, cols ? n / cols : 0, cols, draw, p1, p2, base, &id), "float_random");
  return Tensor(ctx, id, std::move(shape));
}

inline Tensor fill(mi_ctx *ctx, std::vector<int64_t> shape, int elem, uint32_t bits) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_fill(ctx, cols ? n / cols : 0, cols, elem, bits, &id), "fill");
  return Tensor(ctx, id, std::move(shape));
}

// float_empty: contents unspecified until written.
inline Tensor empty(mi_ctx *ctx, std::vector<int64_t> shape, int elem = MI_F32) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const int64_t cols = shape.empty() ? 1 : shape.back();
  mi_id id;
  check(ctx, mi_empty(ctx, cols ? n / cols : 0, cols, elem, &id), "empty");
  return Tensor(ctx, id, std::move(shape));
}

// Result forms holding an F32 result's two BF16 parts ([rows, 2 cols]).
inline bool two_parts(int form) { return form == MI_BF16_PARTS || form == MI_TILES_PARTS; }

// A row-major [r, c] operand in the matrix cores' operand order (mi_tile).
inline Tensor tile(const Tensor &a, int form) {
  mi_id id;
  check(a.ctx(), mi_tile(a.ctx(), a.use(), form, &id), "tile");
  return Tensor(a.ctx(), id, {a.rows(), form == MI_TILES_PARTS ? 2 * a.cols() : a.cols()});
}

// An F32 tensor's BF16 parts ([rows, 2 cols], MI_BF16_PARTS: mi_cast).
inline Tensor parts(const Tensor &a) {
  mi_id id;
  check(a.ctx(), mi_cast(a.ctx(), a.use(), MI_BF16_PARTS, &id), "parts");
  return Tensor(a.ctx(), id, {a.rows(), 2 * a.cols()});
}

inline Tensor float_cast(const Tensor &a, int elem) {
  mi_id id;
  check(a.ctx(), mi_cast(a.ctx(), a.use(), elem, &id), "float_cast");
  return Tensor(a.ctx(), id, a.shape());
}

// Element-wise op by the reference's op id; the result takes a's shape
// unless b (broadcast) is larger.
inline Tensor eltwise(uint32_t kind, const Tensor &a, const Tensor *b = nullptr, const Tensor *c = nullptr,
                      float s1 = 0.0f, float s2 = 0.0f, int out_elem = MI_F32) {
  mi_id id;
  check(a.ctx(), mi_eltwise(a.ctx(), kind, s1, s2, a.use(), b ? b->use() : 0, c ? c->use() : 0, out_elem, &id),
        "eltwise");
  std::vector<int64_t> shape = a.shape();
  if (b && b->numel() > a.numel()) shape = b->shape();
  return Tensor(a.ctx(), id, shape);
}
inline Tensor float_add(const Tensor &a, const Tensor &b) { return eltwise(MI_K_ADD, a, &b); }
inline Tensor float_sub(const Tensor &a, const Tensor &b) { return eltwise(MI_K_SUB, a, &b); }
inline Tensor float_mul(const Tensor &a, const Tensor &b) { return eltwise(MI_K_MUL, a, &b); }
inline Tensor float_mul_scalar(const Tensor &a, float s) { return eltwise(MI_K_MUL_SCALAR, a, nullptr, nullptr, s); }
inline Tensor float_add_scalar(const Tensor &a, float s) { return eltwise(MI_K_ADD_SCALAR, a, nullptr, nullptr, s); }
inline Tensor relu(const Tensor &a) { return eltwise(MI_K_RELU, a); }
inline Tensor relu_backward(const Tensor &out, const Tensor &grad) { return eltwise(MI_K_RELU_BACKWARD, out, &grad); }
inline Tensor gelu(const Tensor &a) { return eltwise(MI_K_GELU, a); }
inline Tensor gelu_backward(const Tensor &x, const Tensor &grad) { return eltwise(MI_K_GELU_BACKWARD, x, &grad); }
inline Tensor float_exp(const Tensor &a) { return eltwise(MI_K_EXP, a); }
inline Tensor float_neg(const Tensor &a) { return eltwise(MI_K_NEG, a); }
// silu(gate) * up in one pass (crates/burn-tt/src/ops.rs:2622-2651).
inline Tensor silu_mul(const Tensor &gate, const Tensor &up) { return eltwise(MI_K_SILU_MUL, gate, &up); }

// float_matmul over the folded matrices: a [.., k] (or, transposed, its
// stored [k, m]) times b [k, n] (or [n, k] transposed).
inline Tensor float_matmul(const Tensor &a, bool ta, const Tensor &b, bool tb, int out_elem = MI_F32) {
  mi_id id;
  check(a.ctx(), mi_matmul(a.ctx(), a.use(), ta, b.use(), tb, out_elem, &id), "float_matmul");
  const int64_t m = ta ? a.cols() : a.rows();
  const int64_t n = tb ? b.rows() : b.cols();
  std::vector<int64_t> shape;
  if (!ta && a.shape().size() > 2) {
    shape.assign(a.shape().begin(), a.shape().end() - 1);
    shape.push_back(n);
  } else {
    shape = {m, n};
  }
  return Tensor(a.ctx(), id, shape);
}

// Cross-entropy against integer targets and its gradient in one pass:
// picked = logp at each row's target ([rows, 1]), dlogits = exp(logp) * s
// minus s at the target.
struct CrossEntropy {
  Tensor picked, dlogits;
};
inline CrossEntropy log_softmax_ce(const Tensor &logits, const Tensor &targets, float grad_scale) {
  mi_id p, d;
  check(logits.ctx(), mi_log_softmax_ce(logits.ctx(), logits.use(), targets.use(), grad_scale, &p, &d),
        "log_softmax_ce");
  return {Tensor(logits.ctx(), p, {logits.rows(), 1}), Tensor(logits.ctx(), d, {logits.rows(), logits.cols()})};
}

// A product left as its split-K slices ([S * m, n]; S = 1: the product),
// for mi_sgd_update to fold.
inline Tensor matmul_slices(const Tensor &a, bool ta, const Tensor &b, bool tb) {
  mi_id id;
  int64_t S = 1;
  check(a.ctx(), mi_matmul_slices(a.ctx(), a.use(), ta, b.use(), tb, &id, &S), "matmul_slices");
  return Tensor(a.ctx(), id, {S * (ta ? a.cols() : a.rows()), tb ? b.rows() : b.cols()});
}

// A Linear forward with an optional residual: residual + (x @ op(w) + bias),
// the adds in the product's epilogue (null pointers omit a term).
inline Tensor linear(const Tensor &x, const Tensor &w, bool tw, const Tensor *bias, const Tensor *residual,
                     int out_elem = MI_F32) {
  mi_id id;
  check(x.ctx(), mi_linear(x.ctx(), x.use(), w.use(), tw, bias ? bias->use() : 0, residual ? residual->use() : 0,
                           out_elem, &id), "linear");
  return Tensor(x.ctx(), id, {x.rows(), tw ? w.rows() : w.cols()});
}

// linear() then rms_norm() of its result in one call: (y, rms_norm(y) gamma
// as norm_elem).
inline std::pair<Tensor, Tensor> linear_add_rms_norm(const Tensor &x, const Tensor &w, bool tw, const Tensor *bias,
                                                     const Tensor *residual, const Tensor &gamma, float eps,
                                                     int norm_elem) {
  mi_id y, yn;
  check(x.ctx(), mi_linear_add_rms_norm(x.ctx(), x.use(), w.use(), tw, bias ? bias->use() : 0,
                                        residual ? residual->use() : 0, gamma.use(), eps, norm_elem, &y, &yn),
        "linear_add_rms_norm");
  const int64_t n = tw ? w.rows() : w.cols();
  return {Tensor(x.ctx(), y, {x.rows(), n}), Tensor(x.ctx(), yn, {x.rows(), two_parts(norm_elem) ? 2 * n : n})};
}

// linear() of an F32 operand given as its BF16 parts ([m, 2 k], MI_BF16_PARTS
// from rms_norm or silu_mul_halves): mi_linear_parts.
inline Tensor linear_parts(const Tensor &x_parts, const Tensor &w, bool tw, const Tensor *bias, const Tensor *residual,
                           int out_elem = MI_F32) {
  mi_id id;
  check(x_parts.ctx(), mi_linear_parts(x_parts.ctx(), x_parts.use(), w.use(), tw, bias ? bias->use() : 0,
                                       residual ? residual->use() : 0, out_elem, &id), "linear_parts");
  return Tensor(x_parts.ctx(), id, {x_parts.rows(), tw ? w.rows() : w.cols()});
}

// silu(x gate^T) * (x up^T) as BF16 parts from x's parts and the gate|up
// weight interleaved in 32-row groups: mi_linear_swiglu_parts.
inline Tensor linear_swiglu_parts(const Tensor &x_parts, const Tensor &w_pairs) {
  mi_id id;
  check(x_parts.ctx(), mi_linear_swiglu_parts(x_parts.ctx(), x_parts.use(), w_pairs.use(), &id), "linear_swiglu_parts");
  return Tensor(x_parts.ctx(), id, {x_parts.rows(), w_pairs.rows()});
}

// The same from BF16 activations, F32 or rounded to BF16: mi_linear_swiglu.
inline Tensor linear_swiglu(const Tensor &x, const Tensor &w_pairs, int out_elem) {
  mi_id id;
  check(x.ctx(), mi_linear_swiglu(x.ctx(), x.use(), w_pairs.use(), out_elem, &id), "linear_swiglu");
  return Tensor(x.ctx(), id, {x.rows(), two_parts(out_elem) ? w_pairs.rows() : w_pairs.rows() / 2});
}

// The q|k|v product and the prefill's q|k|v tail in one launch
// (mi_linear_qkv_rope_cache): q out, as qkv_rope_cache.
inline Tensor linear_qkv_rope_cache(const Tensor &x, bool x_parts, const Tensor &w_qkv, const Tensor &cos,
                                    const Tensor &sin, int64_t seq, int64_t heads, int64_t kv_heads, int64_t pos0,
                                    const Tensor &k_cache, const Tensor &v_cache, bool grouped) {
  mi_id id;
  check(x.ctx(), mi_linear_qkv_rope_cache(x.ctx(), x.use(), x_parts ? 1 : 0, w_qkv.use(), cos.use(), sin.use(), seq,
                                          heads, kv_heads, pos0, k_cache.use(), v_cache.use(), grouped ? 1 : 0, &id),
        "linear_qkv_rope_cache");
  return Tensor(x.ctx(), id, {x.rows() * heads, k_cache.cols()});
}

// Grouped strided products written into `out` in place (item (g, i) of an
// operand at at[0] + g * at[1] + i * at[2], read with its row pitch).
struct Items {
  int64_t offset, group_stride, item_stride;
};
inline void matmul_items(const Tensor &a, bool ta, Items a_at, const Tensor &b, bool tb, Items b_at, int64_t groups,
                         int64_t per_group, int64_t m, int64_t k, int64_t n, const Tensor &out, Items out_at) {
  const int64_t aa[3] = {a_at.offset, a_at.group_stride, a_at.item_stride};
  const int64_t bb[3] = {b_at.offset, b_at.group_stride, b_at.item_stride};
  const int64_t oo[3] = {out_at.offset, out_at.group_stride, out_at.item_stride};
  check(a.ctx(), mi_matmul_items(a.ctx(), a.use(), ta, aa, b.use(), tb, bb, groups, per_group, m, k, n, out.use(), oo),
        "matmul_items");
}

// Products over item blocks of resident buffers (batched_matmul,
// crates/burn-tt/src/ops.rs:2981-3052): result [batch * m, n].
inline Tensor matmul_blocks(const Tensor &a, bool ta, const Tensor &b, bool tb, int64_t batch, int64_t m, int64_t k,
                            int64_t n, int64_t a_off, int64_t a_stride, int64_t b_off, int64_t b_stride) {
  mi_id id;
  check(a.ctx(), mi_matmul_blocks(a.ctx(), a.use(), ta, b.use(), tb, batch, m, k, n, a_off, a_stride, b_off, b_stride,
                                  MI_F32, &id), "matmul_blocks");
  return Tensor(a.ctx(), id, {batch * m, n});
}

inline Tensor reduce(const Tensor &a, int op, int axis) {
  mi_id id;
  check(a.ctx(), mi_reduce(a.ctx(), a.use(), op, axis, &id), "reduce");
  return Tensor(a.ctx(), id, axis == MI_AXIS_COLS ? std::vector<int64_t>{a.rows(), 1} : std::vector<int64_t>{1, a.cols()});
}
inline Tensor reduce_all(const Tensor &a, int op) {
  mi_id id;
  check(a.ctx(), mi_reduce_all(a.ctx(), a.use(), op, &id), "reduce_all");
  return Tensor(a.ctx(), id, {1, 1});
}

inline Tensor softmax_rows(const Tensor &x, const Tensor *mask, float scale, bool log) {
  mi_id id;
  check(x.ctx(), mi_softmax_rows(x.ctx(), x.use(), mask ? mask->use() : 0, scale, log, MI_F32, &id), "softmax_rows");
  return Tensor(x.ctx(), id, x.shape());
}

// RMSNorm over rows: F32, rounded to BF16, or as its BF16 parts ([rows,
// 2 cols]).
inline Tensor rms_norm(const Tensor &x, const Tensor &gamma, float eps, int out_elem = MI_F32) {
  mi_id id;
  check(x.ctx(), mi_rms_norm(x.ctx(), x.use(), gamma.use(), eps, out_elem, &id), "rms_norm");
  if (two_parts(out_elem)) return Tensor(x.ctx(), id, {x.rows(), 2 * x.cols()});
  return Tensor(x.ctx(), id, x.shape());
}

inline Tensor layer_norm(const Tensor &x, const Tensor &gamma, const Tensor &beta, float eps) {
  mi_id id;
  check(x.ctx(), mi_layer_norm(x.ctx(), x.use(), gamma.use(), beta.use(), eps, &id), "layer_norm");
  return Tensor(x.ctx(), id, x.shape());
}

struct NormGrads {
  Tensor dx, dgamma, dbeta;
};
// LayerNorm's gradient (fused); `residual` (may be undefined) is added to dx.
inline NormGrads layer_norm_backward(const Tensor &x, const Tensor &gamma, const Tensor &dy, const Tensor &residual,
                                     float eps) {
  mi_id ids[3];
  check(x.ctx(), mi_layer_norm_backward(x.ctx(), x.use(), gamma.use(), dy.use(), residual.defined() ? residual.use() : 0,
                                        eps, &ids[0], &ids[1], &ids[2]),
        "layer_norm_backward");
  return {Tensor(x.ctx(), ids[0], x.shape()), Tensor(x.ctx(), ids[1], {1, x.cols()}),
          Tensor(x.ctx(), ids[2], {1, x.cols()})};
}

// Softmax's gradient over rows: scale * p * (dp - rowsum(p * dp)).
inline Tensor softmax_backward(const Tensor &p, const Tensor &dp, float scale) {
  mi_id id;
  check(p.ctx(), mi_softmax_backward(p.ctx(), p.use(), dp.use(), scale, &id), "softmax_backward");
  return Tensor(p.ctx(), id, p.shape());
}

// Sgd's step in place over (parameter, gradient) pairs, one launch.
inline void sgd_update(mi_ctx *ctx, const std::vector<const Tensor *> &params, const std::vector<Tensor> &grads,
                       float lr) {
  std::vector<mi_id> p, g;
  for (size_t i = 0; i < params.size(); ++i) {
    p.push_back(params[i]->use());
    g.push_back(grads[i].use());
  }
  check(ctx, mi_sgd_update(ctx, static_cast<int64_t>(p.size()), p.data(), g.data(), lr), "sgd_update");
}

inline Tensor argmax_rows(const Tensor &x) {
  mi_id id;
  check(x.ctx(), mi_argmax_rows(x.ctx(), x.use(), &id), "float_argmax");
  return Tensor(x.ctx(), id, {x.rows(), 1});
}

// embedding: rows of the table for every index, [.., d].
inline Tensor select_rows(const Tensor &table, const Tensor &idx) {
  mi_id id;
  check(table.ctx(), mi_select_rows(table.ctx(), table.use(), idx.use(), &id), "select_rows");
  std::vector<int64_t> shape = idx.shape();
  if (shape.size() >= 2 && shape.back() == 1) shape.pop_back();
  shape.push_back(table.cols());
  return Tensor(table.ctx(), id, shape);
}

// select_rows then float_cast to out_elem (mi_select_rows_as: one launch for
// a BF16 table widened to F32).
inline Tensor select_rows_as(const Tensor &table, const Tensor &idx, int out_elem) {
  mi_id id;
  check(table.ctx(), mi_select_rows_as(table.ctx(), table.use(), idx.use(), out_elem, &id), "select_rows_as");
  std::vector<int64_t> shape = idx.shape();
  if (shape.size() >= 2 && shape.back() == 1) shape.pop_back();
  shape.push_back(table.cols());
  return Tensor(table.ctx(), id, shape);
}

inline Tensor pick_columns(const Tensor &x, const Tensor &idx) {
  mi_id id;
  check(x.ctx(), mi_pick_columns(x.ctx(), x.use(), idx.use(), &id), "pick_columns");
  return Tensor(x.ctx(), id, {x.rows(), 1});
}

inline Tensor scatter_add_columns(const Tensor &x, const Tensor &idx, const Tensor &v) {
  mi_id id;
  check(x.ctx(), mi_scatter_add_columns(x.ctx(), x.use(), idx.use(), v.use(), &id), "scatter_add_columns");
  return Tensor(x.ctx(), id, x.shape());
}

inline Tensor select_add_rows(const Tensor &t, const Tensor &idx, const Tensor &v) {
  mi_id id;
  check(t.ctx(), mi_select_add_rows(t.ctx(), t.use(), idx.use(), v.use(), &id), "select_add_rows");
  return Tensor(t.ctx(), id, t.shape());
}

// A strided 4-D gather into a new [d0 * d1 * d2, d3] tensor (swap_dims,
// head split/merge materialised).
inline Tensor copy4(const Tensor &src, const int64_t dims[4], int64_t off, const int64_t st[4]) {
  mi_id id;
  check(src.ctx(), mi_copy_strided4(src.ctx(), src.use(), dims, off, st, &id), "copy_strided4");
  return Tensor(src.ctx(), id, {dims[0] * dims[1] * dims[2], dims[3]});
}

inline void copy_into4(const Tensor &dst, int64_t doff, const int64_t dst_st[4], const Tensor &src, int64_t soff,
                       const int64_t src_st[4], const int64_t dims[4]) {
  check(dst.ctx(), mi_copy_into4(dst.ctx(), dst.use(), doff, dst_st, src.use(), soff, src_st, dims), "copy_into4");
}

inline Tensor rope(const Tensor &x, const Tensor &cos, const Tensor &sin, int64_t heads, int64_t seq, int64_t pos0) {
  mi_id id;
  check(x.ctx(), mi_rope(x.ctx(), x.use(), cos.use(), sin.use(), heads, seq, pos0, &id), "rope");
  return Tensor(x.ctx(), id, x.shape());
}

// silu(gate) * up of a fused gate|up product's halves (mi_silu_mul_halves),
// F32, rounded to BF16, or as its BF16 parts (twice as many columns).
inline Tensor silu_mul_halves(const Tensor &gate_up, int out_elem = MI_F32) {
  mi_id id;
  check(gate_up.ctx(), mi_silu_mul_halves(gate_up.ctx(), gate_up.use(), out_elem, &id), "silu_mul_halves");
  return Tensor(gate_up.ctx(), id, {gate_up.rows(), out_elem == MI_BF16_PARTS ? gate_up.cols() : gate_up.cols() / 2});
}

// The prefill's q|k|v tail (mi_qkv_rope_cache): RoPE, cache writes, q out.
inline Tensor qkv_rope_cache(const Tensor &qkv, const Tensor &cos, const Tensor &sin, int64_t seq, int64_t heads,
                             int64_t kv_heads, int64_t pos0, const Tensor &k_cache, const Tensor &v_cache,
                             bool grouped) {
  mi_id id;
  check(qkv.ctx(), mi_qkv_rope_cache(qkv.ctx(), qkv.use(), cos.use(), sin.use(), seq, heads, kv_heads, pos0,
                                     k_cache.use(), v_cache.use(), grouped ? 1 : 0, &id), "qkv_rope_cache");
  return Tensor(qkv.ctx(), id, {qkv.rows() * heads, k_cache.cols()});
}

inline Tensor attention_rows(const Tensor &q, const Tensor &k_cache, const Tensor &v_cache, int64_t batch, int64_t t,
                             int64_t heads, int64_t kv_heads, int64_t pos0, float scale) {
  mi_id id;
  check(q.ctx(), mi_attention_rows(q.ctx(), q.use(), k_cache.use(), v_cache.use(), batch, t, heads, kv_heads, pos0,
                                   scale, &id),
        "attention_rows");
  return Tensor(q.ctx(), id, {q.rows(), q.cols()});
}
// The same with its result in `form` (mi_attention_rows_as: rounded to BF16,
// or tiles for an o projection against a tiled weight).
inline Tensor attention_rows_as(const Tensor &q, const Tensor &k_cache, const Tensor &v_cache, int64_t batch, int64_t t,
                                int64_t heads, int64_t kv_heads, int64_t pos0, float scale, int form) {
  mi_id id;
  check(q.ctx(), mi_attention_rows_as(q.ctx(), q.use(), k_cache.use(), v_cache.use(), batch, t, heads, kv_heads, pos0,
                                      scale, form, &id),
        "attention_rows_as");
  return Tensor(q.ctx(), id, {q.rows(), two_parts(form) ? 2 * q.cols() : q.cols()});
}

// attention_rows with the key chunks planned for `span` positions and pos0
// read on the device from `pos` when it is given (mi_attention_rows_at).
inline Tensor attention_rows_at(const Tensor &q, const Tensor &k_cache, const Tensor &v_cache, int64_t batch,
                                int64_t t, int64_t heads, int64_t kv_heads, const Tensor *pos, int64_t pos0,
                                int64_t span, float scale) {
  mi_id id;
  check(q.ctx(), mi_attention_rows_at(q.ctx(), q.use(), k_cache.use(), v_cache.use(), batch, t, heads, kv_heads,
                                      pos ? pos->use() : 0, pos0, span, scale, &id),
        "attention_rows_at");
  return Tensor(q.ctx(), id, {q.rows(), q.cols()});
}

// Fused decode projections (one row per sequence, at most 8 rows).
inline Tensor norm_matvec(const Tensor &x, const Tensor *gamma, float eps, const Tensor &w, const Tensor *residual,
                          bool silu_mul) {
  mi_id id;
  check(x.ctx(), mi_norm_matvec(x.ctx(), x.use(), gamma ? gamma->use() : 0, eps, w.use(),
                                residual ? residual->use() : 0, silu_mul, &id),
        "norm_matvec");
  const int64_t n = silu_mul ? w.rows() / 2 : w.rows();
  return Tensor(x.ctx(), id, {x.rows(), n});
}

// The greedy pick of each row's logits rmsnorm(x) w^T
// (mi_norm_matvec_argmax): [rows, 1] I32.
inline Tensor norm_matvec_argmax(const Tensor &x, const Tensor &gamma, float eps, const Tensor &w) {
  mi_id lg, id;
  check(x.ctx(), mi_norm_matvec_argmax(x.ctx(), x.use(), gamma.use(), eps, w.use(), &lg, &id), "norm_matvec_argmax");
  Tensor logits(x.ctx(), lg, {x.rows(), w.rows()});  // freed here
  return Tensor(x.ctx(), id, {x.rows(), 1});
}

// The attention rows of one new position per sequence from the hidden rows
// (mi_norm_qkv_attention): q|k|v, RoPE, the cache write and the attention.
inline Tensor norm_qkv_attention(const Tensor &x, const Tensor &gamma, float eps, const Tensor &w_qkv,
                                 const Tensor &cos, const Tensor &sin, int64_t heads, int64_t kv_heads,
                                 const Tensor *pos, int64_t pos0, int64_t span, const Tensor &k_cache,
                                 const Tensor &v_cache, float scale) {
  mi_id id;
  check(x.ctx(), mi_norm_qkv_attention(x.ctx(), x.use(), gamma.use(), eps, w_qkv.use(), cos.use(), sin.use(), heads,
                                       kv_heads, pos ? pos->use() : 0, pos0, span, k_cache.use(), v_cache.use(),
                                       scale, &id),
        "norm_qkv_attention");
  return Tensor(x.ctx(), id, {x.rows(), heads * k_cache.cols()});
}

// x + the attention rows times w_o^T (mi_norm_qkv_attention_o): the
// attention block through its output projection and residual.
inline Tensor norm_qkv_attention_o(const Tensor &x, const Tensor &gamma, float eps, const Tensor &w_qkv,
                                   const Tensor &cos, const Tensor &sin, int64_t heads, int64_t kv_heads,
                                   const Tensor *pos, int64_t pos0, int64_t span, const Tensor &k_cache,
                                   const Tensor &v_cache, float scale, const Tensor &w_o) {
  mi_id id;
  check(x.ctx(), mi_norm_qkv_attention_o(x.ctx(), x.use(), gamma.use(), eps, w_qkv.use(), cos.use(), sin.use(),
                                         heads, kv_heads, pos ? pos->use() : 0, pos0, span, k_cache.use(),
                                         v_cache.use(), scale, w_o.use(), &id),
        "norm_qkv_attention_o");
  return Tensor(x.ctx(), id, {x.rows(), x.cols()});
}

inline Tensor norm_qkv_rope(const Tensor &x, const Tensor &gamma, float eps, const Tensor &w_qkv, const Tensor &cos,
                            const Tensor &sin, int64_t heads, int64_t kv_heads, int64_t pos, const Tensor &k_cache,
                            const Tensor &v_cache) {
  mi_id id;
  check(x.ctx(), mi_norm_qkv_rope(x.ctx(), x.use(), gamma.use(), eps, w_qkv.use(), cos.use(), sin.use(), heads,
                                  kv_heads, pos, k_cache.use(), v_cache.use(), &id),
        "norm_qkv_rope");
  return Tensor(x.ctx(), id, {x.rows(), heads * k_cache.cols()});
}

// norm_qkv_rope at the position held on the device in `pos` ([1, 1] I32).
inline Tensor norm_qkv_rope_at(const Tensor &x, const Tensor &gamma, float eps, const Tensor &w_qkv, const Tensor &cos,
                               const Tensor &sin, int64_t heads, int64_t kv_heads, const Tensor &pos,
                               const Tensor &k_cache, const Tensor &v_cache) {
  mi_id id;
  check(x.ctx(), mi_norm_qkv_rope_at(x.ctx(), x.use(), gamma.use(), eps, w_qkv.use(), cos.use(), sin.use(), heads,
                                     kv_heads, pos.use(), k_cache.use(), v_cache.use(), &id),
        "norm_qkv_rope_at");
  return Tensor(x.ctx(), id, {x.rows(), heads * k_cache.cols()});
}

}  // namespace burn
