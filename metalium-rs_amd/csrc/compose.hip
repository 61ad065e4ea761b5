// Engine methods that are compositions of the engine's own ops, each bit for
// bit the sequence of ops the reference's default implementation runs.
//
// Reference: the Engine trait (crates/burn-tt/src/server.rs) --
// reduce with `then` (404-412; ReduceThen, crates/tt-kernels/src/tensor.rs:
// 6038: an exact unary kind applied to the reduction's result),
// add_rms_norm (466-475: s = a + b and s's RMSNorm), and
// matmul_dram_batched over an arbitrary list of operand blocks (229-237;
// Block, crates/tt-kernels/src/tensor.rs:3479-3483).
#include "common.hpp"

#include <vector>

using namespace mi;

namespace {

// Frees an id when it goes out of scope unless released.
struct Owned {
  mi_ctx *ctx;
  mi_id id = 0;
  ~Owned() {
    if (id) mi_free(ctx, id);
  }
  mi_id release() {
    const mi_id r = id;
    id = 0;
    return r;
  }
};

}  // namespace

extern "C" int mi_reduce_then(mi_ctx *ctx, mi_id a, int op, int axis, uint32_t then_kind, float then_scalar,
                              mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  Owned r{ctx};
  int s = mi_reduce(ctx, a, op, axis, &r.id);
  if (s) return s;
  if (then_kind == 0) {
    *out = r.release();
    return MI_OK;
  }
  mi_id t;
  s = mi_eltwise(ctx, then_kind, then_scalar, 0.0f, r.id, 0, 0, MI_F32, &t);
  if (s) return s;
  *out = t;
  return MI_OK;
}

extern "C" int mi_add_rms_norm(mi_ctx *ctx, mi_id a, mi_id b, mi_id gamma, float eps, mi_id *sum, mi_id *norm) {
  MI_ENTER(ctx);
  if (!sum || !norm) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, A, a);
  MI_BUF(ctx, B, b);
  if (A->rows != B->rows || A->cols != B->cols)
    return fail(ctx, MI_E_ARG, "add_rms_norm: a is [%lld, %lld], b [%lld, %lld]", (long long)A->rows,
                (long long)A->cols, (long long)B->rows, (long long)B->cols);
  Owned s_id{ctx};
  int s = mi_eltwise(ctx, MI_K_ADD, 0.0f, 0.0f, a, b, 0, MI_F32, &s_id.id);
  if (s) return s;
  mi_id n;
  s = mi_rms_norm(ctx, s_id.id, gamma, eps, MI_F32, &n);
  if (s) return s;
  *norm = n;
  *sum = s_id.release();
  return MI_OK;
}

extern "C" int mi_matmul_pairs(mi_ctx *ctx, mi_id a, mi_id b, int64_t items, const int64_t *a_at,
                               const int *a_transposed, const int64_t *b_at, const int *b_transposed, int64_t m,
                               int64_t k, int64_t n, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out || !a_at || !b_at || !a_transposed || !b_transposed) return fail(ctx, MI_E_ARG, "null argument");
  MI_BUF(ctx, A, a);
  MI_BUF(ctx, B, b);
  if (items < 1 || m < 1 || k < 1 || n < 1)
    return fail(ctx, MI_E_ARG, "matmul_pairs: %lld items of [%lld, %lld] x [%lld, %lld]", (long long)items,
                (long long)m, (long long)k, (long long)k, (long long)n);
  if (out_elem != MI_F32 && out_elem != MI_BF16) return fail(ctx, MI_E_ARG, "matmul_pairs: result kind");
  // Each block inside its buffer ([r, c] its top-left element).
  for (int64_t i = 0; i < items; ++i) {
    const int64_t ar = a_transposed[i] ? k : m, ac = a_transposed[i] ? m : k;
    const int64_t br = b_transposed[i] ? n : k, bc = b_transposed[i] ? k : n;
    if (a_at[2 * i] < 0 || a_at[2 * i + 1] < 0 || a_at[2 * i] + ar > A->rows || a_at[2 * i + 1] + ac > A->cols)
      return fail(ctx, MI_E_ARG, "matmul_pairs: item %lld's A block [%lld, %lld] at (%lld, %lld) leaves [%lld, %lld]",
                  (long long)i, (long long)ar, (long long)ac, (long long)a_at[2 * i], (long long)a_at[2 * i + 1],
                  (long long)A->rows, (long long)A->cols);
    if (b_at[2 * i] < 0 || b_at[2 * i + 1] < 0 || b_at[2 * i] + br > B->rows || b_at[2 * i + 1] + bc > B->cols)
      return fail(ctx, MI_E_ARG, "matmul_pairs: item %lld's B block [%lld, %lld] at (%lld, %lld) leaves [%lld, %lld]",
                  (long long)i, (long long)br, (long long)bc, (long long)b_at[2 * i], (long long)b_at[2 * i + 1],
                  (long long)B->rows, (long long)B->cols);
  }
  Owned o{ctx};
  int s = mi_empty(ctx, items * m, n, out_elem, &o.id);
  if (s) return s;
  // Runs of items whose blocks step by a constant offset, with one
  // orientation each, are one strided launch; anything else a launch an item.
  auto off = [](const Buffer *t, const int64_t *at, int64_t i) { return at[2 * i] * t->cols + at[2 * i + 1]; };
  int64_t i = 0;
  while (i < items) {
    int64_t j = i + 1;
    int64_t sa = 0, sb = 0;
    if (j < items && a_transposed[j] == a_transposed[i] && b_transposed[j] == b_transposed[i]) {
      sa = off(A, a_at, j) - off(A, a_at, i);
      sb = off(B, b_at, j) - off(B, b_at, i);
      while (sa >= 0 && sb >= 0 && j < items && a_transposed[j] == a_transposed[i] && b_transposed[j] == b_transposed[i] &&
             off(A, a_at, j) - off(A, a_at, j - 1) == sa && off(B, b_at, j) - off(B, b_at, j - 1) == sb &&
             j - i < 65535)
        ++j;
    }
    if (j == i + 1) sa = sb = 0;  // a run of one
    const int64_t at_a[3] = {off(A, a_at, i), 0, sa}, at_b[3] = {off(B, b_at, i), 0, sb};
    const int64_t at_o[3] = {i * m * n, 0, m * n};
    s = mi_matmul_items(ctx, a, a_transposed[i], at_a, b, b_transposed[i], at_b, 1, j - i, m, k, n, o.id, at_o);
    if (s) return s;
    i = j;
  }
  *out = o.release();
  return MI_OK;
}
