// Epilogue tails shared by the product kernels (csrc/gemm.hip, csrc/tiles.hip):
// a SwiGLU MLP's gate|up pairs and a prefill's q|k|v tail, each with the
// arithmetic of the element-wise kernels they replace, so a fused launch
// gives the bits of the product followed by that kernel.
#pragma once

#include "common.hpp"

struct mi_ctx;

namespace mi {

// Result forms of a gate|up product's silu(gate) * up.
enum { SWIGLU_PARTS = 1, SWIGLU_BF16 = 2, SWIGLU_F32 = 3 };

// silu(gate) * up as the element-wise SILU_MUL (mi_silu_mul_halves) forms it.
__device__ __forceinline__ float swiglu_value(float gate, float up) { return (gate * sigmoid2(gate)) * up; }

// A prefill's q|k|v tail (64-wide heads, the product's columns (heads + 2 kv
// heads) x 64, its rows (sequence, position)): RoPE on the q and k heads at
// position pos0 + p, q written to row (b seq + p) heads + h or, grouped,
// ((b kv + j) seq + p) G + g, k and v to cache row (b kv + j) maxc + pos0 + p
// -- mi_qkv_rope_cache's layout and arithmetic.  mode 0: none; QKV_F32 /
// QKV_BF16: the caches' element.
enum { QKV_F32 = 1, QKV_BF16 = 2 };
struct QkvTail {
  int mode = 0;
  const float *cos = nullptr, *sin = nullptr;
  float *q = nullptr;
  void *kc = nullptr, *vc = nullptr;
  int64_t seq = 1, pos0 = 0, maxc = 0;
  int heads = 0, kvh = 1, grouped = 0;
};

// RoPE of the pair (x0, x1) at columns (j, j + 32) of a 64-wide head, with
// the rotary entries c0 = cos[j], c1 = cos[j + 32], s0 = sin[j], s1 =
// sin[j + 32] of its position (sin's first half negated in the table).
__device__ __forceinline__ void rope_pair(float x0, float x1, float c0, float c1, float s0, float s1, float &y0,
                                          float &y1) {
  y0 = __fadd_rn(__fmul_rn(x0, c0), __fmul_rn(x1, s0));
  y1 = __fadd_rn(__fmul_rn(x1, c1), __fmul_rn(x0, s1));
}

// Head h's values y0, y1 at columns j, j + 32 of product row `row` --
// sequence b, position p within it -- to q or to the caches.
__device__ __forceinline__ void qkv_put(const QkvTail &t, int64_t row, int64_t b, int64_t p, int h, int j, float y0,
                                        float y1) {
  if (h < t.heads) {
    const int G = t.heads / t.kvh;
    const int kvh = h / G, gg = h - kvh * G;
    const int64_t qrow = t.grouped ? ((b * t.kvh + kvh) * t.seq + p) * G + gg : row * t.heads + h;
    t.q[qrow * 64 + j] = y0;
    t.q[qrow * 64 + j + 32] = y1;
  } else {
    const bool isk = h < t.heads + t.kvh;
    const int64_t crow = (b * t.kvh + (isk ? h - t.heads : h - t.heads - t.kvh)) * t.maxc + t.pos0 + p;
    if (t.mode == QKV_BF16) {
      uint16_t *c = static_cast<uint16_t *>(isk ? t.kc : t.vc) + crow * 64;
      c[j] = f32_to_bf16_bits(y0);
      c[j + 32] = f32_to_bf16_bits(y1);
    } else {
      float *c = static_cast<float *>(isk ? t.kc : t.vc) + crow * 64;
      c[j] = y0;
      c[j + 32] = y1;
    }
  }
}

// Products against a weight in tiles (csrc/tiles.hip): mi_linear's,
// mi_linear_swiglu's and mi_linear_qkv_rope_cache's short-row path, after
// the caller's own argument checks (bias and residual F32 [n] / [m, n]; the
// q|k|v tail's tables, caches and q buffer).  0, or a failure recorded.
int tiles_linear(mi_ctx *ctx, mi_id x, mi_id w, const float *bias, const float *resid, int out_elem, mi_id *out);
int tiles_swiglu(mi_ctx *ctx, mi_id x, mi_id w_pairs, int out_form, mi_id *out);
int tiles_qkv(mi_ctx *ctx, mi_id x, mi_id w_qkv, const QkvTail &t);

}  // namespace mi
