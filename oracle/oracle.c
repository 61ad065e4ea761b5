/*
 * oracle.c -- CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library, and only as the checker (or
 * the timed CPU baseline).  The product (libmiburn.so) never links or calls
 * it.
 *
 * What it restates.  The reference's CPU oracle is burn-flex 0.21.0, a
 * crates.io dependency that is not vendored under /root/reference and cannot
 * be built here (no Rust toolchain, no network).  Its published semantics, as
 * the reference's own code states and calls them, are restated below, each
 * function citing the reference file:line it follows:
 *  - element-wise meanings: crates/tt-kernels/src/kind.rs:11-27,
 *    crates/tt-kernels/src/sfpu/ops.rs:24-250 and the host model
 *    `reference_op`/`mover` (sfpu/ops.rs:3768-3930);
 *  - scalars converted once to f32 (crates/burn-tt/src/ops.rs:2793-2795);
 *  - reductions and mean = sum / n (ops.rs:3246-3500; sfpu/reduce.rs:1-38);
 *  - softmax / log_softmax (ops.rs:5133-5166), attention's clamps
 *    (ops.rs:4572-4590);
 *  - gather / select / scatter-add, argmax (ops.rs:1001-1240, 2389-2490;
 *    ops/index.rs:27-30; crates/tt-models/src/generate.rs:176-183);
 *  - RMSNorm (crates/burn-tt/src/ops/norm.rs:1-5, ops.rs:2686-2693);
 *  - block floating point storage: the performance contract's BFP8 weights
 *    (crates/tt-models/src/quant.rs:185-235 bfp_round_trip, crates/tt-isa/
 *    src/tile.rs:619-650 the unpacker's decode).
 * Where Flex's exact bits depend on its libm and its summation order, this
 * oracle computes the better answer instead: transcendental functions in
 * double precision rounded once to f32, and every sum or dot product
 * accumulated in double and rounded once.  The tests bound the device's
 * distance from it by the tolerances the north star states (rel 1e-5 for F32
 * element-wise ops and reductions, 2e-2 for BF16 products) -- the same bound
 * Flex's own f32 arithmetic meets against it.  Indexing, gather and argmax are
 * order-free and compared bit for bit.
 *
 * Element kinds and op ids are the C ABI's (include/miburn.h).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#include "../include/miburn.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------ BF16 casts */
/* crates/tt-kernels/README.md:38-42 and Engine::cast_float (server.rs:128):
 * narrowing rounds to nearest, ties to even; a NaN stays a NaN. */
uint16_t or_bf16_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_f32_from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void or_cast_to_bf16(const float *x, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_from_f32(x[i]);
}
void or_cast_from_bf16(const uint16_t *x, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_f32_from_bf16(x[i]);
}

/* -------------------------------------------------------------- products */
/* C = op(A) . op(B) (Engine::matmul_dram, server.rs:178; ops.rs:2833):
 * A is [m, k] (or [k, m] when ta), B is [k, n] (or [n, k] when tb); each
 * output a double-precision dot product rounded once.  `threads` > 1 splits
 * rows of C (OpenMP). */
void or_matmul(const float *A, int ta, const float *B, int tb, float *C, int64_t m, int64_t n, int64_t k,
               int threads) {
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
  {
    double *acc = (double *)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t i = 0; i < m; ++i) {
      for (int64_t j = 0; j < n; ++j) acc[j] = 0.0;
      for (int64_t p = 0; p < k; ++p) {
        const double a = ta ? A[p * m + i] : A[i * k + p];
        if (tb) {
          for (int64_t j = 0; j < n; ++j) acc[j] += a * (double)B[j * k + p];
        } else {
          const float *brow = B + p * n;
          for (int64_t j = 0; j < n; ++j) acc[j] += a * (double)brow[j];
        }
      }
      for (int64_t j = 0; j < n; ++j) C[i * n + j] = (float)acc[j];
    }
    free(acc);
  }
}

/* The same product in f32 arithmetic, k ascending: the order-sensitive
 * product a plain f32 CPU backend computes; used only as the timed CPU
 * baseline.  Each output element is one F32 sum over k in ascending order
 * (a multiply, then an add: no FMA contraction), so the blocking below never
 * changes a bit: C is computed in 4-row x 32-column tiles held in vector
 * registers across the whole k loop (16 8-lane accumulators), threads taking
 * column strips so each strip of B stays in their cache while the rows of A
 * stream past.  Compiled for AVX-512, AVX2 and baseline x86-64, the widest
 * the host supports picked at load time. */
typedef float or_v8 __attribute__((vector_size(32), aligned(4)));

__attribute__((target_clones("avx512f", "avx2", "default")))
static void f32acc_tile(const float *A, const float *Bs, float *C, int64_t i0, int64_t j0, int64_t n, int64_t k) {
  const or_v8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  or_v8 c00 = z, c01 = z, c02 = z, c03 = z, c10 = z, c11 = z, c12 = z, c13 = z;
  or_v8 c20 = z, c21 = z, c22 = z, c23 = z, c30 = z, c31 = z, c32 = z, c33 = z;
  const float *a0 = A + i0 * k, *a1 = a0 + k, *a2 = a1 + k, *a3 = a2 + k;
  for (int64_t p = 0; p < k; ++p) {
    const or_v8 *bp = (const or_v8 *)(Bs + p * 32);
    const or_v8 b0 = bp[0], b1 = bp[1], b2 = bp[2], b3 = bp[3];
    or_v8 av;
#define OR_ROW(ar, x0, x1, x2, x3)                                         \
    av = (or_v8){ar[p], ar[p], ar[p], ar[p], ar[p], ar[p], ar[p], ar[p]}; \
    x0 = x0 + av * b0; x1 = x1 + av * b1; x2 = x2 + av * b2; x3 = x3 + av * b3;
    OR_ROW(a0, c00, c01, c02, c03)
    OR_ROW(a1, c10, c11, c12, c13)
    OR_ROW(a2, c20, c21, c22, c23)
    OR_ROW(a3, c30, c31, c32, c33)
#undef OR_ROW
  }
  or_v8 *c0 = (or_v8 *)(C + i0 * n + j0), *c1 = (or_v8 *)((float *)c0 + n), *c2 = (or_v8 *)((float *)c1 + n),
        *c3 = (or_v8 *)((float *)c2 + n);
  c0[0] = c00; c0[1] = c01; c0[2] = c02; c0[3] = c03;
  c1[0] = c10; c1[1] = c11; c1[2] = c12; c1[3] = c13;
  c2[0] = c20; c2[1] = c21; c2[2] = c22; c2[3] = c23;
  c3[0] = c30; c3[1] = c31; c3[2] = c32; c3[3] = c33;
}

void or_matmul_f32acc(const float *A, const float *B, float *C, int64_t m, int64_t n, int64_t k, int threads) {
  const int64_t mt = m / 4 * 4, nt = n / 32 * 32;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
  {
    /* Each thread packs its 32-column strip of B contiguously ([k, 32]):
     * read in place the strip's rows lie n floats apart, a stride that
     * lands them in the same few cache sets. */
    float *Bs = (float *)malloc((size_t)(k > 0 ? k : 1) * 32 * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int64_t j0 = 0; j0 < nt; j0 += 32) {
      for (int64_t p = 0; p < k; ++p) memcpy(Bs + p * 32, B + p * n + j0, 32 * sizeof(float));
      for (int64_t i0 = 0; i0 < mt; i0 += 4) f32acc_tile(A, Bs, C, i0, j0, n, k);
    }
    free(Bs);
  }
  /* The edges (rows past the last 4-row tile, columns past the last
   * 32-column strip): the same sums, one element at a time. */
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
  for (int64_t i = 0; i < m; ++i) {
    const int64_t j_lo = i < mt ? nt : 0;
    for (int64_t j = j_lo; j < n; ++j) {
      float acc = 0.0f;
      for (int64_t p = 0; p < k; ++p) acc += A[i * k + p] * B[p * n + j];
      C[i * n + j] = acc;
    }
  }
}

/* ------------------------------------------------------------ element-wise */
static float sigmoid2(float x) {
  /* Flex's two branches (crates/burn-tt/src/ops.rs:5287-5291). */
  double d = x;
  if (x >= 0.0f) return (float)(1.0 / (1.0 + exp(-d)));
  double e = exp(d);
  return (float)(e / (1.0 + e));
}

static float opf(uint32_t k, float a, float b, float c, float s1, float s2) {
  const double ad = a;
  switch (k) {
    case MI_K_ADD: case MI_K_ADD_ROW: return a + b;
    case MI_K_SUB: return a - b;
    case MI_K_MUL: return a * b;
    case MI_K_MUL_SCALAR: return a * s1;
    case MI_K_ADD_SCALAR: return a + s1;
    /* kind.rs:19-22 and the mover model (sfpu/ops.rs:3893-3906): a positive
     * `a` passes, everything else (zeros, negatives, NaN) gives +0. */
    case MI_K_RELU: return a > 0.0f ? a : 0.0f;
    case MI_K_RELU_BACKWARD: return a > 0.0f ? b : 0.0f;
    case MI_K_RECIP: return 1.0f / a;
    case MI_K_DIV: return a / b;
    case MI_K_DIV_SCALAR: return a / s1;
    case MI_K_EXP: return (float)exp(ad);
    case MI_K_LOG: return (float)log(ad);
    case MI_K_BOOL_NOT: return a == 0.0f ? 1.0f : 0.0f;
    case MI_K_BOOL_AND: return (a != 0.0f && b != 0.0f) ? 1.0f : 0.0f;
    case MI_K_BOOL_OR: return (a != 0.0f || b != 0.0f) ? 1.0f : 0.0f;
    case MI_K_BOOL_XOR: return ((a != 0.0f) != (b != 0.0f)) ? 1.0f : 0.0f;
    case MI_K_NEG: return -a;
    case MI_K_ABS: return fabsf(a);
    case MI_K_SIGN: return isnan(a) ? a : (a > 0.0f ? 1.0f : (a < 0.0f ? -1.0f : 0.0f));
    case MI_K_CLAMP: return isnan(a) ? a : (a < s1 ? s1 : (a > s2 ? s2 : a));
    /* sfpu/ops.rs:54-58: Flex's clamp_min is f32::max -- a NaN side gives
     * the other, equal values give the scalar. */
    case MI_K_CLAMP_MIN: return isnan(s1) ? a : (a > s1 ? a : s1);
    case MI_K_CLAMP_MAX: return isnan(s1) ? a : (a < s1 ? a : s1);
    case MI_K_LEAKY_RELU: return a >= 0.0f ? a : s1 * a;
    case MI_K_HARD_SIGMOID: {
      volatile float p = s1 * a;
      float t = p + s2;
      return isnan(t) ? t : (t < 0.0f ? 0.0f : (t > 1.0f ? 1.0f : t));
    }
    case MI_K_EQ: return a == b; case MI_K_NE: return a != b;
    case MI_K_GT: return a > b; case MI_K_GE: return a >= b;
    case MI_K_LT: return a < b; case MI_K_LE: return a <= b;
    case MI_K_EQ_S: return a == s1; case MI_K_NE_S: return a != s1;
    case MI_K_GT_S: return a > s1; case MI_K_GE_S: return a >= s1;
    case MI_K_LT_S: return a < s1; case MI_K_LE_S: return a <= s1;
    case MI_K_IS_NAN: return isnan(a) ? 1.0f : 0.0f;
    case MI_K_IS_INF: return isinf(a) ? 1.0f : 0.0f;
    case MI_K_MASK_FILL: return b != 0.0f ? s1 : a;
    case MI_K_MASK_WHERE: return b != 0.0f ? c : a;
    case MI_K_FILL: return s1;
    case MI_K_SQRT: return sqrtf(a);
    case MI_K_RSQRT: return (float)(1.0 / sqrt(ad));
    case MI_K_LOG1P: return (float)log1p(ad);
    case MI_K_POW: return (float)pow(ad, (double)b);
    case MI_K_POW_S: return (float)pow(ad, (double)s1);
    case MI_K_I32_TO_F32: case MI_K_BOOL_TO_F32: return a;
    case MI_K_EXPM1: return (float)expm1(ad);
    case MI_K_SIGMOID: return sigmoid2(a);
    /* sfpu/ops.rs:115-117: g * s * (1 - s), `a` the output s, `b` g. */
    case MI_K_SIGMOID_BACKWARD: return (b * a) * (1.0f - a);
    case MI_K_TANH: return (float)tanh(ad);
    case MI_K_ERF: return (float)erf(ad);
    /* sfpu/ops.rs:135-137: 0.5 a (1 + erf(a / sqrt 2)), as 0.5 a erfc(-a / sqrt 2)
     * -- the same value without the cancellation of 1 + erf below a = -5
     * (the reference's own device program takes the erfc form there,
     * gelu_program, sfpu/ops.rs:2113-2150). */
    case MI_K_GELU: return (float)(0.5 * ad * erfc(-ad * 0.70710678118654752440));
    /* sfpu/ops.rs:128-131: g (Phi(a) + a phi(a)). */
    case MI_K_GELU_BACKWARD: {
      double cdf = 0.5 * (1.0 + erf(ad * 0.70710678118654752440));
      double pdf = 0.39894228040143267794 * exp(-0.5 * ad * ad);
      return (float)((double)b * (cdf + ad * pdf));
    }
    case MI_K_SIN: return (float)sin(ad);
    case MI_K_COS: return (float)cos(ad);
    /* sfpu/ops.rs:235-262: the fused kinds are their compositions. */
    case MI_K_ADD_RELU: { float t = a + b; return t > 0.0f ? t : 0.0f; }
    case MI_K_SILU: return a * sigmoid2(a);
    case MI_K_SILU_MUL: return (a * sigmoid2(a)) * b;
    case MI_K_SUB_EXP: return (float)exp((double)(a - b));
    case MI_K_MUL_ADD: { volatile float p = a * b; return c + p; }
    case MI_K_SCALE_MASK_FILL: return b != 0.0f ? s2 : a * s1;
    case MI_K_RSQRT_ABS_ADD: { float t = fabsf(a) + s1; return (float)(1.0 / sqrt((double)t)); }
    default: return NAN;
  }
}

/* Operand of an element-wise op: `rows` and `cols` each the output's or 1
 * (a broadcast), crates/burn-tt/src/ops.rs:1701-1721, 1830-1872. */
static float at(const float *x, int64_t xr, int64_t xc, int64_t i, int64_t j) {
  return x[(xr == 1 ? 0 : i) * xc + (xc == 1 ? 0 : j)];
}

/* out[R, C] = op(a, b, c); absent operands are NULL.  Bool and I32 operands
 * are passed as floats (0/1, or the integer's value). */
void or_eltwise(uint32_t kind, float s1, float s2, const float *a, int64_t ar, int64_t ac, const float *b,
                int64_t br, int64_t bc, const float *c, int64_t cr, int64_t cc, float *out, int64_t R,
                int64_t C) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (R * C > (1 << 20))
#endif
  for (int64_t i = 0; i < R; ++i)
    for (int64_t j = 0; j < C; ++j) {
      float x = at(a, ar, ac, i, j);
      float y = b ? at(b, br, bc, i, j) : 0.0f;
      float z = c ? at(c, cr, cc, i, j) : 0.0f;
      out[i * C + j] = opf(kind, x, y, z, s1, s2);
    }
}

/* -------------------------------------------------------------- reductions */
static float max_nan(float a, float b) {
  if (isnan(a)) return a;
  if (isnan(b)) return b;
  return b > a ? b : a;
}
static float min_nan(float a, float b) {
  if (isnan(a)) return a;
  if (isnan(b)) return b;
  return b < a ? b : a;
}

/* Engine::reduce (server.rs:404): axis MI_AXIS_ROWS -> [1, C], MI_AXIS_COLS
 * -> [R, 1]; sums in double; a maximum's NaN propagates (sfpu/reduce.rs:
 * 24-28); mean = sum / n (ops.rs:3456-3469). */
void or_reduce(const float *x, int64_t R, int64_t C, int op, int axis, float *out) {
  const int64_t outer = axis == MI_AXIS_COLS ? R : C, inner = axis == MI_AXIS_COLS ? C : R;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (R * C > (1 << 20))
#endif
  for (int64_t o = 0; o < outer; ++o) {
    double s = 0.0;
    float m = op == MI_R_MAX ? -INFINITY : INFINITY;
    for (int64_t t = 0; t < inner; ++t) {
      float v = axis == MI_AXIS_COLS ? x[o * C + t] : x[t * C + o];
      s += v;
      m = op == MI_R_MAX ? max_nan(m, v) : min_nan(m, v);
    }
    float r;
    if (op == MI_R_SUM) r = (float)s;
    else if (op == MI_R_MEAN) r = (float)s / (float)inner;
    else r = m;
    out[o] = r;
  }
}

/* float_sum / float_mean over everything (ops.rs:3246-3400). */
float or_reduce_all(const float *x, int64_t n, int op) {
  double s = 0.0;
  float m = op == MI_R_MAX ? -INFINITY : INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    s += x[i];
    m = op == MI_R_MAX ? max_nan(m, x[i]) : min_nan(m, x[i]);
  }
  if (op == MI_R_SUM) return (float)s;
  if (op == MI_R_MEAN) return (float)s / (float)n;
  return m;
}

/* ----------------------------------------------------------------- softmax */
/* softmax / log_softmax over each row (ops.rs:5133-5166): e = exp(x - max),
 * e / sum(e), or (x - max) - ln(sum).  With a mask (row r reads mask row
 * r % mrows; nonzero = masked to -inf) the max is clamped at -FLT_MAX and
 * the sum at FLT_MIN (ops.rs:4572-4590).  `scale` multiplies x first. */
void or_softmax_rows(const float *x, int64_t R, int64_t C, const uint32_t *mask, int64_t mrows, float scale,
                     int log_mode, float *out) {
  float *v = (float *)malloc((size_t)(C > 0 ? C : 1) * sizeof(float));
  for (int64_t i = 0; i < R; ++i) {
    const uint32_t *mr = mask ? mask + (i % mrows) * C : NULL;
    float m = -INFINITY;
    for (int64_t j = 0; j < C; ++j) {
      float a = x[i * C + j];
      if (scale != 1.0f) a = a * scale;
      if (mr && mr[j]) a = -INFINITY;
      v[j] = a;
      m = max_nan(m, a);
    }
    if (mr && !(m > -FLT_MAX) && !isnan(m)) m = -FLT_MAX;
    double s = 0.0;
    for (int64_t j = 0; j < C; ++j) s += exp((double)(v[j] - m));
    float sf = (float)s;
    if (mr && !(sf > FLT_MIN) && !isnan(sf)) sf = FLT_MIN;
    /* log_softmax's ln(sum) is an F32 tensor, subtracted in F32. */
    const float ls = (float)log((double)sf);
    for (int64_t j = 0; j < C; ++j) {
      float sh = v[j] - m;
      out[i * C + j] = log_mode ? sh - ls : (float)(exp((double)sh) / (double)sf);
    }
  }
  free(v);
}

/* ------------------------------------------------------------------- norms */
/* RMSNorm, x / sqrt(mean(x x) + eps) * gamma (ops/norm.rs:1-5; llama.rs:69). */
void or_rms_norm(const float *x, int64_t R, int64_t C, const float *gamma, float eps, float *out) {
  for (int64_t i = 0; i < R; ++i) {
    double ss = 0.0;
    for (int64_t j = 0; j < C; ++j) ss += (double)x[i * C + j] * x[i * C + j];
    double rms = sqrt(ss / (double)C + (double)eps);
    for (int64_t j = 0; j < C; ++j) {
      double y = (double)x[i * C + j] / rms;
      if (gamma) y *= gamma[j];
      out[i * C + j] = (float)y;
    }
  }
}

/* Burn's LayerNorm: (x - mean) / sqrt(var + eps) * gamma + beta, biased
 * variance (crates/tt-mnist/src/transformer.rs:36-60 builds it). */
void or_layer_norm(const float *x, int64_t R, int64_t C, const float *gamma, const float *beta, float eps,
                   float *out) {
  for (int64_t i = 0; i < R; ++i) {
    double s = 0.0;
    for (int64_t j = 0; j < C; ++j) s += x[i * C + j];
    double mean = s / (double)C, q = 0.0;
    for (int64_t j = 0; j < C; ++j) {
      double d = x[i * C + j] - mean;
      q += d * d;
    }
    double den = sqrt(q / (double)C + (double)eps);
    for (int64_t j = 0; j < C; ++j) {
      double y = (x[i * C + j] - mean) / den;
      if (gamma) y *= gamma[j];
      if (beta) y += beta[j];
      out[i * C + j] = (float)y;
    }
  }
}

/* LayerNorm's gradient (the chain rule through or_layer_norm's formula;
 * Burn's autodiff reaches it through the forward's primitive ops,
 * burn-nn LayerNorm): xh = (x - mean) / den, g = dy * gamma,
 * dx = (g - mean(g) - xh * mean(g * xh)) / den (+ dres), dgamma = sum_rows(dy
 * xh), dbeta = sum_rows(dy).  double throughout, rounded once. */
void or_layer_norm_backward(const float *x, int64_t R, int64_t C, const float *gamma, const float *dy,
                            const float *dres, float eps, float *dx, float *dgamma, float *dbeta) {
  double *xh = (double *)malloc((size_t)(C > 0 ? C : 1) * sizeof(double));
  double *ag = (double *)calloc((size_t)(C > 0 ? C : 1), sizeof(double));
  double *ab = (double *)calloc((size_t)(C > 0 ? C : 1), sizeof(double));
  for (int64_t i = 0; i < R; ++i) {
    const float *xr = x + i * C, *dr = dy + i * C;
    double s = 0.0;
    for (int64_t j = 0; j < C; ++j) s += xr[j];
    const double mean = s / (double)C;
    double q = 0.0;
    for (int64_t j = 0; j < C; ++j) q += (xr[j] - mean) * (xr[j] - mean);
    const double den = sqrt(q / (double)C + (double)eps);
    double sg = 0.0, sgx = 0.0;
    for (int64_t j = 0; j < C; ++j) {
      xh[j] = (xr[j] - mean) / den;
      const double g = (double)dr[j] * (gamma ? gamma[j] : 1.0);
      sg += g;
      sgx += g * xh[j];
      ag[j] += (double)dr[j] * xh[j];
      ab[j] += dr[j];
    }
    for (int64_t j = 0; j < C; ++j) {
      const double g = (double)dr[j] * (gamma ? gamma[j] : 1.0);
      double o = (g - sg / (double)C - xh[j] * sgx / (double)C) / den;
      if (dres) o += dres[i * C + j];
      dx[i * C + j] = (float)o;
    }
  }
  for (int64_t j = 0; j < C; ++j) {
    dgamma[j] = (float)ag[j];
    dbeta[j] = (float)ab[j];
  }
  free(xh);
  free(ag);
  free(ab);
}

/* Softmax's gradient through p = softmax(scale x): ds = scale p (dp -
 * sum_row(p dp)), double, rounded once. */
void or_softmax_backward(const float *p, const float *dp, int64_t R, int64_t C, float scale, float *ds) {
  for (int64_t i = 0; i < R; ++i) {
    double s = 0.0;
    for (int64_t j = 0; j < C; ++j) s += (double)p[i * C + j] * dp[i * C + j];
    for (int64_t j = 0; j < C; ++j)
      ds[i * C + j] = (float)((double)scale * p[i * C + j] * ((double)dp[i * C + j] - s));
  }
}

/* ---------------------------------------------------------------- indexing */
/* argmax over each row: the first maximum, NaN above every number
 * (generate.rs:176-183; ops.rs:2389-2440). */
void or_argmax_rows(const float *x, int64_t R, int64_t C, int32_t *out) {
  for (int64_t i = 0; i < R; ++i) {
    int64_t best = 0;
    for (int64_t j = 1; j < C; ++j) {
      float v = x[i * C + j], b = x[i * C + best];
      if (isnan(b)) break;
      if (isnan(v) || v > b) best = j;
    }
    out[i] = (int32_t)best;
  }
}

/* Raw-bit row gather (select_rows, ops.rs:1177; embedding ops.rs:4958-4972).
 * Returns -1 (DOMAIN) on an out-of-range index, 0 otherwise. */
int or_select_rows(const uint32_t *table, int64_t V, int64_t D, const int32_t *idx, int64_t n, uint32_t *out) {
  for (int64_t i = 0; i < n; ++i) {
    if (idx[i] < 0 || idx[i] >= V) return -1;
    memcpy(out + i * D, table + (int64_t)idx[i] * D, (size_t)D * 4);
  }
  return 0;
}

/* out[r] = x[r, idx[r]] raw bits (pick_columns_native, ops.rs:1001). */
int or_pick_columns(const uint32_t *x, int64_t R, int64_t C, const int32_t *idx, uint32_t *out) {
  for (int64_t r = 0; r < R; ++r) {
    if (idx[r] < 0 || idx[r] >= C) return -1;
    out[r] = x[r * C + idx[r]];
  }
  return 0;
}

/* x with v[r] added at [r, idx[r]] (scatter_add_columns_native,
 * ops.rs:1043-1100). */
int or_scatter_add_columns(const float *x, int64_t R, int64_t C, const int32_t *idx, const float *v, float *out) {
  memcpy(out, x, (size_t)(R * C) * 4);
  for (int64_t r = 0; r < R; ++r) {
    if (idx[r] < 0 || idx[r] >= C) return -1;
    out[r * C + idx[r]] = out[r * C + idx[r]] + v[r];
  }
  return 0;
}

/* t with value row i added to row idx[i], in index order (select_add_rows,
 * server.rs:358; ops/index.rs:27-30). */
int or_select_add_rows(const float *t, int64_t V, int64_t D, const int32_t *idx, int64_t n, const float *value,
                       float *out) {
  memcpy(out, t, (size_t)(V * D) * 4);
  for (int64_t i = 0; i < n; ++i) {
    if (idx[i] < 0 || idx[i] >= V) return -1;
    for (int64_t j = 0; j < D; ++j) out[(int64_t)idx[i] * D + j] = out[(int64_t)idx[i] * D + j] + value[i * D + j];
  }
  return 0;
}

/* Strided 4-D copy (repack / copy_blocks, server.rs:269-284). */
void or_copy_strided4(const uint32_t *src, const int64_t dims[4], int64_t off, const int64_t st[4], uint32_t *out) {
  int64_t e = 0;
  for (int64_t a = 0; a < dims[0]; ++a)
    for (int64_t b = 0; b < dims[1]; ++b)
      for (int64_t c = 0; c < dims[2]; ++c)
        for (int64_t d = 0; d < dims[3]; ++d) out[e++] = src[off + a * st[0] + b * st[1] + c * st[2] + d * st[3]];
}

int or_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------- block floating point */
/* crates/tt-isa/src/tile.rs:619-636 bfp8_to_bf16: the unpacker's decode of
 * one BFP8 datum (sign bit 7, magnitude bits 6..0) under its block's shared
 * exponent byte, to a BF16 bit pattern.  The magnitude shifted left once is
 * normalised by its leading zeros, which come off the exponent byte with
 * uint8 wrap-around; a zero magnitude decodes to +0, or to 0xff80 (-inf)
 * when the sign bit is set (FloatBitPatterns.md:98, tile.rs:1158-1167). */
uint16_t or_bfp8_to_bf16(uint8_t datum, uint8_t exp) {
  const uint16_t sign = (uint16_t)(datum >> 7);
  uint8_t mag = (uint8_t)(datum << 1);
  if (mag == 0) return sign ? 0xff80u : 0u;
  int lz = 0;
  while (!(mag & 0x80u)) {
    mag = (uint8_t)(mag << 1);
    ++lz;
  }
  const uint8_t e = (uint8_t)(exp - (uint8_t)lz);
  return (uint16_t)((sign << 15) | ((uint16_t)e << 7) | (mag & 0x7eu));
}

/* crates/tt-models/src/quant.rs:185-235 bfp_round_trip: `values`, rows of
 * `cols`, held in a block floating point format of `width` datum bits (8:
 * BFP8, 4: BFP4, 2: BFP2) and read back.  Blocks of 16 consecutive columns
 * (the last of a row may be shorter) share the largest biased exponent E of
 * their values; each value truncated to BF16 is scaled by 2^-(E - 133)
 * (double precision), rounded half away from zero, clamped to 127, its low
 * 8 - width bits dropped; a zero magnitude is datum 0, else the sign joins
 * it; the datum decodes through the unpacker (BFP4 / BFP2 datums shifted to
 * the top of the byte first, tile.rs:640-650) and a decoded exponent field
 * of 0 reads as 0.0.  The reference asserts finite values; a non-finite
 * value here gives a NaN output and a return of 1 (0 otherwise).  `exps`,
 * if not null, receives each block's E ([rows, ceil(cols / 16)]). */
int or_bfp_round_trip(const float *x, int64_t rows, int64_t cols, int width, float *out, uint8_t *exps) {
  const int64_t nb = (cols + 15) / 16;
  int bad = 0;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const int64_t c0 = b * 16, c1 = c0 + 16 < cols ? c0 + 16 : cols;
      uint8_t E = 0;
      int finite = 1;
      for (int64_t c = c0; c < c1; ++c) {
        uint32_t u;
        memcpy(&u, &x[r * cols + c], 4);
        const uint8_t e = (uint8_t)(u >> 23);
        if (e > E) E = e;
        if ((u & 0x7f800000u) == 0x7f800000u) finite = 0;
      }
      if (exps) exps[r * nb + b] = E;
      const double quantum = ldexp(1.0, (int)E - 127 - 6);
      for (int64_t c = c0; c < c1; ++c) {
        float *dst = &out[r * cols + c];
        if (!finite) {
          *dst = NAN;
          bad = 1;
          continue;
        }
        uint32_t u;
        memcpy(&u, &x[r * cols + c], 4);
        const uint32_t bits = u & 0xffff0000u;
        double scaled = 0.0;
        if (bits & 0x7f800000u) {
          float t;
          memcpy(&t, &bits, 4);
          scaled = fabs((double)t) / quantum;
        }
        double rd = round(scaled); /* half away from zero, as Rust's f64::round */
        if (rd > 127.0) rd = 127.0;
        const uint8_t magnitude = (uint8_t)((uint8_t)rd >> (8 - width));
        const uint8_t datum = magnitude == 0 ? 0 : (uint8_t)(magnitude | ((bits >> 31) << (width - 1)));
        const uint16_t dec = or_bfp8_to_bf16((uint8_t)(datum << (8 - width)), E);
        if ((dec & 0x7f80u) == 0) {
          *dst = 0.0f;
        } else {
          const uint32_t v = (uint32_t)dec << 16;
          memcpy(dst, &v, 4);
        }
      }
    }
  }
  return bad;
}

/* crates/burn-tt/src/ops.rs:1102-1160 (gather_native): Burn's float_gather
 * along `dim` of a rank <= 4 row-major tensor of dims[4], raw 32-bit
 * payloads; the output has the index tensor's dims idims[4].  Returns 1 if
 * an index is out of range (its output is zero bits), 0 otherwise. */
int or_gather(const uint32_t *x, const int64_t dims[4], int dim, const int32_t *idx, const int64_t idims[4],
              uint32_t *out) {
  int bad = 0;
  for (int64_t a = 0; a < idims[0]; ++a)
    for (int64_t b = 0; b < idims[1]; ++b)
      for (int64_t c = 0; c < idims[2]; ++c)
        for (int64_t d = 0; d < idims[3]; ++d) {
          const int64_t e = ((a * idims[1] + b) * idims[2] + c) * idims[3] + d;
          int64_t co[4] = {a, b, c, d};
          const int32_t k = idx[e];
          if (k < 0 || k >= dims[dim]) {
            out[e] = 0;
            bad = 1;
            continue;
          }
          co[dim] = k;
          out[e] = x[((co[0] * dims[1] + co[1]) * dims[2] + co[2]) * dims[3] + co[3]];
        }
  return bad;
}
