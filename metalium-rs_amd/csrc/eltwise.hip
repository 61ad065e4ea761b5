// Element-wise ops, casts, fills and strided copies.
//
// Reference: the SFPU element-wise family -- op ids and meanings in
// crates/tt-kernels/src/kind.rs:11-27 and crates/tt-kernels/src/sfpu/ops.rs:24-250,
// entered through Engine::eltwise_op_as (crates/burn-tt/src/server.rs:519) and
// the routing `device_op_as` (crates/burn-tt/src/ops.rs:1770) with its row,
// column and scalar broadcasts (ops.rs:1830-1872); casts Engine::cast_float
// (server.rs:128); layout copies Engine::repack / copy_blocks (server.rs:269-284).
//
// MI355X design: one grid-stride kernel per op id, HBM-bound.  The fast form
// reads F32 operands as float4 (16-byte lanes, fully coalesced: a wavefront
// moves 1 KiB per access), with each operand full, a broadcast row, a
// broadcast column or a single value; anything else (BF16/Bool/I32 inputs,
// ragged widths) takes the scalar form with per-operand strides.  Each op is
// computed in F32 with IEEE round-to-nearest arithmetic and the HIP device
// library's expf/logf/erff/tanhf.
#include "common.hpp"

namespace mi {

// Operand addressing: element (i, j) of the output reads p[i * rs + j * cs].
struct Opnd {
  const void *p;
  int64_t rs, cs;
  int elem;
  int mode;  // fast form: 0 full, 1 row broadcast, 2 column broadcast, 3 value
};

__device__ __forceinline__ float load_elem(const Opnd &o, int64_t idx) {
  switch (o.elem) {
    case MI_F32: return static_cast<const float *>(o.p)[idx];
    case MI_BF16: return bf16_bits_to_f32(static_cast<const uint16_t *>(o.p)[idx]);
    case MI_I32: return static_cast<float>(static_cast<const int32_t *>(o.p)[idx]);
    default: return static_cast<float>(static_cast<const uint32_t *>(o.p)[idx]);  // Bool 0/1
  }
}

__device__ __forceinline__ float clamp_min_flex(float a, float s) {
  if (isnan(s)) return a;
  return a > s ? a : s;  // a NaN `a` gives the scalar, equal values the scalar
}
__device__ __forceinline__ float clamp_max_flex(float a, float s) {
  if (isnan(s)) return a;
  return a < s ? a : s;
}

// The op for id K on one element; `a`, `b`, `c` the operands (0 if absent).
template <uint32_t K>
__device__ __forceinline__ float op(float a, float b, float c, float s1, float s2) {
  constexpr float kInvSqrt2 = 0.70710678118654752440f;
  constexpr float kInvSqrt2Pi = 0.39894228040143267794f;
  if constexpr (K == MI_K_ADD || K == MI_K_ADD_ROW) return a + b;
  else if constexpr (K == MI_K_SUB) return a - b;
  else if constexpr (K == MI_K_MUL) return a * b;
  else if constexpr (K == MI_K_MUL_SCALAR) return a * s1;
  else if constexpr (K == MI_K_ADD_SCALAR) return a + s1;
  else if constexpr (K == MI_K_RELU) return a > 0.0f ? a : 0.0f;
  else if constexpr (K == MI_K_RELU_BACKWARD) return a > 0.0f ? b : 0.0f;
  else if constexpr (K == MI_K_RECIP) return 1.0f / a;
  else if constexpr (K == MI_K_DIV) return a / b;
  else if constexpr (K == MI_K_DIV_SCALAR) return a / s1;
  else if constexpr (K == MI_K_EXP) return expf(a);
  else if constexpr (K == MI_K_LOG) return logf(a);
  else if constexpr (K == MI_K_BOOL_NOT) return a == 0.0f ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_BOOL_AND) return (a != 0.0f && b != 0.0f) ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_BOOL_OR) return (a != 0.0f || b != 0.0f) ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_BOOL_XOR) return ((a != 0.0f) != (b != 0.0f)) ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_NEG) return __uint_as_float(__float_as_uint(a) ^ 0x80000000u);
  else if constexpr (K == MI_K_ABS) return __uint_as_float(__float_as_uint(a) & 0x7fffffffu);
  else if constexpr (K == MI_K_SIGN) return isnan(a) ? a : (a > 0.0f ? 1.0f : (a < 0.0f ? -1.0f : 0.0f));
  else if constexpr (K == MI_K_CLAMP) return isnan(a) ? a : (a < s1 ? s1 : (a > s2 ? s2 : a));
  else if constexpr (K == MI_K_CLAMP_MIN) return clamp_min_flex(a, s1);
  else if constexpr (K == MI_K_CLAMP_MAX) return clamp_max_flex(a, s1);
  else if constexpr (K == MI_K_LEAKY_RELU) return a >= 0.0f ? a : s1 * a;
  else if constexpr (K == MI_K_HARD_SIGMOID) {
    float t = __fadd_rn(__fmul_rn(s1, a), s2);
    return isnan(t) ? t : (t < 0.0f ? 0.0f : (t > 1.0f ? 1.0f : t));
  }
  else if constexpr (K == MI_K_EQ) return a == b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_NE) return a != b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_GT) return a > b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_GE) return a >= b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_LT) return a < b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_LE) return a <= b ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_EQ_S) return a == s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_NE_S) return a != s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_GT_S) return a > s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_GE_S) return a >= s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_LT_S) return a < s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_LE_S) return a <= s1 ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_IS_NAN) return isnan(a) ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_IS_INF) return isinf(a) ? 1.0f : 0.0f;
  else if constexpr (K == MI_K_MASK_FILL) return b != 0.0f ? s1 : a;
  else if constexpr (K == MI_K_MASK_WHERE) return b != 0.0f ? c : a;
  else if constexpr (K == MI_K_FILL) return s1;
  // Correctly rounded: the F64 root of an F32 rounded to F32 (double rounding
  // is innocuous for sqrt when 53 >= 2 * 24 + 2, Figueroa 1995).
  else if constexpr (K == MI_K_SQRT) return static_cast<float>(__dsqrt_rn(static_cast<double>(a)));
  else if constexpr (K == MI_K_RSQRT) return __fdiv_rn(1.0f, __fsqrt_rn(a));
  else if constexpr (K == MI_K_LOG1P) return log1pf(a);
  else if constexpr (K == MI_K_POW) return powf(a, b);
  else if constexpr (K == MI_K_POW_S) return powf(a, s1);
  else if constexpr (K == MI_K_I32_TO_F32 || K == MI_K_BOOL_TO_F32) return a;
  else if constexpr (K == MI_K_EXPM1) return expm1f(a);
  else if constexpr (K == MI_K_SIGMOID) return sigmoid2(a);
  else if constexpr (K == MI_K_SIGMOID_BACKWARD) return (b * a) * (1.0f - a);
  else if constexpr (K == MI_K_TANH) return tanhf(a);
  else if constexpr (K == MI_K_ERF) return erff(a);
  else if constexpr (K == MI_K_GELU) {
    // 2 Phi(a) from erfc(|a| / sqrt 2), so the negative tail (where 1 +
    // erf(a / sqrt 2) cancels to zero in F32, a < -5.3) keeps its relative
    // accuracy: for a >= 0, 2 Phi = 2 - erfc; below, erfc itself.  erfc(z) =
    // t exp(-z^2 + P(t)), t = 1 / (1 + z/2), with the Chebyshev fit P of
    // Numerical Recipes in C, 2nd ed., sec. 6.2 (erfcc: fractional error
    // < 1.2e-7 for every z >= 0).  z^2 = a^2 / 2 carries the rounding
    // residual of a^2 into the exponent, and the exponential's argument in
    // base 2 carries its own, so the result is within 4.1e-6 relative down to
    // a = -13 (measured against float64 erfc over [-13, 0] and N(0, 1) draws).
    // Below -13 the value underflows F32's normal range: -0 (NaN for -inf,
    // as 0.5 a (1 + erf) gives); +inf stays +inf, a NaN stays a NaN.
    const float ac = fminf(fmaxf(a, -13.5f), 13.5f);
    const float z = fabsf(ac) * kInvSqrt2;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
    float p = fmaf(t, 0.17087277f, -0.82215223f);
    p = fmaf(t, p, 1.48851587f);
    p = fmaf(t, p, -1.13520398f);
    p = fmaf(t, p, 0.27886807f);
    p = fmaf(t, p, -0.18628806f);
    p = fmaf(t, p, 0.09678418f);
    p = fmaf(t, p, 0.37409196f);
    p = fmaf(t, p, 1.00002368f);
    p = fmaf(t, p, -1.26551223f);
    const float a2 = ac * ac;
    const float arg = fmaf(-0.5f, a2, fmaf(-0.5f, fmaf(ac, ac, -a2), p));  // -z^2 + P(t)
    constexpr float kLog2e = 1.4426950408889634f, kLog2eLo = 1.925963e-08f, kLn2 = 0.6931471805599453f;
    const float y = arg * kLog2e;
    const float yl = fmaf(arg, kLog2e, -y) + arg * kLog2eLo;
    const float h = __builtin_amdgcn_exp2f(y);
    const float e = t * fmaf(h * yl, kLn2, h);
    const float r = a >= 0.0f ? 2.0f - e : (a >= -13.0f ? e : 0.0f);
    return (0.5f * a) * r;
  }
  else if constexpr (K == MI_K_GELU_BACKWARD) {
    float cdf = 0.5f * (1.0f + erff(a * kInvSqrt2));
    float pdf = kInvSqrt2Pi * expf(-0.5f * a * a);
    return b * (cdf + a * pdf);
  }
  else if constexpr (K == MI_K_SIN) return sinf(a);
  else if constexpr (K == MI_K_COS) return cosf(a);
  else if constexpr (K == MI_K_ADD_RELU) { float t = a + b; return t > 0.0f ? t : 0.0f; }
  else if constexpr (K == MI_K_SILU) return a * sigmoid2(a);
  else if constexpr (K == MI_K_SILU_MUL) return (a * sigmoid2(a)) * b;
  else if constexpr (K == MI_K_SUB_EXP) return expf(a - b);
  else if constexpr (K == MI_K_MUL_ADD) return __fadd_rn(c, __fmul_rn(a, b));
  else if constexpr (K == MI_K_SCALE_MASK_FILL) return b != 0.0f ? s2 : a * s1;
  else if constexpr (K == MI_K_RSQRT_ABS_ADD) return __fdiv_rn(1.0f, __fsqrt_rn(fabsf(a) + s1));
  else return __builtin_nanf("");
}

__device__ __forceinline__ void store_elem(void *out, int out_elem, int64_t idx, float v) {
  if (out_elem == MI_F32) static_cast<float *>(out)[idx] = v;
  else if (out_elem == MI_BF16) static_cast<uint16_t *>(out)[idx] = f32_to_bf16_bits(v);
  else static_cast<uint32_t *>(out)[idx] = v != 0.0f ? 1u : 0u;  // Bool
}

// Fast form: F32 operands, the output width a multiple of 4, four lanes of
// one row per thread per step.
template <bool NT>
__device__ __forceinline__ float4 load4(const Opnd &o, int64_t flat, int64_t cols) {
  const float *p = static_cast<const float *>(o.p);
  switch (o.mode) {
    case 0: return ld4<NT>(p + flat);
    case 1: return *reinterpret_cast<const float4 *>(p + (flat % cols));
    case 2: { float v = p[flat / cols]; return make_float4(v, v, v, v); }
    default: { float v = p[0]; return make_float4(v, v, v, v); }
  }
}

// Each thread owns EW_UNROLL float4 lanes spaced a block apart, issuing all
// its loads before any arithmetic.  Two per thread, one pass over up to
// 2^24 float4 (32768 blocks): on [8192, 8192] F32 exp, GELU and SiLU move
// 0.78-0.81 of HBM peak against 0.73-0.77 with four per thread (fewer,
// longer-lived waves whose arithmetic leaves HBM idle longer) and 0.72 for
// GELU / SiLU with one.
constexpr int EW_UNROLL = 2;

template <bool NT>
__device__ __forceinline__ void store4(void *out, int out_elem, int64_t flat, float4 r) {
  if (out_elem == MI_F32) {
    st4<NT>(static_cast<float *>(out) + flat, r);
  } else if (out_elem == MI_BF16) {
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + flat) = make_uint2(bf16x2_bits(r.x, r.y), bf16x2_bits(r.z, r.w));
  } else {
    uint4 m = make_uint4(r.x != 0.f, r.y != 0.f, r.z != 0.f, r.w != 0.f);
    stu4<NT>(static_cast<uint32_t *>(out) + flat, m);
  }
}

template <uint32_t K, int NIN, bool NT>
__global__ void __launch_bounds__(256) ew_vec4(Opnd a, Opnd b, Opnd c, float s1, float s2,
                                               void *out, int out_elem, int64_t n4, int64_t cols) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * EW_UNROLL) + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (256 * EW_UNROLL);
  for (int64_t v0 = base; v0 < n4; v0 += stride) {
    float4 x[EW_UNROLL], y[EW_UNROLL], z[EW_UNROLL];
#pragma unroll
    for (int u = 0; u < EW_UNROLL; ++u) {
      const int64_t v = v0 + u * 256;
      if (v < n4) {
        x[u] = load4<NT>(a, v * 4, cols);
        if constexpr (NIN >= 2) y[u] = load4<NT>(b, v * 4, cols);
        if constexpr (NIN >= 3) z[u] = load4<NT>(c, v * 4, cols);
      }
    }
#pragma unroll
    for (int u = 0; u < EW_UNROLL; ++u) {
      const int64_t v = v0 + u * 256;
      if (v < n4) {
        float4 yy = make_float4(0.f, 0.f, 0.f, 0.f), zz = yy;
        if constexpr (NIN >= 2) yy = y[u];
        if constexpr (NIN >= 3) zz = z[u];
        float4 r;
        r.x = op<K>(x[u].x, yy.x, zz.x, s1, s2);
        r.y = op<K>(x[u].y, yy.y, zz.y, s1, s2);
        r.z = op<K>(x[u].z, yy.z, zz.z, s1, s2);
        r.w = op<K>(x[u].w, yy.w, zz.w, s1, s2);
        store4<NT>(out, out_elem, v * 4, r);
      }
    }
  }
}

template <uint32_t K, int NIN>
__global__ void __launch_bounds__(256) ew_generic(Opnd a, Opnd b, Opnd c, float s1, float s2,
                                                  void *out, int out_elem, int64_t n, int64_t cols) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int64_t i = e / cols, j = e - i * cols;
    float x = load_elem(a, i * a.rs + j * a.cs);
    float y = 0.f, z = 0.f;
    if constexpr (NIN >= 2) y = load_elem(b, i * b.rs + j * b.cs);
    if constexpr (NIN >= 3) z = load_elem(c, i * c.rs + j * c.cs);
    store_elem(out, out_elem, e, op<K>(x, y, z, s1, s2));
  }
}

// Operand count and output class of each op id; 0 operands = unknown id.
struct KindInfo { int nin; bool bool_out; bool bool_in; };

static KindInfo kind_info(uint32_t k) {
  switch (k) {
    case MI_K_ADD: case MI_K_SUB: case MI_K_MUL: case MI_K_ADD_ROW: case MI_K_RELU_BACKWARD:
    case MI_K_DIV: case MI_K_POW: case MI_K_SIGMOID_BACKWARD: case MI_K_GELU_BACKWARD:
    case MI_K_ADD_RELU: case MI_K_SILU_MUL: case MI_K_SUB_EXP:
      return {2, false, false};
    case MI_K_MASK_FILL: case MI_K_SCALE_MASK_FILL:
      return {2, false, false};
    case MI_K_MUL_ADD: case MI_K_MASK_WHERE:
      return {3, false, false};
    case MI_K_EQ: case MI_K_NE: case MI_K_GT: case MI_K_GE: case MI_K_LT: case MI_K_LE:
      return {2, true, false};
    case MI_K_BOOL_AND: case MI_K_BOOL_OR: case MI_K_BOOL_XOR:
      return {2, true, true};
    case MI_K_BOOL_NOT:
      return {1, true, true};
    case MI_K_EQ_S: case MI_K_NE_S: case MI_K_GT_S: case MI_K_GE_S: case MI_K_LT_S: case MI_K_LE_S:
    case MI_K_IS_NAN: case MI_K_IS_INF:
      return {1, true, false};
    case MI_K_MUL_SCALAR: case MI_K_ADD_SCALAR: case MI_K_RELU: case MI_K_RECIP: case MI_K_DIV_SCALAR:
    case MI_K_EXP: case MI_K_LOG: case MI_K_NEG: case MI_K_ABS: case MI_K_SIGN: case MI_K_CLAMP:
    case MI_K_CLAMP_MIN: case MI_K_CLAMP_MAX: case MI_K_LEAKY_RELU: case MI_K_HARD_SIGMOID:
    case MI_K_FILL: case MI_K_SQRT: case MI_K_RSQRT: case MI_K_LOG1P: case MI_K_POW_S:
    case MI_K_I32_TO_F32: case MI_K_BOOL_TO_F32: case MI_K_EXPM1: case MI_K_SIGMOID: case MI_K_TANH:
    case MI_K_ERF: case MI_K_GELU: case MI_K_SIN: case MI_K_COS: case MI_K_SILU: case MI_K_RSQRT_ABS_ADD:
      return {1, false, false};
    default:
      return {0, false, false};
  }
}

#define MI_KIND_LIST(X)                                                                         \
  X(MI_K_ADD) X(MI_K_SUB) X(MI_K_MUL) X(MI_K_MUL_SCALAR) X(MI_K_RELU) X(MI_K_RELU_BACKWARD)      \
  X(MI_K_ADD_ROW) X(MI_K_ADD_SCALAR) X(MI_K_RECIP) X(MI_K_DIV) X(MI_K_DIV_SCALAR) X(MI_K_EXP)   \
  X(MI_K_LOG) X(MI_K_BOOL_NOT) X(MI_K_BOOL_AND) X(MI_K_BOOL_OR) X(MI_K_BOOL_XOR) X(MI_K_NEG)    \
  X(MI_K_ABS) X(MI_K_SIGN) X(MI_K_CLAMP) X(MI_K_CLAMP_MIN) X(MI_K_CLAMP_MAX) X(MI_K_LEAKY_RELU) \
  X(MI_K_HARD_SIGMOID) X(MI_K_EQ) X(MI_K_NE) X(MI_K_GT) X(MI_K_GE) X(MI_K_LT) X(MI_K_LE)        \
  X(MI_K_EQ_S) X(MI_K_NE_S) X(MI_K_GT_S) X(MI_K_GE_S) X(MI_K_LT_S) X(MI_K_LE_S) X(MI_K_IS_NAN)  \
  X(MI_K_IS_INF) X(MI_K_MASK_FILL) X(MI_K_MASK_WHERE) X(MI_K_FILL) X(MI_K_SQRT) X(MI_K_RSQRT)   \
  X(MI_K_LOG1P) X(MI_K_POW) X(MI_K_POW_S) X(MI_K_I32_TO_F32) X(MI_K_EXPM1) X(MI_K_SIGMOID)      \
  X(MI_K_SIGMOID_BACKWARD) X(MI_K_TANH) X(MI_K_ERF) X(MI_K_GELU) X(MI_K_GELU_BACKWARD)          \
  X(MI_K_SIN) X(MI_K_COS) X(MI_K_BOOL_TO_F32) X(MI_K_ADD_RELU) X(MI_K_SILU) X(MI_K_SILU_MUL)    \
  X(MI_K_SUB_EXP) X(MI_K_MUL_ADD) X(MI_K_SCALE_MASK_FILL) X(MI_K_RSQRT_ABS_ADD)

template <uint32_t K>
static void launch_kind(bool fast, int nin, const Opnd &a, const Opnd &b, const Opnd &c, float s1,
                        float s2, void *out, int out_elem, int64_t n, int64_t cols, hipStream_t st) {
  const int threads = 256;
  if (fast) {
    const int64_t n4 = n / 4;
    unsigned g = grid_for(n4, threads * EW_UNROLL, 256 * 128);
    // Stream the accesses when the operation moves more than the last-level
    // cache holds (inputs and output counted at 4 bytes an element).
    const bool nt = n * 4 * (nin + 1) >= kStreamBytes;
    if (nt) {
      if (nin == 1) ew_vec4<K, 1, true><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
      else if (nin == 2) ew_vec4<K, 2, true><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
      else ew_vec4<K, 3, true><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
    } else {
      if (nin == 1) ew_vec4<K, 1, false><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
      else if (nin == 2) ew_vec4<K, 2, false><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
      else ew_vec4<K, 3, false><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n4, cols);
    }
  } else {
    unsigned g = grid_for(n, threads * 4, 256 * 32);
    if (nin == 1) ew_generic<K, 1><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n, cols);
    else if (nin == 2) ew_generic<K, 2><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n, cols);
    else ew_generic<K, 3><<<g, threads, 0, st>>>(a, b, c, s1, s2, out, out_elem, n, cols);
  }
}

// Describe operand `x` against output dims; false if it does not broadcast.
static bool describe(const Buffer *x, int64_t R, int64_t C, Opnd *o) {
  o->p = x->ptr;
  o->elem = x->elem;
  const bool full_r = x->rows == R, full_c = x->cols == C;
  if (!(full_r || x->rows == 1) || !(full_c || x->cols == 1)) return false;
  o->rs = (x->rows == 1 && R != 1) ? 0 : x->cols;
  o->cs = (x->cols == 1 && C != 1) ? 0 : 1;
  if (x->rows == R && x->cols == C) o->mode = 0;
  else if (x->rows == 1 && x->cols == C) o->mode = 1;
  else if (x->rows == R && x->cols == 1) o->mode = 2;
  else o->mode = 3;
  if (x->rows == 1 && x->cols == 1) o->mode = 3;
  return true;
}

}  // namespace mi

using namespace mi;

extern "C" int mi_eltwise(mi_ctx *ctx, uint32_t kind, float scalar, float scalar2, mi_id a, mi_id b,
                          mi_id c, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  KindInfo info = kind_info(kind);
  if (info.nin == 0) return fail(ctx, MI_E_UNSUPPORTED, "element-wise op id %#x is not supported", kind);
  const Buffer *ops[3] = {nullptr, nullptr, nullptr};
  mi_id ids[3] = {a, b, c};
  for (int i = 0; i < 3; ++i) {
    if (i < info.nin) {
      ops[i] = lookup(ctx, ids[i]);
      if (!ops[i]) return fail(ctx, MI_E_ID, "op %#x: operand %d: unknown buffer id %llu", kind, i, (unsigned long long)ids[i]);
    } else if (ids[i] != 0) {
      return fail(ctx, MI_E_ARG, "op %#x takes %d operand(s)", kind, info.nin);
    }
  }
  int64_t R = 1, C = 1;
  for (int i = 0; i < info.nin; ++i) {
    R = std::max(R, ops[i]->rows);
    C = std::max(C, ops[i]->cols);
    if (ops[i]->rows == 0) R = 0;
    if (ops[i]->cols == 0) C = 0;
  }
  Opnd od[3] = {};
  for (int i = 0; i < info.nin; ++i) {
    if (!describe(ops[i], R, C, &od[i]))
      return fail(ctx, MI_E_ARG, "op %#x: operand %d [%lld, %lld] does not broadcast to [%lld, %lld]", kind, i,
                  (long long)ops[i]->rows, (long long)ops[i]->cols, (long long)R, (long long)C);
  }
  // Element kinds: the mask operand of MASK_FILL/MASK_WHERE/SCALE_MASK_FILL is Bool;
  // Bool ops take Bool; everything else takes F32/BF16 (I32 for I32_TO_F32).
  for (int i = 0; i < info.nin; ++i) {
    int e = ops[i]->elem;
    bool mask_slot = (i == 1) && (kind == MI_K_MASK_FILL || kind == MI_K_MASK_WHERE || kind == MI_K_SCALE_MASK_FILL);
    bool ok;
    if (info.bool_in) ok = e == MI_BOOL;
    else if (mask_slot) ok = e == MI_BOOL;
    else if (kind == MI_K_I32_TO_F32) ok = e == MI_I32;
    else if (kind == MI_K_BOOL_TO_F32) ok = e == MI_BOOL;
    else ok = elem_float(e);
    if (!ok) return fail(ctx, MI_E_ARG, "op %#x: operand %d is %s", kind, i, elem_name(e));
  }
  int oe = info.bool_out ? MI_BOOL : out_elem;
  if (!info.bool_out && oe != MI_F32 && oe != MI_BF16)
    return fail(ctx, MI_E_ARG, "op %#x: result kind %s", kind, elem_name(oe));
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, C, oe, &id, &ob);
  if (s) return s;
  const int64_t n = R * C;
  if (n > 0) {
    bool fast = (C % 4 == 0);
    for (int i = 0; i < info.nin; ++i) {
      if (ops[i]->elem != MI_F32) fast = false;
      // A value of one element per row must be 4-aligned to be read as float4 only in mode 0/1.
    }
    switch (kind) {
#define MI_CASE(K) case K: launch_kind<K>(fast, info.nin, od[0], od[1], od[2], scalar, scalar2, ob->ptr, oe, n, C, ctx->stream); break;
      MI_KIND_LIST(MI_CASE)
#undef MI_CASE
      default: break;
    }
    s = check_launch(ctx, "eltwise");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

// ------------------------------------------------------------------ fills
namespace mi {
__global__ void fill32(uint32_t *p, int64_t n, uint32_t bits) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = bits;
}
__global__ void fill16(uint16_t *p, int64_t n, uint16_t bits) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = bits;
}

int fill_zero(Ctx *ctx, void *p, size_t bytes) {
  if (bytes == 0) return MI_OK;
  if (bytes % 4 == 0) {
    const int64_t n = static_cast<int64_t>(bytes / 4);
    fill32<<<grid_for(n, 256 * 4, 256 * 64), 256, 0, ctx->stream>>>(static_cast<uint32_t *>(p), n, 0u);
  } else {
    const int64_t n = static_cast<int64_t>(bytes / 2);
    fill16<<<grid_for(n, 256 * 4, 256 * 64), 256, 0, ctx->stream>>>(static_cast<uint16_t *>(p), n, uint16_t(0));
  }
  return check_launch(ctx, "fill");
}
}  // namespace mi

extern "C" int mi_fill(mi_ctx *ctx, int64_t rows, int64_t cols, int elem, uint32_t bits, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  if (elem == MI_BFP8) return fail(ctx, MI_E_ARG, "fill of a BFP8 buffer (mi_cast_bfp makes one)");
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, rows, cols, elem, &id, &b);
  if (s) return s;
  int64_t n = rows * cols;
  if (n > 0) {
    unsigned g = grid_for(n, 256 * 4, 256 * 32);
    if (elem == MI_BF16) fill16<<<g, 256, 0, ctx->stream>>>(static_cast<uint16_t *>(b->ptr), n, uint16_t(bits));
    else fill32<<<g, 256, 0, ctx->stream>>>(static_cast<uint32_t *>(b->ptr), n, bits);
    s = check_launch(ctx, "fill");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_empty(mi_ctx *ctx, int64_t rows, int64_t cols, int elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  if (elem == MI_BFP8) return fail(ctx, MI_E_ARG, "empty BFP8 buffer (mi_cast_bfp makes one)");
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, rows, cols, elem, &id, &b);
  if (s) return s;
  *out = id;
  return MI_OK;
}

// ------------------------------------------------------------------ casts
namespace mi {
__global__ void cast_kernel(const void *src, int se, void *dst, int de, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v;
    if (se == MI_F32) v = static_cast<const float *>(src)[i];
    else if (se == MI_BF16) v = bf16_bits_to_f32(static_cast<const uint16_t *>(src)[i]);
    else if (se == MI_I32) v = static_cast<float>(static_cast<const int32_t *>(src)[i]);
    else v = static_cast<float>(static_cast<const uint32_t *>(src)[i]);
    if (de == MI_F32) static_cast<float *>(dst)[i] = v;
    else if (de == MI_BF16) static_cast<uint16_t *>(dst)[i] = f32_to_bf16_bits(v);
    else if (de == MI_BOOL) static_cast<uint32_t *>(dst)[i] = v != 0.0f ? 1u : 0u;
    else {
      // F32 -> I32 truncates toward zero, saturating (Rust's `as i32`); a NaN gives 0.
      int32_t r;
      if (isnan(v)) r = 0;
      else if (v >= 2147483648.0f) r = 2147483647;
      else if (v < -2147483648.0f) r = -2147483647 - 1;
      else r = static_cast<int32_t>(v);
      static_cast<int32_t *>(dst)[i] = r;
    }
  }
}
// F32 rows as their BF16 parts ([rows, 2 cols]: a row's heads, then its
// remainders), four values a thread.
__global__ void parts_kernel(const float *src, int64_t rows, int64_t cols, uint16_t *dst) {
  const int64_t q = cols / 4, n = rows * q;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / q, c = (i - r * q) * 4;
    parts4_put(dst + r * 2 * cols + c, dst + r * 2 * cols + cols + c,
               *reinterpret_cast<const float4 *>(src + r * cols + c));
  }
}
}  // namespace mi

extern "C" int mi_cast(mi_ctx *ctx, mi_id a, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, src, a);
  if (out_elem == MI_BF16_PARTS) {  // an F32 buffer's parts (a product's split operand)
    if (src->elem != MI_F32 || src->tiles || src->cols % 4)
      return fail(ctx, MI_E_ARG, "cast of %s [%lld, %lld] to parts: want F32 rows of a multiple of 4",
                  elem_name(src->elem), (long long)src->rows, (long long)src->cols);
    mi_id id; Buffer *b;
    if (int s = new_buffer(ctx, src->rows, 2 * src->cols, MI_BF16, &id, &b)) return s;
    const int64_t n = src->rows * src->cols / 4;
    if (n > 0)
      parts_kernel<<<grid_for(n, 256 * 4, 256 * 32), 256, 0, ctx->stream>>>(static_cast<const float *>(src->ptr),
                                                                          src->rows, src->cols,
                                                                          static_cast<uint16_t *>(b->ptr));
    if (int s = check_launch(ctx, "cast")) {
      mi_free(ctx, id);
      return s;
    }
    *out = id;
    return MI_OK;
  }
  if (!elem_valid(out_elem)) return fail(ctx, MI_E_ARG, "cast to unknown kind %d", out_elem);
  // BFP8 storage: packed or decoded (the reference's cast_bfp).
  if (out_elem == MI_BFP8) return mi_cast_bfp(ctx, a, MI_BFP8, out);
  if (src->elem == MI_BFP8) {
    if (out_elem != MI_F32 && out_elem != MI_BF16)
      return fail(ctx, MI_E_ARG, "cast of BFP8 to %s", elem_name(out_elem));
    return bfp8_decode_to(ctx, src, out_elem, out, nullptr);
  }
  int64_t rows = src->rows, cols = src->cols;
  int se = src->elem;
  const void *sp = src->ptr;
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, rows, cols, out_elem, &id, &b);
  if (s) return s;
  int64_t n = rows * cols;
  if (n > 0) {
    if (se == out_elem) {
      (void)hipMemcpyAsync(b->ptr, sp, n * elem_size(se), hipMemcpyDeviceToDevice, ctx->stream);
    } else {
      cast_kernel<<<grid_for(n, 256 * 4, 256 * 32), 256, 0, ctx->stream>>>(sp, se, b->ptr, out_elem, n);
    }
    s = check_launch(ctx, "cast");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

// --------------------------------------------------------- strided copies
namespace mi {
template <typename T>
__global__ void copy4_kernel(const T *src, T *dst, int64_t d1, int64_t d2, int64_t d3, int64_t n, int64_t off,
                             int64_t s0, int64_t s1, int64_t s2, int64_t s3) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    int64_t i3 = e % d3, r = e / d3;
    int64_t i2 = r % d2; r /= d2;
    int64_t i1 = r % d1, i0 = r / d1;
    dst[e] = src[off + i0 * s0 + i1 * s1 + i2 * s2 + i3 * s3];
  }
}

static int copy4(Ctx *ctx, mi_id srcid, const int64_t dims[4], int64_t offset, const int64_t strides[4], mi_id *out) {
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, src, srcid);
  MI_NO_BFP8(ctx, src, "copy_strided");
  int64_t n = 1;
  for (int i = 0; i < 4; ++i) {
    if (dims[i] < 0) return fail(ctx, MI_E_ARG, "negative copy extent");
    n *= dims[i];
  }
  // Bounds of the addressed range: every element read lies in the source.
  if (n > 0) {
    int64_t lo = offset, hi = offset;
    for (int i = 0; i < 4; ++i) {
      int64_t span = (dims[i] - 1) * strides[i];
      if (span < 0) lo += span; else hi += span;
    }
    if (lo < 0 || hi >= src->numel())
      return fail(ctx, MI_E_ARG, "strided copy reads [%lld, %lld] of a %lld-element buffer", (long long)lo,
                  (long long)hi, (long long)src->numel());
  }
  const void *sp = src->ptr;
  int se = src->elem;
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, dims[0] * dims[1] * dims[2], dims[3], se, &id, &b);
  if (s) return s;
  if (n > 0) {
    unsigned g = grid_for(n, 256 * 4, 256 * 32);
    if (se == MI_BF16)
      copy4_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>(static_cast<const uint16_t *>(sp), static_cast<uint16_t *>(b->ptr),
                                                        dims[1], dims[2], dims[3], n, offset, strides[0], strides[1], strides[2], strides[3]);
    else
      copy4_kernel<uint32_t><<<g, 256, 0, ctx->stream>>>(static_cast<const uint32_t *>(sp), static_cast<uint32_t *>(b->ptr),
                                                        dims[1], dims[2], dims[3], n, offset, strides[0], strides[1], strides[2], strides[3]);
    s = check_launch(ctx, "copy_strided");
    if (s) { mi_free(static_cast<mi_ctx *>(ctx), id); return s; }
  }
  *out = id;
  return MI_OK;
}

template <typename T>
__global__ void assign_kernel(T *dst, int64_t dcols, const T *src, int64_t rows, int64_t cols, int64_t r0, int64_t c0) {
  const int64_t n = rows * cols;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    int64_t i = e / cols, j = e - i * cols;
    dst[(r0 + i) * dcols + c0 + j] = src[e];
  }
}
}  // namespace mi

extern "C" int mi_copy_strided(mi_ctx *ctx, mi_id src, int64_t rows, int64_t cols, int64_t offset, int64_t row_stride,
                               int64_t col_stride, mi_id *out) {
  MI_ENTER(ctx);
  int64_t dims[4] = {1, 1, rows, cols};
  int64_t strides[4] = {0, 0, row_stride, col_stride};
  return copy4(ctx, src, dims, offset, strides, out);
}

extern "C" int mi_copy_strided4(mi_ctx *ctx, mi_id src, const int64_t dims[4], int64_t offset, const int64_t strides[4],
                                mi_id *out) {
  MI_ENTER(ctx);
  if (!dims || !strides) return fail(ctx, MI_E_ARG, "null dims or strides");
  return copy4(ctx, src, dims, offset, strides, out);
}

extern "C" int mi_assign_block(mi_ctx *ctx, mi_id dst, mi_id src, int64_t row0, int64_t col0) {
  MI_ENTER(ctx);
  MI_BUF(ctx, d, dst);
  MI_BUF(ctx, s, src);
  MI_NO_BFP8(ctx, d, "assign_block");
  if (d->elem != s->elem) return fail(ctx, MI_E_ARG, "assign of %s into %s", elem_name(s->elem), elem_name(d->elem));
  if (row0 < 0 || col0 < 0 || row0 + s->rows > d->rows || col0 + s->cols > d->cols)
    return fail(ctx, MI_E_ARG, "block [%lld, %lld] at (%lld, %lld) outside [%lld, %lld]", (long long)s->rows,
                (long long)s->cols, (long long)row0, (long long)col0, (long long)d->rows, (long long)d->cols);
  int64_t n = s->numel();
  if (n == 0) return MI_OK;
  unsigned g = grid_for(n, 256 * 4, 256 * 32);
  if (d->elem == MI_BF16)
    assign_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>(static_cast<uint16_t *>(d->ptr), d->cols,
                                                       static_cast<const uint16_t *>(s->ptr), s->rows, s->cols, row0, col0);
  else
    assign_kernel<uint32_t><<<g, 256, 0, ctx->stream>>>(static_cast<uint32_t *>(d->ptr), d->cols,
                                                       static_cast<const uint32_t *>(s->ptr), s->rows, s->cols, row0, col0);
  return check_launch(ctx, "assign_block");
}

// ------------------------------------------------- strided copy into a buffer
namespace mi {
template <typename T>
__global__ void copy_into4_kernel(T *dst, const T *src, int64_t d1, int64_t d2, int64_t d3, int64_t n, int64_t doff,
                                  int64_t ds0, int64_t ds1, int64_t ds2, int64_t ds3, int64_t soff, int64_t ss0,
                                  int64_t ss1, int64_t ss2, int64_t ss3) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    int64_t i3 = e % d3, r = e / d3;
    int64_t i2 = r % d2; r /= d2;
    int64_t i1 = r % d1, i0 = r / d1;
    dst[doff + i0 * ds0 + i1 * ds1 + i2 * ds2 + i3 * ds3] = src[soff + i0 * ss0 + i1 * ss1 + i2 * ss2 + i3 * ss3];
  }
}

// [lo, hi] element range a 4-D strided index space addresses.
static void span4(const int64_t dims[4], int64_t off, const int64_t st[4], int64_t *lo, int64_t *hi) {
  *lo = off; *hi = off;
  for (int i = 0; i < 4; ++i) {
    const int64_t span = (dims[i] - 1) * st[i];
    if (span < 0) *lo += span; else *hi += span;
  }
}

// RoPE on rows of [rows, d] laid out (sequence, position, head): row r is at
// position pos0 + (r / heads) % seq.  out = x cos + rotate(x) sin, rotate
// swapping the two halves and `sin`'s first half stored negated, two
// roundings (crates/tt-models/src/rope.rs:6-60; ops/rope.rs:27-240).
__global__ void rope_kernel(const float *x, const float *cosp, const float *sinp, float *out, int64_t rows, int64_t d,
                            int64_t heads, int64_t seq, int64_t pos0) {
  const int64_t n = rows * d;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t half = d / 2;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int64_t r = e / d, j = e - r * d;
    const int64_t pos = pos0 + (r / heads) % seq;
    const float xv = x[e];
    const float rv = x[r * d + (j < half ? j + half : j - half)];
    const float c = __fmul_rn(xv, cosp[pos * d + j]);
    out[e] = __fadd_rn(c, __fmul_rn(rv, sinp[pos * d + j]));
  }
}

// silu(gate) * up over the two halves of a fused gate|up product's rows,
// gu [rows, 2 i] -> [rows, i], with SILU_MUL's arithmetic; four columns a
// thread when i is a multiple of 4.  TO: F32, or BF16 (the result rounded once
// as stored, for a product that reads BF16 activations); PARTS (TO = BF16):
// the F32 result's parts, row r's heads at out[2 r i ...] and its remainders
// i further.
template <bool VEC, typename TO, bool PARTS = false>
__global__ void silu_mul_halves_kernel(const float *gu, TO *out, int64_t rows, int64_t inner) {
  static_assert(!PARTS || sizeof(TO) == 2, "parts are BF16");
  const int64_t per = VEC ? inner / 4 : inner, n = rows * per;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int64_t r = e / per, c = e - r * per;
    if constexpr (VEC) {
      const float4 g = *reinterpret_cast<const float4 *>(gu + r * 2 * inner + 4 * c);
      const float4 u = *reinterpret_cast<const float4 *>(gu + r * 2 * inner + inner + 4 * c);
      float4 y;
      y.x = op<MI_K_SILU_MUL>(g.x, u.x, 0.f, 0.f, 0.f);
      y.y = op<MI_K_SILU_MUL>(g.y, u.y, 0.f, 0.f, 0.f);
      y.z = op<MI_K_SILU_MUL>(g.z, u.z, 0.f, 0.f, 0.f);
      y.w = op<MI_K_SILU_MUL>(g.w, u.w, 0.f, 0.f, 0.f);
      if constexpr (PARTS) parts4_put(out + r * 2 * inner + 4 * c, out + r * 2 * inner + inner + 4 * c, y);
      else f32x4_put(out + r * inner + 4 * c, y);
    } else {
      const float y = op<MI_K_SILU_MUL>(gu[r * 2 * inner + c], gu[r * 2 * inner + inner + c], 0.f, 0.f, 0.f);
      if constexpr (PARTS) {
        uint16_t h, l;
        split_bf16(y, h, l);
        out[r * 2 * inner + c] = h;
        out[r * 2 * inner + inner + c] = l;
      } else {
        f32_put(out + r * inner + c, y);
      }
    }
  }
}

// The q|k|v tail of a prefill in one pass over the fused projection's rows
// qkv [batch * seq, (heads + 2 kv) * d], row (sequence b, position p): RoPE
// on the q and k heads at position pos0 + p (rope_kernel's arithmetic), k and
// v written into the caches [batch * kv * maxc, d] at row (b kv + j) maxc +
// pos0 + p, q written to row (b seq + p) heads + h (natural order) or, with
// `grouped`, to row ((b kv + j) seq + p) G + g for head h = j G + g (the
// queries regrouped per kv head, G = heads / kv).  The caches are F32 or BF16
// (KV; k and v rounded to nearest even as they are stored).
template <typename KV>
__global__ void qkv_rope_cache_kernel(const float *qkv, const float *cosp, const float *sinp, float *q, KV *kc,
                                      KV *vc, int64_t rows, int64_t seq, int64_t heads, int64_t kv, int64_t d,
                                      int64_t maxc, int64_t pos0, int grouped) {
  const int64_t w = (heads + 2 * kv) * d, n = rows * w, half = d / 2, G = heads / kv;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int64_t r = e / w, c = e - r * w;
    const int64_t b = r / seq, p = r - b * seq, pos = pos0 + p;
    const int64_t h = c / d, j = c - h * d;  // head index across q, k, v
    const float xv = qkv[e];
    float y = xv;
    if (h < heads + kv) {  // q or k: rotate
      const float rv = qkv[r * w + h * d + (j < half ? j + half : j - half)];
      const float cv = __fmul_rn(xv, cosp[pos * d + j]);
      y = __fadd_rn(cv, __fmul_rn(rv, sinp[pos * d + j]));
    }
    if (h < heads) {
      const int64_t kvh = h / G, g = h - kvh * G;
      const int64_t row = grouped ? ((b * kv + kvh) * seq + p) * G + g : r * heads + h;
      q[row * d + j] = y;
    } else if (h < heads + kv) {
      f32_put(kc + ((b * kv + (h - heads)) * maxc + pos) * d + j, y);
    } else {
      f32_put(vc + ((b * kv + (h - heads - kv)) * maxc + pos) * d + j, y);
    }
  }
}
}  // namespace mi

extern "C" int mi_copy_into4(mi_ctx *ctx, mi_id dst, int64_t dst_offset, const int64_t dst_strides[4], mi_id src,
                             int64_t src_offset, const int64_t src_strides[4], const int64_t dims[4]) {
  MI_ENTER(ctx);
  if (!dst_strides || !src_strides || !dims) return fail(ctx, MI_E_ARG, "null dims or strides");
  MI_BUF(ctx, d, dst);
  MI_BUF(ctx, sb, src);
  MI_NO_BFP8(ctx, d, "copy_into4");
  MI_NO_BFP8(ctx, sb, "copy_into4");
  if (elem_size(d->elem) != elem_size(sb->elem)) return fail(ctx, MI_E_ARG, "copy of %s into %s", elem_name(sb->elem), elem_name(d->elem));
  int64_t n = 1;
  for (int i = 0; i < 4; ++i) {
    if (dims[i] < 0) return fail(ctx, MI_E_ARG, "negative copy extent");
    n *= dims[i];
  }
  if (n == 0) return MI_OK;
  int64_t lo, hi;
  span4(dims, dst_offset, dst_strides, &lo, &hi);
  if (lo < 0 || hi >= d->numel()) return fail(ctx, MI_E_ARG, "copy writes [%lld, %lld] of a %lld-element buffer", (long long)lo, (long long)hi, (long long)d->numel());
  span4(dims, src_offset, src_strides, &lo, &hi);
  if (lo < 0 || hi >= sb->numel()) return fail(ctx, MI_E_ARG, "copy reads [%lld, %lld] of a %lld-element buffer", (long long)lo, (long long)hi, (long long)sb->numel());
  const unsigned g = grid_for(n, 256 * 4, 256 * 32);
  if (elem_size(d->elem) == 2)
    copy_into4_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>(static_cast<uint16_t *>(d->ptr), static_cast<const uint16_t *>(sb->ptr),
        dims[1], dims[2], dims[3], n, dst_offset, dst_strides[0], dst_strides[1], dst_strides[2], dst_strides[3],
        src_offset, src_strides[0], src_strides[1], src_strides[2], src_strides[3]);
  else
    copy_into4_kernel<uint32_t><<<g, 256, 0, ctx->stream>>>(static_cast<uint32_t *>(d->ptr), static_cast<const uint32_t *>(sb->ptr),
        dims[1], dims[2], dims[3], n, dst_offset, dst_strides[0], dst_strides[1], dst_strides[2], dst_strides[3],
        src_offset, src_strides[0], src_strides[1], src_strides[2], src_strides[3]);
  return check_launch(ctx, "copy_into4");
}

extern "C" int mi_rope(mi_ctx *ctx, mi_id x, mi_id cos_table, mi_id sin_table, int64_t heads, int64_t seq, int64_t pos0,
                       mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, cb, cos_table);
  MI_BUF(ctx, sb, sin_table);
  if (xb->elem != MI_F32 || cb->elem != MI_F32 || sb->elem != MI_F32) return fail(ctx, MI_E_ARG, "rope takes F32");
  const int64_t R = xb->rows, D = xb->cols;
  if (D % 2 || cb->cols != D || sb->cols != D || cb->rows != sb->rows) return fail(ctx, MI_E_ARG, "rope tables [%lld, %lld] for width %lld", (long long)cb->rows, (long long)cb->cols, (long long)D);
  if (heads < 1 || seq < 1 || R % (heads * seq) != 0) return fail(ctx, MI_E_ARG, "rope: %lld rows are not sequences of %lld positions x %lld heads", (long long)R, (long long)seq, (long long)heads);
  if (pos0 < 0 || pos0 + seq > cb->rows) return fail(ctx, MI_E_ARG, "rope positions [%lld, %lld) beyond the %lld-row table", (long long)pos0, (long long)(pos0 + seq), (long long)cb->rows);
  const float *xp = static_cast<const float *>(xb->ptr), *cp = static_cast<const float *>(cb->ptr), *sp = static_cast<const float *>(sb->ptr);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, D, MI_F32, &id, &ob);
  if (s) return s;
  if (R * D > 0) {
    rope_kernel<<<grid_for(R * D, 256 * 4, 256 * 32), 256, 0, ctx->stream>>>(xp, cp, sp, static_cast<float *>(ob->ptr), R, D, heads, seq, pos0);
    s = check_launch(ctx, "rope");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

// qkv_rope_cache_kernel's work, one wavefront per row (four a block) and
// four columns a lane (d a multiple of 8, so a float4 of one half of a head
// has its rotation partner at the same place in the other half).  A row's
// loads are all issued before its first store (up to NQ float4 a lane: rows
// of up to 256 NQ columns; wider ones loop).  The head, sequence and position
// come from one small division per lane and one per row, not four 64-bit
// divisions per element.
template <typename KV>
__global__ void __launch_bounds__(256) qkv_rope_cache_row_kernel(const float *qkv, const float *cosp,
                                                                 const float *sinp, float *q, KV *kc, KV *vc,
                                                                 int64_t rows, int64_t seq, int heads, int kv, int d,
                                                                 int64_t maxc, int64_t pos0, int grouped) {
  constexpr int NQ = 4;
  const int w = (heads + 2 * kv) * d, half = d / 2, G = heads / kv;
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t b = r / seq, p = r - b * seq, pos = pos0 + p;
  const float *xr = qkv + r * w;
  for (int c0 = 4 * lane; c0 < w; c0 += 4 * 64 * NQ) {
    float4 y[NQ], rv[NQ], cv[NQ], sv[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int c = c0 + 4 * 64 * u;
      if (c < w) {
        const int h = c / d, j = c - h * d;
        y[u] = *reinterpret_cast<const float4 *>(xr + c);
        if (h < heads + kv) {
          rv[u] = *reinterpret_cast<const float4 *>(xr + h * d + (j < half ? j + half : j - half));
          cv[u] = *reinterpret_cast<const float4 *>(cosp + pos * d + j);
          sv[u] = *reinterpret_cast<const float4 *>(sinp + pos * d + j);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int c = c0 + 4 * 64 * u;
      if (c >= w) break;
      const int h = c / d, j = c - h * d;
      float4 o = y[u];
      if (h < heads + kv) {
        o.x = __fadd_rn(__fmul_rn(y[u].x, cv[u].x), __fmul_rn(rv[u].x, sv[u].x));
        o.y = __fadd_rn(__fmul_rn(y[u].y, cv[u].y), __fmul_rn(rv[u].y, sv[u].y));
        o.z = __fadd_rn(__fmul_rn(y[u].z, cv[u].z), __fmul_rn(rv[u].z, sv[u].z));
        o.w = __fadd_rn(__fmul_rn(y[u].w, cv[u].w), __fmul_rn(rv[u].w, sv[u].w));
      }
      if (h < heads) {
        const int kvh = h / G, g = h - kvh * G;
        const int64_t row = grouped ? ((b * kv + kvh) * seq + p) * G + g : r * heads + h;
        *reinterpret_cast<float4 *>(q + row * d + j) = o;
      } else if (h < heads + kv) {
        f32x4_put(kc + ((b * kv + (h - heads)) * maxc + pos) * d + j, o);
      } else {
        f32x4_put(vc + ((b * kv + (h - heads - kv)) * maxc + pos) * d + j, o);
      }
    }
  }
}

extern "C" int mi_silu_mul_halves(mi_ctx *ctx, mi_id gate_up, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, gb, gate_up);
  if (gb->elem != MI_F32 || gb->cols % 2)
    return fail(ctx, MI_E_ARG, "silu_mul_halves of %s [%lld, %lld]: want F32 with an even width", elem_name(gb->elem),
                (long long)gb->rows, (long long)gb->cols);
  if (out_elem != MI_F32 && out_elem != MI_BF16 && out_elem != MI_BF16_PARTS)
    return fail(ctx, MI_E_ARG, "silu_mul_halves result kind %d", out_elem);
  const int64_t R = gb->rows, I = gb->cols / 2;
  const bool parts = out_elem == MI_BF16_PARTS;
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, parts ? 2 * I : I, parts ? MI_BF16 : out_elem, &id, &ob);
  if (s) return s;
  if (R * I > 0) {
    const float *gp = static_cast<const float *>(gb->ptr);
    const unsigned gv = grid_for(R * I / 4, 256 * 2, 256 * 128), gs = grid_for(R * I, 256 * 4, 256 * 64);
    if (parts) {
      uint16_t *op_ = static_cast<uint16_t *>(ob->ptr);
      if (I % 4 == 0)
        silu_mul_halves_kernel<true, uint16_t, true><<<gv, 256, 0, ctx->stream>>>(gp, op_, R, I);
      else
        silu_mul_halves_kernel<false, uint16_t, true><<<gs, 256, 0, ctx->stream>>>(gp, op_, R, I);
    } else if (out_elem == MI_BF16) {
      uint16_t *op_ = static_cast<uint16_t *>(ob->ptr);
      if (I % 4 == 0)
        silu_mul_halves_kernel<true, uint16_t><<<gv, 256, 0, ctx->stream>>>(gp, op_, R, I);
      else
        silu_mul_halves_kernel<false, uint16_t><<<gs, 256, 0, ctx->stream>>>(gp, op_, R, I);
    } else {
      float *op_ = static_cast<float *>(ob->ptr);
      if (I % 4 == 0)
        silu_mul_halves_kernel<true, float><<<gv, 256, 0, ctx->stream>>>(gp, op_, R, I);
      else
        silu_mul_halves_kernel<false, float><<<gs, 256, 0, ctx->stream>>>(gp, op_, R, I);
    }
    s = check_launch(ctx, "silu_mul_halves");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_qkv_rope_cache(mi_ctx *ctx, mi_id qkv, mi_id cos_table, mi_id sin_table, int64_t seq,
                                 int64_t heads, int64_t kv_heads, int64_t pos0, mi_id k_cache, mi_id v_cache,
                                 int grouped, mi_id *q_out) {
  MI_ENTER(ctx);
  if (!q_out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, qkv);
  MI_BUF(ctx, cb, cos_table);
  MI_BUF(ctx, sb, sin_table);
  MI_BUF(ctx, kb, k_cache);
  MI_BUF(ctx, vb, v_cache);
  if (xb->elem != MI_F32 || cb->elem != MI_F32 || sb->elem != MI_F32 || kb->elem != vb->elem ||
      !elem_float(kb->elem))
    return fail(ctx, MI_E_ARG, "qkv_rope_cache takes F32 rows and tables and two F32 or two BF16 caches");
  const int64_t D = kb->cols, R = xb->rows;
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || D < 2 || D % 2)
    return fail(ctx, MI_E_ARG, "qkv_rope_cache: %lld heads over %lld kv heads of width %lld", (long long)heads,
                (long long)kv_heads, (long long)D);
  if (xb->cols != (heads + 2 * kv_heads) * D)
    return fail(ctx, MI_E_ARG, "qkv_rope_cache: rows of %lld, want (heads + 2 kv_heads) * %lld = %lld",
                (long long)xb->cols, (long long)D, (long long)((heads + 2 * kv_heads) * D));
  if (seq < 1 || R % seq) return fail(ctx, MI_E_ARG, "qkv_rope_cache: %lld rows are not sequences of %lld", (long long)R, (long long)seq);
  const int64_t batch = R / seq;
  if (vb->cols != D || vb->rows != kb->rows || kb->rows % (batch * kv_heads))
    return fail(ctx, MI_E_ARG, "qkv_rope_cache: caches must both be [%lld * %lld * max_ctx, %lld]", (long long)batch,
                (long long)kv_heads, (long long)D);
  const int64_t maxc = kb->rows / (batch * kv_heads);
  if (pos0 < 0 || pos0 + seq > maxc)
    return fail(ctx, MI_E_ARG, "qkv_rope_cache: positions [%lld, %lld) beyond the cache's %lld", (long long)pos0,
                (long long)(pos0 + seq), (long long)maxc);
  if (cb->cols != D || sb->cols != D || cb->rows != sb->rows || pos0 + seq > cb->rows)
    return fail(ctx, MI_E_ARG, "qkv_rope_cache: rope tables [%lld, %lld] for positions below %lld", (long long)cb->rows,
                (long long)cb->cols, (long long)(pos0 + seq));
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R * heads, D, MI_F32, &id, &ob);
  if (s) return s;
  const bool aligned = (reinterpret_cast<uintptr_t>(xb->ptr) | reinterpret_cast<uintptr_t>(ob->ptr) |
                        reinterpret_cast<uintptr_t>(kb->ptr) | reinterpret_cast<uintptr_t>(vb->ptr) |
                        reinterpret_cast<uintptr_t>(cb->ptr) | reinterpret_cast<uintptr_t>(sb->ptr)) % 16 == 0;
  const float *xp = static_cast<const float *>(xb->ptr), *cp = static_cast<const float *>(cb->ptr),
              *sp = static_cast<const float *>(sb->ptr);
  float *qp = static_cast<float *>(ob->ptr);
  const bool kv16 = kb->elem == MI_BF16;
  if (R > 0 && D % 8 == 0 && aligned && R <= INT32_MAX && xb->cols <= INT32_MAX) {
    const unsigned grid = static_cast<unsigned>((R + 3) / 4);
    const int hi = static_cast<int>(heads), kvi = static_cast<int>(kv_heads), di = static_cast<int>(D);
    if (kv16)
      qkv_rope_cache_row_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>(
          xp, cp, sp, qp, static_cast<uint16_t *>(kb->ptr), static_cast<uint16_t *>(vb->ptr), R, seq, hi, kvi, di,
          maxc, pos0, grouped ? 1 : 0);
    else
      qkv_rope_cache_row_kernel<float><<<grid, 256, 0, ctx->stream>>>(
          xp, cp, sp, qp, static_cast<float *>(kb->ptr), static_cast<float *>(vb->ptr), R, seq, hi, kvi, di, maxc,
          pos0, grouped ? 1 : 0);
    s = check_launch(ctx, "qkv_rope_cache");
    if (s) { mi_free(ctx, id); return s; }
  } else if (R > 0) {
    const unsigned grid = grid_for(R * xb->cols, 256 * 4, 256 * 64);
    if (kv16)
      qkv_rope_cache_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>(
          xp, cp, sp, qp, static_cast<uint16_t *>(kb->ptr), static_cast<uint16_t *>(vb->ptr), R, seq, heads, kv_heads,
          D, maxc, pos0, grouped ? 1 : 0);
    else
      qkv_rope_cache_kernel<float><<<grid, 256, 0, ctx->stream>>>(
          xp, cp, sp, qp, static_cast<float *>(kb->ptr), static_cast<float *>(vb->ptr), R, seq, heads, kv_heads, D,
          maxc, pos0, grouped ? 1 : 0);
    s = check_launch(ctx, "qkv_rope_cache");
    if (s) { mi_free(ctx, id); return s; }
  }
  *q_out = id;
  return MI_OK;
}

// ------------------------------------------------------------- SGD update
// The optimizer's `param - grad * lr` (burn-optim `Sgd` without momentum or
// decay) for many parameters in one launch, in place.  Each parameter gets a
// run of blocks; a block finds its parameter by a scan of the (at most
// SGD_MAX_PARAMS) block offsets in the kernel argument, then updates 4 float4
// per thread.  Bits equal the two-op form: grad * lr rounded, then subtracted.
// A gradient of S stacked slices (a split-K product's partials) is their sum
// in slice order first -- the bits split-K's own reduce gives.
namespace mi {
constexpr int SGD_MAX_PARAMS = 48;
constexpr int SGD_BLOCK_ELEMS = 256 * 16;

struct SgdList {
  float *p[SGD_MAX_PARAMS];
  const float *g[SGD_MAX_PARAMS];
  int64_t n[SGD_MAX_PARAMS];
  int S[SGD_MAX_PARAMS];
  int64_t first_block[SGD_MAX_PARAMS + 1];
  int count;
};

__global__ void __launch_bounds__(256) sgd_kernel(SgdList L, float lr) {
  int i = 0;
  while (i + 1 < L.count && static_cast<int64_t>(blockIdx.x) >= L.first_block[i + 1]) ++i;
  float *p = L.p[i];
  const float *g = L.g[i];
  const int64_t n = L.n[i];
  const int S = L.S[i];
  const int64_t base = (static_cast<int64_t>(blockIdx.x) - L.first_block[i]) * SGD_BLOCK_ELEMS;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t e = base + (static_cast<int64_t>(u) * 256 + threadIdx.x) * 4;
    if (e + 3 < n && (S == 1 || (n & 3) == 0)) {  // slices 16-byte aligned too
      float4 pv = *reinterpret_cast<const float4 *>(p + e);
      float4 gv = *reinterpret_cast<const float4 *>(g + e);
      for (int z0 = 1; z0 < S; z0 += 4) {  // four slices' loads before their adds
        float4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (z0 + u < S) q[u] = *reinterpret_cast<const float4 *>(g + (z0 + u) * n + e);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (z0 + u < S) {
            gv.x += q[u].x; gv.y += q[u].y; gv.z += q[u].z; gv.w += q[u].w;
          }
      }
      pv.x = __fsub_rn(pv.x, __fmul_rn(gv.x, lr));
      pv.y = __fsub_rn(pv.y, __fmul_rn(gv.y, lr));
      pv.z = __fsub_rn(pv.z, __fmul_rn(gv.z, lr));
      pv.w = __fsub_rn(pv.w, __fmul_rn(gv.w, lr));
      *reinterpret_cast<float4 *>(p + e) = pv;
    } else {
      for (int64_t k = e; k < n && k < e + 4; ++k) {
        float gk = g[k];
        for (int z = 1; z < S; ++z) gk += g[z * n + k];
        p[k] = __fsub_rn(p[k], __fmul_rn(gk, lr));
      }
    }
  }
}
}  // namespace mi

extern "C" int mi_sgd_update(mi_ctx *ctx, int64_t count, const mi_id *params, const mi_id *grads, float lr) {
  MI_ENTER(ctx);
  if (count < 0 || (count > 0 && (!params || !grads))) return fail(ctx, MI_E_ARG, "sgd_update: null lists");
  SgdList L;
  L.count = 0;
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (L.count == 0) return MI_OK;
    L.first_block[L.count] = blocks;
    sgd_kernel<<<static_cast<unsigned>(blocks), 256, 0, ctx->stream>>>(L, lr);
    L.count = 0;
    blocks = 0;
    return check_launch(ctx, "sgd_update");
  };
  for (int64_t i = 0; i < count; ++i) {
    const Buffer *pb = lookup(ctx, params[i]);
    const Buffer *gb = lookup(ctx, grads[i]);
    if (!pb || !gb) return fail(ctx, MI_E_ID, "sgd_update: unknown id in entry %lld", (long long)i);
    if (pb->elem != MI_F32 || gb->elem != MI_F32) return fail(ctx, MI_E_ARG, "sgd_update: entry %lld is not F32", (long long)i);
    const int64_t n = pb->rows * pb->cols, ng = gb->rows * gb->cols;
    if (n > 0 && (ng % n || ng / n < 1 || ng / n > 64))
      return fail(ctx, MI_E_ARG, "sgd_update: entry %lld: %lld parameters, %lld gradients (1 to 64 slices)",
                  (long long)i, (long long)n, (long long)ng);
    if (n == 0 && ng != 0)
      return fail(ctx, MI_E_ARG, "sgd_update: entry %lld: no parameters, %lld gradients", (long long)i, (long long)ng);
    if (params[i] == grads[i]) return fail(ctx, MI_E_ARG, "sgd_update: entry %lld updates a buffer by itself", (long long)i);
    if (n == 0) continue;
    const int64_t nb = (n + SGD_BLOCK_ELEMS - 1) / SGD_BLOCK_ELEMS;
    if (L.count == SGD_MAX_PARAMS || blocks + nb > INT32_MAX) {
      int s = flush();
      if (s) return s;
    }
    L.p[L.count] = static_cast<float *>(pb->ptr);
    L.g[L.count] = static_cast<const float *>(gb->ptr);
    L.n[L.count] = n;
    L.S[L.count] = static_cast<int>(ng / n);
    L.first_block[L.count] = blocks;
    ++L.count;
    blocks += nb;
  }
  return flush();
}
