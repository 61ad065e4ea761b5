// Reductions over one axis and over a whole buffer, fused row softmax /
// log-softmax (with attention's scale and mask), RMSNorm and LayerNorm.
//
// Reference: Engine::reduce (crates/burn-tt/src/server.rs:404) and
// Session::reduce_then (crates/tt-kernels/src/session.rs:8487) with the order
// contract of crates/tt-kernels/src/sfpu/reduce.rs:1-38; full sums
// (crates/burn-tt/src/ops.rs:3246-3400); mean = sum / count (ops.rs:3456-3469);
// softmax / log_softmax (ops.rs:5133-5166) and attention's clamped softmax
// (ops.rs:4572-4590); Engine::softmax_rows (server.rs:428); Engine::rms_norm
// (server.rs:438, crates/burn-tt/src/ops/norm.rs:39-283).
//
// MI355X design.  Row-wise work (over columns) gives each row to one 64-lane
// wavefront: lanes stride the row with coalesced loads, keep it in registers
// when it fits (softmax reads its row from HBM once and writes it once), and
// fold across lanes with a fixed butterfly, so results are deterministic.
// Softmax takes each quotient by the row sum as a product with the sum's
// reciprocal (one division per row instead of one per element, which would
// make the kernel VALU-bound): at most one rounding more than a division,
// relative error < 2^-22.
// Column sums (over rows) split the rows over a 2-D grid, each block summing a
// strip of columns over its share of the rows as float4 lanes (F32 rows of
// 1024+ columns: every splits-th row, so the grid sweeps the matrix in
// address order), and a second pass folds the partials in a fixed order (16
// interleaved chains, then in chain order) -- deterministic, and enough
// blocks to fill 256 CUs.
#include "common.hpp"
#include "wave.hpp"

#include <cfloat>

namespace mi {

__device__ __forceinline__ float ld(const void *p, int elem, int64_t i) {
  return elem == MI_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]) : static_cast<const float *>(p)[i];
}
__device__ __forceinline__ void st(void *p, int elem, int64_t i, float v) {
  if (elem == MI_BF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  else static_cast<float *>(p)[i] = v;
}

// ------------------------------------------------ reduce over columns (dim 1)
// One wavefront per row; four rows per 256-thread block.
template <bool NT>
__global__ void __launch_bounds__(256) reduce_cols_kernel(const void *x, int elem, float *out, int64_t rows,
                                                          int64_t cols, int op) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float acc = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  if (elem == MI_F32 && (cols % 4) == 0) {
    const float *p = static_cast<const float *>(x) + base;
    const int64_t n4 = cols / 4;
    auto fold = [op](float a, float4 v) {
      if (op == MI_R_MAX) return max_nan(max_nan(max_nan(max_nan(a, v.x), v.y), v.z), v.w);
      if (op == MI_R_MIN) return min_nan(min_nan(min_nan(min_nan(a, v.x), v.y), v.z), v.w);
      return a + ((v.x + v.y) + (v.z + v.w));
    };
    int64_t j = lane;
    // Four float4 per lane in flight, streamed when the input is large.
    for (; j + 192 < n4; j += 256) {
      float4 v0, v1, v2, v3;
      if (NT) { v0 = ld4<true>(p + 4 * j); v1 = ld4<true>(p + 4 * (j + 64)); v2 = ld4<true>(p + 4 * (j + 128)); v3 = ld4<true>(p + 4 * (j + 192)); }
      else { v0 = ld4<false>(p + 4 * j); v1 = ld4<false>(p + 4 * (j + 64)); v2 = ld4<false>(p + 4 * (j + 128)); v3 = ld4<false>(p + 4 * (j + 192)); }
      acc = fold(fold(fold(fold(acc, v0), v1), v2), v3);
    }
    for (; j < n4; j += 64) acc = fold(acc, ld4<false>(p + 4 * j));
  } else {
    for (int64_t j = lane; j < cols; j += 64) {
      float v = ld(x, elem, base + j);
      if (op == MI_R_MAX) acc = max_nan(acc, v);
      else if (op == MI_R_MIN) acc = min_nan(acc, v);
      else acc += v;
    }
  }
  if (op == MI_R_MAX) acc = wave_max(acc);
  else if (op == MI_R_MIN) acc = wave_min(acc);
  else acc = wave_sum(acc);
  if (lane == 0) out[row] = (op == MI_R_MEAN) ? acc / static_cast<float>(cols) : acc;
}

// --------------------------------------------------- reduce over rows (dim 0)
// Block (256 threads) = 4 waves; a wave's 64 lanes cover 256 columns as
// float4 (or 64 columns as scalars).  Wave w adds rows r0 + w, r0 + w + 4, ...
// of the block's row strip; the 4 waves then fold in order through LDS.
template <bool VEC>
__global__ void __launch_bounds__(256) reduce_rows_part(const void *x, int elem, float *part, int64_t rows,
                                                        int64_t cols, int64_t rows_per_split, int op) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  constexpr int CW = VEC ? 256 : 64;  // columns per block
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CW;
  const int64_t split = blockIdx.y;
  const int64_t r_begin = split * rows_per_split;
  const int64_t r_end = r_begin + rows_per_split < rows ? r_begin + rows_per_split : rows;
  const float init = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  float4 acc = make_float4(init, init, init, init);
  __shared__ float4 red[4][64];
  if (VEC) {
    const int64_t c = c0 + lane * 4;
    if (c < cols) {
      const float *p = static_cast<const float *>(x);
#pragma unroll 8
      for (int64_t r = r_begin + w; r < r_end; r += 4) {
        float4 v = *reinterpret_cast<const float4 *>(p + r * cols + c);
        if (op == MI_R_MAX) { acc.x = max_nan(acc.x, v.x); acc.y = max_nan(acc.y, v.y); acc.z = max_nan(acc.z, v.z); acc.w = max_nan(acc.w, v.w); }
        else if (op == MI_R_MIN) { acc.x = min_nan(acc.x, v.x); acc.y = min_nan(acc.y, v.y); acc.z = min_nan(acc.z, v.z); acc.w = min_nan(acc.w, v.w); }
        else { acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w; }
      }
    }
  } else {
    const int64_t c = c0 + lane;
    if (c < cols) {
      for (int64_t r = r_begin + w; r < r_end; r += 4) {
        float v = ld(x, elem, r * cols + c);
        if (op == MI_R_MAX) acc.x = max_nan(acc.x, v);
        else if (op == MI_R_MIN) acc.x = min_nan(acc.x, v);
        else acc.x += v;
      }
    }
  }
  red[w][lane] = acc;
  __syncthreads();
  if (w == 0) {
    float4 s = red[0][lane];
    for (int k = 1; k < 4; ++k) {
      float4 v = red[k][lane];
      if (op == MI_R_MAX) { s.x = max_nan(s.x, v.x); s.y = max_nan(s.y, v.y); s.z = max_nan(s.z, v.z); s.w = max_nan(s.w, v.w); }
      else if (op == MI_R_MIN) { s.x = min_nan(s.x, v.x); s.y = min_nan(s.y, v.y); s.z = min_nan(s.z, v.z); s.w = min_nan(s.w, v.w); }
      else { s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w; }
    }
    float *dst = part + split * cols;
    if (VEC) {
      const int64_t c = c0 + lane * 4;
      if (c < cols) *reinterpret_cast<float4 *>(dst + c) = s;
    } else {
      const int64_t c = c0 + lane;
      if (c < cols) dst[c] = s.x;
    }
  }
}

// Wide rows (F32, at least 1024 columns, a multiple of 4): block (tile,
// split) folds the tile's 1024 columns -- 256 threads, a float4 each -- over
// rows split, split + splits, split + 2 splits, ... in that order, sixteen
// rows' loads in flight, into partial row `split`.  Interleaved rows keep the
// grid's blocks on neighbouring rows at any moment, so the grid sweeps the
// matrix in address order: 0.86 of HBM peak on [8192, 8192] against 0.82
// for blocks of whole rows over contiguous row ranges, and 0.77 for 1024
// columns over contiguous ranges.  (Finishing in the same launch -- the
// last block of a tile folding its partials behind an arrival counter --
// measured ~10 us slower than the second launch: the write-through of the
// partials, the counter's round trip and the coherent reads are serial.)
template <bool NT>
__global__ void __launch_bounds__(256) reduce_rows_strided(const float *x, float *part, int64_t rows, int64_t cols,
                                                           int op) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 1024 + threadIdx.x * 4;
  if (c >= cols) return;
  const int64_t split = blockIdx.y, splits = gridDim.y;
  const int64_t n = rows > split ? (rows - split + splits - 1) / splits : 0;  // rows of this split
  const float init = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  float4 acc = make_float4(init, init, init, init);
  auto fold = [op](float4 &a, float4 v) {
    if (op == MI_R_MAX) { a.x = max_nan(a.x, v.x); a.y = max_nan(a.y, v.y); a.z = max_nan(a.z, v.z); a.w = max_nan(a.w, v.w); }
    else if (op == MI_R_MIN) { a.x = min_nan(a.x, v.x); a.y = min_nan(a.y, v.y); a.z = min_nan(a.z, v.z); a.w = min_nan(a.w, v.w); }
    else { a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w; }
  };
  // Row k of the split is row split + k * splits: a step of `st` floats.
  const int64_t st = splits * cols;
  const float *p = x + split * cols + c;
  int64_t k = 0;
  if (k + 8 <= n) {
    float4 v[8], w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ld4<NT>(p + (k + u) * st);
    for (; k + 16 <= n; k += 16) {
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = ld4<NT>(p + (k + 8 + u) * st);
#pragma unroll
      for (int u = 0; u < 8; ++u) fold(acc, v[u]);
      if (k + 24 <= n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld4<NT>(p + (k + 16 + u) * st);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) fold(acc, w[u]);
    }
    if (k + 8 <= n) {  // v holds rows k .. k + 7
#pragma unroll
      for (int u = 0; u < 8; ++u) fold(acc, v[u]);
      k += 8;
    }
  }
  for (; k < n; ++k) fold(acc, ld4<NT>(p + k * st));
  *reinterpret_cast<float4 *>(part + split * cols + c) = acc;
}

// Fold the partial rows [nb, n] of a split reduction into [1, n].  A block
// of 512 threads takes 32 columns: thread t folds column t % 32 over partial
// rows w, w + 16, w + 32, ... (chain w = t / 32, sixteen loads in flight),
// and the 16 chains fold in chain order through LDS -- a fixed order, so the
// result is deterministic.  Columns below `split_at` go to out0, the rest to
// out1 (two reductions in one pass).
__global__ void __launch_bounds__(512) fold_partials_kernel(const float *part, int64_t nb, int64_t n, int op,
                                                            float div, float *out0, int64_t split_at, float *out1) {
  __shared__ float red[16][32];
  const int col = threadIdx.x & 31, w = threadIdx.x >> 5;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 32 + col;
  auto fold = [op](float a, float b) {
    if (op == MI_R_MAX) return max_nan(a, b);
    if (op == MI_R_MIN) return min_nan(a, b);
    return a + b;
  };
  float acc = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  if (c < n) {
    for (int64_t k = w; k < nb; k += 256) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = (k + 16 * u < nb) ? part[(k + 16 * u) * n + c] : 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (k + 16 * u < nb) acc = fold(acc, v[u]);
    }
  }
  red[w][col] = acc;
  __syncthreads();
  if (w == 0 && c < n) {
    float s = red[0][col];
#pragma unroll
    for (int k = 1; k < 16; ++k) s = fold(s, red[k][col]);
    if (op == MI_R_MEAN) s = s / div;
    if (c < split_at) out0[c] = s;
    else out1[c - split_at] = s;
  }
}

// ---------------------------------------------------------- full reduction
__global__ void __launch_bounds__(256) reduce_all_part(const void *x, int elem, float *part, int64_t n, int op) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  float acc = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = ld(x, elem, i);
    if (op == MI_R_MAX) acc = max_nan(acc, v);
    else if (op == MI_R_MIN) acc = min_nan(acc, v);
    else acc += v;
  }
  __shared__ float red[4];
  if (op == MI_R_MAX) acc = wave_max(acc);
  else if (op == MI_R_MIN) acc = wave_min(acc);
  else acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = red[0];
    for (int k = 1; k < 4; ++k) s = (op == MI_R_MAX) ? max_nan(s, red[k]) : (op == MI_R_MIN ? min_nan(s, red[k]) : s + red[k]);
    part[blockIdx.x] = s;
  }
}

__global__ void reduce_all_final(const float *part, int parts, float *out, int64_t n, int op) {
  // One wave folds the block partials in a fixed order.
  const int lane = threadIdx.x;
  float acc = (op == MI_R_MAX) ? -INFINITY : (op == MI_R_MIN ? INFINITY : 0.0f);
  for (int i = lane; i < parts; i += 64) {
    float v = part[i];
    if (op == MI_R_MAX) acc = max_nan(acc, v);
    else if (op == MI_R_MIN) acc = min_nan(acc, v);
    else acc += v;
  }
  if (op == MI_R_MAX) acc = wave_max(acc);
  else if (op == MI_R_MIN) acc = wave_min(acc);
  else acc = wave_sum(acc);
  if (lane == 0) out[0] = (op == MI_R_MEAN) ? acc / static_cast<float>(n) : acc;
}

// ------------------------------------------------------------ row softmax
// One wavefront per row, the row in registers: lane l holds columns
// l + 64 t (t < T).  `mask` Bool rows read as row % mask_rows.
template <int T>
__global__ void __launch_bounds__(256) softmax_kernel(const void *x, int elem, const uint32_t *mask, int64_t mask_rows,
                                                      float scale, int log_mode, void *out, int out_elem,
                                                      int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  const uint32_t *mrow = mask ? mask + (row % mask_rows) * cols : nullptr;
  float v[T];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    float a = -INFINITY;
    if (j < cols) {
      a = ld(x, elem, base + j);
      if (scale != 1.0f) a = a * scale;
      if (mrow && mrow[j]) a = -INFINITY;
    }
    v[t] = a;
    m = max_nan(m, a);
  }
  m = wave_max(m);
  if (mrow) m = m > -FLT_MAX ? m : (isnan(m) ? m : -FLT_MAX);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    float sh = v[t] - m;
    float e = (j < cols) ? expf(sh) : 0.0f;
    if (log_mode) v[t] = sh; else v[t] = e;
    s += e;
  }
  s = wave_sum(s);
  if (mrow) s = s > FLT_MIN ? s : (isnan(s) ? s : FLT_MIN);
  const float ls = log_mode ? logf(s) : 0.0f;
  const float inv = 1.0f / s;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < cols) st(out, out_elem, base + j, log_mode ? v[t] - ls : v[t] * inv);
  }
}

// Masked F32 rows of at most 1024 columns, a multiple of 4 (attention's
// scores): softmax_kernel with float4 loads of the row and uint4 loads of the
// mask, lane l holding columns 4 (l + 64 t) .. 4 (l + 64 t) + 3.  The max
// ignores NaN (a NaN makes the sum, and so its row, NaN, as a NaN max
// would); the clamps of a fully masked row are softmax_kernel's.  Half the
// load instructions of the scalar form, and no per-element kind switch.
template <int T4>
__global__ void __launch_bounds__(256) softmax_masked4_kernel(const float *x, const uint32_t *mask, int64_t mask_rows,
                                                              float scale, int log_mode, float *out, int64_t rows,
                                                              int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *xr = x + row * cols;
  const uint32_t *mr = mask + (row % mask_rows) * cols;
  float v[4 * T4];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T4; ++t) {
    const int64_t j = 4 * static_cast<int64_t>(lane + 64 * t);
    float4 a = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (j < cols) {
      a = *reinterpret_cast<const float4 *>(xr + j);
      const uint4 mk = *reinterpret_cast<const uint4 *>(mr + j);
      if (scale != 1.0f) { a.x *= scale; a.y *= scale; a.z *= scale; a.w *= scale; }
      a.x = mk.x ? -INFINITY : a.x; a.y = mk.y ? -INFINITY : a.y;
      a.z = mk.z ? -INFINITY : a.z; a.w = mk.w ? -INFINITY : a.w;
    }
    v[4 * t] = a.x; v[4 * t + 1] = a.y; v[4 * t + 2] = a.z; v[4 * t + 3] = a.w;
    m = fmaxf(fmaxf(m, a.x), fmaxf(a.y, fmaxf(a.z, a.w)));
  }
  m = wave_max(m);
  m = m > -FLT_MAX ? m : (isnan(m) ? m : -FLT_MAX);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < 4 * T4; ++t) {
    const float sh = v[t] - m;
    const float e = (4 * static_cast<int64_t>(lane + 64 * (t / 4)) < cols) ? expf(sh) : 0.0f;
    v[t] = log_mode ? sh : e;
    s += e;
  }
  s = wave_sum(s);
  s = s > FLT_MIN ? s : (isnan(s) ? s : FLT_MIN);
  const float ls = log_mode ? logf(s) : 0.0f;
  const float inv = 1.0f / s;
#pragma unroll
  for (int t = 0; t < T4; ++t) {
    const int64_t j = 4 * static_cast<int64_t>(lane + 64 * t);
    if (j < cols) {
      float4 r;
      r.x = log_mode ? v[4 * t] - ls : v[4 * t] * inv;
      r.y = log_mode ? v[4 * t + 1] - ls : v[4 * t + 1] * inv;
      r.z = log_mode ? v[4 * t + 2] - ls : v[4 * t + 2] * inv;
      r.w = log_mode ? v[4 * t + 3] - ls : v[4 * t + 3] * inv;
      *reinterpret_cast<float4 *>(out + row * cols + j) = r;
    }
  }
}

// Long rows: one 256-thread block per row, the row in registers (thread t
// holds float4 lanes t + 256 u, u < VPT, or scalars t + 256 u, u < 4 VPT),
// cross-wave folds through LDS.
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = max_nan(max_nan(red[0], red[1]), max_nan(red[2], red[3]));
  __syncthreads();
  return m;
}
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// FULL: the row is exactly 1024 VPT long (F32, VEC), so no column check.
// LOG: 0 softmax, 1 log-softmax, -1 as `log_mode` says.
// Up to 8192 columns the registers are held to 64, so eight rows' blocks
// share a CU: the 32 rows a CU gets of an 8192-row input then run in four
// full rounds instead of five and a third.
template <int VPT, bool VEC, bool NT, bool FULL = false, int LOG = -1>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(VPT <= 8 ? 8 : 4)))
softmax_block_kernel(const void *x, int elem, const uint32_t *mask,
                                                            int64_t mask_rows, float scale, int log_mode_arg, void *out,
                                                            int out_elem, int64_t cols) {
  static_assert(!FULL || VEC, "full rows are read as float4");
  const bool log_mode = LOG < 0 ? log_mode_arg != 0 : LOG == 1;
  constexpr int T = 4 * VPT;  // elements per thread
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * cols;
  const uint32_t *mrow = mask ? mask + (row % mask_rows) * cols : nullptr;
  const int tid = threadIdx.x;
  float v[T];
  auto col_of = [&](int t) -> int64_t {
    return VEC ? (static_cast<int64_t>(tid + 256 * (t >> 2)) * 4 + (t & 3)) : static_cast<int64_t>(tid + 256 * t);
  };
  if constexpr (VEC) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + base);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int64_t j4 = tid + 256 * u;
      float4 q = (FULL || j4 * 4 < cols) ? ld4<NT>(reinterpret_cast<const float *>(p + j4))
                                         : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      v[4 * u] = q.x; v[4 * u + 1] = q.y; v[4 * u + 2] = q.z; v[4 * u + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = col_of(t);
      v[t] = j < cols ? ld(x, elem, base + j) : -INFINITY;
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = col_of(t);
    if (FULL || j < cols) {
      if (scale != 1.0f) v[t] = v[t] * scale;
      if (mrow && mrow[j]) v[t] = -INFINITY;
    }
    m = max_nan(m, v[t]);
  }
  m = block_max(m, red);
  if (mrow) m = m > -FLT_MAX ? m : (isnan(m) ? m : -FLT_MAX);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = col_of(t);
    const float sh = v[t] - m;
    const float e = (FULL || j < cols) ? expf(sh) : 0.0f;
    v[t] = log_mode ? sh : e;
    s += e;
  }
  s = block_sum(s, red);
  if (mrow) s = s > FLT_MIN ? s : (isnan(s) ? s : FLT_MIN);
  const float ls = log_mode ? logf(s) : 0.0f;
  const float inv = 1.0f / s;
  if (VEC && out_elem == MI_F32) {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + base);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int64_t j4 = tid + 256 * u;
      if (FULL || j4 * 4 < cols) {
        float4 r;
        r.x = log_mode ? v[4 * u] - ls : v[4 * u] * inv;
        r.y = log_mode ? v[4 * u + 1] - ls : v[4 * u + 1] * inv;
        r.z = log_mode ? v[4 * u + 2] - ls : v[4 * u + 2] * inv;
        r.w = log_mode ? v[4 * u + 3] - ls : v[4 * u + 3] * inv;
        st4<NT>(reinterpret_cast<float *>(o + j4), r);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = col_of(t);
      if (j < cols) st(out, out_elem, base + j, log_mode ? v[t] - ls : v[t] * inv);
    }
  }
}

// One row of exactly 1024 VPT F32 columns held in registers (thread t holds
// float4 lanes t + 256 u), unmasked: the softmax_block_kernel<VPT, true, true,
// true, LOG> arithmetic in the same order, so the same bits for every row
// without a NaN.  The row's max ignores NaN (v_max / v_max3, one instruction
// per element or two instead of six for the NaN-ranking max): a NaN makes the
// sum NaN and so every output of its row NaN, as when the max is NaN.  The
// max and the sum fold through separate LDS slots, one barrier each.
template <int N>
__device__ __forceinline__ float tree_sum(const float *r) {
  if constexpr (N == 1) return r[0];
  else return tree_sum<N / 2>(r) + tree_sum<N / 2>(r + N / 2);
}
template <int N>
__device__ __forceinline__ float tree_max(const float *r) {
  if constexpr (N == 1) return r[0];
  else return fmaxf(tree_max<N / 2>(r), tree_max<N / 2>(r + N / 2));
}

template <int VPT, int LOG, int NTH, bool NT>
__device__ __forceinline__ void softmax_row_regs(const float4 (&q)[VPT], float scale, float *o,
                                                 float (&red)[2][NTH / 64]) {
  constexpr int T = 4 * VPT, NW = NTH / 64;
  const int tid = threadIdx.x, w = tid >> 6;
  float v[T];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    v[4 * u] = q[u].x; v[4 * u + 1] = q[u].y; v[4 * u + 2] = q[u].z; v[4 * u + 3] = q[u].w;
  }
  if (scale != 1.0f) {
#pragma unroll
    for (int t = 0; t < T; ++t) v[t] = v[t] * scale;
  }
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; t += 2) m = fmaxf(fmaxf(m, v[t]), v[t + 1]);
  m = wave_max(m);
  if ((tid & 63) == 0) red[0][w] = m;
  __syncthreads();
  m = tree_max<NW>(red[0]);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float sh = v[t] - m;
    const float e = expf(sh);
    v[t] = LOG ? sh : e;
    s += e;
  }
  s = wave_sum(s);
  if ((tid & 63) == 0) red[1][w] = s;
  __syncthreads();
  s = tree_sum<NW>(red[1]);
  const float ls = LOG ? logf(s) : 0.0f;
  const float inv = 1.0f / s;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    float4 r;
    r.x = LOG ? v[4 * u] - ls : v[4 * u] * inv;
    r.y = LOG ? v[4 * u + 1] - ls : v[4 * u + 1] * inv;
    r.z = LOG ? v[4 * u + 2] - ls : v[4 * u + 2] * inv;
    r.w = LOG ? v[4 * u + 3] - ls : v[4 * u + 3] * inv;
    st4<NT>(o + static_cast<int64_t>(tid + NTH * u) * 4, r);
  }
}

// Unmasked F32 rows of exactly 4 NTH VPT columns, one block of NTH threads
// per row, eight waves to a SIMD; NT streams the accesses (large inputs).  Eight values a thread (VPT = 2; 1024
// threads for 8192 columns): on [8192, 8192] 0.78 of HBM peak against 0.75
// with 16 values a thread and 0.73 with 32 -- short-lived waves keep more of
// the chip's loads in flight while others fold and exponentiate.  (Blocks
// that walk several rows with the next row's loads in flight under the
// current row's folds measured no better.)
template <int VPT, int LOG, int NTH, bool NT>
__global__ void __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(8)))
softmax_row_kernel(const float *x, float scale, float *out) {
  constexpr int64_t C = 4 * NTH * VPT;
  __shared__ float red[2][NTH / 64];
  const int64_t lane = static_cast<int64_t>(threadIdx.x) * 4;
  const int64_t row = blockIdx.x;
  float4 a[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) a[u] = ld4<NT>(x + row * C + lane + 4 * NTH * u);
  softmax_row_regs<VPT, LOG, NTH, NT>(a, scale, out + row * C, red);
}

// Cross-entropy over a row of logits and its gradient in one pass: the row's
// log-softmax logp_j = (z_j - m) - ln(sum_k e^(z_k - m)) exactly as the
// log-softmax kernel forms it, the target's value logp_t written to
// picked[row], and dz_j = e^(logp_j) * gscale + (j == t ? -gscale : 0) -- the
// same two roundings as exp, then MUL_ADD against the scattered one-hot --
// written to dz.  A target outside [0, cols) raises the index flag, picks 0
// bits and adds no one-hot term (as pick_columns and scatter_add_columns).
// NTH threads a row: thread t holds float4 lanes t + NTH u (VEC) or values
// t + NTH u, folded as the softmax kernel that runs the log-softmax of the
// same row folds (softmax_row_kernel, NTH = columns / 8, for rows of 2048,
// 4096 or 8192 columns; softmax_block_kernel, NTH = 256, otherwise).
template <int VPT, bool VEC, bool NT, int NTH = 256>
__global__ void __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(VPT <= 8 ? 8 : 4)))
log_softmax_ce_kernel(const float *z, const int32_t *tgt, int64_t cols, float gscale, float *picked, float *dz,
                      uint32_t *flags) {
  constexpr int T = 4 * VPT, NW = NTH / 64;
  __shared__ float red[2][NW];
  const int64_t row = blockIdx.x;
  const int64_t base = row * cols;
  const int tid = threadIdx.x, w = tid >> 6;
  float v[T];
  auto col_of = [&](int t) -> int64_t {
    return VEC ? (static_cast<int64_t>(tid + NTH * (t >> 2)) * 4 + (t & 3)) : static_cast<int64_t>(tid + NTH * t);
  };
  if constexpr (VEC) {
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int64_t j4 = tid + NTH * u;
      const float4 q = (j4 * 4 < cols) ? ld4<NT>(z + base + j4 * 4)
                                       : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      v[4 * u] = q.x; v[4 * u + 1] = q.y; v[4 * u + 2] = q.z; v[4 * u + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = col_of(t);
      v[t] = j < cols ? z[base + j] : -INFINITY;
    }
  }
  // The max ignores NaN (two elements an instruction): a NaN logit makes the
  // sum, and so every value of its row, NaN, as a NaN max would.
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; t += 2) m = fmaxf(fmaxf(m, v[t]), v[t + 1]);
  m = wave_max(m);
  if ((tid & 63) == 0) red[0][w] = m;
  __syncthreads();
  m = tree_max<NW>(red[0]);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float sh = v[t] - m;
    s += col_of(t) < cols ? expf(sh) : 0.0f;
    v[t] = sh;
  }
  s = wave_sum(s);
  if ((tid & 63) == 0) red[1][w] = s;
  __syncthreads();
  s = tree_sum<NW>(red[1]);
  const float ls = logf(s);
  const int32_t target = tgt[row];
  const bool in_range = target >= 0 && target < cols;
  if (tid == 0 && !in_range) {
    atomicOr(flags, FLAG_INDEX_RANGE);
    picked[row] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = col_of(t);
    v[t] = v[t] - ls;  // logp_j
    if (j == target) picked[row] = v[t];
    v[t] = __fadd_rn(j == target ? -gscale : 0.0f, __fmul_rn(expf(v[t]), gscale));
  }
  if constexpr (VEC) {
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int64_t j4 = tid + NTH * u;
      if (j4 * 4 < cols) st4<NT>(dz + base + j4 * 4, make_float4(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]));
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = col_of(t);
      if (j < cols) dz[base + j] = v[t];
    }
  }
}

// The same for rows of at most 1024 logits, a wavefront per row (lane l
// holds columns l + 64 t), in the order of the wavefront softmax.
template <int T>
__global__ void __launch_bounds__(256) log_softmax_ce_wave_kernel(const float *z, const int32_t *tgt, int64_t rows,
                                                                  int64_t cols, float gscale, float *picked, float *dz,
                                                                  uint32_t *flags) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float v[T];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = j < cols ? z[base + j] : -INFINITY;
    m = max_nan(m, v[t]);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    const float sh = v[t] - m;
    s += (j < cols) ? expf(sh) : 0.0f;
    v[t] = sh;
  }
  s = wave_sum(s);
  const float ls = logf(s);
  const int32_t target = tgt[row];
  if (lane == 0 && !(target >= 0 && target < cols)) {
    atomicOr(flags, FLAG_INDEX_RANGE);
    picked[row] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    const float lp = v[t] - ls;
    if (j == target) picked[row] = lp;
    if (j < cols) dz[base + j] = __fadd_rn(j == target ? -gscale : 0.0f, __fmul_rn(expf(lp), gscale));
  }
}

// Rows too long for registers: three passes over the row (from L2).
__global__ void __launch_bounds__(256) softmax_long_kernel(const void *x, int elem, const uint32_t *mask, int64_t mask_rows,
                                                           float scale, int log_mode, void *out, int out_elem,
                                                           int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  const uint32_t *mrow = mask ? mask + (row % mask_rows) * cols : nullptr;
  auto val = [&](int64_t j) {
    float a = ld(x, elem, base + j);
    if (scale != 1.0f) a = a * scale;
    if (mrow && mrow[j]) a = -INFINITY;
    return a;
  };
  float m = -INFINITY;
  for (int64_t j = lane; j < cols; j += 64) m = max_nan(m, val(j));
  m = wave_max(m);
  if (mrow) m = m > -FLT_MAX ? m : (isnan(m) ? m : -FLT_MAX);
  float s = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) s += expf(val(j) - m);
  s = wave_sum(s);
  if (mrow) s = s > FLT_MIN ? s : (isnan(s) ? s : FLT_MIN);
  const float ls = log_mode ? logf(s) : 0.0f;
  const float inv = 1.0f / s;
  for (int64_t j = lane; j < cols; j += 64) {
    float sh = val(j) - m;
    st(out, out_elem, base + j, log_mode ? sh - ls : expf(sh) * inv);
  }
}

// ------------------------------------------------------- RMSNorm, LayerNorm
// XF: the input and the gain F32, fixed at compile time (else read from elem
// and gelem); OE >= 0: the result's form, fixed likewise.  The fixed forms
// carry no element switch around each load and store.
template <int T, bool XF = false, int OE = -1>
__global__ void __launch_bounds__(256) rms_norm_kernel(const void *x, int elem, const void *gamma, int gelem, float eps,
                                                       void *out, int out_elem, int64_t rows, int64_t cols) {
  if constexpr (XF) {
    elem = MI_F32;
    gelem = MI_F32;
  }
  if constexpr (OE >= 0) out_elem = OE;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  // Rows of up to 2048 columns request the gain with the row, so the scaling
  // does not wait for a second memory round trip after the fold; the fold
  // runs on the DPP lane paths.
  constexpr bool GPRE = T <= 32;
  float v[T], gm[GPRE ? T : 1];
  float ss = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = j < cols ? ld(x, elem, base + j) : 0.0f;
    if constexpr (GPRE) gm[t] = (gamma && j < cols) ? ld(gamma, gelem, j) : 1.0f;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) ss += v[t] * v[t];
  ss = fold_sum<64>(ss);
  const float rms = __fsqrt_rn(ss / static_cast<float>(cols) + eps);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < cols) {
      float y = v[t] / rms;
      if constexpr (GPRE) {
        if (gamma) y = y * gm[t];
      } else {
        if (gamma) y = y * ld(gamma, gelem, j);
      }
      if (out_elem == MI_BF16_PARTS) {
        uint16_t h, l;
        split_bf16(y, h, l);
        uint16_t *o = static_cast<uint16_t *>(out) + 2 * base;
        o[j] = h;
        o[cols + j] = l;
      } else if (out_elem == MI_TILES_PARTS) {
        uint16_t h, l;
        split_bf16(y, h, l);
        uint16_t *o = static_cast<uint16_t *>(out) + tile_offset(row, j, cols);
        o[0] = h;
        o[rows * cols] = l;
      } else if (out_elem == MI_TILES_BF16) {
        static_cast<uint16_t *>(out)[tile_offset(row, j, cols)] = f32_to_bf16_bits(y);
      } else {
        st(out, out_elem, base + j, y);
      }
    }
  }
}

template <int T>
__global__ void __launch_bounds__(256) layer_norm_kernel(const float *x, const float *gamma, const float *beta, float eps,
                                                         float *out, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  // As rms_norm_kernel: the gain and bias requested with the row (up to
  // 1024 columns), the folds on the DPP lane paths.
  constexpr bool GPRE = T <= 16;
  float v[T], gm[GPRE ? T : 1], bt[GPRE ? T : 1];
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = j < cols ? x[base + j] : 0.0f;
    if constexpr (GPRE) {
      gm[t] = (gamma && j < cols) ? gamma[j] : 1.0f;
      bt[t] = (beta && j < cols) ? beta[j] : 0.0f;
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) s += v[t];
  const float mean = fold_sum<64>(s) / static_cast<float>(cols);
  float q = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    float d = j < cols ? v[t] - mean : 0.0f;
    q += d * d;
  }
  const float var = fold_sum<64>(q) / static_cast<float>(cols);
  const float den = __fsqrt_rn(var + eps);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < cols) {
      float y = (v[t] - mean) / den;
      if constexpr (GPRE) {
        if (gamma) y = y * gm[t];
        if (beta) y = y + bt[t];
      } else {
        if (gamma) y = y * gamma[j];
        if (beta) y = y + beta[j];
      }
      out[base + j] = y;
    }
  }
}

// Register-row kernels: the smallest T (columns per lane) covering `cols`.
static int pick_t(int64_t cols) {
  const int ts[] = {1, 2, 4, 8, 16, 32, 64, 128};
  for (int t : ts)
    if (cols <= 64 * t) return t;
  return 0;  // too long: a multi-pass kernel
}

}  // namespace mi

using namespace mi;

extern "C" int mi_reduce(mi_ctx *ctx, mi_id a, int op, int axis, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, x, a);
  if (op < MI_R_SUM || op > MI_R_MIN) return fail(ctx, MI_E_ARG, "reduce op %d", op);
  if (!elem_float(x->elem)) return fail(ctx, MI_E_ARG, "reduce of a %s buffer", elem_name(x->elem));
  if (axis != MI_AXIS_ROWS && axis != MI_AXIS_COLS) return fail(ctx, MI_E_ARG, "reduce axis %d", axis);
  const int64_t R = x->rows, C = x->cols;
  const void *xp = x->ptr;
  const int xe = x->elem;
  if ((axis == MI_AXIS_COLS ? C : R) == 0 && op != MI_R_SUM)
    return fail(ctx, MI_E_ARG, "reduce of an empty axis");
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, axis == MI_AXIS_COLS ? R : 1, axis == MI_AXIS_COLS ? 1 : C, MI_F32, &id, &ob);
  if (s) return s;
  float *o = static_cast<float *>(ob->ptr);
  if (axis == MI_AXIS_COLS) {
    if (R > 0) {
      if (C == 0) fill_zero(ctx, o, R * sizeof(float));
      else if (R * C * 4 >= kStreamBytes)
        reduce_cols_kernel<true><<<grid_for(R, 4, INT32_MAX), 256, 0, ctx->stream>>>(xp, xe, o, R, C, op);
      else
        reduce_cols_kernel<false><<<grid_for(R, 4, INT32_MAX), 256, 0, ctx->stream>>>(xp, xe, o, R, C, op);
    }
  } else if (C > 0) {
    if (R == 0) {
      fill_zero(ctx, o, C * sizeof(float));
    } else {
      const bool vec = (xe == MI_F32) && (C % 4 == 0);
      const bool wide = vec && C >= 1024;
      const int64_t cw = wide ? 1024 : (vec ? 256 : 64);
      const int64_t tiles = (C + cw - 1) / cw;
      // Wide rows: about 256 blocks (one a CU), at least 16 rows a split.
      // Otherwise about 2048 blocks, eight a CU, so the row ranges' loads
      // keep HBM busy.  The partials (written and re-read by the fold) stay a
      // few percent of the input.
      const int64_t target = wide ? 256 : 2048;
      int64_t splits = (target + tiles - 1) / tiles;
      int64_t max_splits = (R + 15) / 16;
      if (splits > max_splits) splits = max_splits;
      if (splits > 65535) splits = 65535;
      if (splits < 1) splits = 1;
      const int64_t rps = (R + splits - 1) / splits;
      if (!wide) splits = (R + rps - 1) / rps;
      float *part = static_cast<float *>(scratch(ctx, static_cast<size_t>(splits * C) * sizeof(float)));
      if (!part) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "reduce scratch"); }
      dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits));
      const float *xf = static_cast<const float *>(xp);
      if (wide && R * C * 4 >= kStreamBytes) reduce_rows_strided<true><<<grid, 256, 0, ctx->stream>>>(xf, part, R, C, op);
      else if (wide) reduce_rows_strided<false><<<grid, 256, 0, ctx->stream>>>(xf, part, R, C, op);
      else if (vec) reduce_rows_part<true><<<grid, 256, 0, ctx->stream>>>(xp, xe, part, R, C, rps, op);
      else reduce_rows_part<false><<<grid, 256, 0, ctx->stream>>>(xp, xe, part, R, C, rps, op);
      fold_partials_kernel<<<static_cast<unsigned>((C + 31) / 32), 512, 0, ctx->stream>>>(
          part, splits, C, op, static_cast<float>(R), o, C, nullptr);
    }
  }
  s = check_launch(ctx, "reduce");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

extern "C" int mi_reduce_all(mi_ctx *ctx, mi_id a, int op, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, x, a);
  if (op < MI_R_SUM || op > MI_R_MIN) return fail(ctx, MI_E_ARG, "reduce op %d", op);
  if (!elem_float(x->elem)) return fail(ctx, MI_E_ARG, "reduce of a %s buffer", elem_name(x->elem));
  const int64_t n = x->numel();
  if (n == 0 && op != MI_R_SUM) return fail(ctx, MI_E_ARG, "reduce of an empty buffer");
  const void *xp = x->ptr;
  const int xe = x->elem;
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, 1, 1, MI_F32, &id, &ob);
  if (s) return s;
  const int parts = static_cast<int>(grid_for(n, 256 * 8, 2048));
  float *part = static_cast<float *>(scratch(ctx, parts * sizeof(float)));
  if (!part) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "reduce scratch"); }
  reduce_all_part<<<parts, 256, 0, ctx->stream>>>(xp, xe, part, n, op);
  reduce_all_final<<<1, 64, 0, ctx->stream>>>(part, parts, static_cast<float *>(ob->ptr), n, op);
  s = check_launch(ctx, "reduce_all");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

extern "C" int mi_softmax_rows(mi_ctx *ctx, mi_id x, mi_id mask, float scale, int log, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  if (!elem_float(xb->elem)) return fail(ctx, MI_E_ARG, "softmax of a %s buffer", elem_name(xb->elem));
  if (out_elem != MI_F32 && out_elem != MI_BF16) return fail(ctx, MI_E_ARG, "softmax result kind %s", elem_name(out_elem));
  const uint32_t *mp = nullptr;
  int64_t mrows = 1;
  if (mask) {
    MI_BUF(ctx, mb, mask);
    if (mb->elem != MI_BOOL) return fail(ctx, MI_E_ARG, "softmax mask is %s", elem_name(mb->elem));
    if (mb->cols != xb->cols || mb->rows == 0 || (xb->rows % mb->rows) != 0)
      return fail(ctx, MI_E_ARG, "softmax mask [%lld, %lld] for [%lld, %lld]", (long long)mb->rows, (long long)mb->cols,
                  (long long)xb->rows, (long long)xb->cols);
    mp = static_cast<const uint32_t *>(mb->ptr);
    mrows = mb->rows;
  }
  const int64_t R = xb->rows, C = xb->cols;
  const void *xp = xb->ptr;
  const int xe = xb->elem;
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, C, out_elem, &id, &ob);
  if (s) return s;
  if (R > 0 && C > 0) {
    unsigned g = grid_for(R, 4, INT32_MAX);
    int t = pick_t(C);
    const bool vec = (xe == MI_F32) && (C % 4 == 0);
    if (t != 0 && t <= 16 && mp && xe == MI_F32 && out_elem == MI_F32 && C % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(xp) | reinterpret_cast<uintptr_t>(mp)) % 16 == 0) {
      const float *xf = static_cast<const float *>(xp);
      float *of = static_cast<float *>(ob->ptr);
      switch ((C + 255) / 256) {
        case 1: softmax_masked4_kernel<1><<<g, 256, 0, ctx->stream>>>(xf, mp, mrows, scale, log, of, R, C); break;
        case 2: softmax_masked4_kernel<2><<<g, 256, 0, ctx->stream>>>(xf, mp, mrows, scale, log, of, R, C); break;
        default: softmax_masked4_kernel<4><<<g, 256, 0, ctx->stream>>>(xf, mp, mrows, scale, log, of, R, C); break;
      }
    } else if (t != 0 && t <= 16) {
      // Up to 1024 columns: a wavefront per row.
      switch (t) {
#define MI_SM(T) case T: softmax_kernel<T><<<g, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, R, C); break;
        MI_SM(1) MI_SM(2) MI_SM(4) MI_SM(8) MI_SM(16)
#undef MI_SM
      }
    } else if (C <= 16384) {
      // A block per row: the smallest VPT with 1024 * VPT >= C.
      int vpt = 1;
      while (1024 * vpt < C) vpt *= 2;
      const unsigned rows = static_cast<unsigned>(R);
      // Stream rows the size of the last-level cache and beyond.
      const bool nt = vec && R * C * 8 >= kStreamBytes;
      if (xe == MI_F32 && C == 1024 * vpt && vpt >= 2 && vpt <= 8 && !mp && out_elem == MI_F32) {
        // Unmasked F32 rows of 2048, 4096, 8192: the same folds at any size.
        const float *xf = static_cast<const float *>(xp);
        float *of = static_cast<float *>(ob->ptr);
        switch (vpt * 4 + (log ? 2 : 0) + (nt ? 1 : 0)) {
#define MI_SL(V) case 4 * V: softmax_row_kernel<2, 0, 128 * V, false><<<rows, 128 * V, 0, ctx->stream>>>(xf, scale, of); break; \
                 case 4 * V + 1: softmax_row_kernel<2, 0, 128 * V, true><<<rows, 128 * V, 0, ctx->stream>>>(xf, scale, of); break; \
                 case 4 * V + 2: softmax_row_kernel<2, 1, 128 * V, false><<<rows, 128 * V, 0, ctx->stream>>>(xf, scale, of); break; \
                 case 4 * V + 3: softmax_row_kernel<2, 1, 128 * V, true><<<rows, 128 * V, 0, ctx->stream>>>(xf, scale, of); break;
          MI_SL(2) MI_SL(4) MI_SL(8)
#undef MI_SL
        }
      } else
      switch (vpt) {
#define MI_SB(V) case V: if (nt && C == 1024 * V && log) softmax_block_kernel<V, true, true, true, 1><<<rows, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, C); \
                         else if (nt && C == 1024 * V) softmax_block_kernel<V, true, true, true, 0><<<rows, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, C); \
                         else if (nt) softmax_block_kernel<V, true, true><<<rows, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, C); \
                         else if (vec) softmax_block_kernel<V, true, false><<<rows, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, C); \
                         else softmax_block_kernel<V, false, false><<<rows, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, C); break;
        MI_SB(1) MI_SB(2) MI_SB(4) MI_SB(8) MI_SB(16)
#undef MI_SB
      }
    } else {
      softmax_long_kernel<<<g, 256, 0, ctx->stream>>>(xp, xe, mp, mrows, scale, log, ob->ptr, out_elem, R, C);
    }
  }
  s = check_launch(ctx, "softmax_rows");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

namespace mi {
void rms_norm_launch(Ctx *ctx, const void *xp, int xe, const void *gp, int ge, float eps, void *out, int out_elem,
                     int64_t R, int64_t C) {
  // One wavefront a row; below 4096 rows one a block, so the rows spread
  // over every CU (a 512-row prompt's norms: 128 blocks of four rows left
  // half the chip idle).
  const int per = R < 4096 ? 1 : 4;
  const unsigned g = grid_for(R, per, INT32_MAX);
  const int t = pick_t(C);
  const int form = out_elem == MI_F32 ? 0 : out_elem == MI_BF16 ? 1 : out_elem == MI_BF16_PARTS ? 2
                 : out_elem == MI_TILES_BF16 ? 3 : out_elem == MI_TILES_PARTS ? 4 : -1;
  if (xe == MI_F32 && (gp == nullptr || ge == MI_F32) && t >= 1 && t <= 16 && form >= 0) {
    switch (t * 8 + form) {
#define MI_RN(T)                                                                                                  \
  case 8 * T: rms_norm_kernel<T, true, MI_F32><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break; \
  case 8 * T + 1: rms_norm_kernel<T, true, MI_BF16><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break; \
  case 8 * T + 2: rms_norm_kernel<T, true, MI_BF16_PARTS><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break; \
  case 8 * T + 3: rms_norm_kernel<T, true, MI_TILES_BF16><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break; \
  case 8 * T + 4: rms_norm_kernel<T, true, MI_TILES_PARTS><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break;
      MI_RN(1) MI_RN(2) MI_RN(4) MI_RN(8) MI_RN(16)
#undef MI_RN
    }
    return;
  }
  switch (t) {
#define MI_RN(T) case T: rms_norm_kernel<T><<<g, 64 * per, 0, ctx->stream>>>(xp, xe, gp, ge, eps, out, out_elem, R, C); break;
    MI_RN(1) MI_RN(2) MI_RN(4) MI_RN(8) MI_RN(16) MI_RN(32) MI_RN(64) MI_RN(128)
#undef MI_RN
  }
}
}  // namespace mi

extern "C" int mi_rms_norm(mi_ctx *ctx, mi_id a, mi_id gamma, float eps, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, a);
  if (!elem_float(xb->elem) || xb->tiles)
    return fail(ctx, MI_E_ARG, "rms_norm of a %s buffer%s", elem_name(xb->elem), xb->tiles ? " in tiles" : "");
  if (out_elem != MI_F32 && out_elem != MI_BF16 && out_elem != MI_BF16_PARTS && out_elem != MI_TILES_BF16 &&
      out_elem != MI_TILES_PARTS)
    return fail(ctx, MI_E_ARG, "rms_norm result kind %d", out_elem);
  const bool tiled = out_elem == MI_TILES_BF16 || out_elem == MI_TILES_PARTS;
  if (tiled && (xb->rows % 32 || xb->cols % 16))
    return fail(ctx, MI_E_ARG, "rms_norm: tiles of [%lld, %lld] (rows a multiple of 32, columns of 16)",
                (long long)xb->rows, (long long)xb->cols);
  const void *gp = nullptr;
  int ge = MI_F32;
  if (gamma) {
    MI_BUF(ctx, gb, gamma);
    if (!elem_float(gb->elem) || gb->numel() != xb->cols) return fail(ctx, MI_E_ARG, "rms_norm gamma must be [1, %lld] float", (long long)xb->cols);
    gp = gb->ptr; ge = gb->elem;
  }
  const int64_t R = xb->rows, C = xb->cols;
  int t = pick_t(C);
  if (t == 0) return fail(ctx, MI_E_UNSUPPORTED, "rms_norm rows longer than 8192");
  const void *xp = xb->ptr;
  const int xe = xb->elem;
  mi_id id; Buffer *ob;
  const bool parts = out_elem == MI_BF16_PARTS || out_elem == MI_TILES_PARTS;
  int s = new_buffer(ctx, R, parts ? 2 * C : C, parts || tiled ? MI_BF16 : out_elem, &id, &ob);
  if (s) return s;
  ob->tiles = tiled ? out_elem : 0;
  if (R > 0 && C > 0) rms_norm_launch(ctx, xp, xe, gp, ge, eps, ob->ptr, out_elem, R, C);
  s = check_launch(ctx, "rms_norm");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

extern "C" int mi_layer_norm(mi_ctx *ctx, mi_id a, mi_id gamma, mi_id beta, float eps, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, a);
  if (xb->elem != MI_F32) return fail(ctx, MI_E_ARG, "layer_norm of a %s buffer", elem_name(xb->elem));
  const float *gp = nullptr, *bp = nullptr;
  if (gamma) {
    MI_BUF(ctx, gb, gamma);
    if (gb->elem != MI_F32 || gb->numel() != xb->cols) return fail(ctx, MI_E_ARG, "layer_norm gamma must be [1, %lld] F32", (long long)xb->cols);
    gp = static_cast<const float *>(gb->ptr);
  }
  if (beta) {
    MI_BUF(ctx, bb, beta);
    if (bb->elem != MI_F32 || bb->numel() != xb->cols) return fail(ctx, MI_E_ARG, "layer_norm beta must be [1, %lld] F32", (long long)xb->cols);
    bp = static_cast<const float *>(bb->ptr);
  }
  const int64_t R = xb->rows, C = xb->cols;
  int t = pick_t(C);
  if (t == 0) return fail(ctx, MI_E_UNSUPPORTED, "layer_norm rows longer than 8192");
  const float *xp = static_cast<const float *>(xb->ptr);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, C, MI_F32, &id, &ob);
  if (s) return s;
  if (R > 0 && C > 0) {
    unsigned g = grid_for(R, 4, INT32_MAX);
    float *o = static_cast<float *>(ob->ptr);
    switch (t) {
#define MI_LN(T) case T: layer_norm_kernel<T><<<g, 256, 0, ctx->stream>>>(xp, gp, bp, eps, o, R, C); break;
      MI_LN(1) MI_LN(2) MI_LN(4) MI_LN(8) MI_LN(16) MI_LN(32) MI_LN(64) MI_LN(128)
#undef MI_LN
    }
  }
  s = check_launch(ctx, "layer_norm");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

namespace mi {

// ------------------------------------------------------------ backward rows
// LayerNorm's backward, fused (Burn's autodiff composes it from the forward's
// primitive ops -- mean, subtract, square, mean, sqrt, divide, scale, shift):
// with xh = (x - mean) / den, den = sqrt(var + eps) and g = dy * gamma,
//   dx = (g - mean(g) - xh * mean(g * xh)) / den   (+ an incoming residual
//   gradient, added in the same pass),
//   dgamma = sum over rows of dy * xh,  dbeta = sum over rows of dy.
// One wavefront per row with the row in registers (T columns per lane);
// each block of 4 waves takes LNB_ROWS rows and writes its column partials
// of dgamma and dbeta; a second pass folds the blocks' partials.
// Rows a block of four wavefronts takes: one each, so a [2048, 256] gradient
// spreads over 512 blocks with one load round trip a wavefront (16 rows, four
// dependent ones a wavefront on 128 blocks: transformer step 1.87 -> 1.81 ms).
constexpr int LNB_ROWS = 4;

template <int T>
__global__ void __launch_bounds__(256) layer_norm_backward_kernel(const float *x, const float *gamma, const float *dy,
                                                                  const float *dres, float eps, float *dx,
                                                                  float *part, int64_t rows, int64_t cols) {
  __shared__ float red[4][2][64 * T];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float pg[T], pb[T];
#pragma unroll
  for (int t = 0; t < T; ++t) pg[t] = pb[t] = 0.0f;
  for (int r = wave; r < LNB_ROWS; r += 4) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * LNB_ROWS + r;
    if (row >= rows) break;
    const int64_t base = row * cols;
    float v[T], g[T], d[T];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = lane + 64 * t;
      v[t] = j < cols ? x[base + j] : 0.0f;
      d[t] = j < cols ? dy[base + j] : 0.0f;
      g[t] = j < cols ? d[t] * (gamma ? gamma[j] : 1.0f) : 0.0f;
      s += v[t];
    }
    const float inv_n = 1.0f / static_cast<float>(cols);
    const float mean = wave_sum(s) / static_cast<float>(cols);
    float q = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = lane + 64 * t;
      const float c = j < cols ? v[t] - mean : 0.0f;
      q += c * c;
    }
    const float den = __fsqrt_rn(wave_sum(q) / static_cast<float>(cols) + eps);
    float sg = 0.0f, sgx = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      v[t] = (v[t] - mean) / den;  // xh
      sg += g[t];
      sgx += g[t] * v[t];
    }
    const float mg = wave_sum(sg) * inv_n, mgx = wave_sum(sgx) * inv_n;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t j = lane + 64 * t;
      if (j < cols) {
        float o = (g[t] - mg - v[t] * mgx) / den;
        if (dres) o = o + dres[base + j];
        dx[base + j] = o;
        pg[t] += d[t] * v[t];
        pb[t] += d[t];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    red[wave][0][lane + 64 * t] = pg[t];
    red[wave][1][lane + 64 * t] = pb[t];
  }
  __syncthreads();
  float *pp = part + static_cast<int64_t>(blockIdx.x) * 2 * cols;
  for (int64_t j = threadIdx.x; j < 2 * cols; j += 256) {
    const int w = j < cols ? 0 : 1;
    const int64_t c = j < cols ? j : j - cols;
    pp[j] = ((red[0][w][c] + red[1][w][c]) + red[2][w][c]) + red[3][w][c];
  }
}

// Softmax's backward over rows (Burn composes it from the forward's ops):
// ds = scale * p * (dp - sum_row(p * dp)).  One wavefront per row; the row
// is read twice, the second time from cache.
__global__ void __launch_bounds__(256) softmax_backward_kernel(const float *p, const float *dp, float scale, float *ds,
                                                               int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float s = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) s += p[base + j] * dp[base + j];
  s = wave_sum(s);
  for (int64_t j = lane; j < cols; j += 64) ds[base + j] = scale * (p[base + j] * (dp[base + j] - s));
}

}  // namespace mi

using namespace mi;

extern "C" int mi_layer_norm_backward(mi_ctx *ctx, mi_id x, mi_id gamma, mi_id dy, mi_id residual_grad, float eps,
                                      mi_id *dx, mi_id *dgamma, mi_id *dbeta) {
  MI_ENTER(ctx);
  if (!dx || !dgamma || !dbeta) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, db, dy);
  const Buffer *gb = nullptr, *rb = nullptr;
  if (gamma) { gb = lookup(ctx, gamma); if (!gb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)gamma); }
  if (residual_grad) {
    rb = lookup(ctx, residual_grad);
    if (!rb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)residual_grad);
  }
  const int64_t R = xb->rows, C = xb->cols;
  if (xb->elem != MI_F32 || db->elem != MI_F32 || db->rows != R || db->cols != C)
    return fail(ctx, MI_E_ARG, "layer_norm_backward: x and dy must be F32 of one shape");
  if (gb && (gb->elem != MI_F32 || gb->rows * gb->cols != C)) return fail(ctx, MI_E_ARG, "layer_norm_backward: gamma");
  if (rb && (rb->elem != MI_F32 || rb->rows != R || rb->cols != C))
    return fail(ctx, MI_E_ARG, "layer_norm_backward: residual gradient shape");
  const int t = pick_t(C);
  if (t == 0 || t > 16) return fail(ctx, MI_E_UNSUPPORTED, "layer_norm_backward: %lld columns (at most 1024)", (long long)C);
  const int64_t nb = (R + LNB_ROWS - 1) / LNB_ROWS;
  if (nb > INT32_MAX) return fail(ctx, MI_E_UNSUPPORTED, "layer_norm_backward: too many rows");
  float *part = nullptr;
  if (R > 0) {
    part = static_cast<float *>(scratch(ctx, static_cast<size_t>(nb * 2 * C) * sizeof(float)));
    if (!part) return fail(ctx, MI_E_OOM, "layer_norm_backward scratch");
  }
  mi_id ids[3];
  Buffer *bx, *bg, *bb;
  int s = new_buffer(ctx, R, C, MI_F32, &ids[0], &bx);
  if (s) return s;
  s = new_buffer(ctx, 1, C, MI_F32, &ids[1], &bg);
  if (s) { mi_free(ctx, ids[0]); return s; }
  s = new_buffer(ctx, 1, C, MI_F32, &ids[2], &bb);
  if (s) { mi_free(ctx, ids[0]); mi_free(ctx, ids[1]); return s; }
  if (R == 0) {
    fill_zero(ctx, bg->ptr, C * sizeof(float));
    fill_zero(ctx, bb->ptr, C * sizeof(float));
  } else {
    const float *xp = static_cast<const float *>(xb->ptr), *dp = static_cast<const float *>(db->ptr);
    const float *gp = gb ? static_cast<const float *>(gb->ptr) : nullptr;
    const float *rp = rb ? static_cast<const float *>(rb->ptr) : nullptr;
    float *o = static_cast<float *>(bx->ptr);
    const unsigned g = static_cast<unsigned>(nb);
    switch (t) {
#define MI_LNB(T) case T: layer_norm_backward_kernel<T><<<g, 256, 0, ctx->stream>>>(xp, gp, dp, rp, eps, o, part, R, C); break;
      MI_LNB(1) MI_LNB(2) MI_LNB(4) MI_LNB(8) MI_LNB(16)
#undef MI_LNB
    }
    fold_partials_kernel<<<static_cast<unsigned>((2 * C + 31) / 32), 512, 0, ctx->stream>>>(
        part, nb, 2 * C, MI_R_SUM, 1.0f, static_cast<float *>(bg->ptr), C, static_cast<float *>(bb->ptr));
  }
  s = check_launch(ctx, "layer_norm_backward");
  if (s) { for (mi_id i : ids) mi_free(ctx, i); return s; }
  *dx = ids[0]; *dgamma = ids[1]; *dbeta = ids[2];
  return MI_OK;
}

extern "C" int mi_log_softmax_ce(mi_ctx *ctx, mi_id logits, mi_id targets, float grad_scale, mi_id *picked,
                                 mi_id *dlogits) {
  MI_ENTER(ctx);
  if (!picked || !dlogits) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, zb, logits);
  MI_BUF(ctx, tb, targets);
  if (zb->elem != MI_F32) return fail(ctx, MI_E_ARG, "log_softmax_ce of a %s buffer", elem_name(zb->elem));
  const int64_t R = zb->rows, C = zb->cols;
  if (tb->elem != MI_I32 || tb->numel() != R)
    return fail(ctx, MI_E_ARG, "log_softmax_ce: targets must be %lld I32 values", (long long)R);
  if (C < 1 || C > 16384)
    return fail(ctx, MI_E_UNSUPPORTED, "log_softmax_ce: rows of %lld logits (1 to 16384)", (long long)C);
  mi_id pid, did;
  Buffer *pb, *db;
  int s = new_buffer(ctx, R, 1, MI_F32, &pid, &pb);
  if (s) return s;
  s = new_buffer(ctx, R, C, MI_F32, &did, &db);
  if (s) { mi_free(ctx, pid); return s; }
  const float *zp = static_cast<const float *>(zb->ptr);
  const int32_t *tp = static_cast<const int32_t *>(tb->ptr);
  float *pp = static_cast<float *>(pb->ptr), *dp = static_cast<float *>(db->ptr);
  if (R > 0 && C <= 1024) {
    // The row lengths the log-softmax runs a wavefront per row on.
    const unsigned g = grid_for(R, 4, INT32_MAX);
    switch (pick_t(C)) {
#define MI_CEW(T) case T: log_softmax_ce_wave_kernel<T><<<g, 256, 0, ctx->stream>>>(zp, tp, R, C, grad_scale, pp, dp, flags(ctx)); break;
      MI_CEW(1) MI_CEW(2) MI_CEW(4) MI_CEW(8) MI_CEW(16)
#undef MI_CEW
    }
    s = check_launch(ctx, "log_softmax_ce");
    if (s) { mi_free(ctx, pid); mi_free(ctx, did); return s; }
  } else if (R > 0) {
    int vpt = 1;
    while (1024 * vpt < C) vpt *= 2;
    const bool vec = C % 4 == 0;
    const bool nt = vec && R * C * 8 >= kStreamBytes;
    const unsigned g = static_cast<unsigned>(R);
    // Rows of 2048, 4096 or 8192: the layout of softmax_row_kernel.
    if (C == 1024 * vpt && vpt >= 2 && vpt <= 8) {
      switch (vpt * 2 + (nt ? 1 : 0)) {
#define MI_CER(V) case 2 * V: log_softmax_ce_kernel<2, true, false, 128 * V><<<g, 128 * V, 0, ctx->stream>>>(zp, tp, C, grad_scale, pp, dp, flags(ctx)); break; \
                  case 2 * V + 1: log_softmax_ce_kernel<2, true, true, 128 * V><<<g, 128 * V, 0, ctx->stream>>>(zp, tp, C, grad_scale, pp, dp, flags(ctx)); break;
        MI_CER(2) MI_CER(4) MI_CER(8)
#undef MI_CER
      }
    } else
    switch (vpt) {
#define MI_CE(V) case V: if (nt) log_softmax_ce_kernel<V, true, true><<<g, 256, 0, ctx->stream>>>(zp, tp, C, grad_scale, pp, dp, flags(ctx)); \
                         else if (vec) log_softmax_ce_kernel<V, true, false><<<g, 256, 0, ctx->stream>>>(zp, tp, C, grad_scale, pp, dp, flags(ctx)); \
                         else log_softmax_ce_kernel<V, false, false><<<g, 256, 0, ctx->stream>>>(zp, tp, C, grad_scale, pp, dp, flags(ctx)); break;
      MI_CE(1) MI_CE(2) MI_CE(4) MI_CE(8) MI_CE(16)
#undef MI_CE
    }
    s = check_launch(ctx, "log_softmax_ce");
    if (s) { mi_free(ctx, pid); mi_free(ctx, did); return s; }
  }
  *picked = pid;
  *dlogits = did;
  return MI_OK;
}

extern "C" int mi_softmax_backward(mi_ctx *ctx, mi_id p, mi_id dp, float scale, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, pb, p);
  MI_BUF(ctx, db, dp);
  if (pb->elem != MI_F32 || db->elem != MI_F32 || pb->rows != db->rows || pb->cols != db->cols)
    return fail(ctx, MI_E_ARG, "softmax_backward: p and dp must be F32 of one shape");
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, pb->rows, pb->cols, MI_F32, &id, &ob);
  if (s) return s;
  if (pb->rows > 0 && pb->cols > 0)
    softmax_backward_kernel<<<grid_for(pb->rows, 4, INT32_MAX), 256, 0, ctx->stream>>>(
        static_cast<const float *>(pb->ptr), static_cast<const float *>(db->ptr), scale, static_cast<float *>(ob->ptr),
        pb->rows, pb->cols);
  s = check_launch(ctx, "softmax_backward");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}
