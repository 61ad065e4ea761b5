// Indexing: row select (embedding), column pick (cross-entropy gather) and
// its scatter-add backward, row select-add (embedding backward), row argmax.
//
// Reference: Engine::select_rows / pick_columns / select_add_rows / argmax_row
// (crates/burn-tt/src/server.rs:300, 349, 358, 477); their routing
// `select_rows_native`, `pick_columns_native`, `scatter_add_columns_native`
// (crates/burn-tt/src/ops.rs:1001-1240); duplicates folded in index order
// (crates/burn-tt/src/ops/index.rs:27-30); argmax's first maximum with NaN
// above every number (crates/tt-models/src/generate.rs:176-183,
// crates/burn-tt/src/ops.rs:2389-2490).
//
// Every copy here moves raw bits, so results are bit-exact.  An index outside
// its range sets the context's device flag (reported as MI_E_DOMAIN at the
// next wait) and the element is written as zero bits, never read out of
// bounds.
#include <utility>

#include "common.hpp"


namespace mi {

// ---------------------------------------------------------- select_rows
// A block of 256 threads copies rows: each wave one output row per step,
// 16-byte lanes when the row width allows.
template <typename V, bool NT>
__global__ void __launch_bounds__(256) select_rows_kernel(const V *table, int64_t vrows, int64_t vcols,
                                                          const int32_t *idx, int64_t n, V *out,
                                                          uint32_t *flags) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t waves = (static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6;
  for (int64_t i = wave; i < n; i += waves) {
    const int32_t r = idx[i];
    V *dst = out + i * vcols;
    if (r < 0 || r >= vrows) {
      if (lane == 0) atomicOr(flags, FLAG_INDEX_RANGE);
      for (int64_t j = lane; j < vcols; j += 64) dst[j] = V{};
      continue;
    }
    const V *src = table + static_cast<int64_t>(r) * vcols;
    // Up to four loads per lane in flight before the stores.
    for (int64_t j0 = lane; j0 < vcols; j0 += 256) {
      V v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (j0 + 64 * u < vcols) v[u] = src[j0 + 64 * u];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (j0 + 64 * u < vcols) {
          if constexpr (NT && sizeof(V) == 16) stu4<true>(dst + j0 + 64 * u, v[u]);
          else dst[j0 + 64 * u] = v[u];
        }
      }
    }
  }
}

// ---------------------------------------------------------- pick_columns
__global__ void pick_columns_kernel(const uint32_t *x, int64_t rows, int64_t cols, const int32_t *idx,
                                    uint32_t *out, uint32_t *flags) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int32_t c = idx[r];
  if (c < 0 || c >= cols) { atomicOr(flags, FLAG_INDEX_RANGE); out[r] = 0; return; }
  out[r] = x[r * cols + c];
}

__global__ void scatter_add_columns_kernel(float *out, int64_t rows, int64_t cols, const int32_t *idx,
                                           const float *v, uint32_t *flags) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int32_t c = idx[r];
  if (c < 0 || c >= cols) { atomicOr(flags, FLAG_INDEX_RANGE); return; }
  out[r * cols + c] = out[r * cols + c] + v[r];
}

// ------------------------------------------------------- select_add_rows
// After a stable sort of (index, position) pairs, each run of one index is a
// segment; one wave per segment start adds the segment's value rows into the
// destination row in position order, so duplicates fold in index order.
__global__ void iota_kernel(int32_t *p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = static_cast<int32_t>(i);
}

__global__ void __launch_bounds__(256) select_add_segments(float *out, int64_t vrows, int64_t cols,
                                                           const int32_t *keys, const int32_t *pos, int64_t n,
                                                           const float *value, uint32_t *flags) {
  const int lane = threadIdx.x & 63;
  const int64_t p = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (p >= n) return;
  const int32_t key = keys[p];
  if (p > 0 && keys[p - 1] == key) return;  // not a segment start
  if (key < 0 || key >= vrows) {
    if (lane == 0) atomicOr(flags, FLAG_INDEX_RANGE);
    return;
  }
  int64_t end = p + 1;
  while (end < n && keys[end] == key) ++end;
  float *dst = out + static_cast<int64_t>(key) * cols;
  for (int64_t j = lane; j < cols; j += 64) {
    float acc = dst[j];
    for (int64_t q = p; q < end; ++q) acc = acc + value[static_cast<int64_t>(pos[q]) * cols + j];
    dst[j] = acc;
  }
}

// Up to SORT_BLOCK_MAX indices: one block sorts the (index, position) pairs
// in LDS with a bitonic network -- as 64-bit keys (index bits above position
// bits), so equal indices keep position order and negative (invalid) indices
// group above every valid one.  No library sort and no memset: the path a
// captured trace can hold.
constexpr int SORT_BLOCK_MAX = 8192;

__global__ void __launch_bounds__(1024) sort_pairs_block(const int32_t *idx, int64_t n, int32_t *keys_out,
                                                         int32_t *pos_out) {
  __shared__ uint64_t k[SORT_BLOCK_MAX];
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = threadIdx.x; i < np; i += 1024)
    k[i] = i < n ? (static_cast<uint64_t>(static_cast<uint32_t>(idx[i])) << 32) | static_cast<uint32_t>(i) : ~0ull;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < np / 2; t += 1024) {
        const int lo = 2 * t - (t & (stride - 1));  // first element of the pair
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = k[lo], b = k[hi];
        if ((a > b) == up) {
          k[lo] = b;
          k[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < n; i += 1024) {
    keys_out[i] = static_cast<int32_t>(k[i] >> 32);
    pos_out[i] = static_cast<int32_t>(k[i] & 0xffffffffu);
  }
}

// More indices: each block sorts a chunk of SORT_BLOCK_MAX keys in LDS with
// the same network, then merge passes double the sorted runs.  The keys are
// unique (the position is part of each), so an element's place in the merged
// run is its place in its own run plus the number of the other run's keys
// below it (a binary search): no ties, no atomics, one order.
__global__ void __launch_bounds__(1024) sort_keys_chunks(const int32_t *idx, int64_t n, uint64_t *out) {
  __shared__ uint64_t k[SORT_BLOCK_MAX];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * SORT_BLOCK_MAX;
  const int64_t m = n - base < SORT_BLOCK_MAX ? n - base : SORT_BLOCK_MAX;
  int np = 1;
  while (np < m) np <<= 1;
  for (int i = threadIdx.x; i < np; i += 1024)
    k[i] = i < m ? (static_cast<uint64_t>(static_cast<uint32_t>(idx[base + i])) << 32) |
                       static_cast<uint32_t>(base + i)
                 : ~0ull;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < np / 2; t += 1024) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = k[lo], b = k[hi];
        if ((a > b) == up) {
          k[lo] = b;
          k[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < m; i += 1024) out[base + i] = k[i];
}

// Keys of [lo, hi) below `key`: a binary search over a sorted run.
__device__ __forceinline__ int64_t keys_below(const uint64_t *k, int64_t lo, int64_t hi, uint64_t key) {
  int64_t a = lo, b = hi;
  while (a < b) {
    const int64_t mid = a + ((b - a) >> 1);
    if (k[mid] < key) a = mid + 1;
    else b = mid;
  }
  return a - lo;
}

// One merge pass: sorted runs of `run` keys pairwise into runs of 2 run.
__global__ void __launch_bounds__(256) merge_runs(const uint64_t *src, uint64_t *dst, int64_t n, int64_t run) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t a0 = i / (2 * run) * (2 * run);
  const int64_t b0 = a0 + run < n ? a0 + run : n, b1 = b0 + run < n ? b0 + run : n;
  const uint64_t key = src[i];
  const int64_t at = i < b0 ? a0 + (i - a0) + keys_below(src, b0, b1, key)
                            : a0 + (i - b0) + keys_below(src, a0, b0, key);
  dst[at] = key;
}

__global__ void __launch_bounds__(256) split_keys(const uint64_t *k, int64_t n, int32_t *keys, int32_t *pos) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  keys[i] = static_cast<int32_t>(k[i] >> 32);
  pos[i] = static_cast<int32_t>(k[i] & 0xffffffffu);
}

// BF16 table rows gathered and widened to F32 (exact) in one pass: a wave a
// row, eight columns a lane per access; an index outside the table raises
// the range flag and gives a zero row, as select_rows_kernel does.
__global__ void __launch_bounds__(256) select_rows_widen_kernel(const uint16_t *table, int64_t vrows, int64_t cols,
                                                                const int32_t *idx, int64_t n, float *out,
                                                                uint32_t *flags) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t waves = (static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6;
  for (int64_t i = wave; i < n; i += waves) {
    const int32_t r = idx[i];
    float *dst = out + i * cols;
    if (r < 0 || r >= vrows) {
      if (lane == 0) atomicOr(flags, FLAG_INDEX_RANGE);
      for (int64_t j = lane; j < cols; j += 64) dst[j] = 0.0f;
      continue;
    }
    const uint16_t *src = table + static_cast<int64_t>(r) * cols;
    for (int64_t j = 8 * lane; j < cols; j += 512) {
      const uint4 u = *reinterpret_cast<const uint4 *>(src + j);
      *reinterpret_cast<float4 *>(dst + j) = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                                                         __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
      *reinterpret_cast<float4 *>(dst + j + 4) = make_float4(__uint_as_float(u.z << 16),
                                                             __uint_as_float(u.z & 0xffff0000u),
                                                             __uint_as_float(u.w << 16),
                                                             __uint_as_float(u.w & 0xffff0000u));
    }
  }
}

// --------------------------------------------------------------- argmax

__global__ void __launch_bounds__(256) argmax_rows_kernel(const void *x, int elem, int64_t rows, int64_t cols,
                                                          int32_t *out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  ArgBest best{-INFINITY, INT32_MAX};
  for (int64_t j = lane; j < cols; j += 64) {
    float v = elem == MI_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(x)[base + j])
                              : static_cast<const float *>(x)[base + j];
    best = better(best, ArgBest{v, static_cast<int32_t>(j)});
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ArgBest other{__shfl_xor(best.v, o, 64), __shfl_xor(best.i, o, 64)};
    best = better(best, other);
  }
  if (lane == 0) out[row] = best.i == INT32_MAX ? 0 : best.i;
}

// Long rows (a vocabulary's logits): blocks of 256 threads over column
// chunks of a row, eight loads per thread in flight, folded by the same
// (value, index) rule -- a total order, so the fold order does not matter.
// One chunk per row writes the index; several write (value, index) partials
// that argmax_fold_kernel folds, one wavefront per row.
__global__ void __launch_bounds__(256) argmax_chunk_kernel(const void *x, int elem, int64_t cols, int64_t ch,
                                                           int32_t *out, float *pv, int32_t *pi) {
  const int64_t row = blockIdx.y, chunk = blockIdx.x, nch = gridDim.x;
  const int64_t lo = chunk * ch, hi = lo + ch < cols ? lo + ch : cols;
  const int64_t base = row * cols;
  ArgBest best{-INFINITY, INT32_MAX};
  for (int64_t j0 = lo + threadIdx.x; j0 < hi; j0 += 256 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t j = j0 + 256 * u;
      v[u] = j < hi ? (elem == MI_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(x)[base + j])
                                       : static_cast<const float *>(x)[base + j])
                    : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t j = j0 + 256 * u;
      if (j < hi) best = better(best, ArgBest{v[u], static_cast<int32_t>(j)});
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ArgBest other{__shfl_xor(best.v, o, 64), __shfl_xor(best.i, o, 64)};
    best = better(best, other);
  }
  __shared__ float rv[4];
  __shared__ int32_t ri[4];
  if ((threadIdx.x & 63) == 0) { rv[threadIdx.x >> 6] = best.v; ri[threadIdx.x >> 6] = best.i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgBest b{rv[0], ri[0]};
    for (int w = 1; w < 4; ++w) b = better(b, ArgBest{rv[w], ri[w]});
    if (nch == 1) {
      out[row] = b.i == INT32_MAX ? 0 : b.i;
    } else {
      pv[row * nch + chunk] = b.v;
      pi[row * nch + chunk] = b.i;
    }
  }
}

__global__ void __launch_bounds__(256) argmax_fold_kernel(const float *pv, const int32_t *pi, int64_t nch,
                                                          int64_t rows, int32_t *out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  ArgBest best{-INFINITY, INT32_MAX};
  for (int64_t c = lane; c < nch; c += 64) best = better(best, ArgBest{pv[row * nch + c], pi[row * nch + c]});
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ArgBest other{__shfl_xor(best.v, o, 64), __shfl_xor(best.i, o, 64)};
    best = better(best, other);
  }
  if (lane == 0) out[row] = best.i == INT32_MAX ? 0 : best.i;
}

}  // namespace mi

using namespace mi;

extern "C" int mi_select_rows(mi_ctx *ctx, mi_id table, mi_id idx, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, t, table);
  MI_BUF(ctx, ix, idx);
  MI_NO_BFP8(ctx, t, "select_rows");
  if (ix->elem != MI_I32) return fail(ctx, MI_E_ARG, "select_rows indices are %s, not I32", elem_name(ix->elem));
  const int64_t n = ix->numel(), V = t->rows, D = t->cols;
  const void *tp = t->ptr;
  const int32_t *ip = static_cast<const int32_t *>(ix->ptr);
  const int te = t->elem;
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, n, D, te, &id, &ob);
  if (s) return s;
  if (n > 0 && D > 0) {
    const size_t row_bytes = static_cast<size_t>(D) * elem_size(te);
    const unsigned g = grid_for(n, 4, 256 * 64);
    // The gathered rows are streamed out when the result outgrows the
    // last-level cache; the table is read through the caches (ids repeat).
    const bool nt = n * row_bytes >= kStreamBytes;
    if (row_bytes % 16 == 0 && nt)
      select_rows_kernel<uint4, true><<<g, 256, 0, ctx->stream>>>(static_cast<const uint4 *>(tp), V, row_bytes / 16, ip,
                                                                  n, static_cast<uint4 *>(ob->ptr), flags(ctx));
    else if (row_bytes % 16 == 0)
      select_rows_kernel<uint4, false><<<g, 256, 0, ctx->stream>>>(static_cast<const uint4 *>(tp), V, row_bytes / 16, ip,
                                                                   n, static_cast<uint4 *>(ob->ptr), flags(ctx));
    else if (row_bytes % 4 == 0)
      select_rows_kernel<uint32_t, false><<<g, 256, 0, ctx->stream>>>(static_cast<const uint32_t *>(tp), V,
                                                                      row_bytes / 4, ip, n,
                                                                      static_cast<uint32_t *>(ob->ptr), flags(ctx));
    else
      select_rows_kernel<uint16_t, false><<<g, 256, 0, ctx->stream>>>(static_cast<const uint16_t *>(tp), V,
                                                                      row_bytes / 2, ip, n,
                                                                      static_cast<uint16_t *>(ob->ptr), flags(ctx));
    s = check_launch(ctx, "select_rows");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_select_rows_as(mi_ctx *ctx, mi_id table, mi_id idx, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, t, table);
  MI_BUF(ctx, ix, idx);
  if (ix->elem != MI_I32) return fail(ctx, MI_E_ARG, "select_rows_as indices are %s, not I32", elem_name(ix->elem));
  if (!elem_float(t->elem) || (out_elem != MI_F32 && out_elem != MI_BF16))
    return fail(ctx, MI_E_ARG, "select_rows_as of a %s table to %d", elem_name(t->elem), out_elem);
  const int64_t n = ix->numel(), D = t->cols;
  if (out_elem == t->elem) return mi_select_rows(ctx, table, idx, out);
  if (t->elem == MI_BF16 && D % 8 == 0 && n > 0) {
    // BF16 rows widened (exactly) as they are gathered: one launch.
    mi_id id; Buffer *ob;
    int s = new_buffer(ctx, n, D, MI_F32, &id, &ob);
    if (s) return s;
    const unsigned g = grid_for(n, 4, 256 * 64);
    select_rows_widen_kernel<<<g, 256, 0, ctx->stream>>>(static_cast<const uint16_t *>(t->ptr), t->rows, D,
                                                          static_cast<const int32_t *>(ix->ptr), n,
                                                          static_cast<float *>(ob->ptr), flags(ctx));
    s = check_launch(ctx, "select_rows_as");
    if (s) { mi_free(ctx, id); return s; }
    *out = id;
    return MI_OK;
  }
  // Any other pair: the gather, then the cast.
  mi_id g;
  int s = mi_select_rows(ctx, table, idx, &g);
  if (s) return s;
  s = mi_cast(ctx, g, out_elem, out);
  mi_free(ctx, g);
  return s;
}

extern "C" int mi_pick_columns(mi_ctx *ctx, mi_id x, mi_id idx, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, ix, idx);
  if (ix->elem != MI_I32) return fail(ctx, MI_E_ARG, "pick_columns indices are %s, not I32", elem_name(ix->elem));
  if (elem_size(xb->elem) != 4) return fail(ctx, MI_E_ARG, "pick_columns of a %s buffer", elem_name(xb->elem));
  if (ix->numel() != xb->rows) return fail(ctx, MI_E_ARG, "pick_columns: %lld indices for %lld rows", (long long)ix->numel(), (long long)xb->rows);
  const int64_t R = xb->rows, C = xb->cols;
  const void *xp = xb->ptr;
  const int32_t *ip = static_cast<const int32_t *>(ix->ptr);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, 1, xb->elem, &id, &ob);
  if (s) return s;
  if (R > 0) {
    pick_columns_kernel<<<grid_for(R, 256, INT32_MAX), 256, 0, ctx->stream>>>(static_cast<const uint32_t *>(xp), R, C, ip,
                                                                            static_cast<uint32_t *>(ob->ptr), flags(ctx));
    s = check_launch(ctx, "pick_columns");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

namespace mi {
// One thread an output element: its coordinates from its flat position in
// the index tensor's dims, the source with the gathered dim replaced.
template <typename T>
__global__ void __launch_bounds__(256) gather_dim_kernel(const T *x, int64_t d1, int64_t d2, int64_t d3, int dim,
                                                         int64_t ddim, const int32_t *idx, int64_t i1, int64_t i2,
                                                         int64_t i3, int64_t n, T *out, uint32_t *flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    int64_t c[4];
    int64_t r = e;
    c[3] = r % i3; r /= i3;
    c[2] = r % i2; r /= i2;
    c[1] = r % i1; r /= i1;
    c[0] = r;
    const int32_t k = idx[e];
    if (k < 0 || k >= ddim) {
      atomicOr(flags, FLAG_INDEX_RANGE);
      out[e] = T(0);
      continue;
    }
    c[dim] = k;
    out[e] = x[((c[0] * d1 + c[1]) * d2 + c[2]) * d3 + c[3]];
  }
}
}  // namespace mi

extern "C" int mi_gather(mi_ctx *ctx, mi_id x, const int64_t dims[4], int dim, mi_id idx, const int64_t idims[4],
                         mi_id *out) {
  MI_ENTER(ctx);
  if (!out || !dims || !idims) return fail(ctx, MI_E_ARG, "null pointer argument");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, ib, idx);
  MI_NO_BFP8(ctx, xb, "gather");
  if (ib->elem != MI_I32) return fail(ctx, MI_E_ARG, "gather indices are %s, not I32", elem_name(ib->elem));
  if (dim < 0 || dim > 3) return fail(ctx, MI_E_ARG, "gather dim %d (0 to 3)", dim);
  int64_t nx = 1, ni = 1;
  for (int d = 0; d < 4; ++d) {
    if (dims[d] < 1 || idims[d] < 0 || (d != dim && idims[d] != dims[d]))
      return fail(ctx, MI_E_ARG, "gather: dims [%lld, %lld, %lld, %lld], index dims [%lld, %lld, %lld, %lld] along %d",
                  (long long)dims[0], (long long)dims[1], (long long)dims[2], (long long)dims[3], (long long)idims[0],
                  (long long)idims[1], (long long)idims[2], (long long)idims[3], dim);
    nx *= dims[d];
    ni *= idims[d];
  }
  if (nx != xb->numel() || ni != ib->numel())
    return fail(ctx, MI_E_ARG, "gather: %lld and %lld elements for dims of %lld and %lld", (long long)xb->numel(),
                (long long)ib->numel(), (long long)nx, (long long)ni);
  if (dims[dim] > INT32_MAX) return fail(ctx, MI_E_ARG, "gather: dim of %lld", (long long)dims[dim]);
  const size_t es = elem_size(xb->elem);
  if (es != 4 && es != 2) return fail(ctx, MI_E_ARG, "gather of a %s buffer", elem_name(xb->elem));
  const int64_t rows = idims[0] * idims[1] * idims[2], cols = idims[3];
  const void *xp = xb->ptr;
  const int32_t *ip = static_cast<const int32_t *>(ib->ptr);
  mi_id id;
  Buffer *ob;
  int s = new_buffer(ctx, rows, cols, xb->elem, &id, &ob);
  if (s) return s;
  if (ni > 0) {
    const unsigned g = grid_for(ni, 256, 256 * 64);
    if (es == 4)
      gather_dim_kernel<uint32_t><<<g, 256, 0, ctx->stream>>>(static_cast<const uint32_t *>(xp), dims[1], dims[2], dims[3],
                                                               dim, dims[dim], ip, idims[1], idims[2], idims[3], ni,
                                                               static_cast<uint32_t *>(ob->ptr), flags(ctx));
    else
      gather_dim_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>(static_cast<const uint16_t *>(xp), dims[1], dims[2], dims[3],
                                                               dim, dims[dim], ip, idims[1], idims[2], idims[3], ni,
                                                               static_cast<uint16_t *>(ob->ptr), flags(ctx));
    s = check_launch(ctx, "gather");
    if (s) {
      mi_free(ctx, id);
      return s;
    }
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_scatter_add_columns(mi_ctx *ctx, mi_id x, mi_id idx, mi_id v, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, ix, idx);
  MI_BUF(ctx, vb, v);
  if (xb->elem != MI_F32 || vb->elem != MI_F32) return fail(ctx, MI_E_ARG, "scatter_add_columns takes F32 values");
  if (ix->elem != MI_I32) return fail(ctx, MI_E_ARG, "scatter_add_columns indices are %s, not I32", elem_name(ix->elem));
  if (ix->numel() != xb->rows || vb->numel() != xb->rows)
    return fail(ctx, MI_E_ARG, "scatter_add_columns: %lld indices, %lld values for %lld rows", (long long)ix->numel(),
                (long long)vb->numel(), (long long)xb->rows);
  const int64_t R = xb->rows, C = xb->cols;
  const void *xp = xb->ptr;
  const int32_t *ip = static_cast<const int32_t *>(ix->ptr);
  const float *vp = static_cast<const float *>(vb->ptr);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, C, MI_F32, &id, &ob);
  if (s) return s;
  if (R * C > 0) {
    (void)hipMemcpyAsync(ob->ptr, xp, R * C * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
    scatter_add_columns_kernel<<<grid_for(R, 256, INT32_MAX), 256, 0, ctx->stream>>>(static_cast<float *>(ob->ptr), R, C, ip,
                                                                                   vp, flags(ctx));
    s = check_launch(ctx, "scatter_add_columns");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_select_add_rows(mi_ctx *ctx, mi_id t, mi_id idx, mi_id value, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, tb, t);
  MI_BUF(ctx, ix, idx);
  MI_BUF(ctx, vb, value);
  if (tb->elem != MI_F32 || vb->elem != MI_F32) return fail(ctx, MI_E_ARG, "select_add_rows takes F32 values");
  if (ix->elem != MI_I32) return fail(ctx, MI_E_ARG, "select_add_rows indices are %s, not I32", elem_name(ix->elem));
  const int64_t n = ix->numel(), V = tb->rows, D = tb->cols;
  if (vb->rows != n || vb->cols != D)
    return fail(ctx, MI_E_ARG, "select_add_rows: value [%lld, %lld] for %lld indices of width %lld", (long long)vb->rows,
                (long long)vb->cols, (long long)n, (long long)D);
  if (n > INT32_MAX) return fail(ctx, MI_E_ARG, "select_add_rows: too many indices");
  const void *tp = tb->ptr;
  const int32_t *ip = static_cast<const int32_t *>(ix->ptr);
  const float *vp = static_cast<const float *>(vb->ptr);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, V, D, MI_F32, &id, &ob);
  if (s) return s;
  if (V * D > 0) (void)hipMemcpyAsync(ob->ptr, tp, V * D * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
  if (n > 0 && D > 0 && n <= SORT_BLOCK_MAX) {
    const size_t arr = (static_cast<size_t>(n) * 4 + 255) & ~size_t(255);
    char *sc = static_cast<char *>(scratch(ctx, 2 * arr));
    if (!sc) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "select_add_rows scratch"); }
    int32_t *keys_out = reinterpret_cast<int32_t *>(sc);
    int32_t *pos_out = reinterpret_cast<int32_t *>(sc + arr);
    sort_pairs_block<<<1, 1024, 0, ctx->stream>>>(ip, n, keys_out, pos_out);
    select_add_segments<<<grid_for(n, 4, INT32_MAX), 256, 0, ctx->stream>>>(static_cast<float *>(ob->ptr), V, D, keys_out,
                                                                           pos_out, n, vp, flags(ctx));
  } else if (n > 0 && D > 0) {
    const size_t arr = (static_cast<size_t>(n) * 4 + 255) & ~size_t(255);
    const size_t arr8 = (static_cast<size_t>(n) * 8 + 255) & ~size_t(255);
    char *sc = static_cast<char *>(scratch(ctx, 2 * arr + 2 * arr8));
    if (!sc) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "select_add_rows scratch"); }
    int32_t *keys_out = reinterpret_cast<int32_t *>(sc);
    int32_t *pos_out = reinterpret_cast<int32_t *>(sc + arr);
    uint64_t *ka = reinterpret_cast<uint64_t *>(sc + 2 * arr), *kb = reinterpret_cast<uint64_t *>(sc + 2 * arr + arr8);
    sort_keys_chunks<<<static_cast<unsigned>((n + SORT_BLOCK_MAX - 1) / SORT_BLOCK_MAX), 1024, 0, ctx->stream>>>(ip, n,
                                                                                                                ka);
    const unsigned g = grid_for(n, 256, INT32_MAX);
    for (int64_t run = SORT_BLOCK_MAX; run < n; run *= 2) {
      merge_runs<<<g, 256, 0, ctx->stream>>>(ka, kb, n, run);
      std::swap(ka, kb);
    }
    split_keys<<<g, 256, 0, ctx->stream>>>(ka, n, keys_out, pos_out);
    select_add_segments<<<grid_for(n, 4, INT32_MAX), 256, 0, ctx->stream>>>(static_cast<float *>(ob->ptr), V, D, keys_out,
                                                                           pos_out, n, vp, flags(ctx));
  }
  s = check_launch(ctx, "select_add_rows");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

namespace mi {
// One block: every thread reads the position before thread 0 advances it.
__global__ void __launch_bounds__(1024) decode_advance_kernel(const int32_t *next, int32_t *ids, int32_t *pos,
                                                                int32_t *log, int64_t B, int64_t cols,
                                                                uint32_t *flags) {
  const int32_t p = *pos;
  const bool ok = p >= 0 && static_cast<int64_t>(p) + 1 < cols;
  for (int64_t b = threadIdx.x; b < B; b += blockDim.x) {
    const int32_t v = next[b];
    ids[b] = v;
    if (ok) log[b * cols + p + 1] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (ok) *pos = p + 1;
    else atomicOr(flags, FLAG_INDEX_RANGE);
  }
}
}  // namespace mi

extern "C" int mi_decode_advance(mi_ctx *ctx, mi_id next, mi_id ids, mi_id pos, mi_id log) {
  MI_ENTER(ctx);
  MI_BUF(ctx, nb, next);
  MI_BUF(ctx, ib, ids);
  MI_BUF(ctx, pb, pos);
  MI_BUF(ctx, lb, log);
  const int64_t B = nb->numel();
  if (nb->elem != MI_I32 || ib->elem != MI_I32 || lb->elem != MI_I32 || pb->elem != MI_I32 || pb->numel() != 1 ||
      ib->numel() != B || lb->rows != B || B < 1)
    return fail(ctx, MI_E_ARG, "decode_advance: next [%lld] %s, ids [%lld] %s, position %s [%lld], log %s [%lld, %lld]; "
                "want I32 with ids and log rows matching next and one position", (long long)B, elem_name(nb->elem),
                (long long)ib->numel(), elem_name(ib->elem), elem_name(pb->elem), (long long)pb->numel(),
                elem_name(lb->elem), (long long)lb->rows, (long long)lb->cols);
  decode_advance_kernel<<<1, 256, 0, ctx->stream>>>(static_cast<const int32_t *>(nb->ptr), static_cast<int32_t *>(ib->ptr),
                                                    static_cast<int32_t *>(pb->ptr), static_cast<int32_t *>(lb->ptr), B,
                                                    lb->cols, flags(ctx));
  return check_launch(ctx, "decode_advance");
}

extern "C" int mi_argmax_rows(mi_ctx *ctx, mi_id a, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, a);
  if (!elem_float(xb->elem)) return fail(ctx, MI_E_ARG, "argmax of a %s buffer", elem_name(xb->elem));
  if (xb->cols == 0) return fail(ctx, MI_E_ARG, "argmax of an empty row");
  if (xb->cols > (int64_t(1) << 31) - 1) return fail(ctx, MI_E_ARG, "argmax row too long");
  const int64_t R = xb->rows, C = xb->cols;
  const void *xp = xb->ptr;
  const int xe = xb->elem;
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R, 1, MI_I32, &id, &ob);
  if (s) return s;
  if (R > 0) {
    if (C > 2048 && R <= 65535) {
      // Chunks of at least 2048 columns, enough of them for ~256 blocks.
      int64_t nch = (256 + R - 1) / R;
      const int64_t cap = (C + 2047) / 2048;
      if (nch > cap) nch = cap;
      const int64_t ch = (C + nch - 1) / nch;
      nch = (C + ch - 1) / ch;
      float *pv = nullptr;
      int32_t *pi = nullptr;
      if (nch > 1) {
        char *sc = static_cast<char *>(scratch(ctx, static_cast<size_t>(R * nch) * 8));
        if (!sc) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "argmax scratch"); }
        pv = reinterpret_cast<float *>(sc);
        pi = reinterpret_cast<int32_t *>(sc + static_cast<size_t>(R * nch) * 4);
      }
      int32_t *o = static_cast<int32_t *>(ob->ptr);
      argmax_chunk_kernel<<<dim3(static_cast<unsigned>(nch), static_cast<unsigned>(R)), 256, 0, ctx->stream>>>(
          xp, xe, C, ch, o, pv, pi);
      if (nch > 1) argmax_fold_kernel<<<grid_for(R, 4, INT32_MAX), 256, 0, ctx->stream>>>(pv, pi, nch, R, o);
    } else
      argmax_rows_kernel<<<grid_for(R, 4, INT32_MAX), 256, 0, ctx->stream>>>(xp, xe, R, C, static_cast<int32_t *>(ob->ptr));
    s = check_launch(ctx, "argmax_rows");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}
