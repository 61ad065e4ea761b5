// Attention of a few query rows against a KV cache, as one operation.
//
// Reference: Engine::attention_rows (crates/burn-tt/src/server.rs:255-265;
// crates/tt-kernels/src/attention.rs:1-20) -- per key/value head, the
// composition of ops.rs:4520-4595: scores = Q K^T, scaled, masked to -inf
// above the causal diagonal, max clamped below at -FLT_MAX, exp(x - max), sum
// clamped below at FLT_MIN, divide, then P V.
//
// MI355X design.  The cache of one (sequence, kv head) item is [max_ctx, D],
// position-major, so a key or value row is one contiguous read; its elements
// are F32 (the reference numeric contract) or BF16 (the performance
// contract's cache, llama.rs:1276-1278: half the bytes), widened to F32 as
// they are loaded -- every product and sum is F32 either way.
// A block of 4 wavefronts takes one (item, query position, key chunk); the
// group's G query heads share every key and value row read.
// D/4 lanes read a row as float4s (a wavefront covers 64/(D/4) rows per
// access, coalesced), dot products fold over those lanes with xor shuffles,
// the scores [G, chunk] stay in LDS, each softmax row is one wavefront's, and
// the value product accumulates per lane and folds across lanes and waves in
// a fixed order.
//
// Decode has only batch * kv_heads query groups -- 3 for SmolLM2 at batch 1,
// far too few blocks for 256 CUs -- so the keys are split into chunks across
// blocks (split-K over the context): each chunk writes its own max, exp-sum
// and unnormalised P V to scratch, and a combine pass rescales them by
// exp(max_s - max) and divides.  One chunk writes the normalised result
// directly, the composition's exact formula order.  A block loads the value
// rows of its first pass before computing the scores (one HBM round trip
// less on a short chunk).
#include "combine.hpp"
#include "common.hpp"
#include "wave.hpp"

#include <atomic>
#include <cfloat>
#include <mutex>
#include <type_traits>

namespace mi {

constexpr int ATT_MAX_GROUP = 8;       // query heads per kv head
constexpr int64_t ATT_MAX_CHUNK = 1024;
constexpr int64_t ATT_MIN_CHUNK = 64;
constexpr int64_t ATT_TARGET_BLOCKS = 512;
constexpr int ATT_WAVES = 4;  // wavefronts per chunk block

// The first new position of the queries: an immediate value, or (a traced
// decode step's) read from the device, where it must keep pos0 + T <= span
// (the positions the key chunks were planned for, at most the cache's);
// outside that the rows attend from position 0 -- every read stays in the
// cache -- and the range flag is raised for the next wait.
struct AttPos {
  int64_t pos0;
  const int32_t *dev;
  int64_t span;
  uint32_t *flags;
};

__device__ __forceinline__ int64_t att_pos0(const AttPos &pa, int64_t T) {
  if (!pa.dev) return pa.pos0;
  const int64_t v = scalar_read_i32(pa.dev);
  const bool ok = v >= 0 && v + T <= pa.span;
  if (!ok && threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0) atomicOr(pa.flags, FLAG_INDEX_RANGE);
  return ok ? v : 0;
}

// scores[g] = q[g] . k for one key row per lane group, folded over the row's
// D/4 lanes.
template <int G, int LPR>
__device__ __forceinline__ void dots(const float4 (&qv)[G], float4 kv, float (&part)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) part[g] = (qv[g].x * kv.x + qv[g].y * kv.y) + (qv[g].z * kv.z + qv[g].w * kv.w);
#pragma unroll
  for (int g = 0; g < G; ++g) part[g] = fold_sum<LPR>(part[g]);
}

// One (item, position, chunk).  DIRECT: the only chunk -- write normalised
// rows of `out`.  Else write part[(item * S + s)] = {m[G], l[G], o[G][D]}.
template <int D, int G, int NW, typename KV>
__global__ void __launch_bounds__(NW * 64) attention_chunk_kernel(const float *q, const KV *kc, const KV *vc,
                                                              float *out, float *part, int64_t T, int64_t H,
                                                              int64_t KVH, AttPos pa, int64_t maxc, int64_t chunk,
                                                              float scale, int direct) {
  constexpr int LPR = D / 4;     // lanes per row
  constexpr int KPW = 64 / LPR;  // rows per wavefront access
  constexpr int U = 4;            // accesses in flight per wavefront
  constexpr int STEP = NW * KPW;  // rows per block access
  constexpr int NT = NW * 64;
  extern __shared__ float sm[];
  const int s = blockIdx.y;
  const int64_t item = blockIdx.x;  // (sequence, kv head, position), position fastest
  const int64_t p = item % T, bj = item / T;
  const int64_t j = bj % KVH, b = bj / KVH;
  const int64_t n = att_pos0(pa, T) + p + 1;  // causal: cache positions 0 .. pos0 + p
  const int64_t lo = static_cast<int64_t>(s) * chunk;
  const int64_t len = n > lo ? (n - lo < chunk ? n - lo : chunk) : 0;
  const KV *K = kc + ((bj)*maxc + lo) * D;
  const KV *V = vc + ((bj)*maxc + lo) * D;
  float *scores = sm;                     // [G][chunk]
  float *red = sm + G * chunk;            // [NW][G][D]
  float *stat = red + NW * G * D;         // [G] max, [G] sum
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sl = lane % LPR, kk = lane / LPR;
  const float *qrow = q + (b * T + p) * H * D + j * G * D;
  float4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = *reinterpret_cast<const float4 *>(qrow + g * D + 4 * sl);
  // The value rows of the first P V pass are independent of the scores:
  // their loads are issued now and land while the scores and softmax run.
  // Key and value rows are loaded unconditionally, rows past the chunk's end
  // clamped to its last (row lo when the chunk is empty, still below the
  // context): a load under a condition compiles to a branch that waits for
  // it.  Those lanes' scores are never written and their values never used.
  const int64_t first = static_cast<int64_t>(wave) * KPW + kk;
  const int64_t last = len > 0 ? len - 1 : 0;
  float4 vv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = first + u * STEP;
    vv[u] = f32x4_get(V + (c < len ? c : last) * D + 4 * sl);
  }

  // Scores, U accesses in flight per wavefront.
  for (int64_t c0 = first; c0 < len + kk; c0 += STEP * U) {
    float4 kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      kv[u] = f32x4_get(K + (c < len ? c : last) * D + 4 * sl);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      float pr[G];
      dots<G, LPR>(qv, kv[u], pr);
      if (sl == 0 && c < len)
#pragma unroll
        for (int g = 0; g < G; ++g) scores[g * chunk + c] = pr[g] * scale;
    }
  }
  __syncthreads();

  // Softmax statistics of each row (one wavefront per row).
  for (int g = wave; g < G; g += NW) {
    float *row = scores + g * chunk;
    float m = -INFINITY;
    for (int64_t c = lane; c < len; c += 64) m = max_nan(m, row[c]);
    m = fold_max<64>(m);
    m = isnan(m) ? m : (m > -FLT_MAX ? m : -FLT_MAX);
    float sum = 0.0f;
    for (int64_t c = lane; c < len; c += 64) {
      const float e = expf(row[c] - m);
      row[c] = e;
      sum += e;
    }
    sum = fold_sum<64>(sum);
    if (direct) {
      sum = isnan(sum) ? sum : (sum > FLT_MIN ? sum : FLT_MIN);
      for (int64_t c = lane; c < len; c += 64) row[c] = row[c] / sum;
    }
    if (lane == 0) {
      stat[g] = m;
      stat[G + g] = sum;
    }
  }
  __syncthreads();

  // P V.
  float4 acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t c0 = first; c0 < len + kk; c0 += STEP * U) {
    if (c0 != first) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + u * STEP;
        vv[u] = f32x4_get(V + (c < len ? c : last) * D + 4 * sl);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      if (c < len) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pg = scores[g * chunk + c];
          acc[g].x += pg * vv[u].x;
          acc[g].y += pg * vv[u].y;
          acc[g].z += pg * vv[u].z;
          acc[g].w += pg * vv[u].w;
        }
      }
    }
  }
  // Fold the row groups of a wavefront (lanes with equal sl), then the waves.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    acc[g].x = fold_columns<LPR>(acc[g].x);
    acc[g].y = fold_columns<LPR>(acc[g].y);
    acc[g].z = fold_columns<LPR>(acc[g].z);
    acc[g].w = fold_columns<LPR>(acc[g].w);
  }
  if (kk == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) *reinterpret_cast<float4 *>(red + (wave * G + g) * D + 4 * sl) = acc[g];
  __syncthreads();
  float *dst;
  if (direct) {
    dst = out + (b * T + p) * H * D + j * G * D;
  } else {
    float *pb = part + (item * gridDim.y + s) * static_cast<int64_t>(G * (D + 2));
    if (tid < 2 * G) pb[tid] = stat[tid];
    dst = pb + 2 * G;
  }
  for (int e = tid; e < G * D; e += NT) {
    float t = red[e];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w * G * D + e];
    dst[e] = t;
  }
}

// Where an attention result value (row, col) of [R, C] goes: F32 rows (the
// plain form), BF16 rows rounded once, an F32 value's BF16 parts in rows
// (MI_BF16_PARTS: a row's heads, then its remainders), or the tiles an o
// projection reads (MI_TILES_BF16, or MI_TILES_PARTS: heads' plane then
// remainders').
struct AttOut {
  void *p = nullptr;
  int form = MI_F32;
  int64_t R = 0, C = 0;
};
__device__ __forceinline__ void att_put(const AttOut &o, int64_t r, int64_t c, float v) {
  uint16_t *h = static_cast<uint16_t *>(o.p);
  switch (o.form) {
    case MI_F32: static_cast<float *>(o.p)[r * o.C + c] = v; break;
    case MI_BF16: h[r * o.C + c] = f32_to_bf16_bits(v); break;
    case MI_TILES_BF16: h[tile_offset(r, c, o.C)] = f32_to_bf16_bits(v); break;
    case MI_BF16_PARTS: {
      uint16_t hi, lo;
      split_bf16(v, hi, lo);
      h[r * 2 * o.C + c] = hi;
      h[r * 2 * o.C + o.C + c] = lo;
      break;
    }
    default: {
      uint16_t hi, lo;
      split_bf16(v, hi, lo);
      const int64_t t = tile_offset(r, c, o.C);
      h[t] = hi;
      h[o.R * o.C + t] = lo;
    }
  }
}
// Four consecutive values (c a multiple of 4) of one row.
__device__ __forceinline__ void att_put4(const AttOut &o, int64_t r, int64_t c, float4 v) {
  uint16_t *h = static_cast<uint16_t *>(o.p);
  switch (o.form) {
    case MI_F32: *reinterpret_cast<float4 *>(static_cast<float *>(o.p) + r * o.C + c) = v; break;
    case MI_BF16: f32x4_put(h + r * o.C + c, v); break;
    case MI_TILES_BF16: f32x4_put(h + tile_offset(r, c, o.C), v); break;
    case MI_BF16_PARTS: parts4_put(h + r * 2 * o.C + c, h + r * 2 * o.C + o.C + c, v); break;
    default: {
      const int64_t t = tile_offset(r, c, o.C);
      parts4_put(h + t, h + o.R * o.C + t, v);
    }
  }
}

// Combine the chunks of one (item, position): out = sum_s w_s o_s / sum_s w_s
// l_s with w_s = exp(m_s - max_s m_s), the sum clamped below at FLT_MIN.  The
// chunks' statistics go to LDS in one pass and the weights are formed there,
// so each output element then issues its S loads back to back.
// RUNS: the matrix-core kernel's split wrote the partials, its 32-position
// runs on XCD (run % 8) (T a multiple of 256): block c takes an item whose
// run lies on c's own XCD (c % 8), so the partials are read from the L2 they
// were written to.
// chunk > 0 (the matrix-core kernel's split, causal): position p's keys
// reach only its first (pos0 + p) / chunk + 1 ranges, and only those are
// read (the others carry no keys and were not written).
template <int D, int G, bool FORMS = false>
__global__ void __launch_bounds__(256) attention_combine_kernel(const float *part, AttOut out, int64_t T, int64_t H,
                                                                int64_t KVH, int S, int runs = 0, int64_t pos0 = 0,
                                                                int64_t chunk = 0) {
  extern __shared__ float st[];  // [S][2G] statistics, then [S][G] weights, [G] denominators
  int64_t item = blockIdx.x;
  if (runs) {
    const int64_t x = item & 7, sl = item >> 3, per = T >> 3;  // items of one XCD per (sequence, kv head)
    const int64_t bjx = sl / per, r = sl - bjx * per;
    item = bjx * T + 32 * (x + 8 * (r >> 5)) + (r & 31);
  }
  const int64_t p = item % T, bj = item / T;
  const int64_t j = bj % KVH, b = bj / KVH;
  constexpr int PS = G * (D + 2);  // floats per chunk partial
  const float *pb = part + item * S * static_cast<int64_t>(PS);
  const int64_t reach = chunk > 0 ? (pos0 + p) / chunk + 1 : S;
  const int SR = static_cast<int>(reach < S ? reach : S);  // the ranges read
  float *w = st + 2 * G * S;
  float *den = w + G * S;
  // A thread's output elements e = tid + 256 i: their first CS chunks'
  // values requested with the statistics, so the combine is one round trip
  // for up to CS chunks.
  constexpr int EP = (G * D + 255) / 256, CS = EP <= 2 ? 16 : 8;
  float ov[EP][CS];
#pragma unroll
  for (int i = 0; i < EP; ++i) {
    const int e = threadIdx.x + 256 * i, ec = e < G * D ? e : 0;
#pragma unroll
    for (int s = 0; s < CS; ++s) ov[i][s] = s < SR ? pb[s * PS + 2 * G + ec] : 0.0f;
  }
  for (int e = threadIdx.x; e < 2 * G * SR; e += 256) st[e] = pb[(e / (2 * G)) * PS + e % (2 * G)];
  __syncthreads();
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < SR; ++s) M = max_nan(M, st[s * 2 * G + g]);
    float l = 0.0f;
    for (int s = 0; s < SR; ++s) {
      const float ws = expf(st[s * 2 * G + g] - M);
      w[s * G + g] = ws;
      l += ws * st[s * 2 * G + G + g];
    }
    den[g] = isnan(l) ? l : (l > FLT_MIN ? l : FLT_MIN);
  }
  __syncthreads();
  const int64_t orow = b * T + p, ocol = j * G * D;
#pragma unroll
  for (int i = 0; i < EP; ++i) {
    const int e = threadIdx.x + 256 * i;
    if (e < G * D) {
      const int g = e / D;
      float num = 0.0f;
#pragma unroll
      for (int s = 0; s < CS; ++s)
        if (s < SR) num += w[s * G + g] * ov[i][s];
      for (int s = CS; s < SR; ++s) num += w[s * G + g] * pb[s * PS + 2 * G + e];
      if constexpr (FORMS) att_put(out, orow, ocol + e, num / den[g]);
      else static_cast<float *>(out.p)[orow * out.C + ocol + e] = num / den[g];
    }
  }
}

// ------------------------------------------- long prompts: matrix cores
// Causal attention of many new positions (a prefill) flash style on the
// matrix cores: one block per (sequence, kv head, two runs of 32 query
// positions -- a long and a short run of keys paired, so causal blocks carry
// equal work), one wavefront per query head of the group; the scores never
// leave registers.  Per block of 32 keys (staged in LDS, shared by the
// group's heads, the next block's loads in flight under the current one) a
// wavefront forms S^T = K Q^T -- keys as the rows of its 32 x 32
// accumulator, its lane's query as the column, so each query's keys sit in
// one lane and its partner (lane ^ 32) -- scales and masks it, takes the
// running softmax (max clamped as the composition's; the sum of a causal row
// is never empty; exponentials in base 2, v_exp_f32, within a few ulps,
// against a reference max allowed to trail the running max by < 8, so the
// accumulators are rescaled only when the max outruns it), and adds V^T P^T
// to its 64 x 32 output accumulator.  Only the order of the sums differs from
// the composition.  D = 64.
constexpr int FLASH_MIN_T = 64;  // new positions per sequence that take it
// Below FLASH_MIN_BLOCKS (run, sequence, kv head) blocks the kernel splits
// its keys into ranges of 128 -- 64 where that still leaves fewer than
// FLASH_MIN_BLOCKS (run, item, range) blocks -- and the combine pass adds
// the ranges (512-token prompts, ms: batch 1 2.98 -> 2.74 at 64 keys,
// batch 2 3.98 -> 3.59 and batch 4 6.69 -> 6.52 at 128).
constexpr int64_t FLASH_MIN_BLOCKS = 256;

typedef float flash_f32x16 __attribute__((ext_vector_type(16)));

// The products run on the BF16 matrix cores (v_mfma_f32_32x32x16_bf16:
// 16 K multiply-adds a 32-cycle instruction, against 2 K a 64-cycle one on
// F32: 138.5 -> 122.5 us a layer for the batch-32 prompt, the rest being the
// staging, the splits and the softmax).  Every F32 operand is split into three BF16 parts (head truncated,
// remainders rounded to nearest: |a - hi - mid - lo| <= 2^-25 |a|) and each
// product taken as the part products down to 2^-16 of its size -- hi hi, hi
// mid, mid hi, hi lo, mid mid, lo hi -- so the scores and P V keep the F32
// products' accuracy; a BF16 cache holds its keys and values exactly: one
// part, three products.  The key and value blocks are split as they are
// staged into LDS (keys [32 keys][64 d], values transposed [64 d][32 keys],
// one array per part), the queries once per run into registers, P^T from
// its accumulator registers after the softmax.  The contraction over keys
// for V^T P^T takes k slots in the order P^T's registers hold the keys
// (slot i of half-wave h: key 16 j + 8 (i / 4) + 4 h + i % 4), so P^T is
// the B operand as it lies; the value fragments are read in that order.
// D = 64.
typedef __bf16 fl_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 fl_bf16x4 __attribute__((ext_vector_type(4)));
// LDS row pitches (bf16): a key part [32 keys][64 d] at 72 (a lane's 16-byte
// fragment reads of one 16-lane group start 36 dwords apart: no two share a
// bank), a value part transposed [64 d][32 keys] at 36 (a half-wave's 8-byte
// reads start 18 dwords apart: none shared).
constexpr int FL3_KS = 72;
constexpr int FL3_VS = 36;

__device__ __forceinline__ void fl_split(float v, __bf16 &hi, __bf16 &mid, __bf16 &lo) {
  const uint32_t hb = __float_as_uint(v) & 0xffff0000u;
  const float r1 = v - __uint_as_float(hb);
  const bool fin = r1 == r1;  // an infinite or NaN value: its head carries it alone
  const __bf16 m = static_cast<__bf16>(fin ? r1 : 0.0f);
  const float r2 = fin ? r1 - static_cast<float>(m) : 0.0f;
  hi = __builtin_bit_cast(__bf16, static_cast<uint16_t>(hb >> 16));
  mid = m;
  lo = static_cast<__bf16>(r2);
}

// fl_split of two exponentials (finite, < 2^8 here, or a quiet NaN) as
// packed pairs: a quiet NaN's truncated head is itself NaN (its quiet bit is
// in the head), so no finiteness check is needed -- a NaN gives NaN
// products either way; the remainders rounded two at a time.
__device__ __forceinline__ void fl_split2_exp(float a, float b, uint32_t &hi, uint32_t &mid, uint32_t &lo) {
  const uint32_t ha = __float_as_uint(a) & 0xffff0000u, hb = __float_as_uint(b) & 0xffff0000u;
  const float ra = a - __uint_as_float(ha), rb = b - __uint_as_float(hb);
  mid = bf16x2_bits(ra, rb);
  const float sa = ra - __uint_as_float(mid << 16), sb = rb - __uint_as_float(mid & 0xffff0000u);
  lo = bf16x2_bits(sa, sb);
  hi = (ha >> 16) | hb;
}

// The part products of one k step: A parts a[], B parts b[] (NA and NB of them).
template <int NA, int NB>
__device__ __forceinline__ flash_f32x16 fl_mfma(const fl_bf16x8 (&a)[NA], const fl_bf16x8 (&b)[NB], flash_f32x16 c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], c, 0, 0, 0);
  if constexpr (NB > 1) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], c, 0, 0, 0);
  if constexpr (NA > 1) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], c, 0, 0, 0);
  if constexpr (NB > 2) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], c, 0, 0, 0);
  if constexpr (NA > 1 && NB > 1) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], c, 0, 0, 0);
  if constexpr (NA > 2) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], c, 0, 0, 0);
  return c;
}

// FORMS: the result's form -- 0 F32 rows, 1 BF16 parts in rows, 3 BF16
// rows, 2 any (the store's form switch); each compiles only its own store,
// so the row-form kernels keep two waves a SIMD.
template <int G, typename KV, int FORMS>
__global__ void __launch_bounds__(G * 64)
flash3_prefill_kernel(const float *q, const KV *kc, const KV *vc, AttOut out, int64_t T, int64_t H, int64_t KVH,
                      int64_t pos0, int64_t maxc, float scale, int64_t kchunk, float *part, int item_major) {
  constexpr int D = 64, NT = G * 64;
  constexpr bool EXACT = sizeof(KV) == 2;  // a BF16 cache: one part
  constexpr int KP = EXACT ? 1 : 3;
  __shared__ __attribute__((aligned(16))) __bf16 ks[2][KP][32 * FL3_KS];
  __shared__ __attribute__((aligned(16))) __bf16 vs[2][KP][64 * FL3_VS];
  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  // item_major 0: block (pair of runs x, item y).  1 (many items): the
  // grid's x the item, so every block of an item is on one XCD (workgroup w
  // runs on XCD w % 8) and its keys and values are read into one L2.  2 (the
  // items a multiple of 8): one run a block, blocks in order of falling work
  // -- block w takes run nqb - 1 - w / items of item w % items -- so the
  // dispatcher, handing blocks out in order as CUs free up, fills the last
  // ones with the shortest runs (equal pairs left the chip's second round of
  // blocks half empty), each item still on one XCD.
  const int64_t nqb = (T + 31) / 32;
  const int64_t nitems = static_cast<int64_t>(item_major == 2 ? gridDim.x / nqb : 0);
  const int64_t bx = item_major == 2 ? nqb - 1 - blockIdx.x / nitems : item_major ? blockIdx.y : blockIdx.x;
  const int64_t bj = item_major == 2 ? blockIdx.x % nitems : item_major ? blockIdx.x : blockIdx.y;  // (sequence, kv head)
  const int64_t j = bj % KVH, b = bj / KVH;
  const int n = lane & 31, half = lane >> 5;
  const int64_t ctx = pos0 + T;
  const int64_t h = j * G + g;
  const float scale2 = scale * 1.4426950408889634f;
  const KV *K = kc + bj * maxc * D, *V = vc + bj * maxc * D;
  const int ctx32 = static_cast<int>(ctx);  // the host keeps a cache item below 2^31 / D rows
  // Split over keys (kchunk > 0): block (query run x, item y, key range z)
  // takes keys [z kchunk, (z + 1) kchunk) of its run's and writes the
  // range's partials (max, sum, unnormalised P V) for the combine pass;
  // one run a block, no pairing.
  const bool split = kchunk > 0;
  for (int pass = 0; pass < (split || item_major == 2 ? 1 : 2); ++pass) {
    const int64_t qb = pass == 0 ? bx : nqb - 1 - bx;
    if (pass == 1 && qb == bx) break;
    const int64_t p0 = qb * 32, p = p0 + n;
    const bool live = p < T;
    const int64_t pq = live ? p : T - 1;
    const int64_t qpos = pos0 + pq;
    // Q^T as the B operand of step s: q[p][16 s + 8 half .. + 7], three
    // parts -- its loads issued here, split once the first key and value
    // block's loads are in flight too.
    float4 qv[4][2];
    {
      const float *qrow = q + (b * T + pq) * H * D + h * D + 8 * half;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        qv[s2][0] = *reinterpret_cast<const float4 *>(qrow + 16 * s2);
        qv[s2][1] = *reinterpret_cast<const float4 *>(qrow + 16 * s2 + 4);
      }
    }
    flash_f32x16 o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o0[r] = 0.0f; o1[r] = 0.0f; }
    float m = -INFINITY, l = 0.0f;
    const int64_t kend_run = pos0 + (p0 + 32 < T ? p0 + 32 : T);
    const int64_t kbeg = split ? static_cast<int64_t>(blockIdx.z) * kchunk : 0;
    const int64_t kend = split ? (kbeg + kchunk < kend_run ? kbeg + kchunk : kend_run) : kend_run;
    // A key range past every position of the run: no partials (the combine
    // reads only the ranges a position's keys reach).
    if (split && kbeg >= kend_run) return;
    // Key and value blocks as 512 groups of 4 values, loaded into registers
    // for the next block while the current one is used: key group e is key
    // e / 16, d 4 (e % 16) .. + 3 (a 16-byte load); value group e is d e % 64
    // of keys 4 (e / 64) .. + 3 (four loads, each a half-wave's row segment),
    // so that it is stored transposed as one 8-byte run a part.
    constexpr int PER = (32 * 16 + NT - 1) / NT;
    using Raw = typename std::conditional<EXACT, uint2, float4>::type;
    Raw kr[PER];
    KV vr[PER][4];
    auto fetch = [&](int64_t j0) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int e0 = tid + u * NT, e = e0 < 32 * 16 ? e0 : tid;
        const int r = static_cast<int>(j0) + (e >> 4) < ctx32 ? static_cast<int>(j0) + (e >> 4) : ctx32 - 1;
        kr[u] = *reinterpret_cast<const Raw *>(K + r * D + (e & 15) * 4);
        const int d = e & 63, k4 = static_cast<int>(j0) + 4 * (e >> 6);
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[u][i] = V[(k4 + i < ctx32 ? k4 + i : ctx32 - 1) * D + d];
      }
    };
    auto stage = [&](int buf) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int e = tid + u * NT;
        if (e < 32 * 16) {
          const int r = e >> 4, c4 = (e & 15) * 4;
          const int vofs = (e & 63) * FL3_VS + 4 * (e >> 6);
          if constexpr (EXACT) {
            *reinterpret_cast<uint2 *>(&ks[buf][0][r * FL3_KS + c4]) = kr[u];
            const fl_bf16x4 v4 = {__builtin_bit_cast(__bf16, vr[u][0]), __builtin_bit_cast(__bf16, vr[u][1]),
                                  __builtin_bit_cast(__bf16, vr[u][2]), __builtin_bit_cast(__bf16, vr[u][3])};
            *reinterpret_cast<fl_bf16x4 *>(&vs[buf][0][vofs]) = v4;
          } else {
            const float k4[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
            fl_bf16x4 kp0, kp1, kp2, vp0, vp1, vp2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              __bf16 a0, a1, a2;
              fl_split(k4[i], a0, a1, a2);
              kp0[i] = a0; kp1[i] = a1; kp2[i] = a2;
              fl_split(vr[u][i], a0, a1, a2);
              vp0[i] = a0; vp1[i] = a1; vp2[i] = a2;
            }
            *reinterpret_cast<fl_bf16x4 *>(&ks[buf][0][r * FL3_KS + c4]) = kp0;
            *reinterpret_cast<fl_bf16x4 *>(&ks[buf][1 % KP][r * FL3_KS + c4]) = kp1;
            *reinterpret_cast<fl_bf16x4 *>(&ks[buf][2 % KP][r * FL3_KS + c4]) = kp2;
            *reinterpret_cast<fl_bf16x4 *>(&vs[buf][0][vofs]) = vp0;
            *reinterpret_cast<fl_bf16x4 *>(&vs[buf][1 % KP][vofs]) = vp1;
            *reinterpret_cast<fl_bf16x4 *>(&vs[buf][2 % KP][vofs]) = vp2;
          }
        }
      }
    };
    fetch(kbeg < kend ? kbeg : 0);
    fl_bf16x8 qp[4][3];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const float vv[8] = {qv[s2][0].x, qv[s2][0].y, qv[s2][0].z, qv[s2][0].w,
                           qv[s2][1].x, qv[s2][1].y, qv[s2][1].z, qv[s2][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        __bf16 a0, a1, a2;
        fl_split(vv[e], a0, a1, a2);
        qp[s2][0][e] = a0;
        qp[s2][1][e] = a1;
        qp[s2][2][e] = a2;
      }
    }
    stage(0);
    __syncthreads();
    for (int64_t j0 = kbeg, it = 0; j0 < kend; j0 += 32, ++it) {
      const int buf = static_cast<int>(it & 1);
      const bool more = j0 + 32 < kend;
      if (more) fetch(j0 + 32);

      // S^T = K Q^T over d: step s takes d 16 s .. 16 s + 15, half-wave h
      // supplying d 16 s + 8 h .. + 7.
      flash_f32x16 st;
#pragma unroll
      for (int r = 0; r < 16; ++r) st[r] = 0.0f;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        fl_bf16x8 ka[KP];
#pragma unroll
        for (int pp = 0; pp < KP; ++pp)
          ka[pp] = *reinterpret_cast<const fl_bf16x8 *>(&ks[buf][pp][n * FL3_KS + 16 * s2 + 8 * half]);
        st = fl_mfma<KP, 3>(ka, qp[s2], st);
      }
      float mx = -INFINITY;
      if (j0 + 31 <= pos0 + p0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          st[r] *= scale2;
          mx = max_nan(mx, st[r]);
        }
      } else {
        const int lim = static_cast<int>((qpos < ctx - 1 ? qpos : ctx - 1) - j0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kofs = 8 * (r >> 2) + 4 * half + (r & 3);
          st[r] = kofs > lim ? -INFINITY : st[r] * scale2;
          mx = max_nan(mx, st[r]);
        }
      }
      mx = max_nan(mx, __shfl_xor(mx, 32, 64));
      if (__any(!(mx <= m + 8.0f))) {
        float mnew = max_nan(m, mx);
        mnew = isnan(mnew) ? mnew : (mnew > -FLT_MAX ? mnew : -FLT_MAX);
        const float corr = __builtin_amdgcn_exp2f(m - mnew);
        l *= corr;
#pragma unroll
        for (int r = 0; r < 16; ++r) { o0[r] *= corr; o1[r] *= corr; }
        m = mnew;
      }
      float ls = 0.0f;
      uint32_t pw[2][3][4];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float e0 = __builtin_amdgcn_exp2f(st[r] - m), e1 = __builtin_amdgcn_exp2f(st[r + 1] - m);
        ls += e0;
        ls += e1;
        fl_split2_exp(e0, e1, pw[r >> 3][0][(r & 7) >> 1], pw[r >> 3][1][(r & 7) >> 1], pw[r >> 3][2][(r & 7) >> 1]);
      }
      fl_bf16x8 pb[2][3];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int pp = 0; pp < 3; ++pp)
          pb[i][pp] = __builtin_bit_cast(fl_bf16x8, make_uint4(pw[i][pp][0], pw[i][pp][1], pw[i][pp][2], pw[i][pp][3]));
      ls += __shfl_xor(ls, 32, 64);
      l += ls;
      // O^T += V^T P^T: step s2 contracts the keys of P^T's registers 8 s2 .. 8 s2 + 7.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        fl_bf16x8 va0[KP], va1[KP];
#pragma unroll
        for (int pp = 0; pp < KP; ++pp) {
          const __bf16 *v0 = &vs[buf][pp][n * FL3_VS + 16 * s2 + 4 * half];
          const __bf16 *v1 = &vs[buf][pp][(32 + n) * FL3_VS + 16 * s2 + 4 * half];
          const fl_bf16x4 a = *reinterpret_cast<const fl_bf16x4 *>(v0), c = *reinterpret_cast<const fl_bf16x4 *>(v0 + 8);
          const fl_bf16x4 a1 = *reinterpret_cast<const fl_bf16x4 *>(v1), c1 = *reinterpret_cast<const fl_bf16x4 *>(v1 + 8);
          va0[pp] = fl_bf16x8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
          va1[pp] = fl_bf16x8{a1[0], a1[1], a1[2], a1[3], c1[0], c1[1], c1[2], c1[3]};
        }
        o0 = fl_mfma<KP, 3>(va0, pb[s2], o0);
        o1 = fl_mfma<KP, 3>(va1, pb[s2], o1);
      }
      if (more) stage(buf ^ 1);
      __syncthreads();
    }
    if (split) {
      if (live) {
        // The combine's layout: item (sequence, kv head, position), range z;
        // the max in natural units (the scores here are in base 2).
        float *pbk = part + (((b * KVH + j) * T + p) * gridDim.z + blockIdx.z) * static_cast<int64_t>(G * (D + 2));
        if (half == 0) {
          const float mc = isnan(m) ? m : (m > -FLT_MAX ? m : -FLT_MAX);
          pbk[g] = mc > -FLT_MAX ? mc * 0.6931471805599453f : mc;
          pbk[G + g] = l;
        }
        float *orow = pbk + 2 * G + g * D + 4 * half;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            orow[8 * c + i] = o0[4 * c + i];
            orow[32 + 8 * c + i] = o1[4 * c + i];
          }
      }
    } else if (live) {
      const float den = isnan(l) ? l : (l > FLT_MIN ? l : FLT_MIN);
      const int64_t orow = b * T + p, ocol = h * D + 4 * half;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 y0 = make_float4(o0[4 * c] / den, o0[4 * c + 1] / den, o0[4 * c + 2] / den, o0[4 * c + 3] / den);
        const float4 y1 = make_float4(o1[4 * c] / den, o1[4 * c + 1] / den, o1[4 * c + 2] / den, o1[4 * c + 3] / den);
        if constexpr (FORMS == 1) {
          uint16_t *h = static_cast<uint16_t *>(out.p) + orow * 2 * out.C + ocol;
          parts4_put(h + 8 * c, h + out.C + 8 * c, y0);
          parts4_put(h + 32 + 8 * c, h + out.C + 32 + 8 * c, y1);
        } else if constexpr (FORMS == 3) {
          uint16_t *h = static_cast<uint16_t *>(out.p) + orow * out.C + ocol;
          f32x4_put(h + 8 * c, y0);
          f32x4_put(h + 32 + 8 * c, y1);
        } else if constexpr (FORMS == 2) {
          att_put4(out, orow, ocol + 8 * c, y0);
          att_put4(out, orow, ocol + 32 + 8 * c, y1);
        } else {
          float *orp = static_cast<float *>(out.p) + orow * out.C + ocol;
          *reinterpret_cast<float4 *>(orp + 8 * c) = y0;
          *reinterpret_cast<float4 *>(orp + 32 + 8 * c) = y1;
        }
      }
    }
  }
}

template <int G, typename KV>
void launch_flash(hipStream_t st, const float *q, const KV *k, const KV *v, const AttOut &out, int64_t batch, int64_t T,
                  int64_t H, int64_t KVH, int64_t pos0, int64_t maxc, float scale, int64_t kchunk, int S,
                  float *part) {
  if (kchunk > 0) {
    const dim3 grid(static_cast<unsigned>((T + 31) / 32), static_cast<unsigned>(batch * KVH), static_cast<unsigned>(S));
    flash3_prefill_kernel<G, KV, 0><<<grid, G * 64, 0, st>>>(q, k, v, out, T, H, KVH, pos0, maxc, scale, kchunk,
                                                                   part, 0);
    // With the runs a multiple of 8 the split's blocks of a run share an XCD
    // (run % 8): the combine reads each item's partials there.
    const int runs = T % 256 == 0 ? 1 : 0;
    const unsigned items = static_cast<unsigned>(batch * KVH * T);
    const size_t smem = static_cast<size_t>(3 * G * S + G) * sizeof(float);
    if (out.form == MI_F32)
      attention_combine_kernel<64, G, false><<<items, 256, smem, st>>>(part, out, T, H, KVH, S, runs, pos0, kchunk);
    else
      attention_combine_kernel<64, G, true><<<items, 256, smem, st>>>(part, out, T, H, KVH, S, runs, pos0, kchunk);
    return;
  }
  // Many items (a multiple of 8): one run a block, the longest first, each
  // item's blocks on one XCD; else pairs of runs of equal total work.
  const int64_t pairs = ((T + 31) / 32 + 1) / 2, items = batch * KVH, nqb = (T + 31) / 32;
  const int im = items % 8 == 0 ? 2 : 0;
  const dim3 grid = im ? dim3(static_cast<unsigned>(nqb * items)) : dim3(static_cast<unsigned>(pairs), static_cast<unsigned>(items));
  if (out.form == MI_F32)
    flash3_prefill_kernel<G, KV, 0><<<grid, G * 64, 0, st>>>(q, k, v, out, T, H, KVH, pos0, maxc, scale, 0, nullptr, im);
  else if (out.form == MI_BF16_PARTS)
    flash3_prefill_kernel<G, KV, 1><<<grid, G * 64, 0, st>>>(q, k, v, out, T, H, KVH, pos0, maxc, scale, 0, nullptr, im);
  else if (out.form == MI_BF16)
    flash3_prefill_kernel<G, KV, 3><<<grid, G * 64, 0, st>>>(q, k, v, out, T, H, KVH, pos0, maxc, scale, 0, nullptr, im);
  else
    flash3_prefill_kernel<G, KV, 2><<<grid, G * 64, 0, st>>>(q, k, v, out, T, H, KVH, pos0, maxc, scale, 0, nullptr, im);
}

template <typename KV>
bool flash_dispatch(int64_t G, hipStream_t st, const float *q, const KV *k, const KV *v, const AttOut &out, int64_t batch,
                    int64_t T, int64_t H, int64_t KVH, int64_t pos0, int64_t maxc, float scale, int64_t kchunk,
                    int S, float *part) {
  switch (G) {
#define MI_FLASH_G(gg) \
  case gg: launch_flash<gg, KV>(st, q, k, v, out, batch, T, H, KVH, pos0, maxc, scale, kchunk, S, part); return true;
    MI_FLASH_G(1) MI_FLASH_G(2) MI_FLASH_G(3) MI_FLASH_G(4) MI_FLASH_G(5) MI_FLASH_G(6) MI_FLASH_G(7) MI_FLASH_G(8)
#undef MI_FLASH_G
    default:
      return false;
  }
}

// LDS bytes of a chunk kernel with `nw` wavefronts.
inline size_t attention_smem(int64_t G, int64_t D, int64_t chunk, int nw) {
  return static_cast<size_t>(G * chunk + nw * G * D + 2 * G) * sizeof(float);
}

template <int D, int G, typename KV>
void launch_attention(hipStream_t st, const float *q, const KV *k, const KV *v, float *out, float *part,
                      int64_t items, int S, int64_t T, int64_t H, int64_t KVH, const AttPos &pa, int64_t maxc,
                      int64_t chunk, float scale) {
  const dim3 grid(static_cast<unsigned>(items), static_cast<unsigned>(S));
  const size_t smem = attention_smem(G, D, chunk, ATT_WAVES);
  attention_chunk_kernel<D, G, ATT_WAVES, KV><<<grid, ATT_WAVES * 64, smem, st>>>(q, k, v, out, part, T, H, KVH, pa, maxc,
                                                                            chunk, scale, S == 1);
  if (S > 1) {
    AttOut o;  // F32 rows of H D columns (the form reads no row count)
    o.p = out;
    o.C = H * D;
    attention_combine_kernel<D, G><<<static_cast<unsigned>(items), 256, static_cast<size_t>(3 * G * S + G) * sizeof(float),
                                     st>>>(part, o, T, H, KVH, S);
  }
}

template <int D, typename KV>
bool dispatch_group(int64_t G, hipStream_t st, const float *q, const KV *k, const KV *v, float *out,
                    float *part, int64_t items, int S, int64_t T, int64_t H, int64_t KVH, const AttPos &pa,
                    int64_t maxc, int64_t chunk, float scale) {
  switch (G) {
#define MI_ATT_G(g)                                                                                   \
  case g:                                                                                             \
    launch_attention<D, g, KV>(st, q, k, v, out, part, items, S, T, H, KVH, pa, maxc, chunk, scale); \
    return true;
    MI_ATT_G(1) MI_ATT_G(2) MI_ATT_G(3) MI_ATT_G(4) MI_ATT_G(5) MI_ATT_G(6) MI_ATT_G(7) MI_ATT_G(8)
#undef MI_ATT_G
    default:
      return false;
  }
}


// ------------------------------ a decode step's q|k|v and attention, fused
// One new position per sequence (a decode step) of up to 6 sequences with
// 64-wide heads: the RMSNorm of the hidden row, the q|k|v projection, RoPE,
// the cache write and the attention's key chunks in one launch (the
// composition mi_norm_qkv_rope then mi_attention_rows_at runs as two, the
// second waiting for the first's queries and cache row).  Two kinds of block:
//   - (sequence, query head, key chunk): the block forms its head's 64 query
//     values itself -- the norm into LDS, a 64-row GEMV, RoPE -- and attends
//     over its chunk of the keys before the new position, whose rows are
//     requested at the start so they land under the GEMV;
//   - (sequence, kv head, k or v): 64 rows of the new key (rotated) or value,
//     stored into the cache at the position.
// The new key itself is one more chunk, added by the combine pass: score
// q . k_new (read back from the cache, as stored), weight 1, value v_new.
// So every block of the launch is independent; the queries of the head's
// first chunk block go to memory for the combine.  The 9 chunk blocks of a
// head read the same 64 weight rows (74 KB for k = 576); they run on
// different XCDs, each with its own L2, so the repeats are fetched from the
// fabric (8.7 MB a SmolLM2 launch against 2.0 MB of weights and cache), at a
// rate that does not bound the launch.
constexpr int DQA_MAX_CH = 32;  // k <= 32 DQA_MAX_CH = 1024
// Wavefronts a block of the fused step, and so the lanes of each of its 64
// weight rows: 8 (two a SIMD: the GEMV's and the chunk passes' instruction
// latencies hide behind the other wavefront's; 7.2 -> 6.4 us a SmolLM2 layer).
constexpr int DQA_NW = 8, DQA_NT = 64 * DQA_NW, DQA_RL = DQA_NT / 64;
constexpr int DQA_D = 64;
// Sequences up to which the fused launch serves a decode step: beyond, its
// blocks' query GEMVs (each (sequence, head, chunk) block its own) cost more
// than the composition's one matrix-core product (batch 8: 1.34 ms a
// SmolLM2 step either way).
constexpr int64_t DQA_MAX_B = 6;

struct DqaArgs {
  const float *x;  // [B, K] F32 hidden rows
  int64_t K;
  const float *gamma;  // [1, K] RMSNorm gain
  float eps;
  const uint16_t *w;       // [(H + 2 KVH) 64, K] BF16: q, k, v heads
  const int8_t *wq;        // or BFP8: datums [(H + 2 KVH) 64, K] and
  const uint8_t *we;       //   block exponents [(H + 2 KVH) 64, K / 16]
  const float *cos, *sin;  // rotary tables, rows by position
  void *kc, *vc;           // caches [B KVH maxc, 64], F32 or BF16
  int64_t maxc;
  int H, KVH, G, B;
  AttPos pa;  // the new position
  int64_t S, chunk;
  float scale;
  float *q;     // [B, H 64] rotated queries, for the combine
  float *part;  // [B KVH][S][G (64 + 2)] chunk partials
  float *kvn;   // [B KVH][2][64] the new key and value rows as stored, for the combine
};

// How the fused step reads eight consecutive q|k|v weights of row r from k
// (a multiple of 8): a BF16 weight as one 16-byte load, a BFP8 weight as its
// 8 datum bytes and the block's exponent byte -- decoded exactly to the
// values a BF16 weight holding them gives, so the step's bits are the same.
struct DqaBf16 {
  using Raw = uint4;
  static __device__ __forceinline__ Raw load(const DqaArgs &g, int64_t r, int64_t k) {
    return *reinterpret_cast<const uint4 *>(g.w + r * g.K + k);
  }
  static __device__ __forceinline__ void f32(const Raw &q, float (&w)[8]) {
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[2 * e] = __uint_as_float(u[e] << 16);
      w[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
    }
  }
};
struct DqaBfp8 {
  struct Raw {
    uint2 d;
    int e;
  };
  static __device__ __forceinline__ Raw load(const DqaArgs &g, int64_t r, int64_t k) {
    Raw q;
    q.d = *reinterpret_cast<const uint2 *>(g.wq + r * g.K + k);
    q.e = g.we[r * (g.K >> 4) + (k >> 4)];
    return q;
  }
  static __device__ __forceinline__ void f32(const Raw &q, float (&w)[8]) { bfp8x8(q.d, q.e, w); }
};

// The fused step's device-held position (or, without one, the flags word:
// read, never used) through the scalar cache (scalar_read_i32), unconditionally.
__device__ __forceinline__ int32_t dqa_pos_read(const AttPos &pa) {
  return scalar_read_i32(pa.dev ? pa.dev : reinterpret_cast<const int32_t *>(pa.flags));
}

// Ids of the fused step's chunk blocks in the XCD-aware order (dqa_work): 8
// XCDs times ceil(heads / 8) heads' S chunks.  (Measured against the plain
// order and against all G S blocks of a (sequence, kv head) on one XCD: the
// same batch-1 and batch-4 step times, 0.703 / 0.705 / 0.714 ms at batch 1;
// this order halves the launch's fetched bytes, 8.7 -> 4.1 MB.)
__host__ __device__ __forceinline__ int64_t dqa_chunk_ids(const DqaArgs &g) {
  const int64_t ni = static_cast<int64_t>(g.B) * g.KVH;
  return 8 * ((ni + 7) / 8) * g.G * g.S;
}

// Block (DQA_NT threads): 64 rows (from row0, each K weights) times the
// staged row in LDS xn; thread t takes row t / RL and the 8-weight chunks t %
// RL, + RL, ... (RL = DQA_RL); the partial sums fold over the row's lanes.
// wr: the chunks, loaded by dqa_wload.  NCH > 0: K / 8 is NCH, known when
// compiled (no chunk past the row to clamp or skip).
template <int CH, typename WT, int NCH = 0>
__device__ __forceinline__ void dqa_wload(const DqaArgs &g, int64_t row0, typename WT::Raw (&wr)[CH]) {
  const int tid = threadIdx.x, r = tid / DQA_RL, kq = tid % DQA_RL;
  const int64_t nch = NCH > 0 ? NCH : g.K / 8;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int64_t c = kq + DQA_RL * i;
    wr[i] = WT::load(g, row0 + r, 8 * (c < nch ? c : nch - 1));
  }
}
template <int CH, typename WT, int NCH = 0>
__device__ __forceinline__ float dqa_dot(const float *xn, int64_t K, const typename WT::Raw (&wr)[CH]) {
  const int kq = threadIdx.x % DQA_RL;
  const int64_t nch = NCH > 0 ? NCH : K / 8;
  // Four independent sums (an FMA's latency is not hidden by the SIMD's
  // other wavefront alone), added at the end.
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int64_t c = kq + DQA_RL * i;
    if (c < nch) {
      const float4 a0 = *reinterpret_cast<const float4 *>(xn + 8 * c);
      const float4 a1 = *reinterpret_cast<const float4 *>(xn + 8 * c + 4);
      float w[8];
      WT::f32(wr[i], w);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] = fmaf(av[2 * e], w[2 * e], acc[e]);
        acc[e] = fmaf(av[2 * e + 1], w[2 * e + 1], acc[e]);
      }
    }
  }
  return fold_sum<DQA_RL>((acc[0] + acc[1]) + (acc[2] + acc[3]));
}

// A thread's operands of the norm and the rotation, requested with the
// weights so neither phase waits for a round trip of its own: the float4 of
// the hidden row b and of the gain at 4 tid (k <= 1024: one a thread) --
// requested before a device-held position is read, so the norm does not wait
// for that read -- and for tid < 32 the rotary table entries of pair (tid,
// tid + 32) at the position.
struct DqaPre {
  float4 x, gm;
  float cs0, cs1, sn0, sn1;
};
__device__ __forceinline__ void dqa_pre_x(const DqaArgs &g, int64_t b, DqaPre &e) {
  const int64_t k = 4 * threadIdx.x < g.K ? 4 * threadIdx.x : g.K - 4;
  e.x = *reinterpret_cast<const float4 *>(g.x + b * g.K + k);
  e.gm = *reinterpret_cast<const float4 *>(g.gamma + k);
}
__device__ __forceinline__ void dqa_pre_rot(const DqaArgs &g, int64_t pos, DqaPre &e) {
  constexpr int half = DQA_D / 2;
  const int i = threadIdx.x & (half - 1);
  const float *cs = g.cos + pos * DQA_D, *sn = g.sin + pos * DQA_D;
  e.cs0 = cs[i];
  e.cs1 = cs[i + half];
  e.sn0 = sn[i];
  e.sn1 = sn[i + half];
}

// The hidden row times the gain into LDS, xg[k] = x[k] gamma[k], and the
// RMSNorm's rms = sqrt(mean(x x) + eps), which divides the finished
// products (sum_k x g w / rms: the GEMV need not wait for the norm's fold).
__device__ __forceinline__ float dqa_stage(const DqaArgs &g, const DqaPre &pre, float *xg, float *red4) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool mine = 4 * tid < g.K;
  const float4 v = pre.x, gm = pre.gm;
  float ss = mine ? fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, v.w * v.w))) : 0.0f;
  if (mine) *reinterpret_cast<float4 *>(xg + 4 * tid) = make_float4(v.x * gm.x, v.y * gm.y, v.z * gm.z, v.w * gm.w);
  ss = fold_sum<64>(ss);
  if (lane == 0) red4[wave] = ss;
  __syncthreads();
  float t = red4[0];
#pragma unroll
  for (int w = 1; w < DQA_NW; ++w) t += red4[w];
  return __fsqrt_rn(t / static_cast<float>(g.K) + g.eps);
}

// RoPE of a 64-wide head in LDS (raw -> rot): the rotation of pair (i, i +
// 32) as the decode projections apply it, the table entries from dqa_pre_rot.
__device__ __forceinline__ void dqa_rope(const DqaPre &pre, const float *raw, float *rot) {
  const int tid = threadIdx.x;
  constexpr int half = DQA_D / 2;
  if (tid < half) {
    const float y0 = raw[tid], y1 = raw[tid + half];
    rot[tid] = __fadd_rn(__fmul_rn(y0, pre.cs0), __fmul_rn(y1, pre.sn0));
    rot[tid + half] = __fadd_rn(__fmul_rn(y1, pre.cs1), __fmul_rn(y0, pre.sn1));
  }
}

// The combine of a fused step: the S chunks of each (sequence, kv head) and
// the new key as one more -- score scale (q . k_new), weight exp(score -
// max), value row v_new -- with the key-chunked combine's formula: out =
// (sum_s w_s o_s + w_new v_new) / max(sum_s w_s l_s + w_new, FLT_MIN), w_s =
// exp(m_s - max) (ChunkCombine).  Item bj, one block: its G query heads on
// rows of 16 lanes (a row past the last head repeats the last and writes
// nothing); wl: 16 S floats of LDS for each wavefront's rows.
template <int CS>
__device__ __forceinline__ void combine_new_item(const DqaArgs &g, int64_t bj, float *out, float *wl) {
  constexpr int D = DQA_D;
  const int G = g.G, S = static_cast<int>(g.S);
  const int row = threadIdx.x >> 4, r = threadIdx.x & 15, gg = row < G ? row : G - 1;
  const int64_t b = bj / g.KVH, j = bj % g.KVH, h = j * G + gg;
  const float *pitem = g.part + bj * S * dqa_part_stride(G);
  ChunkCombine<CS> cc;
  cc.load(pitem, G, gg, S, r, g.q + (b * g.H + h) * D, g.kvn + bj * 2 * D, g.kvn + bj * 2 * D + D);
  const float4 o = cc.finish(pitem, G, gg, S, r, g.scale, wl + row * S);
  if (row < G) *reinterpret_cast<float4 *>(out + (b * g.H + h) * D + 4 * r) = o;
}

// The block's part of the launch (its item, sequence and kv head, is
// returned).  (Counting the blocks in and letting the last of an item combine -- device
// fences before and after the count -- costs more than the combine's own
// launch: batch-1 SmolLM2 decode 0.694 -> 0.938 ms a step.)
template <typename KV, int CH, typename WT, int NCH>
__device__ __forceinline__ int64_t dqa_work(const DqaArgs &g, float *dqa_sm) {
  constexpr int D = DQA_D, NW = DQA_NW, LPR = D / 4, KPW = 64 / LPR, U = 2, STEP = NW * KPW;
  float *xn = dqa_sm;            // [K]
  float *qraw = xn + g.K;        // [64]
  float *qrot = qraw + D;        // [64]
  float *red4 = qrot + D;        // [NW]
  float *scores = red4 + NW;     // [chunk]
  float *red = scores + g.chunk; // [NW][D]
  float *wsum = red + NW * D;    // [NW]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Block order, XCD-aware: workgroup p runs on XCD p % 8, and the G S
  // chunk blocks of kv item i (i = sequence KVH + kv head) take the ids p =
  // i % 8 + 8 (slot), slot = (i / 8) G S + g S + chunk, so every block that
  // reads the item's key and value chunks, and a query head's 64 weight
  // rows, runs on one XCD and they come once into its L2 (ids with i past
  // the last item are empty blocks).  Then the key / value blocks.
  const int64_t nchunk = dqa_chunk_ids(g);
  const int64_t bid = blockIdx.x;

  if (bid >= nchunk) {  // the new key or value row of (sequence, kv head)
    const int64_t kb = bid - nchunk, which = kb & 1, bj = kb >> 1, b = bj / g.KVH, j = bj % g.KVH;
    // A device-held position through the scalar cache (dqa_pos_read): its
    // wait covers it alone, not the weights requested around it.
    const int32_t pdev = dqa_pos_read(g.pa);
    typename WT::Raw wr[CH];
    dqa_wload<CH, WT, NCH>(g, (g.H + which * g.KVH + j) * D, wr);
    DqaPre pre;
    dqa_pre_x(g, b, pre);
    int64_t pos = g.pa.pos0;
    bool ok = true;
    if (g.pa.dev) {
      pos = pdev;
      ok = pos >= 0 && pos + 1 <= g.pa.span;
      pos = ok ? pos : 0;
    }
    dqa_pre_rot(g, pos, pre);
    const float rms = dqa_stage(g, pre, xn, red4);
    const float y = dqa_dot<CH, WT, NCH>(xn, g.K, wr) / rms;
    if (tid % DQA_RL == 0) qraw[tid / DQA_RL] = y;
    __syncthreads();
    if (!ok) {
      // Refused position (the chunk blocks raise the flag): no cache row is
      // written, and the step attends from position 0, so the combine's new
      // row is the cache's row at position 0 as stored.
      const KV *row0 = static_cast<const KV *>(which ? g.vc : g.kc) + bj * g.maxc * D;
      if (tid < D) {
        float held;
        if constexpr (sizeof(KV) == 2) held = bf16_bits_to_f32(row0[tid]);
        else held = row0[tid];
        g.kvn[(bj * 2 + which) * D + tid] = held;
      }
      return bj;
    }
    KV *dst = static_cast<KV *>(which ? g.vc : g.kc) + (bj * g.maxc + pos) * D;
    // The row as the cache holds it, also where the combine reads it
    // without the position.
    auto put = [&](float y) {
      f32_put(dst + tid, y);
      float held = y;
      if constexpr (sizeof(KV) == 2) held = bf16_bits_to_f32(f32_to_bf16_bits(y));
      g.kvn[(bj * 2 + which) * D + tid] = held;
    };
    if (which == 0) {
      dqa_rope(pre, qraw, qrot);
      __syncthreads();
      if (tid < D) put(qrot[tid]);
    } else if (tid < D) {
      put(qraw[tid]);
    }
    return bj;
  }

  // (sequence, query head, key chunk)
  const int64_t GS = static_cast<int64_t>(g.G) * g.S;
  const int64_t slot = bid >> 3, bj = (bid & 7) + 8 * (slot / GS), rem = slot % GS;
  if (bj >= static_cast<int64_t>(g.B) * g.KVH) return 0;  // an empty id of the XCD-aware order
  const int64_t gg = rem / g.S, s = rem - gg * g.S;
  const int64_t b = bj / g.KVH, j = bj % g.KVH, hq = j * g.G + gg;
  // A device-held position through the scalar cache (dqa_pos_read: its wait
  // covers it alone), the weights and the hidden row, which do not wait for it.
  const int32_t pdev = dqa_pos_read(g.pa);
  typename WT::Raw wr[CH];
  dqa_wload<CH, WT, NCH>(g, hq * D, wr);
  DqaPre pre;
  dqa_pre_x(g, b, pre);
  int64_t pos = g.pa.pos0;
  if (g.pa.dev) {  // att_pos0's check for one new position
    const int64_t v = pdev;
    const bool ok = v >= 0 && v + 1 <= g.pa.span;
    if (!ok && tid == 0 && blockIdx.x == 0) atomicOr(g.pa.flags, FLAG_INDEX_RANGE);
    pos = ok ? v : 0;
  }
  const int64_t lo = s * g.chunk, len = pos > lo ? (pos - lo < g.chunk ? pos - lo : g.chunk) : 0;
  float *pb = g.part + (bj * g.S + s) * dqa_part_stride(g.G);
  float *pacc = pb + dqa_part_acc0(g.G) + gg * D;
  if (len == 0 && s != 0) {  // past the keys: the empty chunk's statistics
    if (tid == 0) {
      pb[gg] = -FLT_MAX;
      pb[g.G + gg] = 0.0f;
    }
    if (tid < D) pacc[tid] = 0.0f;
    return bj;
  }
  const KV *Kc = static_cast<const KV *>(g.kc) + (bj * g.maxc + lo) * D;
  const KV *Vc = static_cast<const KV *>(g.vc) + (bj * g.maxc + lo) * D;
  const int sl = lane % LPR, kk = lane / LPR;
  const int64_t first = static_cast<int64_t>(wave) * KPW + kk, last = len > 0 ? len - 1 : 0;
  // The first pass's key and value rows: in flight with the weights before
  // the norm waits.
  float4 kpre[U], vv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = first + u * STEP;
    kpre[u] = f32x4_get(Kc + (c < len ? c : last) * D + 4 * sl);
    vv[u] = f32x4_get(Vc + (c < len ? c : last) * D + 4 * sl);
  }
  dqa_pre_rot(g, pos, pre);
  const float rms = dqa_stage(g, pre, xn, red4);
  {
    const float y = dqa_dot<CH, WT, NCH>(xn, g.K, wr) / rms;
    if (tid % DQA_RL == 0) qraw[tid / DQA_RL] = y;
  }
  __syncthreads();
  dqa_rope(pre, qraw, qrot);
  __syncthreads();
  if (s == 0 && tid < D) g.q[(b * g.H + hq) * D + tid] = qrot[tid];

  // Scores, softmax statistics and P V of the chunk: the key-chunked
  // kernel's steps for one query head.  Each wavefront keeps the maximum of
  // its own scores (every lane of a key's LPR lanes holds the key's score),
  // so the block's maximum is a fold of NW values after the one barrier, and
  // the P V pass forms exp(score - max) and the sums itself: no pass over
  // the scores between.
  const float4 qv[1] = {*reinterpret_cast<const float4 *>(qrot + 4 * sl)};
  float mx = -INFINITY;
  for (int64_t c0 = first; c0 < len + kk; c0 += STEP * U) {
    float4 kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      kv[u] = c0 == first ? kpre[u] : f32x4_get(Kc + (c < len ? c : last) * D + 4 * sl);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      float pr[1];
      dots<1, LPR>(qv, kv[u], pr);
      const float sc = pr[0] * g.scale;
      if (c < len) {
        mx = max_nan(mx, sc);
        if (sl == 0) scores[c] = sc;
      }
    }
  }
  mx = fold_max<64>(mx);
  if (lane == 0) red4[wave] = mx;  // the norm's sums are read before the q barriers
  __syncthreads();
  float m = red4[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = max_nan(m, red4[w]);
  m = isnan(m) ? m : (m > -FLT_MAX ? m : -FLT_MAX);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.0f;
  for (int64_t c0 = first; c0 < len + kk; c0 += STEP * U) {
    if (c0 != first) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + u * STEP;
        vv[u] = f32x4_get(Vc + (c < len ? c : last) * D + 4 * sl);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + u * STEP;
      if (c < len) {
        const float pg = expf(scores[c] - m);
        if (sl == 0) lsum += pg;
        acc.x += pg * vv[u].x;
        acc.y += pg * vv[u].y;
        acc.z += pg * vv[u].z;
        acc.w += pg * vv[u].w;
      }
    }
  }
  acc.x = fold_columns<LPR>(acc.x);
  acc.y = fold_columns<LPR>(acc.y);
  acc.z = fold_columns<LPR>(acc.z);
  acc.w = fold_columns<LPR>(acc.w);
  lsum = fold_sum<64>(lsum);
  if (kk == 0) *reinterpret_cast<float4 *>(red + wave * D + 4 * sl) = acc;
  if (lane == 0) wsum[wave] = lsum;
  __syncthreads();
  if (tid == 0) {
    float l = wsum[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) l += wsum[w];
    pb[gg] = m;
    pb[g.G + gg] = l;
  }
  if (tid < D) {
    float t = red[tid];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w * D + tid];
    pacc[tid] = t;
  }
  return bj;
}

template <typename KV, int CH, typename WT, int NCH = 0>
__global__ void __launch_bounds__(DQA_NT) decode_qkv_attention_kernel(DqaArgs g) {
  extern __shared__ float dqa_sm[];
  dqa_work<KV, CH, WT, NCH>(g, dqa_sm);
}

// The combine: one block an item, the launch after the fused one.
template <int CS>
__global__ void __launch_bounds__(128) attention_combine_new_kernel(DqaArgs g, float *out) {
  extern __shared__ float wl[];
  combine_new_item<CS>(g, blockIdx.x, out, wl);
}

}  // namespace mi

// The no-allocation form's partials (mi_attention_rows_into): a file-scope
// device array, one copy per GPU the library runs on, held until the process
// ends.  Host code never passes the array's name to a kernel (in host code it
// is a stand-in, not a device address): attention_scratch_setup looks up each
// device's address once, with that device current, and the entry point uses
// that address.
constexpr size_t ATT_NOALLOC_BYTES = size_t(4) << 20;  // 1 Mi floats
static __device__ __align__(256) float scratch[ATT_NOALLOC_BYTES / sizeof(float)];

namespace mi {

constexpr int ATT_MAX_DEVICES = 64;
static std::atomic<float *> g_att_scratch[ATT_MAX_DEVICES];
static std::mutex g_att_scratch_mu;

// At context creation (mi_ctx_create), once per device: the address of this
// device's copy of `scratch`.  A failure is kept and reported by
// mi_attention_rows_into, which cannot run without it.
int attention_scratch_setup(Ctx *ctx) {
  if (ctx->device < 0 || ctx->device >= ATT_MAX_DEVICES) return MI_OK;
  std::lock_guard<std::mutex> lk(g_att_scratch_mu);
  if (g_att_scratch[ctx->device].load()) return MI_OK;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return fail(ctx, MI_E_HIP, "attention scratch: no current device");
  if (cur != ctx->device && hipSetDevice(ctx->device) != hipSuccess)
    return fail(ctx, MI_E_HIP, "attention scratch: hipSetDevice(%d)", ctx->device);
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
  if (cur != ctx->device) (void)hipSetDevice(cur);
  if (e != hipSuccess || !p)
    return fail(ctx, MI_E_HIP, "attention scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
  g_att_scratch[ctx->device].store(static_cast<float *>(p));
  return MI_OK;
}

namespace {

// A checked attention call: shapes, the key-chunk split and the partials'
// size, shared by the allocating and the no-allocation entry points so both
// run the same kernels on the same chunks.
struct AttPlan {
  const float *q;
  const void *k, *v;
  bool kv16;  // BF16 caches (else F32)
  int64_t D, G, maxc, items, S, chunk;
  size_t part_bytes;
  bool flash;  // many new positions: the matrix-core kernel
  int64_t fchunk, fS;  // its key ranges when split (fchunk 0: whole runs, no partials)
  AttPos pos;
};

// pos_dev null: the immediate pos0, chunks planned for span = pos0 + t when
// span is 0.  pos_dev set: pos0 read on the device, chunks for `span`.
int attention_plan(Ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache, int64_t batch, int64_t t, int64_t heads,
                   int64_t kv_heads, int64_t pos0, const int32_t *pos_dev, int64_t span, AttPlan *P) {
  MI_BUF(ctx, qb, q);
  MI_BUF(ctx, kb, k_cache);
  MI_BUF(ctx, vb, v_cache);
  if (qb->elem != MI_F32 || kb->elem != vb->elem || !elem_float(kb->elem))
    return fail(ctx, MI_E_ARG, "attention_rows takes F32 queries and two F32 or two BF16 caches (q %s, k %s, v %s)",
                elem_name(qb->elem), elem_name(kb->elem), elem_name(vb->elem));
  if (batch < 1 || t < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads)
    return fail(ctx, MI_E_ARG, "attention_rows: batch %lld, t %lld, heads %lld, kv heads %lld", (long long)batch,
                (long long)t, (long long)heads, (long long)kv_heads);
  const int64_t D = kb->cols, G = heads / kv_heads;
  if (G > ATT_MAX_GROUP)
    return fail(ctx, MI_E_UNSUPPORTED, "attention_rows: %lld query heads per kv head (at most %d)", (long long)G,
                ATT_MAX_GROUP);
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail(ctx, MI_E_UNSUPPORTED, "attention_rows: head width %lld (16, 32, 64 or 128)", (long long)D);
  if (qb->rows != batch * t || qb->cols != heads * D)
    return fail(ctx, MI_E_ARG, "attention_rows: q is [%lld, %lld], want [%lld, %lld]", (long long)qb->rows,
                (long long)qb->cols, (long long)(batch * t), (long long)(heads * D));
  if (vb->cols != D || vb->rows != kb->rows || kb->rows % (batch * kv_heads))
    return fail(ctx, MI_E_ARG, "attention_rows: caches must both be [batch * kv_heads * max_ctx, %lld]", (long long)D);
  const int64_t maxc = kb->rows / (batch * kv_heads);
  if (pos_dev) {
    if (span < t || span > maxc)
      return fail(ctx, MI_E_ARG, "attention_rows: span %lld for %lld new positions in a cache of %lld", (long long)span,
                  (long long)t, (long long)maxc);
  } else {
    if (pos0 < 0 || pos0 + t > maxc)
      return fail(ctx, MI_E_ARG, "attention_rows: positions %lld..%lld beyond the cache's %lld", (long long)pos0,
                  (long long)(pos0 + t), (long long)maxc);
    if (span == 0) span = pos0 + t;
    if (span < pos0 + t || span > maxc)
      return fail(ctx, MI_E_ARG, "attention_rows: span %lld for positions %lld..%lld in a cache of %lld",
                  (long long)span, (long long)pos0, (long long)(pos0 + t), (long long)maxc);
  }
  // Chunks: at least enough that none exceeds ATT_MAX_CHUNK keys, more (down
  // to ATT_MIN_CHUNK keys each) until the grid has ATT_TARGET_BLOCKS blocks --
  // decode has only batch * kv_heads query groups, and one block's chain of
  // dependent loads over a long context is slower than several short chains
  // and a combine pass.  Chunks are a multiple of 4 keys, so the LDS fold area
  // after the scores stays 16-byte aligned for its float4 stores.
  const int64_t items = batch * kv_heads * t, nmax = span;
  int64_t S = (nmax + ATT_MAX_CHUNK - 1) / ATT_MAX_CHUNK;
  const int64_t want = (ATT_TARGET_BLOCKS + items - 1) / items;
  // With many items (a batch of sequences) longer chunks: fewer blocks and
  // partials to combine (batch-32 decode 1.94 -> 1.89 ms a step at 128 keys;
  // batch 1 is fastest at 64).
  const int64_t min_chunk = items >= 64 ? 2 * ATT_MIN_CHUNK : ATT_MIN_CHUNK;
  const int64_t cap = (nmax + min_chunk - 1) / min_chunk;
  if (want > S) S = want < cap ? want : cap;
  if (S < 1) S = 1;
  const int64_t chunk = ((nmax + S - 1) / S + 3) / 4 * 4;
  S = (nmax + chunk - 1) / chunk;
  if (items > INT32_MAX || S > 65535) return fail(ctx, MI_E_UNSUPPORTED, "attention_rows: grid too large");
  if (static_cast<size_t>(3 * G * S + G) * sizeof(float) > 65536)
    return fail(ctx, MI_E_UNSUPPORTED, "attention_rows: context of %lld keys too long", (long long)nmax);
  P->q = static_cast<const float *>(qb->ptr);
  P->k = kb->ptr;
  P->v = vb->ptr;
  P->kv16 = kb->elem == MI_BF16;
  P->D = D; P->G = G; P->maxc = maxc; P->items = items; P->S = S; P->chunk = chunk;
  // The matrix-core kernel for 64+ new positions with 64-wide heads, its
  // keys split into ranges on small grids (whole, paired runs of a 512-token
  // prompt at batch 1 took 4.27 ms against 3.92 on the key-chunked kernel).
  P->flash = !pos_dev && span == pos0 + t && D == 64 && t >= FLASH_MIN_T && batch * kv_heads <= 65535;
  P->fchunk = P->fS = 0;
  const int64_t runs = (t + 31) / 32 * batch * kv_heads;
  if (P->flash && runs < FLASH_MIN_BLOCKS) {
    P->fchunk = runs * ((pos0 + t + 127) / 128) >= FLASH_MIN_BLOCKS ? 128 : 64;
    P->fS = (pos0 + t + P->fchunk - 1) / P->fchunk;
    if (P->fS > 65535 || static_cast<size_t>(3 * G * P->fS + G) * sizeof(float) > 65536) P->flash = false;
  }
  P->pos = AttPos{pos0, pos_dev, span, flags(ctx)};
  if (P->flash)
    P->part_bytes = P->fchunk ? static_cast<size_t>(items * P->fS * G * (D + 2)) * sizeof(float) : 0;
  else
    P->part_bytes = S > 1 ? static_cast<size_t>(items * S * G * (D + 2)) * sizeof(float) : 0;
  return MI_OK;
}

template <typename KV>
void attention_launch_kv(Ctx *ctx, const AttPlan &P, const AttOut &ao, float *part, int64_t batch, int64_t t,
                         int64_t heads, int64_t kv_heads, float scale) {
  const KV *k = static_cast<const KV *>(P.k), *v = static_cast<const KV *>(P.v);
  if (P.flash) {
    flash_dispatch<KV>(P.G, ctx->stream, P.q, k, v, ao, batch, t, heads, kv_heads, P.pos.pos0, P.maxc, scale,
                       P.fchunk, static_cast<int>(P.fS), part);
    return;
  }
  float *out = static_cast<float *>(ao.p);  // the chunk kernels write F32 rows
  const int Si = static_cast<int>(P.S);
  switch (P.D) {
    case 16: dispatch_group<16, KV>(P.G, ctx->stream, P.q, k, v, out, part, P.items, Si, t, heads, kv_heads, P.pos, P.maxc, P.chunk, scale); break;
    case 32: dispatch_group<32, KV>(P.G, ctx->stream, P.q, k, v, out, part, P.items, Si, t, heads, kv_heads, P.pos, P.maxc, P.chunk, scale); break;
    case 64: dispatch_group<64, KV>(P.G, ctx->stream, P.q, k, v, out, part, P.items, Si, t, heads, kv_heads, P.pos, P.maxc, P.chunk, scale); break;
    default: dispatch_group<128, KV>(P.G, ctx->stream, P.q, k, v, out, part, P.items, Si, t, heads, kv_heads, P.pos, P.maxc, P.chunk, scale); break;
  }
}

// The result in `ao`: any form on the matrix-core (flash) path, F32 rows on
// the chunk kernels'.
void attention_launch(Ctx *ctx, const AttPlan &P, const AttOut &ao, float *part, int64_t batch, int64_t t,
                      int64_t heads, int64_t kv_heads, float scale) {
  if (P.kv16)
    attention_launch_kv<uint16_t>(ctx, P, ao, part, batch, t, heads, kv_heads, scale);
  else
    attention_launch_kv<float>(ctx, P, ao, part, batch, t, heads, kv_heads, scale);
}
void attention_launch(Ctx *ctx, const AttPlan &P, float *out, float *part, int64_t batch, int64_t t, int64_t heads,
                      int64_t kv_heads, float scale) {
  AttOut o;
  o.p = out;
  o.R = batch * t;
  o.C = heads * P.D;
  attention_launch(ctx, P, o, part, batch, t, heads, kv_heads, scale);
}

// The result of a planned call into a new buffer (partials in the context's
// scratch).
int attention_new(mi_ctx *ctx, const AttPlan &P, int64_t batch, int64_t t, int64_t heads, int64_t kv_heads, float scale,
                  const char *what, mi_id *out, int form = MI_F32) {
  const int64_t R = batch * t, C = heads * P.D;
  const bool tiled = form == MI_TILES_BF16 || form == MI_TILES_PARTS;
  if (tiled && (R % 32 || C % 16))
    return fail(ctx, MI_E_ARG, "%s: tiles of [%lld, %lld] (rows a multiple of 32, columns of 16)", what, (long long)R,
                (long long)C);
  // The chunk kernels write F32 rows: another form from them is converted.
  if (form != MI_F32 && !P.flash) {
    mi_id f;
    if (int s = attention_new(ctx, P, batch, t, heads, kv_heads, scale, what, &f)) return s;
    const int s = tiled ? mi_tile(ctx, f, form, out) : mi_cast(ctx, f, form, out);
    mi_free(ctx, f);  // stream-ordered
    return s;
  }
  float *part = nullptr;
  if (P.part_bytes) {
    part = static_cast<float *>(mi::scratch(ctx, P.part_bytes));
    if (!part) return fail(ctx, MI_E_OOM, "%s scratch", what);
  }
  mi_id id;
  Buffer *ob;
  const bool parts = form == MI_TILES_PARTS || form == MI_BF16_PARTS;
  int s = new_buffer(ctx, R, parts ? 2 * C : C, form == MI_F32 ? MI_F32 : MI_BF16, &id, &ob);
  if (s) return s;
  ob->tiles = tiled ? form : 0;
  AttOut o;
  o.p = ob->ptr;
  o.form = form;
  o.R = R;
  o.C = C;
  attention_launch(ctx, P, o, part, batch, t, heads, kv_heads, scale);
  s = check_launch(ctx, what);
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}

}  // namespace

}  // namespace mi

using namespace mi;

extern "C" int mi_attention_rows(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache, int64_t batch, int64_t t,
                                 int64_t heads, int64_t kv_heads, int64_t pos0, float scale, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  AttPlan P;
  int s = attention_plan(ctx, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, nullptr, 0, &P);
  if (s) return s;
  return attention_new(ctx, P, batch, t, heads, kv_heads, scale, "attention_rows", out);
}

extern "C" int mi_attention_rows_as(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache, int64_t batch, int64_t t,
                                    int64_t heads, int64_t kv_heads, int64_t pos0, float scale, int out_form,
                                    mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  if (out_form != MI_F32 && out_form != MI_BF16 && out_form != MI_BF16_PARTS && out_form != MI_TILES_BF16 &&
      out_form != MI_TILES_PARTS)
    return fail(ctx, MI_E_ARG, "attention_rows_as: result form %d", out_form);
  AttPlan P;
  int s = attention_plan(ctx, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, nullptr, 0, &P);
  if (s) return s;
  return attention_new(ctx, P, batch, t, heads, kv_heads, scale, "attention_rows_as", out, out_form);
}

extern "C" int mi_attention_rows_at(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache, int64_t batch, int64_t t,
                                    int64_t heads, int64_t kv_heads, mi_id pos, int64_t pos0, int64_t span,
                                    float scale, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  const int32_t *pos_dev = nullptr;
  if (pos) {
    MI_BUF(ctx, pb, pos);
    if (pb->elem != MI_I32 || pb->numel() != 1)
      return fail(ctx, MI_E_ARG, "attention_rows_at: the position is %s [%lld, %lld], want I32 [1, 1]",
                  elem_name(pb->elem), (long long)pb->rows, (long long)pb->cols);
    pos_dev = static_cast<const int32_t *>(pb->ptr);
  }
  if (span < 1) return fail(ctx, MI_E_ARG, "attention_rows_at: span %lld", (long long)span);
  AttPlan P;
  int s = attention_plan(ctx, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, pos_dev, span, &P);
  if (s) return s;
  return attention_new(ctx, P, batch, t, heads, kv_heads, scale, "attention_rows_at", out);
}

extern "C" int mi_attention_rows_into(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache, int64_t batch, int64_t t,
                                      int64_t heads, int64_t kv_heads, int64_t pos0, float scale, mi_id out) {
  MI_ENTER(ctx);
  AttPlan P;
  int s = attention_plan(ctx, q, k_cache, v_cache, batch, t, heads, kv_heads, pos0, nullptr, 0, &P);
  if (s) return s;
  MI_BUF(ctx, ob, out);
  if (out == q || out == k_cache || out == v_cache)
    return fail(ctx, MI_E_ARG, "attention_rows_into: the output is one of the inputs");
  if (ob->elem != MI_F32 || ob->rows != batch * t || ob->cols != heads * P.D)
    return fail(ctx, MI_E_ARG, "attention_rows_into: output is [%lld, %lld] %s, want [%lld, %lld] F32",
                (long long)ob->rows, (long long)ob->cols, elem_name(ob->elem), (long long)(batch * t),
                (long long)(heads * P.D));
  if (P.part_bytes > ATT_NOALLOC_BYTES)
    return fail(ctx, MI_E_UNSUPPORTED,
                "attention_rows_into: %zu bytes of key-chunk partials, beyond the %zu the no-allocation form holds",
                P.part_bytes, ATT_NOALLOC_BYTES);
  float *part = nullptr;
  if (P.part_bytes) {
    part = ctx->device >= 0 && ctx->device < ATT_MAX_DEVICES ? g_att_scratch[ctx->device].load() : nullptr;
    if (!part) return fail(ctx, MI_E_HIP, "attention_rows_into: no scratch address for device %d", ctx->device);
  }
  attention_launch(ctx, P, static_cast<float *>(ob->ptr), part, batch, t, heads, kv_heads, scale);
  return check_launch(ctx, "attention_rows_into");
}

namespace mi {
namespace {

// The fused launch, then the combine's.
template <typename KV, typename WT>
void launch_dqa_w(hipStream_t st, const DqaArgs &g, unsigned blocks, size_t lds) {
  const int64_t ch = (g.K / 8 + DQA_RL - 1) / DQA_RL;  // chunks a thread
  if (g.K == 576)  // SmolLM2's width: 9 chunks a thread exactly
    decode_qkv_attention_kernel<KV, 9, WT, 576 / 8><<<blocks, DQA_NT, lds, st>>>(g);
  else if (ch <= 4) decode_qkv_attention_kernel<KV, 4, WT><<<blocks, DQA_NT, lds, st>>>(g);
  else if (ch <= 8) decode_qkv_attention_kernel<KV, 8, WT><<<blocks, DQA_NT, lds, st>>>(g);
  else if (ch <= 12) decode_qkv_attention_kernel<KV, 12, WT><<<blocks, DQA_NT, lds, st>>>(g);
  else decode_qkv_attention_kernel<KV, DQA_MAX_CH * 4 / DQA_RL, WT><<<blocks, DQA_NT, lds, st>>>(g);
}

// out null: the fused launch only (its combine is the caller's).
template <typename KV>
void launch_dqa(hipStream_t st, const DqaArgs &g, float *out) {
  const unsigned blocks = static_cast<unsigned>(dqa_chunk_ids(g) + 2 * static_cast<int64_t>(g.B) * g.KVH);
  const size_t lds = static_cast<size_t>(g.K + 2 * DQA_D + DQA_NW + g.chunk + DQA_NW * DQA_D + DQA_NW) * sizeof(float);
  if (g.wq) launch_dqa_w<KV, DqaBfp8>(st, g, blocks, lds);
  else launch_dqa_w<KV, DqaBf16>(st, g, blocks, lds);
  if (!out) return;
  const unsigned threads = g.G <= 4 ? 64 : 128, items = static_cast<unsigned>(static_cast<int64_t>(g.B) * g.KVH);
  const size_t comb = static_cast<size_t>(threads / 16 * g.S) * sizeof(float);
  switch (combine_cs(g.S)) {
    case 4: attention_combine_new_kernel<4><<<items, threads, comb, st>>>(g, out); break;
    case 8: attention_combine_new_kernel<8><<<items, threads, comb, st>>>(g, out); break;
    case 12: attention_combine_new_kernel<12><<<items, threads, comb, st>>>(g, out); break;
    default: attention_combine_new_kernel<16><<<items, threads, comb, st>>>(g, out); break;
  }
}

}  // namespace
}  // namespace mi

// w_o 0: the attention rows (mi_norm_qkv_attention); else x + those rows
// times w_o^T (mi_norm_qkv_attention_o).
static int norm_qkv_attention(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table,
                              mi_id sin_table, int64_t heads, int64_t kv_heads, mi_id pos, int64_t pos0, int64_t span,
                              mi_id k_cache, mi_id v_cache, float scale, mi_id w_o, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  // With w_o and no launch of its own: the attention rows, then the
  // projection (which checks w_o against them and x).
  auto project = [&](int s, mi_id o) {
    if (s || !w_o) {
      if (!s) *out = o;
      return s;
    }
    s = mi_norm_matvec(ctx, o, 0, 0.0f, w_o, x, 0, out);
    mi_free(ctx, o);
    return s;
  };
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, wb, w_qkv);
  MI_BUF(ctx, cb, cos_table);
  MI_BUF(ctx, sb, sin_table);
  MI_BUF(ctx, kb, k_cache);
  MI_BUF(ctx, vb, v_cache);
  const Buffer *gb = nullptr;
  if (gamma) {
    gb = lookup(ctx, gamma);
    if (!gb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)gamma);
  }
  const int32_t *pos_dev = nullptr;
  if (pos) {
    MI_BUF(ctx, pb, pos);
    if (pb->elem != MI_I32 || pb->numel() != 1)
      return fail(ctx, MI_E_ARG, "norm_qkv_attention: the position is %s [%lld, %lld], want I32 [1, 1]",
                  elem_name(pb->elem), (long long)pb->rows, (long long)pb->cols);
    pos_dev = static_cast<const int32_t *>(pb->ptr);
  }
  const int64_t B = xb->rows, K = xb->cols, D = kb->cols;
  const int64_t G = kv_heads > 0 ? heads / kv_heads : 0;
  const int64_t maxc = B > 0 && kv_heads > 0 ? kb->rows / (B * kv_heads) : 0;
  const Buffer *wob = nullptr;
  if (w_o) {  // checked before anything is written
    wob = lookup(ctx, w_o);
    if (!wob) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)w_o);
    if ((wob->elem != MI_BF16 && wob->elem != MI_BFP8) || wob->rows != K || wob->cols != heads * D ||
        xb->elem != MI_F32)
      return fail(ctx, MI_E_ARG, "norm_qkv_attention_o: the o weight is %s [%lld, %lld], want BF16 or BFP8 [%lld, %lld]",
                  elem_name(wob->elem), (long long)wob->rows, (long long)wob->cols, (long long)K,
                  (long long)(heads * D));
  }
  // The fused launch: up to DQA_MAX_B sequences, 64-wide heads, k a
  // multiple of 32 up to 1024, a gain, aligned operands; else the two calls
  // composed (which check every argument themselves).
  const bool fused = B >= 1 && B <= DQA_MAX_B && D == DQA_D && K % 32 == 0 && K <= 32 * DQA_MAX_CH && gb &&
                     xb->elem == MI_F32 && (wb->elem == MI_BF16 || (wb->elem == MI_BFP8 && K % 16 == 0)) &&
                     wb->cols == K && heads >= 1 && kv_heads >= 1 &&
                     heads % kv_heads == 0 && G <= ATT_MAX_GROUP && wb->rows == (heads + 2 * kv_heads) * D &&
                     kb->elem == vb->elem && elem_float(kb->elem) && vb->cols == D && vb->rows == kb->rows &&
                     kb->rows % (B * kv_heads) == 0 && gb->elem == MI_F32 && gb->rows * gb->cols == K &&
                     cb->elem == MI_F32 && sb->elem == MI_F32 && cb->cols == D && sb->cols == D &&
                     cb->rows >= maxc && sb->rows >= maxc &&
                     ((reinterpret_cast<uintptr_t>(xb->ptr) | reinterpret_cast<uintptr_t>(wb->ptr) |
                       reinterpret_cast<uintptr_t>(gb->ptr)) & 15) == 0;
  if (!fused) {
    mi_id q = 0, o = 0;
    int s = pos_dev ? mi_norm_qkv_rope_at(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, pos,
                                          k_cache, v_cache, &q)
                    : mi_norm_qkv_rope(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, pos0,
                                       k_cache, v_cache, &q);
    if (s) return s;
    s = mi_attention_rows_at(ctx, q, k_cache, v_cache, B, 1, heads, kv_heads, pos, pos0, span, scale, &o);
    mi_free(ctx, q);
    return project(s, o);
  }
  if (span < 1 || span > maxc)
    return fail(ctx, MI_E_ARG, "norm_qkv_attention: span %lld in a cache of %lld", (long long)span, (long long)maxc);
  if (!pos_dev && (pos0 < 0 || pos0 + 1 > span))
    return fail(ctx, MI_E_ARG, "norm_qkv_attention: position %lld beyond the span %lld", (long long)pos0,
                (long long)span);
  // The key chunks as mi_attention_rows_at plans them for one new position.
  const int64_t items = B * kv_heads;
  int64_t S = (span + ATT_MAX_CHUNK - 1) / ATT_MAX_CHUNK;
  const int64_t want = (ATT_TARGET_BLOCKS + items - 1) / items;
  const int64_t min_chunk = items >= 64 ? 2 * ATT_MIN_CHUNK : ATT_MIN_CHUNK;
  const int64_t cap = (span + min_chunk - 1) / min_chunk;
  if (want > S) S = want < cap ? want : cap;
  if (S < 1) S = 1;
  const int64_t chunk = ((span + S - 1) / S + 3) / 4 * 4;
  S = (span + chunk - 1) / chunk;
  if (static_cast<size_t>(16 * S) * sizeof(float) > 65536 || 8 * (B * heads + 8 * G) * S + 2 * items > INT32_MAX)
    return fail(ctx, MI_E_UNSUPPORTED, "norm_qkv_attention: context of %lld keys too long", (long long)span);
  const size_t part_floats = static_cast<size_t>(items * S * dqa_part_stride(G));
  const size_t q_floats = static_cast<size_t>(B * heads * D), kvn_floats = static_cast<size_t>(items * 2 * D);
  float *sc = static_cast<float *>(mi::scratch(ctx, (part_floats + q_floats + kvn_floats) * sizeof(float)));
  if (!sc) return fail(ctx, MI_E_OOM, "norm_qkv_attention scratch");
  // One sequence, a BF16 or BFP8 o weight [K, heads 64]: the combine runs
  // inside the o projection's launch.
  const bool fuse_o = wob && B == 1 && (wob->elem == MI_BF16 || wob->elem == MI_BFP8) && wob->rows == K &&
                      wob->cols == heads * D && attention_o_fits(heads, S) &&
                      (reinterpret_cast<uintptr_t>(wob->ptr) & 15) == 0;
  mi_id id;
  Buffer *ob;
  int s = new_buffer(ctx, B, fuse_o ? K : heads * D, MI_F32, &id, &ob);
  if (s) return s;
  DqaArgs g{};
  g.x = static_cast<const float *>(xb->ptr);
  g.K = K;
  g.gamma = static_cast<const float *>(gb->ptr);
  g.eps = eps;
  if (wb->elem == MI_BFP8) {
    g.wq = static_cast<const int8_t *>(wb->ptr);
    g.we = static_cast<const uint8_t *>(wb->ptr) + bfp8_exp_offset(wb->rows, wb->cols);
  } else {
    g.w = static_cast<const uint16_t *>(wb->ptr);
  }
  g.cos = static_cast<const float *>(cb->ptr);
  g.sin = static_cast<const float *>(sb->ptr);
  g.kc = kb->ptr;
  g.vc = vb->ptr;
  g.maxc = maxc;
  g.H = static_cast<int>(heads);
  g.KVH = static_cast<int>(kv_heads);
  g.G = static_cast<int>(G);
  g.B = static_cast<int>(B);
  g.pa = AttPos{pos0, pos_dev, span, flags(ctx)};
  g.S = S;
  g.chunk = chunk;
  g.scale = scale;
  g.part = sc;
  g.q = sc + part_floats;
  g.kvn = g.q + q_floats;
  float *o = static_cast<float *>(ob->ptr);
  if (fuse_o) {
    if (kb->elem == MI_BF16) launch_dqa<uint16_t>(ctx->stream, g, nullptr);
    else launch_dqa<float>(ctx->stream, g, nullptr);
    s = check_launch(ctx, "norm_qkv_attention");
    if (!s)
      s = attention_o_launch(ctx, AttnCombine{g.part, g.q, g.kvn, g.H, g.G, static_cast<int>(S), scale}, wob,
                             static_cast<const float *>(xb->ptr), o);
    if (s) {
      mi_free(ctx, id);
      return s;
    }
    *out = id;
    return MI_OK;
  }
  if (kb->elem == MI_BF16) launch_dqa<uint16_t>(ctx->stream, g, o);
  else launch_dqa<float>(ctx->stream, g, o);
  s = check_launch(ctx, "norm_qkv_attention");
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  return project(MI_OK, id);
}

extern "C" int mi_norm_qkv_attention(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table,
                                     mi_id sin_table, int64_t heads, int64_t kv_heads, mi_id pos, int64_t pos0,
                                     int64_t span, mi_id k_cache, mi_id v_cache, float scale, mi_id *out) {
  return norm_qkv_attention(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, pos, pos0, span,
                            k_cache, v_cache, scale, 0, out);
}

extern "C" int mi_norm_qkv_attention_o(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table,
                                       mi_id sin_table, int64_t heads, int64_t kv_heads, mi_id pos, int64_t pos0,
                                       int64_t span, mi_id k_cache, mi_id v_cache, float scale, mi_id w_o,
                                       mi_id *out) {
  MI_ENTER(ctx);
  if (!w_o) return fail(ctx, MI_E_ARG, "norm_qkv_attention_o: no o weight");
  return norm_qkv_attention(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, pos, pos0, span,
                            k_cache, v_cache, scale, w_o, out);
}
