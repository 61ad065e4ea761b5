// Fused decode projections: a few activation rows (one per sequence) times a
// BF16 weight, with the neighbouring element-wise work folded in so that a
// decoder layer's step is six launches instead of eighteen.
//
// Reference: the fused projections of crates/tt-models/src/llama.rs:655-672
// (`Llama::fused`: each layer's q|k|v and gate|up weights one matrix each,
// every output column keeping its own accumulation) composed with the ops the
// decode step runs around them -- Engine::rms_norm_as (crates/burn-tt/src/
// server.rs:449; ops/norm.rs:39-283), Engine::rope_blocks (server.rs:566;
// ops/rope.rs:27-240), the KV-cache `slice_assign` (llama.rs:415-435), the
// residual add, and silu(gate) * up (ops.rs:2622-2651).
//
// MI355X design.  Decode reads every weight once per step: the kernels are
// HBM-latency-bound GEMVs.  Up to 6 activation rows (up to 8 where the
// matrix-core form below does not fit the shape) a wavefront owns two output
// rows of the weight and all M activation rows; each lane streams 16 bytes
// (8 BF16) of both weight rows per step, so a 576-wide row is read by the
// wavefront in two coalesced passes.  The activation rows (a few KB) are
// re-read from cache by every wavefront; when a gain is given each wavefront
// multiplies the rows by it on the fly and divides its finished sums by the
// rows' rms (folded from the same values), so the normalised rows never touch
// HBM.  The two rows a
// wavefront owns are chosen so that the epilogue is local: a RoPE pair
// (i, i + d/2) of one head, or a gate row and its up row.
#include <cfloat>
#include <type_traits>

#include "combine.hpp"
#include "common.hpp"
#include "wave.hpp"

namespace mi {

enum DecodeMode { DM_PLAIN = 0, DM_SILU_MUL = 1, DM_QKV = 2 };
constexpr int DECODE_MAX_M = 32;

struct DecodeArgs {
  const float *x;  // [M, K] F32, rows ldx apart
  int64_t ldx, K;
  const float *gamma;  // [1, K] RMSNorm gain, or null for no norm
  float eps;
  const uint16_t *w;  // [N, K] BF16, k-contiguous
  // Or a BFP8 weight (WBfp8 below): datums [N, K] signed bytes and block
  // exponents [N, K / 16] bytes, K a multiple of 16.
  const int8_t *wq;
  const uint8_t *we;
  int64_t N, npairs;
  // DM_PLAIN: pair p = rows (2p, 2p + 1), out [M, N] (+ resid [M, N]).
  // DM_SILU_MUL: pair p = rows (p, p + inter), out [M, inter].
  const float *resid;
  float *out;
  int64_t ldo, inter;
  // DM_QKV: pair p = rows (h d + i, h d + i + d / 2) of head h = p / (d / 2)
  // over heads q 0..H-1, k H..H+KVH-1, v H+KVH..H+2KVH-1; q to `out`, k and v
  // into the caches at position pos of item (row m, kv head): F32, or BF16
  // (kv16; rounded to nearest even as stored).  pos_dev set: the position is
  // read on the device (a traced decode step's input); outside [0, maxc) the
  // step writes no cache row and no q, and raises the range flag.
  int d, H, KVH;
  int64_t pos, maxc;
  const float *cos, *sin;
  void *kc, *vc;
  int kv16;
  const int32_t *pos_dev;
  uint32_t *flags;
  // Split-k matrix-core form: S partial sums per output and each activation
  // row's partial sum of squares (see decode_mfma_split_kernel).
  float *part;
  int split;
};

// Two values of one cache row, elements hi and hi + half of the row at `at`.
__device__ __forceinline__ void cache_pair(const DecodeArgs &g, void *base, int64_t at, int64_t hi, int64_t half,
                                           float a, float b) {
  if (g.kv16) {
    uint16_t *o = static_cast<uint16_t *>(base) + at;
    o[hi] = f32_to_bf16_bits(a);
    o[hi + half] = f32_to_bf16_bits(b);
  } else {
    float *o = static_cast<float *>(base) + at;
    o[hi] = a;
    o[hi + half] = b;
  }
}

__device__ __forceinline__ void bf16x8(uint4 q, float (&w)[8]) {
  const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    w[2 * e] = __uint_as_float(u[e] << 16);
    w[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
  }
}

// How a kernel reads eight consecutive weights of row r from k (a multiple
// of 8): a BF16 weight as one 16-byte load; a BFP8 weight as its 8 datum
// bytes and the block's exponent byte, decoded exactly to the values the
// BF16 weight holding them would give -- so a product over BFP8 weights has
// the BF16 kernel's bits.  Raw is what is held in registers between the
// load and the use.
struct WBf16 {
  using Raw = uint4;
  template <bool NT>
  static __device__ __forceinline__ Raw load(const DecodeArgs &g, int64_t r, int64_t k) {
    return ldu4<NT>(g.w + r * g.K + k);
  }
  static __device__ __forceinline__ void f32(const Raw &q, float (&w)[8]);
  static __device__ __forceinline__ uint4 bf16(const Raw &q) { return q; }
};
struct WBfp8 {
  struct Raw {
    uint2 d;
    int e;
  };
  template <bool NT>
  static __device__ __forceinline__ Raw load(const DecodeArgs &g, int64_t r, int64_t k) {
    Raw q;
    q.d = *reinterpret_cast<const uint2 *>(g.wq + r * g.K + k);
    q.e = g.we[r * (g.K >> 4) + (k >> 4)];
    return q;
  }
  static __device__ __forceinline__ void f32(const Raw &q, float (&w)[8]) { bfp8x8(q.d, q.e, w); }
  static __device__ __forceinline__ uint4 bf16(const Raw &q) {
    float w[8];
    bfp8x8(q.d, q.e, w);
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = (__float_as_uint(w[2 * i]) >> 16) | (__float_as_uint(w[2 * i + 1]) & 0xffff0000u);
    return make_uint4(h[0], h[1], h[2], h[3]);
  }
};
__device__ __forceinline__ void WBf16::f32(const Raw &q, float (&w)[8]) { bf16x8(q, w); }

__device__ __forceinline__ float silu2(float a) {
  // a * sigmoid(a), the sigmoid in the two-branch form of the element-wise op.
  const float s = sigmoid2(a);
  return a * s;
}

// The two weight rows of pair p, chosen so the epilogue is local.
struct PairRows {
  int64_t r0, r1, head, hi;
  bool has1;
};
template <int MODE>
__device__ __forceinline__ PairRows pair_rows(const DecodeArgs &g, int64_t p) {
  PairRows q{0, 0, 0, 0, true};
  if constexpr (MODE == DM_PLAIN) {
    q.r0 = 2 * p;
    q.r1 = 2 * p + 1;
  } else if constexpr (MODE == DM_SILU_MUL) {
    q.r0 = p;
    q.r1 = p + g.inter;
  } else {
    const int half = g.d / 2;
    q.head = p / half;
    q.hi = p % half;
    q.r0 = q.head * g.d + q.hi;
    q.r1 = q.r0 + half;
  }
  q.has1 = q.r1 < g.N;
  return q;
}

// The epilogue's operands of activation row m, requested with the weights so
// they have landed by the time the sums are folded: the residual values
// (DM_PLAIN; without a residual a harmless read of the output), or the
// rotary table entries at the position (DM_QKV; a position read on the
// device and out of range reads row 0 and is refused at the write).
struct PairPre {
  float v0, v1, v2, v3;
  int64_t pos;
  bool ok;
};
template <int MODE>
__device__ __forceinline__ PairPre pair_pre(const DecodeArgs &g, const PairRows &q, int64_t m) {
  PairPre e{0.0f, 0.0f, 0.0f, 0.0f, g.pos, true};
  if constexpr (MODE == DM_PLAIN) {
    const float *rp = g.resid ? g.resid : g.out;
    e.v0 = rp[m * g.ldo + q.r0];
    e.v1 = rp[m * g.ldo + (q.has1 ? q.r1 : q.r0)];
  } else if constexpr (MODE == DM_QKV) {
    if (g.pos_dev) {
      const int64_t v = scalar_read_i32(g.pos_dev);
      e.ok = v >= 0 && v < g.maxc;
      e.pos = e.ok ? v : 0;
    }
    const int64_t half = g.d / 2;
    const float *cs = g.cos + e.pos * g.d, *sn = g.sin + e.pos * g.d;
    e.v0 = cs[q.hi];
    e.v1 = cs[q.hi + half];
    e.v2 = sn[q.hi];
    e.v3 = sn[q.hi + half];
  }
  return e;
}

// Activation row m's outputs of the pair: y0, y1 its two products, the
// epilogue's operands e from pair_pre.
template <int MODE>
__device__ __forceinline__ void pair_write_pre(const DecodeArgs &g, const PairRows &q, int64_t m, float y0, float y1,
                                               const PairPre &e) {
  if constexpr (MODE == DM_PLAIN) {
    float *o = g.out + m * g.ldo;
    o[q.r0] = g.resid ? __fadd_rn(e.v0, y0) : y0;
    if (q.has1) o[q.r1] = g.resid ? __fadd_rn(e.v1, y1) : y1;
  } else if constexpr (MODE == DM_SILU_MUL) {
    g.out[m * g.ldo + q.r0] = silu2(y0) * y1;
  } else {
    const int64_t half = g.d / 2, hi = q.hi, head = q.head, pos = e.pos;
    if (!e.ok) {
      if (m == 0 && hi == 0 && head == 0) atomicOr(g.flags, FLAG_INDEX_RANGE);
      return;
    }
    if (head < g.H + g.KVH) {
      const float o0 = __fadd_rn(__fmul_rn(y0, e.v0), __fmul_rn(y1, e.v2));
      const float o1 = __fadd_rn(__fmul_rn(y1, e.v1), __fmul_rn(y0, e.v3));
      if (head < g.H) {
        float *o = g.out + m * g.ldo + head * g.d;
        o[hi] = o0;
        o[hi + half] = o1;
      } else {
        cache_pair(g, g.kc, ((m * g.KVH + (head - g.H)) * g.maxc + pos) * g.d, hi, half, o0, o1);
      }
    } else {
      cache_pair(g, g.vc, ((m * g.KVH + (head - g.H - g.KVH)) * g.maxc + pos) * g.d, hi, half, y0, y1);
    }
  }
}

template <int MODE>
__device__ __forceinline__ void pair_write(const DecodeArgs &g, const PairRows &q, int64_t m, float y0, float y1) {
  pair_write_pre<MODE>(g, q, m, y0, y1, pair_pre<MODE>(g, q, m));
}

// PRE: 16-byte chunks a lane requested up front (k <= 512 PRE), 2 or 4.
// NTW: the weights streamed (non-temporal loads), for a weight larger than
// the caches keep between steps -- the vocabulary head -- so it does not
// displace the layers' weights from the last-level cache (batch-1 SmolLM2
// decode 0.713 -> 0.697 ms a step).
template <int M, int MODE, int PRE = 4, bool NTW = false, typename WT = WBf16>
__global__ void __launch_bounds__(256) decode_matvec_kernel(DecodeArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t p = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (p >= g.npairs) return;  // whole wavefronts
  const PairRows q = pair_rows<MODE>(g, p);
  const int64_t r1c = q.has1 ? q.r1 : q.r0;

  // The weight rows are independent of the norm: with K <= 512 PRE all of
  // them are requested first, and up to 4 rows the activation rows and the
  // gain with them into registers, so the products wait for one round trip.
  // The norm scales the finished sums -- sum_k x g w / rms -- so the
  // products do not wait for its fold either.  The loads are unconditional,
  // from clamped rows and columns: a load under a condition compiles to a
  // branch that waits for it before the next is issued (0.956 -> 0.922 ms a
  // batch-1 SmolLM2 decode step).  Without a second row (a lone last row)
  // the first is read twice and the second product is discarded by
  // pair_write.
  constexpr bool XPRE = M <= 4;
  constexpr int XM = XPRE ? M : 1, XC = XPRE ? PRE : 1;
  typename WT::Raw pw0[PRE], pw1[PRE];
  float4 px[XM][XC][2], pg[XC][2];
  const bool pre_k = g.K <= 512 * PRE;
  if (pre_k) {
    const float *gp = g.gamma ? g.gamma : g.x;  // without a gain: read, never used
#pragma unroll
    for (int c = 0; c < PRE; ++c) {
      const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * c;
      const int64_t kc = k < g.K ? k : g.K - 8;
      pw0[c] = WT::template load<NTW>(g, q.r0, kc);
      pw1[c] = WT::template load<NTW>(g, r1c, kc);
      if constexpr (XPRE) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          px[m][c][0] = *reinterpret_cast<const float4 *>(g.x + m * g.ldx + kc);
          px[m][c][1] = *reinterpret_cast<const float4 *>(g.x + m * g.ldx + kc + 4);
        }
        pg[c][0] = *reinterpret_cast<const float4 *>(gp + kc);
        pg[c][1] = *reinterpret_cast<const float4 *>(gp + kc + 4);
      }
    }
  }
  const PairPre pre = pair_pre<MODE>(g, q, lane < M ? lane : 0);
  const bool inreg = XPRE && pre_k;

  // Activation row m at k (chunk c of the prefetch): its 8 values.
  auto xrow = [&](int m, int c, int64_t k, float4 &a0, float4 &a1) {
    if (inreg) {
      a0 = px[XPRE ? m : 0][XPRE ? c : 0][0];
      a1 = px[XPRE ? m : 0][XPRE ? c : 0][1];
    } else {
      a0 = *reinterpret_cast<const float4 *>(g.x + m * g.ldx + k);
      a1 = *reinterpret_cast<const float4 *>(g.x + m * g.ldx + k + 4);
    }
  };

  float acc[M][2];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m][0] = acc[m][1] = 0.0f;
  float ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) ss[m] = 0.0f;
  // One 8-wide k step: the activations times the gain, times both rows; and
  // the rows' sums of squares for the norm.
  auto step = [&](int c, int64_t k, const float (&w0)[8], const float (&w1)[8]) {
    float gm[8];
    if (g.gamma) {
      float4 g0, g1;
      if (inreg) {
        g0 = pg[XPRE ? c : 0][0];
        g1 = pg[XPRE ? c : 0][1];
      } else {
        g0 = *reinterpret_cast<const float4 *>(g.gamma + k);
        g1 = *reinterpret_cast<const float4 *>(g.gamma + k + 4);
      }
      gm[0] = g0.x; gm[1] = g0.y; gm[2] = g0.z; gm[3] = g0.w;
      gm[4] = g1.x; gm[5] = g1.y; gm[6] = g1.z; gm[7] = g1.w;
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float av[8];
      {
        float4 a0, a1;
        xrow(m, c, k, a0, a1);
        av[0] = a0.x; av[1] = a0.y; av[2] = a0.z; av[3] = a0.w;
        av[4] = a1.x; av[5] = a1.y; av[6] = a1.z; av[7] = a1.w;
      }
      if (g.gamma) {
        float t = ss[m];
#pragma unroll
        for (int e = 0; e < 8; ++e) t = fmaf(av[e], av[e], t);
        ss[m] = t;
#pragma unroll
        for (int e = 0; e < 8; ++e) av[e] *= gm[e];
      }
      float t0 = acc[m][0], t1 = acc[m][1];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        t0 = fmaf(av[e], w0[e], t0);
        t1 = fmaf(av[e], w1[e], t1);
      }
      acc[m][0] = t0;
      acc[m][1] = t1;
    }
  };
  if (pre_k) {
#pragma unroll
    for (int c = 0; c < PRE; ++c) {
      const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * c;
      if (k < g.K) {
        float w0[8], w1[8];
        WT::f32(pw0[c], w0);
        WT::f32(pw1[c], w1);
        step(c, k, w0, w1);
      }
    }
  } else {
    for (int64_t k = static_cast<int64_t>(lane) * 8; k < g.K; k += 512) {
      float w0[8], w1[8];
      WT::f32(WT::template load<false>(g, q.r0, k), w0);
      WT::f32(WT::template load<false>(g, r1c, k), w1);
      step(0, k, w0, w1);
    }
  }
  // RMSNorm: rms = sqrt(mean(x x) + eps), dividing the finished sums.
  float rms[M];
#pragma unroll
  for (int m = 0; m < M; ++m)
    rms[m] = g.gamma ? __fsqrt_rn(fold_sum<64>(ss[m]) / static_cast<float>(g.K) + g.eps) : 1.0f;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float y0 = fold_sum<64>(acc[m][0]), y1 = fold_sum<64>(acc[m][1]);
    if (g.gamma) {
      y0 = y0 / rms[m];
      y1 = y1 / rms[m];
    }
    // Lane m writes activation row m's outputs.
    if (lane == m) pair_write_pre<MODE>(g, q, m, y0, y1, pre);
  }
}

// The streamed product of one activation row (the vocabulary head at batch
// 1): decode_matvec_kernel<1, DM_PLAIN, 2, true>'s arithmetic per pair (so
// its bits), R pairs a wavefront.  That kernel reads the row and the gain
// again for every pair, two thirds of what its CUs load, and the loads
// through each CU's vector cache (64 bytes a clock), not HBM, bound it; here
// the row, the gain and the norm's sum of squares serve R pairs, whose 4 R
// weight chunks a lane are all requested first.  K <= 1024, BF16 weights.
// ARG: also the block's best output by argmax's rule (better), written to
// (pv, pi)[block] for argmax_partials_kernel -- the greedy pick's first
// pass over the logits done where they are formed.
template <int R, bool ARG = false>
__global__ void __launch_bounds__(256) decode_head_kernel(DecodeArgs g, float *pv = nullptr, int32_t *pi = nullptr) {
  constexpr int PRE = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t p0 = ((static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6) * R;
  if (!ARG && p0 >= g.npairs) return;  // whole wavefronts (with ARG: clamped, to reach the barrier)
  uint4 pw[R][2][PRE];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t p = p0 + r < g.npairs ? p0 + r : g.npairs - 1;
    const int64_t r0 = 2 * p, r1 = r0 + 1 < g.N ? r0 + 1 : r0;
#pragma unroll
    for (int c = 0; c < PRE; ++c) {
      const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * c;
      const int64_t kc = k < g.K ? k : g.K - 8;
      pw[r][0][c] = ldu4<true>(g.w + r0 * g.K + kc);
      pw[r][1][c] = ldu4<true>(g.w + r1 * g.K + kc);
    }
  }
  const float *gp = g.gamma ? g.gamma : g.x;  // without a gain: read, never used
  float4 px[PRE][2], pg[PRE][2];
#pragma unroll
  for (int c = 0; c < PRE; ++c) {
    const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * c;
    const int64_t kc = k < g.K ? k : g.K - 8;
    px[c][0] = *reinterpret_cast<const float4 *>(g.x + kc);
    px[c][1] = *reinterpret_cast<const float4 *>(g.x + kc + 4);
    pg[c][0] = *reinterpret_cast<const float4 *>(gp + kc);
    pg[c][1] = *reinterpret_cast<const float4 *>(gp + kc + 4);
  }
  float ev[R][2];
  if (g.resid) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t p = p0 + r < g.npairs ? p0 + r : g.npairs - 1;
      ev[r][0] = g.resid[2 * p];
      ev[r][1] = g.resid[2 * p + 1 < g.N ? 2 * p + 1 : 2 * p];
    }
  }
  // The row times the gain, and the norm's sum of squares, as the plain
  // kernel forms them lane by lane.
  float xg[PRE][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < PRE; ++c) {
    const float av[8] = {px[c][0].x, px[c][0].y, px[c][0].z, px[c][0].w,
                         px[c][1].x, px[c][1].y, px[c][1].z, px[c][1].w};
    const float gm[8] = {pg[c][0].x, pg[c][0].y, pg[c][0].z, pg[c][0].w,
                         pg[c][1].x, pg[c][1].y, pg[c][1].z, pg[c][1].w};
    const bool in = static_cast<int64_t>(lane) * 8 + 512 * c < g.K;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (g.gamma) {
        if (in) ss = fmaf(av[e], av[e], ss);
        xg[c][e] = av[e] * gm[e];
      } else {
        xg[c][e] = av[e];
      }
    }
  }
  const float rms = g.gamma ? __fsqrt_rn(fold_sum<64>(ss) / static_cast<float>(g.K) + g.eps) : 1.0f;
  ArgBest best{-INFINITY, INT32_MAX};
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
    for (int c = 0; c < PRE; ++c) {
      if (static_cast<int64_t>(lane) * 8 + 512 * c < g.K) {
        float w0[8], w1[8];
        bf16x8(pw[r][0][c], w0);
        bf16x8(pw[r][1][c], w1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          t0 = fmaf(xg[c][e], w0[e], t0);
          t1 = fmaf(xg[c][e], w1[e], t1);
        }
      }
    }
    float y0 = fold_sum<64>(t0), y1 = fold_sum<64>(t1);
    if (g.gamma) {
      y0 = y0 / rms;
      y1 = y1 / rms;
    }
    const int64_t p = p0 + r;
    const float o0 = g.resid ? __fadd_rn(ev[r][0], y0) : y0, o1 = g.resid ? __fadd_rn(ev[r][1], y1) : y1;
    if (lane == r && p < g.npairs) {
      g.out[2 * p] = o0;
      if (2 * p + 1 < g.N) g.out[2 * p + 1] = o1;
    }
    if constexpr (ARG) {
      if (p < g.npairs) best = better(best, ArgBest{o0, static_cast<int32_t>(2 * p)});
      if (2 * p + 1 < g.N) best = better(best, ArgBest{o1, static_cast<int32_t>(2 * p + 1)});
    }
  }
  if constexpr (ARG) {  // every lane holds the wavefront's best
    __shared__ float bv[4];
    __shared__ int32_t bi[4];
    if (lane == 0) {
      bv[wave] = best.v;
      bi[wave] = best.i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      ArgBest b{bv[0], bi[0]};
      for (int w = 1; w < 4; ++w) b = better(b, ArgBest{bv[w], bi[w]});
      pv[blockIdx.x] = b.v;
      pi[blockIdx.x] = b.i;
    }
  }
}

// The greedy pick's last pass: the n partial bests of one row, by argmax's
// rule, into out[0] (0 when every partial is empty).
__global__ void __launch_bounds__(256) argmax_partials_kernel(const float *pv, const int32_t *pi, int64_t n,
                                                              int32_t *out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  ArgBest best{-INFINITY, INT32_MAX};
  for (int64_t c = threadIdx.x; c < n; c += 256) best = better(best, ArgBest{pv[c], pi[c]});
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) best = better(best, ArgBest{__shfl_xor(best.v, o, 64), __shfl_xor(best.i, o, 64)});
  __shared__ float bv[4];
  __shared__ int32_t bi[4];
  if (lane == 0) {
    bv[wave] = best.v;
    bi[wave] = best.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgBest b{bv[0], bi[0]};
    for (int w = 1; w < 4; ++w) b = better(b, ArgBest{bv[w], bi[w]});
    out[0] = b.i == INT32_MAX ? 0 : b.i;
  }
}
constexpr int HEAD_R = 4;  // pairs a wavefront of decode_head_kernel

// A one-sequence decode step's attention combine and o projection in one
// launch.  The block's 16 rows of 16 lanes first form the whole attention row
// into LDS -- row h query head h (ChunkCombine, the combine kernel's code, so
// its bits) -- then its 4 wavefronts (output rows 8 b .. 8 b + 7, a pair
// each) multiply it as decode_matvec_kernel<1, DM_PLAIN, 2> does (its bits
// again).  The weight rows are requested first and the combine's partials,
// queries and new rows after them with no wait between, so the launch waits
// for one round trip as the plain product does, and the combine's own launch
// is gone.  H <= 16 heads (a row past the last repeats it and writes
// nothing); LDS: the row's H 64 floats, then 16 S chunk weights.
template <typename WT, int CS>
__global__ void __launch_bounds__(256) attention_o_kernel(DecodeArgs g, AttnCombine c) {
  constexpr int D = 64, PRE = 2;
  extern __shared__ float sm[];
  const int H = c.H, G = c.G, S = c.S;
  float *xs = sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const bool live = p < g.npairs;  // a wavefront past the last pair still combines and syncs
  const int64_t r0 = live ? 2 * p : 0;
  const bool has1 = live && r0 + 1 < g.N;
  const int64_t r1 = has1 ? r0 + 1 : r0;

  typename WT::Raw pw0[PRE], pw1[PRE];
#pragma unroll
  for (int cc = 0; cc < PRE; ++cc) {
    const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * cc;
    const int64_t kc = k < g.K ? k : g.K - 8;
    pw0[cc] = WT::template load<false>(g, r0, kc);
    pw1[cc] = WT::template load<false>(g, r1, kc);
  }
  const float *rp = g.resid ? g.resid : g.out;
  const float e0 = rp[r0], e1 = rp[r1];
  const int row = tid >> 4, r = tid & 15, h = row < H ? row : H - 1, j = h / G, gg = h - j * G;
  const float *pitem = c.part + static_cast<int64_t>(j) * S * dqa_part_stride(G);
  ChunkCombine<CS> comb;
  comb.load(pitem, G, gg, S, r, c.q + h * D, c.kvn + j * 2 * D, c.kvn + j * 2 * D + D);
  const float4 o = comb.finish(pitem, G, gg, S, r, c.scale, xs + H * D + row * S);
  if (row < H) *reinterpret_cast<float4 *>(xs + h * D + 4 * r) = o;
  __syncthreads();
  float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
  for (int cc = 0; cc < PRE; ++cc) {
    const int64_t k = static_cast<int64_t>(lane) * 8 + 512 * cc;
    if (k < g.K) {
      float w0[8], w1[8];
      WT::f32(pw0[cc], w0);
      WT::f32(pw1[cc], w1);
      const float4 a0 = *reinterpret_cast<const float4 *>(xs + k);
      const float4 a1 = *reinterpret_cast<const float4 *>(xs + k + 4);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        t0 = fmaf(av[e], w0[e], t0);
        t1 = fmaf(av[e], w1[e], t1);
      }
    }
  }
  const float y0 = fold_sum<64>(t0), y1 = fold_sum<64>(t1);
  if (live && lane == 0) {
    g.out[r0] = g.resid ? __fadd_rn(e0, y0) : y0;
    if (has1) g.out[r1] = g.resid ? __fadd_rn(e1, y1) : y1;
  }
}

// LDS of attention_o_kernel for H heads over S chunks, in floats.
static int64_t attention_o_lds(int64_t H, int64_t S) { return H * 64 + 16 * S; }

bool attention_o_fits(int64_t H, int64_t S) {
  return H >= 1 && H <= 16 && S >= 1 && attention_o_lds(H, S) * 4 <= 65536;
}

template <typename WT>
static void attention_o_cs(unsigned grid, size_t lds, hipStream_t st, const DecodeArgs &g, const AttnCombine &c) {
  switch (combine_cs(c.S)) {
    case 4: attention_o_kernel<WT, 4><<<grid, 256, lds, st>>>(g, c); break;
    case 8: attention_o_kernel<WT, 8><<<grid, 256, lds, st>>>(g, c); break;
    case 12: attention_o_kernel<WT, 12><<<grid, 256, lds, st>>>(g, c); break;
    default: attention_o_kernel<WT, 16><<<grid, 256, lds, st>>>(g, c); break;
  }
}

int attention_o_launch(Ctx *ctx, const AttnCombine &c, const Buffer *w, const float *resid, float *out) {
  if (!attention_o_fits(c.H, c.S) || c.G < 1 || c.H % c.G || w->cols != c.H * 64 || w->rows < 1 ||
      (w->elem != MI_BF16 && w->elem != MI_BFP8))
    return fail(ctx, MI_E_ARG, "attention_o: %d heads over %d chunks against a %s [%lld, %lld] weight", c.H, c.S,
                elem_name(w->elem), (long long)w->rows, (long long)w->cols);
  DecodeArgs g{};
  g.K = w->cols;
  g.N = w->rows;
  g.npairs = (w->rows + 1) / 2;
  g.resid = resid;
  g.out = out;
  g.ldo = w->rows;
  const unsigned grid = static_cast<unsigned>((g.npairs + 3) / 4);
  const size_t lds = static_cast<size_t>(attention_o_lds(c.H, c.S)) * sizeof(float);
  if (w->elem == MI_BFP8) {
    g.wq = static_cast<const int8_t *>(w->ptr);
    g.we = static_cast<const uint8_t *>(w->ptr) + bfp8_exp_offset(w->rows, w->cols);
    attention_o_cs<WBfp8>(grid, lds, ctx->stream, g, c);
  } else {
    g.w = static_cast<const uint16_t *>(w->ptr);
    attention_o_cs<WBf16>(grid, lds, ctx->stream, g, c);
  }
  return check_launch(ctx, "attention_o");
}

// 9 to 32 activation rows: a block's 4 wavefronts (8 weight rows) share each
// 256-wide k chunk of the rows (times the gain) through LDS, read from cache
// once per block instead of once per wavefront.  Lane l takes 4 k of the chunk
// (8 bytes of each weight row, 512 contiguous bytes a wavefront) and
// accumulates the 2 x 32 products; a halving butterfly leaves lane l holding
// product l (row l / 2, weight row l % 2) after 63 shuffles.  Latency is
// hidden rather than waited for: a wavefront requests all its weight chunks
// (K <= 2048) at the start, and the next chunk of rows is loaded into
// registers while the current one is multiplied.  The RMSNorm divides the
// finished products -- sum_k x g w / rms -- with the sums of squares folded
// from the staged values, so no pass over the rows precedes the products.
constexpr int WIDE_M = 32;
constexpr int WIDE_KC = 256;
constexpr int WIDE_PRE = 8;  // weight chunks requested up front (K <= 2048)

template <int MODE>
__global__ void __launch_bounds__(256) decode_matvec_wide_kernel(DecodeArgs g, int M) {
  __shared__ float4 xs[WIDE_M][WIDE_KC / 4];
  __shared__ float rms_s[WIDE_M];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const bool live = p < g.npairs;  // a wavefront past the last pair still stages and syncs
  const PairRows q = pair_rows<MODE>(g, live ? p : 0);
  const int nch = static_cast<int>((g.K + WIDE_KC - 1) / WIDE_KC);
  const bool pre = nch <= WIDE_PRE;

  uint2 pw0[WIDE_PRE], pw1[WIDE_PRE];
  auto wload = [&](int c, uint2 &a, uint2 &b) {
    const int64_t k = static_cast<int64_t>(c) * WIDE_KC + 4 * lane;
    a = make_uint2(0u, 0u);
    b = make_uint2(0u, 0u);
    if (live && k < g.K) {
      a = *reinterpret_cast<const uint2 *>(g.w + q.r0 * g.K + k);
      if (q.has1) b = *reinterpret_cast<const uint2 *>(g.w + q.r1 * g.K + k);
    }
  };
  if (pre) {
#pragma unroll
    for (int c = 0; c < WIDE_PRE; ++c)
      if (c < nch) wload(c, pw0[c], pw1[c]);
  }

  // Staging: thread (wave w, lane l) owns rows w + 4 i (i < 8) at float4 l.
  float4 xr[8];
  float ssq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ssq[i] = 0.0f;
  auto xload = [&](int c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = wave + 4 * i;
      const int64_t k = static_cast<int64_t>(c) * WIDE_KC + 4 * lane;
      xr[i] = (m < M && k < g.K) ? *reinterpret_cast<const float4 *>(g.x + m * g.ldx + k)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  xload(0);

  float acc[2 * WIDE_M];
#pragma unroll
  for (int i = 0; i < 2 * WIDE_M; ++i) acc[i] = 0.0f;
  for (int c = 0; c < nch; ++c) {
    const int64_t k = static_cast<int64_t>(c) * WIDE_KC + 4 * lane;
    float4 gm = make_float4(1.f, 1.f, 1.f, 1.f);
    if (g.gamma && k < g.K) gm = *reinterpret_cast<const float4 *>(g.gamma + k);
    __syncthreads();  // the previous chunk's reads are done
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xr[i];
      ssq[i] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      xs[wave + 4 * i][lane] = make_float4(v.x * gm.x, v.y * gm.y, v.z * gm.z, v.w * gm.w);
    }
    __syncthreads();
    if (c + 1 < nch) xload(c + 1);  // lands while this chunk is multiplied
    uint2 a, b;
    if (pre) {
      a = pw0[0];
      b = pw1[0];
#pragma unroll
      for (int j = 1; j < WIDE_PRE; ++j)
        if (j == c) { a = pw0[j]; b = pw1[j]; }
    } else {
      wload(c, a, b);
    }
    const float w0[4] = {__uint_as_float(a.x << 16), __uint_as_float(a.x & 0xffff0000u),
                         __uint_as_float(a.y << 16), __uint_as_float(a.y & 0xffff0000u)};
    const float w1[4] = {__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xffff0000u),
                         __uint_as_float(b.y << 16), __uint_as_float(b.y & 0xffff0000u)};
#pragma unroll
    for (int m = 0; m < WIDE_M; ++m) {
      const float4 v = xs[m][lane];
      acc[2 * m] += v.x * w0[0] + v.y * w0[1] + v.z * w0[2] + v.w * w0[3];
      acc[2 * m + 1] += v.x * w1[0] + v.y * w1[1] + v.z * w1[2] + v.w * w1[3];
    }
  }
  if (g.gamma) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = wave_sum(ssq[i]);
      const int m = wave + 4 * i;
      if (lane == 0 && m < M) rms_s[m] = __fsqrt_rn(s / static_cast<float>(g.K) + g.eps);
    }
  }
  // Halving butterfly: after the step with offset o each lane keeps the half
  // of its values whose index bit matches its own lane bit, plus the
  // partner's matching half; lane l ends with the full sum of value l.
#pragma unroll
  for (int o = 32, n = 64; o >= 1; o >>= 1, n >>= 1) {
    const bool upper = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i < n / 2) {
        const float keep = upper ? acc[i + n / 2] : acc[i];
        const float send = upper ? acc[i] : acc[i + n / 2];
        acc[i] = keep + __shfl_xor(send, o, 64);
      }
    }
  }
  __syncthreads();  // the norms are visible
  // Lane l: row l / 2, weight row l % 2; the pair's other product from lane l ^ 1.
  const int m = lane >> 1;
  float y = acc[0];
  if (g.gamma && m < M) y = y / rms_s[m];
  const float other = __shfl_xor(y, 1, 64);
  if (live && m < M && (lane & 1) == 0) pair_write<MODE>(g, q, m, y, other);
}

// ------------------------------------ 3 to 32 rows on the matrix cores
// One 512-thread block per tile of weight rows -- 32 consecutive rows
// (DM_PLAIN), or two blocks of 32 whose rows pair up lane by lane: gate rows
// and their up rows (DM_SILU_MUL), the two halves of one 64-wide head
// (DM_QKV) -- against all M <= 32 activation rows, on
// v_mfma_f32_32x32x16_bf16 (A: the activation rows times the gain, B: the
// weight rows; lane l holds row l % 32, k group l / 32 of both).  Each F32
// activation is split into three BF16 parts (hi + mid + lo = a to within
// 2^-25 |a|, each remainder exact in F32), so the products keep F32
// accuracy.  The block's sixteen wavefronts take the k16 steps w, w + 16, ...;
// each lane issues all its weight, activation and gain loads before any
// arithmetic (STEPS steps a wavefront, fixed at compile time), then the
// sixteen partial accumulators and the rows' sums of squares fold through LDS
// in wavefront order and the pair epilogue writes.  Against the LDS-staged
// VALU form, which re-reads every activation row from LDS for every weight
// pair, a 32-row step does one MFMA per 16K multiply-adds.
typedef __bf16 dm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float dm_f32x16 __attribute__((ext_vector_type(16)));
constexpr int DMFMA_WAVES = 16;

// Three BF16 parts of eight F32 values: the head truncated (it cannot
// overflow, and a - head is exact), the two remainders rounded to nearest by
// the hardware conversion; |a - hi - mid - lo| <= 2^-25 |a|.  An infinite or
// NaN value leaves a NaN remainder: its head carries it alone.
__device__ __forceinline__ void split3x8(const float (&v)[8], dm_bf16x8 &hi, dm_bf16x8 &mid, dm_bf16x8 &lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t hb = __float_as_uint(v[e]) & 0xffff0000u;
    const float r1 = v[e] - __uint_as_float(hb);
    const bool fin = r1 == r1;
    const __bf16 m = static_cast<__bf16>(fin ? r1 : 0.0f);
    const float r2 = fin ? r1 - static_cast<float>(m) : 0.0f;
    hi[e] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(hb >> 16));
    mid[e] = m;
    lo[e] = static_cast<__bf16>(r2);
  }
}

template <int MODE, int STEPS, int NB, bool GAMMA, typename WT = WBf16>
__global__ void __launch_bounds__(64 * DMFMA_WAVES)
decode_mfma_kernel(DecodeArgs g, int M) {
  constexpr int NW = DMFMA_WAVES;
  __shared__ float red[NW][NB * 16][64];
  __shared__ float sq[NW][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t = blockIdx.x;
  const int n = lane & 31, kg = lane >> 5;
  // The weight row of column n in each block, and whether it exists.
  int64_t row[NB];
  bool rv[NB];
  if constexpr (MODE == DM_PLAIN) {
    row[0] = 32 * t + n;
    rv[0] = row[0] < g.N;
  } else if constexpr (MODE == DM_SILU_MUL) {
    row[0] = 32 * t + n;
    row[1] = g.inter + row[0];
    rv[0] = rv[1] = row[0] < g.inter;
  } else {
    row[0] = t * g.d + n;  // g.d == 64: the head's two halves
    row[1] = row[0] + 32;
    rv[0] = rv[1] = true;
  }
  const int m = lane & 31;
  const bool mv = m < M;
  const int64_t nsteps = g.K / 16;

  // Every load is unconditional from an address inside its buffer (the last
  // step, row 0 of the weight, row 0 of the activations): a load under a
  // condition compiles to a load through a selected pointer, one that may
  // point at a private zero.  Steps past the end are skipped below, missing
  // weight rows and activation rows zeroed.
  typename WT::Raw wb[STEPS][NB];
  float4 xa[STEPS][2], ga[GAMMA ? STEPS : 1][2];
  const int64_t mc = mv ? m : 0;
  int64_t rowc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rowc[b] = rv[b] ? row[b] : 0;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t step = w + NW * s;
    const int64_t k = (step < nsteps ? step : nsteps - 1) * 16 + 8 * kg;
#pragma unroll
    for (int b = 0; b < NB; ++b) wb[s][b] = WT::template load<false>(g, rowc[b], k);
    xa[s][0] = *reinterpret_cast<const float4 *>(g.x + mc * g.ldx + k);
    xa[s][1] = *reinterpret_cast<const float4 *>(g.x + mc * g.ldx + k + 4);
    if constexpr (GAMMA) {
      ga[s][0] = *reinterpret_cast<const float4 *>(g.gamma + k);
      ga[s][1] = *reinterpret_cast<const float4 *>(g.gamma + k + 4);
    }
  }
  // The residual value this thread's epilogue adds (row mo below), requested
  // with the weights rather than after the fold.
  float rpre = 0.0f;
  if constexpr (MODE == DM_PLAIN) {
    if (g.resid) {
      const int mo = 8 * (w >> 2) + 4 * kg + (w & 3);
      rpre = g.resid[(mo < M ? mo : 0) * g.ldo + rowc[0]];
    }
  }
  dm_f32x16 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
  float ssq = 0.0f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    if (w + NW * s < nsteps) {
      float v[8] = {xa[s][0].x, xa[s][0].y, xa[s][0].z, xa[s][0].w, xa[s][1].x, xa[s][1].y, xa[s][1].z, xa[s][1].w};
      if (!mv) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
      }
      if constexpr (GAMMA) {
        const float gm[8] = {ga[s][0].x, ga[s][0].y, ga[s][0].z, ga[s][0].w,
                             ga[s][1].x, ga[s][1].y, ga[s][1].z, ga[s][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ssq += v[e] * v[e];
          v[e] = v[e] * gm[e];
        }
      }
      dm_bf16x8 hi, mid, lo;
      split3x8(v, hi, mid, lo);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const dm_bf16x8 wv = __builtin_bit_cast(dm_bf16x8, rv[b] ? WT::bf16(wb[s][b]) : make_uint4(0, 0, 0, 0));
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, wv, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, wv, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, wv, acc[b], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[w][b * 16 + r][lane] = acc[b][r];
  sq[w][lane] = ssq;
  __syncthreads();
  // Wavefront w finishes value r = w of every block: rows
  // m = 8 (r / 4) + 4 (lane / 32) + r % 4, column n = lane % 32.
  static_assert(NW == 16, "one accumulator value a wavefront");
  {
    const int r = w;
    const int mo = 8 * (r >> 2) + 4 * kg + (r & 3);
    if (mo >= M) return;
    float y[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float a = red[0][b * 16 + r][lane];
#pragma unroll
      for (int v = 1; v < NW; ++v) a += red[v][b * 16 + r][lane];
      y[b] = a;
    }
    if constexpr (GAMMA) {
      float ss = sq[0][mo] + sq[0][mo + 32];
#pragma unroll
      for (int v = 1; v < NW; ++v) ss += sq[v][mo] + sq[v][mo + 32];
      const float rms = __fsqrt_rn(ss / static_cast<float>(g.K) + g.eps);
#pragma unroll
      for (int b = 0; b < NB; ++b) y[b] = y[b] / rms;
    }
    if constexpr (MODE == DM_PLAIN) {
      if (rv[0]) {
        float *o = g.out + mo * g.ldo + row[0];
        *o = g.resid ? __fadd_rn(rpre, y[0]) : y[0];
      }
    } else if constexpr (MODE == DM_SILU_MUL) {
      if (rv[0]) g.out[mo * g.ldo + row[0]] = silu2(y[0]) * y[1];
    } else {
      PairRows q{row[0], row[1], t, n, true};
      pair_write<MODE>(g, q, mo, y[0], y[1]);
    }
  }
}

// The same products split over k for grids of few tiles (the q|k|v heads and
// the down projection: 15 and 18 tiles of a 256-CU chip, each block pulling
// every activation row and its weight rows through one CU): block (tile, s)
// takes k16 steps [s per, (s + 1) per) on four wavefronts and writes its raw
// sums -- no RMS, no epilogue -- to part[(s M + m) N + weight row], and,
// from the first tile's blocks, each activation row's sum of squares over
// its steps to part[S M N + s M + m].  decode_fold_kernel adds the S
// partials in split order and runs the mode's epilogue.  In a batch-32
// SmolLM2 decode step the down projection takes 6.9 + 3.6 us (split, fold)
// against 13.6, the q|k|v heads 6.7 + 3.8 against 11.1: 1.88 -> 1.755 ms a
// step.
constexpr int DSPLIT_WAVES = 4;

template <int MODE, int STEPS, int NB, bool GAMMA, typename WT = WBf16>
__global__ void __launch_bounds__(64 * DSPLIT_WAVES) decode_mfma_split_kernel(DecodeArgs g, int M) {
  constexpr int NW = DSPLIT_WAVES;
  __shared__ float red[NW][NB * 16][64];
  __shared__ float sq[NW][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t = blockIdx.x, sp = blockIdx.y, S = gridDim.y;
  const int n = lane & 31, kg = lane >> 5;
  int64_t row[NB];
  bool rv[NB];
  if constexpr (MODE == DM_PLAIN) {
    row[0] = 32 * t + n;
    rv[0] = row[0] < g.N;
  } else if constexpr (MODE == DM_SILU_MUL) {
    row[0] = 32 * t + n;
    row[1] = g.inter + row[0];
    rv[0] = rv[1] = row[0] < g.inter;
  } else {
    row[0] = t * g.d + n;
    row[1] = row[0] + 32;
    rv[0] = rv[1] = true;
  }
  const int m = lane & 31;
  const bool mv = m < M;
  const int64_t nsteps = g.K / 16, per = (nsteps + S - 1) / S;
  const int64_t s0 = sp * per, s1 = s0 + per < nsteps ? s0 + per : nsteps;  // s0 < s1: the host keeps S <= nsteps / per
  // Unconditional loads from addresses inside the buffers, as the unsplit
  // kernel's: steps past the split's end reread its last step.
  typename WT::Raw wb[STEPS][NB];
  float4 xa[STEPS][2], ga[GAMMA ? STEPS : 1][2];
  const int64_t mc = mv ? m : 0;
  int64_t rowc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rowc[b] = rv[b] ? row[b] : 0;
#pragma unroll
  for (int si = 0; si < STEPS; ++si) {
    const int64_t step = s0 + w + NW * si;
    const int64_t k = (step < s1 ? step : s1 - 1) * 16 + 8 * kg;
#pragma unroll
    for (int b = 0; b < NB; ++b) wb[si][b] = WT::template load<false>(g, rowc[b], k);
    xa[si][0] = *reinterpret_cast<const float4 *>(g.x + mc * g.ldx + k);
    xa[si][1] = *reinterpret_cast<const float4 *>(g.x + mc * g.ldx + k + 4);
    if constexpr (GAMMA) {
      ga[si][0] = *reinterpret_cast<const float4 *>(g.gamma + k);
      ga[si][1] = *reinterpret_cast<const float4 *>(g.gamma + k + 4);
    }
  }
  dm_f32x16 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
  float ssq = 0.0f;
#pragma unroll
  for (int si = 0; si < STEPS; ++si) {
    if (s0 + w + NW * si < s1) {
      float v[8] = {xa[si][0].x, xa[si][0].y, xa[si][0].z, xa[si][0].w, xa[si][1].x, xa[si][1].y, xa[si][1].z,
                    xa[si][1].w};
      if (!mv) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
      }
      if constexpr (GAMMA) {
        const float gm[8] = {ga[si][0].x, ga[si][0].y, ga[si][0].z, ga[si][0].w,
                             ga[si][1].x, ga[si][1].y, ga[si][1].z, ga[si][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ssq += v[e] * v[e];
          v[e] = v[e] * gm[e];
        }
      }
      dm_bf16x8 hi, mid, lo;
      split3x8(v, hi, mid, lo);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const dm_bf16x8 wv = __builtin_bit_cast(dm_bf16x8, rv[b] ? WT::bf16(wb[si][b]) : make_uint4(0, 0, 0, 0));
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, wv, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, wv, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, wv, acc[b], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[w][b * 16 + r][lane] = acc[b][r];
  sq[w][lane] = ssq;
  __syncthreads();
  // Wavefront w finishes values r = w, w + 4, ... of every block: rows
  // m = 8 (r / 4) + 4 (lane / 32) + r % 4, weight row row[b].
  for (int r = w; r < 16; r += NW) {
    const int mo = 8 * (r >> 2) + 4 * kg + (r & 3);
    if (mo >= M) continue;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float a = red[0][b * 16 + r][lane];
#pragma unroll
      for (int v = 1; v < NW; ++v) a += red[v][b * 16 + r][lane];
      if (rv[b]) g.part[(sp * M + mo) * g.N + row[b]] = a;
    }
  }
  if (GAMMA && t == 0 && tid < M) {
    float ss = sq[0][tid] + sq[0][tid + 32];
#pragma unroll
    for (int v = 1; v < NW; ++v) ss += sq[v][tid] + sq[v][tid + 32];
    g.part[S * M * g.N + sp * M + tid] = ss;
  }
}

// The split products' partials added in split order, then the mode's
// epilogue (RMS, residual, SiLU-mul, RoPE and the cache write): one thread
// per (activation row, output pair).  Every partial, sum of squares and
// epilogue operand is requested before the first add (the split count is at
// most DSPLIT_MAX), so the fold is one memory round trip, not one per split.
constexpr int DSPLIT_MAX = 8;
template <int MODE>
__global__ void __launch_bounds__(256) decode_fold_kernel(DecodeArgs g, int M) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= M * g.npairs) return;
  const int64_t m = i / g.npairs, p = i - m * g.npairs;
  const PairRows q = pair_rows<MODE>(g, p);
  const int S = g.split;
  const float *ssq = g.part + static_cast<int64_t>(S) * M * g.N;
  float p0[DSPLIT_MAX], p1[DSPLIT_MAX], sq[DSPLIT_MAX];
#pragma unroll
  for (int s = 0; s < DSPLIT_MAX; ++s) {
    if (s < S) {
      p0[s] = g.part[(s * M + m) * g.N + q.r0];
      p1[s] = q.has1 ? g.part[(s * M + m) * g.N + q.r1] : 0.0f;
      sq[s] = g.gamma ? ssq[s * M + m] : 0.0f;
    }
  }
  const PairPre e = pair_pre<MODE>(g, q, m);
  float y0 = p0[0], y1 = p1[0];
#pragma unroll
  for (int s = 1; s < DSPLIT_MAX; ++s) {
    if (s < S) {
      y0 += p0[s];
      y1 += p1[s];
    }
  }
  if (g.gamma) {
    float ss = sq[0];
#pragma unroll
    for (int s = 1; s < DSPLIT_MAX; ++s)
      if (s < S) ss += sq[s];
    const float rms = __fsqrt_rn(ss / static_cast<float>(g.K) + g.eps);
    y0 = y0 / rms;
    y1 = y1 / rms;
  }
  pair_write_pre<MODE>(g, q, m, y0, y1, e);
}

// Rows up to which the GEMV beats the matrix-core form (SmolLM2 decode step
// with the fused q|k|v attention up to the same batch, ms: batch 3 0.89
// against 1.26, batch 4 0.99 against 1.29, batch 6 1.22 against 1.32, batch
// 8 1.40 against 1.33).
constexpr int64_t DECODE_GEMV_MAX_M = 6;

// Splits for the split-k form, or 1: grids of fewer than 32 tiles whose
// blocks carry paired rows (the q|k|v heads) or long rows (k >= 1024); each
// split at most four wavefronts' STEPS steps.  (Splitting the o and gate|up
// products too: batch-32 decode 1.755 -> 1.735 ms a step, batch 8 1.371 ->
// 1.419.)
template <int MODE>
static int dsplit_count(int64_t M, const DecodeArgs &g) {
  if (M <= DECODE_GEMV_MAX_M || g.K % 16) return 1;
  if (MODE == DM_QKV && g.d != 64) return 1;
  constexpr int NB = MODE == DM_PLAIN ? 1 : 2;
  const int64_t tiles = MODE == DM_PLAIN ? (g.N + 31) / 32 : (MODE == DM_SILU_MUL ? (g.inter + 31) / 32 : g.H + 2 * g.KVH);
  // A gate|up grid below 64 tiles splits too (batch 32: 48 tiles, 12.1 us
  // unsplit against 6.3 + 2.8 split and folded); the o product's 18 tiles at
  // k 576 do not (7.3 against 6.7 + 2.7).
  if (tiles >= (MODE == DM_SILU_MUL ? 64 : 32) || !(NB == 2 || g.K >= 1024)) return 1;
  const int64_t nsteps = g.K / 16, per = DSPLIT_WAVES * (NB == 1 ? 6 : 3);
  int64_t S = (nsteps + per - 1) / per;
  if (S < 2) return 1;
  if (S > DSPLIT_MAX) S = DSPLIT_MAX;
  return static_cast<int>(S);
}

// Steps a wavefront takes for k = 16 * nsteps, or 0 past what the registers
// hold without spilling: the loads of every step are in flight at once (4 NB
// + 8, plus 8 with a gain, registers a step) within the 128 registers of four
// wavefronts a SIMD -- k up to 1536 plain, 768 for paired rows with a gain.
template <int NB, bool GAMMA>
constexpr int dmfma_most() { return NB == 1 ? (GAMMA ? 5 : 6) : (GAMMA ? 3 : 5); }

static int dmfma_steps(int64_t K, int nb, bool gamma) {
  const int64_t need = (K / 16 + DMFMA_WAVES - 1) / DMFMA_WAVES;
  const int most = nb == 1 ? (gamma ? dmfma_most<1, true>() : dmfma_most<1, false>())
                           : (gamma ? dmfma_most<2, true>() : dmfma_most<2, false>());
  return need <= most ? static_cast<int>(need) : 0;  // longer rows: the LDS-staged kernel
}

template <int MODE, int NB, bool GAMMA, int S, typename WT>
static void launch_dmfma_s(unsigned grid, const DecodeArgs &g, int M, hipStream_t st) {
  if constexpr (S <= dmfma_most<NB, GAMMA>())
    decode_mfma_kernel<MODE, S, NB, GAMMA, WT><<<grid, 64 * DMFMA_WAVES, 0, st>>>(g, M);
}

template <int MODE, int NB, bool GAMMA, typename WT>
static void launch_dmfma(int steps, unsigned grid, const DecodeArgs &g, int M, hipStream_t st) {
  switch (steps) {
    case 1: launch_dmfma_s<MODE, NB, GAMMA, 1, WT>(grid, g, M, st); break;
    case 2: launch_dmfma_s<MODE, NB, GAMMA, 2, WT>(grid, g, M, st); break;
    case 3: launch_dmfma_s<MODE, NB, GAMMA, 3, WT>(grid, g, M, st); break;
    case 4: launch_dmfma_s<MODE, NB, GAMMA, 4, WT>(grid, g, M, st); break;
    case 5: launch_dmfma_s<MODE, NB, GAMMA, 5, WT>(grid, g, M, st); break;
    case 6: launch_dmfma_s<MODE, NB, GAMMA, 6, WT>(grid, g, M, st); break;
  }
}

// The matrix-core form for 3 to 32 rows; false when the shape does not fit it.
template <int MODE, typename WT>
static bool launch_dmfma_mode(int64_t M, const DecodeArgs &g, hipStream_t st) {
  if (g.K % 16) return false;
  constexpr int NB = MODE == DM_PLAIN ? 1 : 2;
  if (MODE == DM_QKV && g.d != 64) return false;
  const int steps = dmfma_steps(g.K, NB, g.gamma != nullptr);
  if (!steps) return false;
  const int64_t tiles = MODE == DM_PLAIN ? (g.N + 31) / 32 : (MODE == DM_SILU_MUL ? (g.inter + 31) / 32 : g.H + 2 * g.KVH);
  if (g.split > 1 && g.part) {
    // Per split: four wavefronts of STEPS steps cover ceil(nsteps / S) steps.
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(g.split));
    const int per = static_cast<int>((g.K / 16 + g.split - 1) / g.split);
    const int Mi = static_cast<int>(M);
    if constexpr (NB == 1) {
      if (per > DSPLIT_WAVES * 6) return false;
      if (g.gamma) decode_mfma_split_kernel<MODE, 6, 1, true, WT><<<grid, 64 * DSPLIT_WAVES, 0, st>>>(g, Mi);
      else decode_mfma_split_kernel<MODE, 6, 1, false, WT><<<grid, 64 * DSPLIT_WAVES, 0, st>>>(g, Mi);
    } else {
      if (per > DSPLIT_WAVES * 3) return false;
      if (g.gamma) decode_mfma_split_kernel<MODE, 3, 2, true, WT><<<grid, 64 * DSPLIT_WAVES, 0, st>>>(g, Mi);
      else decode_mfma_split_kernel<MODE, 3, 2, false, WT><<<grid, 64 * DSPLIT_WAVES, 0, st>>>(g, Mi);
    }
    decode_fold_kernel<MODE><<<static_cast<unsigned>((M * g.npairs + 255) / 256), 256, 0, st>>>(g, Mi);
    return true;
  }
  const unsigned grid = static_cast<unsigned>(tiles);
  if (g.gamma) launch_dmfma<MODE, NB, true, WT>(steps, grid, g, static_cast<int>(M), st);
  else launch_dmfma<MODE, NB, false, WT>(steps, grid, g, static_cast<int>(M), st);
  return true;
}

// Weights of at least this many bytes are streamed (NTW).
constexpr int64_t DECODE_STREAM_BYTES = int64_t(32) << 20;

// false: a BFP8 weight of a shape only the LDS-staged kernel takes (the
// caller runs it on the weight decoded to BF16 instead).
template <int MODE, typename WT = WBf16>
static bool launch_decode(int64_t M, const DecodeArgs &g, hipStream_t st) {
  constexpr bool Q = !std::is_same<WT, WBf16>::value;
  const unsigned grid = static_cast<unsigned>((g.npairs + 3) / 4);
  if (M > DECODE_GEMV_MAX_M && launch_dmfma_mode<MODE, WT>(M, g, st)) return true;
  if (M > 8) {
    if constexpr (Q) return false;
    decode_matvec_wide_kernel<MODE><<<grid, 256, 0, st>>>(g, static_cast<int>(M));
    return true;
  }
  if (M <= DECODE_GEMV_MAX_M && g.K <= 1024) {  // two chunks a lane: half the registers of four
    // One wavefront a block (a pair each): the few hundred pairs of a layer's
    // products spread over that many CUs (batch-1 SmolLM2 step 0.703 ->
    // 0.695 ms); the streamed head keeps four.
    // (The streamed form is for the BF16 head; a BFP8 weight is a layer's.)
    const bool nt = !Q && g.N * g.K * 2 >= DECODE_STREAM_BYTES;
    const unsigned g1 = static_cast<unsigned>(g.npairs);
    switch (M) {
      case 1:
        if (nt && MODE == DM_PLAIN && g.w)
          decode_head_kernel<HEAD_R><<<static_cast<unsigned>((g.npairs + 4 * HEAD_R - 1) / (4 * HEAD_R)), 256, 0, st>>>(g);
        else if (nt) decode_matvec_kernel<1, MODE, 2, true><<<grid, 256, 0, st>>>(g);
        else decode_matvec_kernel<1, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g);
        break;
      case 2:
        if (nt) decode_matvec_kernel<2, MODE, 2, true><<<grid, 256, 0, st>>>(g);
        else decode_matvec_kernel<2, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g);
        break;
      case 3: decode_matvec_kernel<3, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g); break;
      case 4: decode_matvec_kernel<4, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g); break;
      case 5: decode_matvec_kernel<5, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g); break;
      default: decode_matvec_kernel<6, MODE, 2, false, WT><<<g1, 64, 0, st>>>(g); break;
    }
    return true;
  }
  // One row past k 1024 (a layer's down product): one wavefront a block too
  // (batch-1 SmolLM2 down 3.38 -> 2.90 us, decode 0.569 -> 0.560 ms a step).
  if (M == 1 && g.N * g.K * 2 < DECODE_STREAM_BYTES) {
    decode_matvec_kernel<1, MODE, 4, false, WT><<<static_cast<unsigned>(g.npairs), 64, 0, st>>>(g);
    return true;
  }
  switch (M) {
#define MI_DEC(m) case m: decode_matvec_kernel<m, MODE, 4, false, WT><<<grid, 256, 0, st>>>(g); break;
    MI_DEC(1) MI_DEC(2) MI_DEC(3) MI_DEC(4) MI_DEC(5) MI_DEC(6) MI_DEC(7) MI_DEC(8)
#undef MI_DEC
  }
  return true;
}

// A projection's launch for its weight: BF16, or BFP8 read as such where
// the kernels take it, else decoded to BF16 into a buffer freed after the
// launch (stream-ordered: no later op gets the memory before the launch
// has run).
template <int MODE>
static int launch_weight(Ctx *ctx, int64_t M, DecodeArgs &g, const Buffer *wb) {
  if (wb->elem != MI_BFP8) {
    launch_decode<MODE>(M, g, ctx->stream);
    return MI_OK;
  }
  g.wq = static_cast<const int8_t *>(wb->ptr);
  g.we = static_cast<const uint8_t *>(wb->ptr) + bfp8_exp_offset(wb->rows, wb->cols);
  if (launch_decode<MODE, WBfp8>(M, g, ctx->stream)) return MI_OK;
  mi_id t;
  Buffer *tb;
  if (int s = bfp8_decode_to(ctx, wb, MI_BF16, &t, &tb)) return s;
  g.w = static_cast<const uint16_t *>(tb->ptr);
  launch_decode<MODE>(M, g, ctx->stream);
  mi_free(static_cast<mi_ctx *>(ctx), t);
  return MI_OK;
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The split-k form's partials in the context's scratch, when the shape takes
// it (without scratch the unsplit form runs).
template <int MODE>
static void split_setup(Ctx *ctx, int64_t M, DecodeArgs &g) {
  g.split = dsplit_count<MODE>(M, g);
  g.part = nullptr;
  if (g.split > 1) {
    const size_t bytes = (static_cast<size_t>(g.split) * M * g.N + static_cast<size_t>(g.split) * M) * sizeof(float);
    g.part = static_cast<float *>(scratch(ctx, bytes));
    if (!g.part) g.split = 1;
  }
}

// Shared checks: x [M <= 32, K] F32, w [N, K] BF16, K % 8 == 0, gamma [1, K].
static int check_common(mi_ctx *ctx, const Buffer *xb, const Buffer *wb, const Buffer *gb, const char *what) {
  if (xb->elem != MI_F32) return fail(ctx, MI_E_ARG, "%s: activations are %s, not F32", what, elem_name(xb->elem));
  if (wb->elem != MI_BF16 && wb->elem != MI_BFP8)
    return fail(ctx, MI_E_ARG, "%s: weight is %s, not BF16 or BFP8", what, elem_name(wb->elem));
  if (wb->elem == MI_BFP8 && xb->cols % 16)
    return fail(ctx, MI_E_UNSUPPORTED, "%s: a BFP8 weight of width %lld (a multiple of 16 is read)", what,
                (long long)xb->cols);
  if (xb->rows < 1 || xb->rows > DECODE_MAX_M)
    return fail(ctx, MI_E_UNSUPPORTED, "%s: %lld activation rows (1 to %d)", what, (long long)xb->rows, DECODE_MAX_M);
  if (wb->cols != xb->cols) return fail(ctx, MI_E_ARG, "%s: weight is [%lld, %lld], activations [%lld, %lld]", what,
                                        (long long)wb->rows, (long long)wb->cols, (long long)xb->rows, (long long)xb->cols);
  if (xb->cols < 8 || xb->cols % 8)
    return fail(ctx, MI_E_UNSUPPORTED, "%s: width %lld is not a positive multiple of 8", what, (long long)xb->cols);
  if (gb && (gb->elem != MI_F32 || gb->rows * gb->cols != xb->cols))
    return fail(ctx, MI_E_ARG, "%s: gain must be [1, %lld] F32", what, (long long)xb->cols);
  if (!aligned16(xb->ptr) || !aligned16(wb->ptr) || (gb && !aligned16(gb->ptr)))
    return fail(ctx, MI_E_ARG, "%s: buffers must be 16-byte aligned", what);
  return MI_OK;
}

}  // namespace mi

using namespace mi;

extern "C" int mi_norm_matvec(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w, mi_id residual, int silu_mul,
                              mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, wb, w);
  const Buffer *gb = nullptr, *rb = nullptr;
  if (gamma) {
    gb = lookup(ctx, gamma);
    if (!gb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)gamma);
  }
  if (residual) {
    rb = lookup(ctx, residual);
    if (!rb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)residual);
  }
  int s = check_common(ctx, xb, wb, gb, "norm_matvec");
  if (s) return s;
  const int64_t M = xb->rows, K = xb->cols, N = wb->rows;
  if (silu_mul && (N % 2 || rb))
    return fail(ctx, MI_E_ARG, "norm_matvec: silu_mul takes a [2 * inter, K] weight and no residual");
  const int64_t ncols = silu_mul ? N / 2 : N;
  if (rb && (rb->elem != MI_F32 || rb->rows != M || rb->cols != N))
    return fail(ctx, MI_E_ARG, "norm_matvec: residual must be [%lld, %lld] F32", (long long)M, (long long)N);
  mi_id id;
  Buffer *ob;
  s = new_buffer(ctx, M, ncols, MI_F32, &id, &ob);
  if (s) return s;
  if (ncols > 0) {
    DecodeArgs g{};
    g.x = static_cast<const float *>(xb->ptr);
    g.ldx = K;
    g.K = K;
    g.gamma = gb ? static_cast<const float *>(gb->ptr) : nullptr;
    g.eps = eps;
    g.w = wb->elem == MI_BF16 ? static_cast<const uint16_t *>(wb->ptr) : nullptr;
    g.N = N;
    g.resid = rb ? static_cast<const float *>(rb->ptr) : nullptr;
    g.out = static_cast<float *>(ob->ptr);
    g.ldo = ncols;
    if (silu_mul) {
      g.inter = ncols;
      g.npairs = ncols;
      split_setup<DM_SILU_MUL>(ctx, M, g);
      s = launch_weight<DM_SILU_MUL>(ctx, M, g, wb);
    } else {
      g.npairs = (N + 1) / 2;
      split_setup<DM_PLAIN>(ctx, M, g);
      s = launch_weight<DM_PLAIN>(ctx, M, g, wb);
    }
    if (s) {
      mi_free(ctx, id);
      return s;
    }
  }
  s = check_launch(ctx, "norm_matvec");
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}

extern "C" int mi_norm_matvec_argmax(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w, mi_id *logits,
                                     mi_id *ids) {
  MI_ENTER(ctx);
  if (!logits || !ids) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, xb, x);
  MI_BUF(ctx, wb, w);
  const Buffer *gb = nullptr;
  if (gamma) {
    gb = lookup(ctx, gamma);
    if (!gb) return fail(ctx, MI_E_ID, "unknown id %llu", (unsigned long long)gamma);
  }
  int s = check_common(ctx, xb, wb, gb, "norm_matvec_argmax");
  if (s) return s;
  const int64_t M = xb->rows, K = xb->cols, N = wb->rows;
  // One row against a streamed BF16 weight: the head kernel with the pick's
  // first pass, then one block over its partials.  Else the two calls.
  const bool fused = M == 1 && N >= 1 && wb->elem == MI_BF16 && K <= 1024 && N * K * 2 >= DECODE_STREAM_BYTES &&
                     N <= INT32_MAX;
  if (!fused) {
    mi_id lg = 0, id = 0;
    s = mi_norm_matvec(ctx, x, gamma, eps, w, 0, 0, &lg);
    if (s) return s;
    s = mi_argmax_rows(ctx, lg, &id);
    if (s) {
      mi_free(ctx, lg);
      return s;
    }
    *logits = lg;
    *ids = id;
    return MI_OK;
  }
  const int64_t npairs = (N + 1) / 2, blocks = (npairs + 4 * HEAD_R - 1) / (4 * HEAD_R);
  char *sc = static_cast<char *>(scratch(ctx, static_cast<size_t>(blocks) * 8));
  if (!sc) return fail(ctx, MI_E_OOM, "norm_matvec_argmax scratch");
  mi_id lid, iid;
  Buffer *lb, *ib;
  s = new_buffer(ctx, 1, N, MI_F32, &lid, &lb);
  if (s) return s;
  s = new_buffer(ctx, 1, 1, MI_I32, &iid, &ib);
  if (s) {
    mi_free(ctx, lid);
    return s;
  }
  DecodeArgs g{};
  g.x = static_cast<const float *>(xb->ptr);
  g.ldx = K;
  g.K = K;
  g.gamma = gb ? static_cast<const float *>(gb->ptr) : nullptr;
  g.eps = eps;
  g.w = static_cast<const uint16_t *>(wb->ptr);
  g.N = N;
  g.npairs = npairs;
  g.out = static_cast<float *>(lb->ptr);
  g.ldo = N;
  float *pv = reinterpret_cast<float *>(sc);
  int32_t *pi = reinterpret_cast<int32_t *>(sc + static_cast<size_t>(blocks) * 4);
  decode_head_kernel<HEAD_R, true><<<static_cast<unsigned>(blocks), 256, 0, ctx->stream>>>(g, pv, pi);
  argmax_partials_kernel<<<1, 256, 0, ctx->stream>>>(pv, pi, blocks, static_cast<int32_t *>(ib->ptr));
  s = check_launch(ctx, "norm_matvec_argmax");
  if (s) {
    mi_free(ctx, lid);
    mi_free(ctx, iid);
    return s;
  }
  *logits = lid;
  *ids = iid;
  return MI_OK;
}

// pos_dev null: the immediate position `pos`; else read on the device.
static int norm_qkv_rope(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table, mi_id sin_table,
                         int64_t heads, int64_t kv_heads, int64_t pos, const int32_t *pos_dev, mi_id k_cache,
                         mi_id v_cache, mi_id *q_out) {
  if (!q_out) return fail(ctx, MI_E_ARG, "null out pointer");
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
  int s = check_common(ctx, xb, wb, gb, "norm_qkv_rope");
  if (s) return s;
  const int64_t M = xb->rows, D = kb->cols;
  if (heads < 1 || kv_heads < 1 || D < 2 || D % 2)
    return fail(ctx, MI_E_ARG, "norm_qkv_rope: heads %lld, kv heads %lld, head width %lld", (long long)heads,
                (long long)kv_heads, (long long)D);
  if (wb->rows != (heads + 2 * kv_heads) * D)
    return fail(ctx, MI_E_ARG, "norm_qkv_rope: weight has %lld rows, want (heads + 2 kv_heads) * %lld = %lld",
                (long long)wb->rows, (long long)D, (long long)((heads + 2 * kv_heads) * D));
  if (kb->elem != vb->elem || !elem_float(kb->elem) || vb->cols != D || vb->rows != kb->rows ||
      kb->rows % (M * kv_heads))
    return fail(ctx, MI_E_ARG, "norm_qkv_rope: caches must both be [rows * kv_heads * max_ctx, %lld], both F32 or both BF16",
                (long long)D);
  const int64_t maxc = kb->rows / (M * kv_heads);
  // A position read on the device may be any below max_ctx: the tables must
  // cover them all.
  const int64_t need = pos_dev ? maxc - 1 : pos;
  if (!pos_dev && (pos < 0 || pos >= maxc))
    return fail(ctx, MI_E_ARG, "norm_qkv_rope: position %lld beyond the cache's %lld", (long long)pos, (long long)maxc);
  if (cb->elem != MI_F32 || sb->elem != MI_F32 || cb->cols != D || sb->cols != D || cb->rows <= need || sb->rows <= need)
    return fail(ctx, MI_E_ARG, "norm_qkv_rope: rotary tables must be [> %lld, %lld] F32", (long long)need, (long long)D);
  mi_id id;
  Buffer *ob;
  s = new_buffer(ctx, M, heads * D, MI_F32, &id, &ob);
  if (s) return s;
  DecodeArgs g{};
  g.x = static_cast<const float *>(xb->ptr);
  g.ldx = xb->cols;
  g.K = xb->cols;
  g.gamma = gb ? static_cast<const float *>(gb->ptr) : nullptr;
  g.eps = eps;
  g.w = wb->elem == MI_BF16 ? static_cast<const uint16_t *>(wb->ptr) : nullptr;
  g.N = wb->rows;
  g.npairs = wb->rows / 2;
  g.out = static_cast<float *>(ob->ptr);
  g.ldo = heads * D;
  g.d = static_cast<int>(D);
  g.H = static_cast<int>(heads);
  g.KVH = static_cast<int>(kv_heads);
  g.pos = pos;
  g.maxc = maxc;
  g.cos = static_cast<const float *>(cb->ptr);
  g.sin = static_cast<const float *>(sb->ptr);
  g.kc = kb->ptr;
  g.vc = vb->ptr;
  g.kv16 = kb->elem == MI_BF16 ? 1 : 0;
  g.pos_dev = pos_dev;
  g.flags = flags(ctx);
  split_setup<DM_QKV>(ctx, M, g);
  s = launch_weight<DM_QKV>(ctx, M, g, wb);
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  s = check_launch(ctx, "norm_qkv_rope");
  if (s) {
    mi_free(ctx, id);
    return s;
  }
  *q_out = id;
  return MI_OK;
}

extern "C" int mi_norm_qkv_rope(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table,
                                mi_id sin_table, int64_t heads, int64_t kv_heads, int64_t pos, mi_id k_cache,
                                mi_id v_cache, mi_id *q_out) {
  MI_ENTER(ctx);
  return norm_qkv_rope(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, pos, nullptr, k_cache,
                       v_cache, q_out);
}

extern "C" int mi_norm_qkv_rope_at(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w_qkv, mi_id cos_table,
                                   mi_id sin_table, int64_t heads, int64_t kv_heads, mi_id pos, mi_id k_cache,
                                   mi_id v_cache, mi_id *q_out) {
  MI_ENTER(ctx);
  MI_BUF(ctx, pb, pos);
  if (pb->elem != MI_I32 || pb->numel() != 1)
    return fail(ctx, MI_E_ARG, "norm_qkv_rope_at: the position is %s [%lld, %lld], want I32 [1, 1]", elem_name(pb->elem),
                (long long)pb->rows, (long long)pb->cols);
  return norm_qkv_rope(ctx, x, gamma, eps, w_qkv, cos_table, sin_table, heads, kv_heads, 0,
                       static_cast<const int32_t *>(pb->ptr), k_cache, v_cache, q_out);
}

