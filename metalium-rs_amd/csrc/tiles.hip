// Products for short row counts -- a batch-1 prefill's 512 rows -- with the
// weight, and where the producer can, the activations in the matrix cores'
// operand order ("tiles", MI_TILES_BF16 / MI_TILES_PARTS).
//
// At 512 rows a decoder's products have 72-384 output tiles of 64 x 64: too
// few to fill 256 CUs whole, so the tiled kernels had split k over launches
// (a reduce launch after each) and still ran each k tile as a chain of
// global load -> LDS -> barrier -> matrix-core steps.  Here one block owns a
// 32 x 32 TN output tile and splits its k range over its KW waves; each wave
// issues every load of its range at once, straight into the operand
// registers of v_mfma_f32_32x32x16_bf16 (a tiled operand's step is one
// contiguous KiB across the wave: no LDS staging and no barrier in the k
// loop), sums its range in k order, and the block adds the waves' partial
// tiles in wave order through LDS.  The epilogue then stores the result with
// a linear layer's bias and residual, or forms a SwiGLU MLP's silu(gate) * up
// (gate|up pairs in one wave tile) or a prefill's q|k|v tail (RoPE, cache
// writes, q's layout; one 64-wide head a wave tile).
//
// The reference tiles its weights for its own cores (tt-layout,
// crates/tt-layout/src/lib.rs) and runs a Linear as float_matmul + float_add
// (crates/burn-tt/src/generated/ops.rs:532, 159); there is no counterpart
// of this kernel beyond that.
#include "common.hpp"
#include "tails.hpp"

namespace mi {

typedef __bf16 tbf16x8 __attribute__((ext_vector_type(8)));
typedef float tf32x16 __attribute__((ext_vector_type(16)));

// The A operand: tiles of an F32 operand's parts (two MFMAs a step, the
// remainder's first), tiles of BF16 values, or row-major F32 (split into
// parts in registers: the fast matmul mode's product) or BF16 rows.
enum { TA_PARTS = 0, TA_BF16 = 1, TA_ROWS_F32 = 2, TA_ROWS_BF16 = 3 };
// The epilogue: store (bias, residual), SwiGLU pairs, q|k|v tail.
enum { TE_STORE = 0, TE_SWIGLU = 1, TE_QKV = 2 };

struct TileArgs {
  const void *a = nullptr;
  const uint16_t *b = nullptr;  // the weight [N, K] in tiles
  int64_t M = 0, N = 0, K = 0;
  int64_t lda = 0;    // row-major A: row pitch in elements
  int64_t plane = 0;  // A's parts in tiles: elements of the heads' plane (M K)
  int tiles_m = 0, tiles_n = 0;
  // TE_STORE: C [M, N] F32 or BF16 (c_form), C = resid + (A B^T + bias).
  // TE_SWIGLU: [M, N / 2] in c_form (MI_F32, MI_BF16, MI_BF16_PARTS,
  // MI_TILES_BF16, MI_TILES_PARTS).
  void *c = nullptr;
  int c_form = MI_F32;
  const float *bias = nullptr;
  const float *resid = nullptr;
  int64_t ldr = 0;
  QkvTail qkv;  // TE_QKV
};

// Blocks run on XCD (block id % 8): consecutive tiles (in m-major order) go
// to one XCD, sharing its L2 for their rows of A.
__device__ __forceinline__ void tiles_block(const TileArgs &g, int *tm, int *tn) {
  const int total = g.tiles_m * g.tiles_n;
  int t = blockIdx.x;
  if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
  *tm = t / g.tiles_n;
  *tn = t - *tm * g.tiles_n;
}

template <int AM, int TN, int KW, int NS, int EPI>
__global__ void __launch_bounds__(KW * 64) gemm_tiles_kernel(TileArgs g) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [KW / 2][TN 16][64]
  constexpr bool PARTS = AM == TA_PARTS || AM == TA_ROWS_F32;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tm, tn;
  tiles_block(g, &tm, &tn);
  const int64_t KS = g.K >> 4;
  const int64_t s0 = (w * KS) / KW, s1 = ((w + 1) * KS) / KW;
  const int ns = static_cast<int>(s1 - s0);

  // Every load of this wave's k steps, issued together.  Steps past the
  // wave's range (its range may be a step shorter than NS) hold zeros, so the
  // matrix-core sequence below runs unconditionally: adding 0 x 0 changes no
  // partial sum but a -0 into a +0, and every product against one weight
  // runs the same sequence.
  uint4 ah[NS], al[NS], bw[NS][TN];
  float4 af[NS][2];
  const int64_t row = static_cast<int64_t>(tm) * 32 + (lane & 31);
  const int64_t kl = s0 * 16 + 8 * (lane >> 5);  // this lane's first k (row-major A)
  const uint4 z4 = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    ah[s] = al[s] = z4;
    af[s][0] = af[s][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < TN; ++j) bw[s][j] = z4;
    if (s < ns) {
      if constexpr (AM == TA_PARTS || AM == TA_BF16) {
        const uint16_t *ap = static_cast<const uint16_t *>(g.a) + ((tm * KS + s0 + s) * 64 + lane) * 8;
        ah[s] = *reinterpret_cast<const uint4 *>(ap);
        if constexpr (AM == TA_PARTS) al[s] = *reinterpret_cast<const uint4 *>(ap + g.plane);
      } else if constexpr (AM == TA_ROWS_F32) {
        const float *ap = static_cast<const float *>(g.a) + row * g.lda + kl + 16 * s;
        af[s][0] = *reinterpret_cast<const float4 *>(ap);
        af[s][1] = *reinterpret_cast<const float4 *>(ap + 4);
      } else {
        ah[s] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g.a) + row * g.lda + kl + 16 * s);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[s][j] = *reinterpret_cast<const uint4 *>(g.b + (((tn * TN + j) * KS + s0 + s) * 64 + lane) * 8);
    }
  }
  tf32x16 acc[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if constexpr (AM == TA_ROWS_F32) {
      split_bf16x2(af[s][0].x, af[s][0].y, ah[s].x, al[s].x);
      split_bf16x2(af[s][0].z, af[s][0].w, ah[s].y, al[s].y);
      split_bf16x2(af[s][1].x, af[s][1].y, ah[s].z, al[s].z);
      split_bf16x2(af[s][1].z, af[s][1].w, ah[s].w, al[s].w);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (PARTS)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(tbf16x8, al[s]),
                                                         __builtin_bit_cast(tbf16x8, bw[s][j]), acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(tbf16x8, ah[s]),
                                                       __builtin_bit_cast(tbf16x8, bw[s][j]), acc[j], 0, 0, 0);
    }
  }

  // The waves' partial tiles, added in a fixed order through LDS: wave w + H
  // into wave w (w < H = KW / 2), then those H sums in wave order -- half the
  // LDS of one slot a wave, so more blocks share a CU.  Accumulator value e
  // of fragment j is row 8 (e / 4) + 4 (lane / 32) + e % 4, column
  // 32 j + lane % 32.
  constexpr int H = KW > 1 ? KW / 2 : 1;
  static_assert(KW == 1 || KW % 2 == 0, "waves pair up");
  float *slot = red + static_cast<int64_t>(w % H) * TN * 16 * 64;
  if (KW > 1 && w >= H) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) slot[(j * 16 + e) * 64 + lane] = acc[j][e];
  }
  if constexpr (KW > 1) __syncthreads();
  if (w < H) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float v = acc[j][e];
        if constexpr (KW > 1) v += slot[(j * 16 + e) * 64 + lane];
        slot[(j * 16 + e) * 64 + lane] = v;
      }
  }
  __syncthreads();
  auto total = [&](int q) {
    float v = red[q * 64 + lane];
#pragma unroll
    for (int p = 1; p < H; ++p) v += red[(p * TN * 16 + q) * 64 + lane];
    return v;
  };
  const int64_t m0 = static_cast<int64_t>(tm) * 32;
  const int col = lane & 31;
  if constexpr (EPI == TE_STORE) {
    for (int q = w; q < TN * 16; q += KW) {
      const int j = q >> 4, e = q & 15;
      const int64_t r = m0 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      const int64_t c = (static_cast<int64_t>(tn) * TN + j) * 32 + col;
      float x = total(q);
      if (g.bias) x = __fadd_rn(x, g.bias[c]);
      if (g.resid) x = __fadd_rn(g.resid[r * g.ldr + c], x);
      if (g.c_form == MI_BF16) static_cast<uint16_t *>(g.c)[r * g.N + c] = f32_to_bf16_bits(x);
      else static_cast<float *>(g.c)[r * g.N + c] = x;
    }
  } else if constexpr (EPI == TE_SWIGLU) {
    static_assert(TN == 2, "gate|up pairs");
    const int64_t I = g.N >> 1;
    for (int e = w; e < 16; e += KW) {
      const int64_t r = m0 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      const int64_t c = static_cast<int64_t>(tn) * 32 + col;
      const float y = swiglu_value(total(e), total(16 + e));
      uint16_t *P = static_cast<uint16_t *>(g.c);
      switch (g.c_form) {
        case MI_F32: static_cast<float *>(g.c)[r * I + c] = y; break;
        case MI_BF16: P[r * I + c] = f32_to_bf16_bits(y); break;
        case MI_TILES_BF16: P[tile_offset(r, c, I)] = f32_to_bf16_bits(y); break;
        default: {
          uint16_t h, l;
          split_bf16(y, h, l);
          if (g.c_form == MI_BF16_PARTS) {
            P[r * 2 * I + c] = h;
            P[r * 2 * I + I + c] = l;
          } else {
            const int64_t o = tile_offset(r, c, I);
            P[o] = h;
            P[g.M * I + o] = l;
          }
        }
      }
    }
  } else {
    static_assert(TN == 2, "one 64-wide head a tile");
    const QkvTail &t = g.qkv;
    const int h = tn;
    const bool rope = h < t.heads + t.kvh;
    for (int e = w; e < 16; e += KW) {
      const int64_t r = m0 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      const int64_t b = r / t.seq, p = r - b * t.seq;
      float y0 = total(e), y1 = total(16 + e);
      if (rope) {
        const int64_t pos = t.pos0 + p;
        rope_pair(y0, y1, t.cos[pos * 64 + col], t.cos[pos * 64 + col + 32], t.sin[pos * 64 + col],
                  t.sin[pos * 64 + col + 32], y0, y1);
      }
      qkv_put(t, r, b, p, h, col, y0, y1);
    }
  }
}

// A row-major F32 or BF16 [R, K] as tiles: one thread per 8 consecutive
// values of a row, stored as one 16-byte lane chunk (and its remainders').
template <typename S, bool PARTS>
__global__ void __launch_bounds__(256) tile_pack_kernel(const S *a, int64_t R, int64_t K, uint16_t *out) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_row = K >> 3;
  if (u >= R * per_row) return;
  const int64_t r = u / per_row, k = (u - r * per_row) * 8;
  uint4 hv, lv;
  if constexpr (sizeof(S) == 4) {
    const float4 v0 = *reinterpret_cast<const float4 *>(a + r * K + k);
    const float4 v1 = *reinterpret_cast<const float4 *>(a + r * K + k + 4);
    if constexpr (PARTS) {
      split_bf16x2(v0.x, v0.y, hv.x, lv.x);
      split_bf16x2(v0.z, v0.w, hv.y, lv.y);
      split_bf16x2(v1.x, v1.y, hv.z, lv.z);
      split_bf16x2(v1.z, v1.w, hv.w, lv.w);
    } else {
      hv = make_uint4(bf16x2_bits(v0.x, v0.y), bf16x2_bits(v0.z, v0.w), bf16x2_bits(v1.x, v1.y),
                      bf16x2_bits(v1.z, v1.w));
    }
  } else {
    hv = *reinterpret_cast<const uint4 *>(a + r * K + k);
  }
  const int64_t o = tile_offset(r, k, K);
  *reinterpret_cast<uint4 *>(out + o) = hv;
  if constexpr (PARTS) *reinterpret_cast<uint4 *>(out + R * K + o) = lv;
}

// -------------------------------------------------------------- launching
// One block a 32 x 32 TN output tile.  Its wave count depends on k alone --
// up to 3 steps a wave on 1, 4, 8, 12 or 16 waves, then 6 steps on 16 (k <=
// 1536) -- so every product against the same weight adds the same k ranges
// in the same order, whatever its epilogue (TN 2 for pairs and heads).  The
// waves' partial tiles take KW / 2 x TN x 4 KiB of LDS.
template <int AM, int TN, int EPI, int KW, int NS>
static hipError_t launch_tiles_kw(const TileArgs &g, hipStream_t st) {
  constexpr int LDS = (KW > 1 ? KW / 2 : 1) * TN * 16 * 64 * 4;
  auto kern = gemm_tiles_kernel<AM, TN, KW, NS, EPI>;
  static bool attr = false;
  if (!attr) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  kern<<<dim3(static_cast<unsigned>(g.tiles_m * g.tiles_n)), KW * 64, LDS, st>>>(g);
  return hipGetLastError();
}

// The waves of a block for k / 16 = ks steps (0: more than 96 steps).
static int tiles_waves(int64_t ks) {
  if (ks <= 3) return 1;
  if (ks <= 12) return 4;
  if (ks <= 24) return 8;
  if (ks <= 36) return 12;
  if (ks <= 96) return 16;
  return 0;
}

template <int AM, int TN, int EPI>
static hipError_t launch_tiles_am(const TileArgs &g, hipStream_t st) {
  const int64_t ks = g.K >> 4;
  switch (tiles_waves(ks)) {
    case 1: return launch_tiles_kw<AM, TN, EPI, 1, 3>(g, st);
    case 4: return launch_tiles_kw<AM, TN, EPI, 4, 3>(g, st);
    case 8: return launch_tiles_kw<AM, TN, EPI, 8, 3>(g, st);
    case 12: return launch_tiles_kw<AM, TN, EPI, 12, 3>(g, st);
    default:
      if (ks <= 48) return launch_tiles_kw<AM, TN, EPI, 16, 3>(g, st);
      return launch_tiles_kw<AM, TN, EPI, 16, 6>(g, st);
  }
}

template <int TN, int EPI>
static hipError_t launch_tiles(int am, const TileArgs &g, hipStream_t st) {
  switch (am) {
    case TA_PARTS: return launch_tiles_am<TA_PARTS, TN, EPI>(g, st);
    case TA_BF16: return launch_tiles_am<TA_BF16, TN, EPI>(g, st);
    case TA_ROWS_F32: return launch_tiles_am<TA_ROWS_F32, TN, EPI>(g, st);
    default: return launch_tiles_am<TA_ROWS_BF16, TN, EPI>(g, st);
  }
}

// The A operand of a product against the tiled weight W [N, K]: its form,
// and the operand fields of g.  0, or a failure recorded.
static int tiles_operands(Ctx *ctx, const char *op, const Buffer *X, const Buffer *W, int pair_cols, TileArgs *g,
                          int *am) {
  if (W->tiles != MI_TILES_BF16 || W->elem != MI_BF16)
    return fail(ctx, MI_E_ARG, "%s: the weight is not BF16 tiles", op);
  const int64_t N = W->rows, K = W->cols;
  int64_t M, XK;
  if (X->tiles == MI_TILES_PARTS) {
    *am = TA_PARTS;
    M = X->rows;
    XK = X->cols / 2;
  } else if (X->tiles == MI_TILES_BF16) {
    *am = TA_BF16;
    M = X->rows;
    XK = X->cols;
  } else if (X->tiles) {
    return fail(ctx, MI_E_ARG, "%s: activations in unknown tiles", op);
  } else if (X->elem == MI_F32) {
    if (ctx->matmul_mode != MI_MATMUL_FAST)
      return fail(ctx, MI_E_UNSUPPORTED, "%s: F32 activations against a tiled weight in the accurate matmul mode", op);
    *am = TA_ROWS_F32;
    M = X->rows;
    XK = X->cols;
  } else if (X->elem == MI_BF16) {
    *am = TA_ROWS_BF16;
    M = X->rows;
    XK = X->cols;
  } else {
    return fail(ctx, MI_E_ARG, "%s: activations %s", op, elem_name(X->elem));
  }
  if (XK != K)
    return fail(ctx, MI_E_ARG, "%s: x is [%lld, %lld], the weight [%lld, %lld]", op, (long long)M, (long long)XK,
                (long long)N, (long long)K);
  const int tn = pair_cols ? 2 : 1;
  if (M % 32 || N % (32 * tn) || K % 16 || K < 16 || !tiles_waves(K / 16) || M < 32)
    return fail(ctx, MI_E_UNSUPPORTED, "%s: [%lld, %lld] x [%lld, %lld]^T in tiles (m a multiple of 32, n of %d, k of 16 "
                "up to 1536)", op, (long long)M, (long long)K, (long long)N, (long long)K, 32 * tn);
  if ((M / 32) * (N / (32 * tn)) > INT32_MAX) return fail(ctx, MI_E_UNSUPPORTED, "%s: too many tiles", op);
  g->a = X->ptr;
  g->b = static_cast<const uint16_t *>(W->ptr);
  g->M = M; g->N = N; g->K = K;
  g->lda = X->cols;
  g->plane = M * K;
  g->tiles_m = static_cast<int>(M / 32);
  g->tiles_n = static_cast<int>(N / (32 * tn));
  return MI_OK;
}

int tiles_linear(mi_ctx *ctx, mi_id x, mi_id w, const float *bias, const float *resid, int out_elem, mi_id *out) {
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w);
  if (out_elem != MI_F32 && out_elem != MI_BF16) return fail(ctx, MI_E_ARG, "linear: result kind %d", out_elem);
  TileArgs g;
  int am;
  // 32 x 64 tiles for long k where 32 x 32 ones would take more than a round
  // of the chip's 256 CUs and the wider ones fit in one (a 512-row prompt's
  // down product: 288 blocks -> 144, 11.3 -> 10.1 us; its o product, k 576,
  // measured slower so); the k ranges, hence the sums, are the same either way.
  const int64_t tiles32 = (X->rows / 32) * (W->rows / 32);
  const bool wide = W->rows % 64 == 0 && W->cols > 768 && tiles32 > 256 && tiles32 / 2 <= 256;
  if (int s = tiles_operands(ctx, "linear", X, W, wide, &g, &am)) return s;
  mi_id id;
  Buffer *ob;
  if (int s = new_buffer(ctx, g.M, g.N, out_elem, &id, &ob)) return s;
  g.c = ob->ptr;
  g.c_form = out_elem;
  g.bias = bias;
  g.resid = resid;
  g.ldr = g.N;
  const hipError_t e = wide ? launch_tiles<2, TE_STORE>(am, g, ctx->stream) : launch_tiles<1, TE_STORE>(am, g, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear (tiles) launch: %s", hipGetErrorString(e));
  }
  if (int s = check_launch(ctx, "linear (tiles)")) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}

int tiles_swiglu(mi_ctx *ctx, mi_id x, mi_id w_pairs, int out_form, mi_id *out) {
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w_pairs);
  if (out_form != MI_F32 && out_form != MI_BF16 && out_form != MI_BF16_PARTS && out_form != MI_TILES_BF16 &&
      out_form != MI_TILES_PARTS)
    return fail(ctx, MI_E_ARG, "linear_swiglu: result kind %d", out_form);
  TileArgs g;
  int am;
  if (int s = tiles_operands(ctx, "linear_swiglu", X, W, 1, &g, &am)) return s;
  const int64_t I = g.N / 2;
  const bool parts = out_form == MI_BF16_PARTS || out_form == MI_TILES_PARTS;
  const bool tiled = out_form == MI_TILES_BF16 || out_form == MI_TILES_PARTS;
  mi_id id;
  Buffer *ob;
  if (int s = new_buffer(ctx, g.M, parts ? 2 * I : I, out_form == MI_F32 ? MI_F32 : MI_BF16, &id, &ob)) return s;
  ob->tiles = tiled ? out_form : 0;
  g.c = ob->ptr;
  g.c_form = out_form;
  const hipError_t e = launch_tiles<2, TE_SWIGLU>(am, g, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear_swiglu (tiles) launch: %s", hipGetErrorString(e));
  }
  if (int s = check_launch(ctx, "linear_swiglu (tiles)")) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}

int tiles_qkv(mi_ctx *ctx, mi_id x, mi_id w_qkv, const QkvTail &t) {
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w_qkv);
  TileArgs g;
  int am;
  if (int s = tiles_operands(ctx, "linear_qkv_rope_cache", X, W, 1, &g, &am)) return s;
  g.qkv = t;
  const hipError_t e = launch_tiles<2, TE_QKV>(am, g, ctx->stream);
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "linear_qkv_rope_cache (tiles) launch: %s", hipGetErrorString(e));
  return check_launch(ctx, "linear_qkv_rope_cache (tiles)");
}

}  // namespace mi

using namespace mi;

extern "C" int mi_tile(mi_ctx *ctx, mi_id a, int form, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, A, a);
  if (A->tiles || !elem_float(A->elem))
    return fail(ctx, MI_E_ARG, "tile of a %s buffer%s", elem_name(A->elem), A->tiles ? " already in tiles" : "");
  if (form != MI_TILES_BF16 && form != MI_TILES_PARTS) return fail(ctx, MI_E_ARG, "tile: form %d", form);
  if (form == MI_TILES_PARTS && A->elem != MI_F32) return fail(ctx, MI_E_ARG, "tile: parts of a BF16 buffer");
  const int64_t R = A->rows, K = A->cols;
  if (R % 32 || K % 16)
    return fail(ctx, MI_E_ARG, "tile: [%lld, %lld] (rows a multiple of 32, columns of 16)", (long long)R, (long long)K);
  const bool parts = form == MI_TILES_PARTS;
  mi_id id;
  Buffer *ob;
  if (int s = new_buffer(ctx, R, parts ? 2 * K : K, MI_BF16, &id, &ob)) return s;
  ob->tiles = form;
  const int64_t units = R * (K / 8);
  if (units > 0) {
    const unsigned grid = static_cast<unsigned>((units + 255) / 256);
    uint16_t *o = static_cast<uint16_t *>(ob->ptr);
    if (A->elem == MI_BF16)
      tile_pack_kernel<uint16_t, false><<<grid, 256, 0, ctx->stream>>>(static_cast<const uint16_t *>(A->ptr), R, K, o);
    else if (parts)
      tile_pack_kernel<float, true><<<grid, 256, 0, ctx->stream>>>(static_cast<const float *>(A->ptr), R, K, o);
    else
      tile_pack_kernel<float, false><<<grid, 256, 0, ctx->stream>>>(static_cast<const float *>(A->ptr), R, K, o);
  }
  if (int s = check_launch(ctx, "tile")) {
    mi_free(ctx, id);
    return s;
  }
  *out = id;
  return MI_OK;
}
