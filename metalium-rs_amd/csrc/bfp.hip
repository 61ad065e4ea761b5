// Block floating point storage (MI_BFP8): the performance contract's weight
// format.
//
// Reference: Engine::cast_bfp (crates/burn-tt/src/server.rs:141-147,
// 1035-1050; Session::store_bfp / bfp_to_f32), StorageFormat::Bfp8
// (crates/burn-tt/src/storage.rs:24-40), the packer's rule as the host
// restates it (crates/tt-models/src/quant.rs:185-235, bfp_round_trip) and the
// unpacker's decode (crates/tt-isa/src/tile.rs:619-636, bfp8_to_bf16).
//
// A row is cut into blocks of 16 consecutive columns.  A block keeps E, the
// largest biased F32 exponent of its values, and each value as q, its BF16
// truncation in quanta of 2^(E - 133) rounded half away from zero and
// clamped to 127 (sign kept).  The unpacker's decode of such a datum is
// q * 2^(E - 133) exactly: for a normal value the decoded exponent is the
// value's own (one more after a round-up), so its exponent arithmetic never
// wraps, and a zero or subnormal value has q = 0.  The device therefore
// stores q as a two's-complement byte -- one sign-extending conversion to
// decode -- where the Tensix datum is sign and magnitude; the values are the
// same.
//
// MI355X design.  Packing and decoding are HBM-bound streams: one thread per
// block of 16 values, its 64 (F32) or 32 (BF16) source bytes as 16-byte
// loads, its 16 datum bytes as one 16-byte store and its exponent byte
// beside its neighbours'.  The consumers (decode GEMVs, the fused decode
// attention, the matrix-core decode projections) read the datums and the
// exponents themselves and form each weight as q * 2^(E - 133) before the
// product, so a BFP8 weight's products are the BF16 weight's products on the
// same values.
#include "common.hpp"

namespace mi {

__device__ __forceinline__ uint32_t src_bits(const float *p, int64_t i) { return __float_as_uint(p[i]); }
__device__ __forceinline__ uint32_t src_bits(const uint16_t *p, int64_t i) { return static_cast<uint32_t>(p[i]) << 16; }

// VEC: cols a multiple of 16 (every block whole, every access aligned).
template <typename SRC, bool VEC>
__global__ void __launch_bounds__(256) bfp8_pack_kernel(const SRC *x, int64_t rows, int64_t cols, int8_t *dat,
                                                          uint8_t *ex, uint32_t *flags) {
  const int64_t nb = (cols + 15) / 16;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * nb) return;
  const int64_t r = t / nb, b = t - r * nb, c0 = b * 16;
  const int n = VEC ? 16 : (cols - c0 < 16 ? static_cast<int>(cols - c0) : 16);
  const SRC *src = x + r * cols + c0;
  uint32_t u[16];
  if constexpr (VEC) {
    if constexpr (sizeof(SRC) == 4) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint4 w = *reinterpret_cast<const uint4 *>(src + 4 * v);
        u[4 * v] = w.x; u[4 * v + 1] = w.y; u[4 * v + 2] = w.z; u[4 * v + 3] = w.w;
      }
    } else {
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const uint4 w = *reinterpret_cast<const uint4 *>(src + 8 * v);
        const uint32_t h[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          u[8 * v + 2 * e] = h[e] << 16;
          u[8 * v + 2 * e + 1] = h[e] & 0xffff0000u;
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) u[j] = j < n ? src_bits(src, j) : 0u;
  }
  uint32_t E = 0;
  bool finite = true;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t e = (u[j] >> 23) & 0xffu;
    E = e > E ? e : E;
    finite = finite && e != 0xffu;
  }
  uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t bt = u[j] & 0xffff0000u;  // the BF16 truncation
    int m = 0;
    if (finite && (bt & 0x7f800000u)) {
      // |bt| < 2^(E - 126), so this is below 128 quanta; ldexp is exact.
      const float s = ldexpf(fabsf(__uint_as_float(bt)), 133 - static_cast<int>(E));
      const int rd = static_cast<int>(roundf(s));  // half away from zero
      m = rd < 127 ? rd : 127;
    }
    const int q = (bt & 0x80000000u) ? -m : m;
    packed[j >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (j & 3));
  }
  if (!finite) atomicOr(flags, FLAG_NOT_FINITE);
  int8_t *d = dat + r * cols + c0;
  if constexpr (VEC) {
    *reinterpret_cast<uint4 *>(d) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < n) d[j] = static_cast<int8_t>((packed[j >> 2] >> (8 * (j & 3))) & 0xffu);
  }
  ex[r * nb + b] = static_cast<uint8_t>(E);
}

__device__ __forceinline__ void put_val(float *p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void put_val(uint16_t *p, int64_t i, float v) { p[i] = static_cast<uint16_t>(__float_as_uint(v) >> 16); }

template <typename DST, bool VEC>
__global__ void __launch_bounds__(256) bfp8_unpack_kernel(const int8_t *dat, const uint8_t *ex, int64_t rows,
                                                            int64_t cols, DST *y) {
  const int64_t nb = (cols + 15) / 16;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * nb) return;
  const int64_t r = t / nb, b = t - r * nb, c0 = b * 16;
  const int e = ex[r * nb + b];
  DST *dst = y + r * cols + c0;
  if constexpr (VEC) {
    const uint4 w = *reinterpret_cast<const uint4 *>(dat + r * cols + c0);
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = bfp8_val(d[j >> 2], j & 3, e);
    if constexpr (sizeof(DST) == 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4 *>(dst + 4 * q) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
      // Exact in BF16: the F32 value's top half.
      uint32_t h[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) h[q] = (__float_as_uint(v[2 * q]) >> 16) | (__float_as_uint(v[2 * q + 1]) & 0xffff0000u);
      *reinterpret_cast<uint4 *>(dst) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4 *>(dst + 8) = make_uint4(h[4], h[5], h[6], h[7]);
    }
  } else {
    const int n = cols - c0 < 16 ? static_cast<int>(cols - c0) : 16;
    const int8_t *s = dat + r * cols + c0;
    for (int j = 0; j < n; ++j) put_val(dst, j, ldexpf(static_cast<float>(s[j]), e - 133));
  }
}

int bfp8_decode_to(Ctx *ctx, const Buffer *src, int elem, mi_id *id, Buffer **out) {
  if (src->elem != MI_BFP8 || (elem != MI_F32 && elem != MI_BF16))
    return fail(ctx, MI_E_ARG, "BFP8 decode of a %s buffer to %s", elem_name(src->elem), elem_name(elem));
  const int64_t rows = src->rows, cols = src->cols;
  const int8_t *dat = static_cast<const int8_t *>(src->ptr);
  const uint8_t *ex = static_cast<const uint8_t *>(src->ptr) + bfp8_exp_offset(rows, cols);
  Buffer *ob;
  int s = new_buffer(ctx, rows, cols, elem, id, &ob);
  if (s) return s;
  if (out) *out = ob;
  const int64_t blocks = rows * bfp_blocks(cols);
  if (blocks == 0) return MI_OK;
  const unsigned g = grid_for(blocks, 256, INT32_MAX);
  const bool vec = cols % 16 == 0;
  if (elem == MI_F32) {
    float *y = static_cast<float *>(ob->ptr);
    if (vec) bfp8_unpack_kernel<float, true><<<g, 256, 0, ctx->stream>>>(dat, ex, rows, cols, y);
    else bfp8_unpack_kernel<float, false><<<g, 256, 0, ctx->stream>>>(dat, ex, rows, cols, y);
  } else {
    uint16_t *y = static_cast<uint16_t *>(ob->ptr);
    if (vec) bfp8_unpack_kernel<uint16_t, true><<<g, 256, 0, ctx->stream>>>(dat, ex, rows, cols, y);
    else bfp8_unpack_kernel<uint16_t, false><<<g, 256, 0, ctx->stream>>>(dat, ex, rows, cols, y);
  }
  s = check_launch(ctx, "bfp8 decode");
  if (s) mi_free(static_cast<mi_ctx *>(ctx), *id);
  return s;
}

// F32 or BF16 `A` into a new BFP8 buffer.
static int bfp8_pack(Ctx *ctx, const Buffer *A, mi_id *out) {
  const int64_t rows = A->rows, cols = A->cols;
  const void *x = A->ptr;
  const int se = A->elem;
  mi_id id;
  Buffer *ob;
  int s = new_buffer(ctx, rows, cols, MI_BFP8, &id, &ob);
  if (s) return s;
  const int64_t blocks = rows * bfp_blocks(cols);
  if (blocks > 0) {
    int8_t *dat = static_cast<int8_t *>(ob->ptr);
    uint8_t *ex = static_cast<uint8_t *>(ob->ptr) + bfp8_exp_offset(rows, cols);
    const unsigned g = grid_for(blocks, 256, INT32_MAX);
    const bool vec = cols % 16 == 0;
    if (se == MI_F32) {
      const float *xp = static_cast<const float *>(x);
      if (vec) bfp8_pack_kernel<float, true><<<g, 256, 0, ctx->stream>>>(xp, rows, cols, dat, ex, flags(ctx));
      else bfp8_pack_kernel<float, false><<<g, 256, 0, ctx->stream>>>(xp, rows, cols, dat, ex, flags(ctx));
    } else {
      const uint16_t *xp = static_cast<const uint16_t *>(x);
      if (vec) bfp8_pack_kernel<uint16_t, true><<<g, 256, 0, ctx->stream>>>(xp, rows, cols, dat, ex, flags(ctx));
      else bfp8_pack_kernel<uint16_t, false><<<g, 256, 0, ctx->stream>>>(xp, rows, cols, dat, ex, flags(ctx));
    }
    s = check_launch(ctx, "bfp8 pack");
    if (s) {
      mi_free(static_cast<mi_ctx *>(ctx), id);
      return s;
    }
  }
  *out = id;
  return MI_OK;
}

}  // namespace mi

using namespace mi;

extern "C" int mi_cast_bfp(mi_ctx *ctx, mi_id a, int format, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, A, a);
  if (format == MI_BFP8) {
    if (A->elem != MI_F32 && A->elem != MI_BF16)
      return fail(ctx, MI_E_ARG, "cast_bfp stores an F32 or BF16 buffer, not %s", elem_name(A->elem));
    return bfp8_pack(ctx, A, out);
  }
  if (format == 0) {
    if (A->elem != MI_BFP8) return fail(ctx, MI_E_ARG, "cast_bfp decodes a BFP8 buffer, not %s", elem_name(A->elem));
    return bfp8_decode_to(ctx, A, MI_F32, out, nullptr);
  }
  return fail(ctx, MI_E_UNSUPPORTED, "cast_bfp: format %d (MI_BFP8 is held; BFP4 and BFP2 are not)", format);
}
