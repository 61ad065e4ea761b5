// Shared definitions of the MI355X engine: the context (device, stream,
// buffer table, caching allocator, sticky error), element helpers and the
// launch-check helpers every kernel file uses.
//
// The context restates the reference's device server state -- the buffer
// table `DramBuffers` (crates/burn-tt/src/server.rs:868), the id counter that
// never reuses an id (server.rs:2421-2446) and the first recorded failure
// (server.rs:2390-2425) -- for a GPU driven through one HIP stream instead of
// a server thread.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/miburn.h"

namespace mi {

// ---------------------------------------------------------------- elements
inline size_t elem_size(int elem) { return elem == MI_BF16 ? 2 : elem == MI_BFP8 ? 1 : 4; }
// BFP8 storage: rows x cols datum bytes, then from the next multiple of 256
// bytes the block exponents, rows x ceil(cols / 16) bytes.
inline int64_t bfp_blocks(int64_t cols) { return (cols + 15) / 16; }
inline size_t bfp8_exp_offset(int64_t rows, int64_t cols) {
  return (static_cast<size_t>(rows) * static_cast<size_t>(cols) + 255) & ~static_cast<size_t>(255);
}
// Bytes a buffer of `elem` [rows, cols] holds.
inline size_t storage_bytes(int elem, int64_t rows, int64_t cols) {
  if (elem == MI_BFP8) return bfp8_exp_offset(rows, cols) + static_cast<size_t>(rows) * bfp_blocks(cols);
  return static_cast<size_t>(rows) * static_cast<size_t>(cols) * elem_size(elem);
}
inline bool elem_valid(int elem) { return (elem >= MI_F32 && elem <= MI_BF16) || elem == MI_BFP8; }
inline bool elem_float(int elem) { return elem == MI_F32 || elem == MI_BF16; }
const char *elem_name(int elem);

// BF16 <-> F32 on the device.  Narrowing rounds to nearest, ties to even,
// keeps subnormals (F32 denormals are on) and keeps a NaN a quiet NaN with
// its sign and top payload bits: gfx950's v_cvt_pk_bf16_f32, whose result
// for every one of the 2^32 F32 bit patterns u was checked on the device to
// equal the integer form the host oracle uses -- (u >> 16) | 0x40 for a NaN,
// else (u + 0x7fff + ((u >> 16) & 1)) >> 16.  Widening is exact.
typedef __bf16 mi_bf16x2 __attribute__((ext_vector_type(2)));
typedef float mi_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Two values narrowed in one instruction: a in the low half, b in the high.
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const mi_f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, mi_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return static_cast<uint16_t>(bf16x2_bits(f, 0.0f));
}

// An F32 value as two BF16 parts, hi + lo within 2^-17 relative of it: hi
// rounded to nearest even, lo the BF16 of the exact F32 remainder a - hi.  A
// finite value above the largest BF16 would round to infinity: it keeps the
// truncated head instead (its remainder is still exact in F32).  An infinite
// or NaN value is carried by its head alone.
__device__ __forceinline__ void split_bf16(float a, uint16_t &hi, uint16_t &lo) {
  hi = f32_to_bf16_bits(a);
  if (((hi & 0x7fffu) == 0x7f80u) && ((__float_as_uint(a) & 0x7f800000u) != 0x7f800000u))
    hi = static_cast<uint16_t>(__float_as_uint(a) >> 16);
  const float r = a - bf16_bits_to_f32(hi);
  lo = (r == r) ? f32_to_bf16_bits(r) : 0;
}
// split_bf16 of two values, their heads and remainders packed in pairs (a in
// the low halves).  A head with an all-ones exponent (an infinity or NaN
// input, or a finite one rounding to infinity) is rare: such a pair takes
// split_bf16 per value.
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
  const uint32_t h = bf16x2_bits(a, b);
  if (__builtin_expect((h & 0x7f80u) == 0x7f80u || (h & 0x7f800000u) == 0x7f800000u, 0)) {
    uint16_t h0, l0, h1, l1;
    split_bf16(a, h0, l0);
    split_bf16(b, h1, l1);
    hi = uint32_t(h0) | (uint32_t(h1) << 16);
    lo = uint32_t(l0) | (uint32_t(l1) << 16);
    return;
  }
  hi = h;
  lo = bf16x2_bits(a - __uint_as_float(h << 16), b - __uint_as_float(h & 0xffff0000u));
}

// Four consecutive F32 values of a row as parts: their heads at hp, their
// remainders at lp (a row of MI_BF16_PARTS keeps its heads, then its
// remainders).
__device__ __forceinline__ void parts4_put(uint16_t *hp, uint16_t *lp, float4 v) {
  uint32_t h0, l0, h1, l1;
  split_bf16x2(v.x, v.y, h0, l0);
  split_bf16x2(v.z, v.w, h1, l1);
  *reinterpret_cast<uint2 *>(hp) = make_uint2(h0, h1);
  *reinterpret_cast<uint2 *>(lp) = make_uint2(l0, l1);
}

// F32 values in F32 or BF16 (uint16_t bits) storage -- a KV cache under the
// reference or the performance numeric contract, an activation stored for a
// product's operand: four consecutive values widened to F32, and F32 values
// stored (BF16 rounded to nearest, ties to even).
__device__ __forceinline__ float4 f32x4_get(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 f32x4_get(const uint16_t *p) {
  const uint2 u = *reinterpret_cast<const uint2 *>(p);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xffff0000u));
}
__device__ __forceinline__ void f32x4_put(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ void f32x4_put(uint16_t *p, float4 v) {
  *reinterpret_cast<uint2 *>(p) = make_uint2(bf16x2_bits(v.x, v.y), bf16x2_bits(v.z, v.w));
}
__device__ __forceinline__ void f32_put(float *p, float v) { *p = v; }
__device__ __forceinline__ void f32_put(uint16_t *p, float v) { *p = f32_to_bf16_bits(v); }

// Element (r, k) of an [R, K] operand in tiles (MI_TILES_BF16 / one plane of
// MI_TILES_PARTS): block (r / 32, k / 16) of 64 lanes x 8 values, lane
// r % 32 + 32 ((k / 8) % 2), value k % 8.
__device__ __host__ __forceinline__ int64_t tile_offset(int64_t r, int64_t k, int64_t K) {
  return (((r >> 5) * (K >> 4) + (k >> 4)) * 64 + (r & 31) + 32 * ((k >> 3) & 1)) * 8 + (k & 7);
}

// The logistic function in its two-branch form, so neither exponential
// overflows: 1 / (1 + e^-x) for x >= 0 and e^x / (1 + e^x) below.  Both
// share t = e^-|x| (which is e^-x above zero and e^x below), so it is
// computed branch-free: r = 1 / (1 + t), then r or t r -- one exponential,
// no divergence within a wavefront.  t is the hardware 2^y (v_exp_f32) of
// y = -|x| log2(e) and r the hardware reciprocal (v_rcp_f32), each within
// 1 ulp; y's rounding and the F32 log2(e) (0.22 2^-24 below the true one)
// add up to 1.23 |x| 2^-24 of relative error to t, so with the sum's and the
// product's roundings the result is within (6 + 1.25 |x|) 2^-24 relative of
// the exact logistic (for |x| < 87, where t is normal) -- 2-3x faster than
// the library exponential and an IEEE division, which made it most of a
// SwiGLU epilogue's cost.
__device__ __forceinline__ float sigmoid2(float x) {
  const float t = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  const float r = __builtin_amdgcn_rcpf(1.0f + t);
  return x >= 0.0f ? r : t * r;
}

// A word written by an earlier launch and only read in this one (a decode
// step's device-held position), read through the scalar cache: a scalar load
// completes on its own counter, so what waits for it does not also wait for
// the vector loads issued around it (those complete in order, and making a
// vector-loaded value uniform waits for all of them).  p: a uniform address.
typedef __attribute__((address_space(4))) const int32_t mi_const_i32;
__device__ __forceinline__ int32_t scalar_read_i32(const int32_t *p) { return *(mi_const_i32 *)p; }

// Argmax's rule (crates/burn-tt/src/ops.rs:2389-2490): the largest value,
// a NaN above every number, the lowest index among equals -- a total order
// on (value, index), so partial bests fold in any order.
struct ArgBest { float v; int32_t i; };
__device__ __forceinline__ ArgBest better(ArgBest a, ArgBest b) {
  const bool an = isnan(a.v), bn = isnan(b.v);
  if (an || bn) {
    if (an && bn) return a.i <= b.i ? a : b;
    return an ? a : b;
  }
  if (a.v > b.v) return a;
  if (b.v > a.v) return b;
  return a.i <= b.i ? a : b;
}

// Streaming (non-temporal) 16-byte accesses: the line is not kept in the
// caches.  On an MI355X a stream of them moves ~80% of the 8 TB/s peak
// against ~70% for ordinary accesses; they suit operands far larger than the
// caches that no later kernel re-reads soon.  NT = false gives the ordinary
// access, so one kernel body serves both.
typedef float mi_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mi_u32x4 __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ float4 ld4(const float *p) {
  if constexpr (NT) {
    const mi_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const mi_f32x4 *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const float4 *>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void st4(float *p, float4 v) {
  if constexpr (NT) {
    const mi_f32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<mi_f32x4 *>(p));
  } else {
    *reinterpret_cast<float4 *>(p) = v;
  }
}
template <bool NT>
__device__ __forceinline__ uint4 ldu4(const void *p) {
  if constexpr (NT) {
    const mi_u32x4 v = __builtin_nontemporal_load(static_cast<const mi_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *static_cast<const uint4 *>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void stu4(void *p, uint4 v) {
  if constexpr (NT) {
    const mi_u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<mi_u32x4 *>(p));
  } else {
    *static_cast<uint4 *>(p) = v;
  }
}
// BFP8 values (MI_BFP8): datum q, a signed byte, under its block's exponent
// byte e is q * 2^(e - 133) -- at most 7 significant bits, so exact in F32
// and in BF16 (the F32 value's top half).  ldexp keeps it exact for every e,
// including the blocks of tiny values whose factor 2^(e - 133) alone would
// be subnormal.
__device__ __forceinline__ float bfp8_val(uint32_t word, int byte, int e) {
  return ldexpf(static_cast<float>(static_cast<int8_t>(word >> (8 * byte))), e - 133);
}
// Eight consecutive datums (one 8-byte load) of one block.
__device__ __forceinline__ void bfp8x8(uint2 d, int e, float (&w)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w[j] = bfp8_val(d.x, j, e);
    w[4 + j] = bfp8_val(d.y, j, e);
  }
}

// Host side: stream an operation's accesses when it moves at least this many
// bytes -- beyond what the 256 MB last-level cache would keep for the next
// kernel to re-read.
constexpr int64_t kStreamBytes = int64_t(128) << 20;

// ------------------------------------------------------------------ buffers
struct Buffer {
  void *ptr = nullptr;
  size_t bytes = 0;  // bytes the allocator handed out (>= datum bytes)
  int64_t rows = 0, cols = 0;
  int elem = MI_F32;
  uint64_t trace = 0;  // the trace whose capture allocated it (its memory is the trace's until released)
  int tiles = 0;       // MI_TILES_BF16 / MI_TILES_PARTS: datums in the matrix cores' operand order; 0 row-major
  int64_t numel() const { return rows * cols; }
  size_t storage() const { return storage_bytes(elem, rows, cols); }
};

// Device error flags a kernel may raise; read back at the next wait.
enum DeviceFlag : uint32_t { FLAG_INDEX_RANGE = 1u, FLAG_NOT_FINITE = 2u };

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;

  std::unordered_map<mi_id, Buffer> bufs;
  // Caching allocator: exact rounded size -> free blocks.  One stream orders
  // every use, so a block freed by the host is safe to hand out to the next
  // op on the same stream.
  std::map<size_t, std::vector<void *>> free_blocks;
  size_t cached_bytes = 0, live_bytes = 0;

  // Pinned staging ring for host transfers.
  static constexpr int kStageSlots = 4;
  static constexpr size_t kStageBytes = size_t(32) << 20;
  void *stage[kStageSlots] = {};
  hipEvent_t stage_done[kStageSlots] = {};
  bool stage_pending[kStageSlots] = {};
  int stage_next = 0;

  uint32_t *dev_flags = nullptr;  // DeviceFlag bits, device memory

  hipEvent_t events[16] = {};
  std::string last_error;
  int sticky = MI_OK;  // first asynchronous failure not yet reported
  std::string sticky_msg;

  mi_report report{};

  int matmul_mode = MI_MATMUL_FAST;  // how F32 products run (mi_set_matmul_mode)

  // Traces (HIP graphs captured from the stream).  Memory a capture's kernels
  // touch must not be handed to other work while the trace can replay: the
  // buffers a capture allocates go back to the trace, not to the allocator,
  // when freed, and scratch that grows while any trace lives is retired, not
  // freed.
  struct Trace {
    hipGraphExec_t exec = nullptr;
    std::vector<std::pair<void *, size_t>> held;
  };
  std::map<uint64_t, Trace> traces;
  // Blocks freed during the current capture: the capture records one
  // stream's launches in order, so a later allocation of the same capture
  // may take one (its graph runs the freeing kernels first); they stay the
  // trace's.
  std::map<size_t, std::vector<void *>> capture_free;
  bool capturing = false;
  uint64_t capture_id = 0, next_trace = 1;
  std::vector<void *> retired_scratch;

  // Scratch for multi-pass kernels (reductions' partials), grown on demand.
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
};

// Status with a formatted message stored on the context.
int fail(Ctx *ctx, int code, const char *fmt, ...);
// Record a launch failure (hipGetLastError) for `what`; returns its status.
int check_launch(Ctx *ctx, const char *what);

// Buffer table.
Buffer *lookup(Ctx *ctx, mi_id id);
mi_id insert(Ctx *ctx, const Buffer &b);
// A new buffer of `rows x cols` of `elem`; returns its id or 0 (status set).
int new_buffer(Ctx *ctx, int64_t rows, int64_t cols, int elem, mi_id *id,
               Buffer **out);
void *device_alloc(Ctx *ctx, size_t bytes, size_t *got);
void device_release(Ctx *ctx, void *p, size_t bytes);
void *scratch(Ctx *ctx, size_t bytes);
// Looks up, once per device, the device address of the no-allocation
// attention form's file-scope partials (attention.hip); called at context
// creation.
int attention_scratch_setup(Ctx *ctx);
// Zero `bytes` (a multiple of 2) at p with a kernel: safe inside a captured
// trace, where a memset node is not.
int fill_zero(Ctx *ctx, void *p, size_t bytes);
// RMSNorm of R rows of C <= 8192 columns (x of kind xe, gain of kind ge or
// null) into `out` as out_elem (F32, BF16 or MI_BF16_PARTS): mi_rms_norm's
// launch.
void rms_norm_launch(Ctx *ctx, const void *xp, int xe, const void *gp, int ge, float eps, void *out, int out_elem,
                     int64_t R, int64_t C);
// A new buffer holding the decoded values of BFP8 buffer `src` as `elem`
// (MI_F32, or MI_BF16: exact either way); what a consumer without a BFP8
// read of its own takes instead.  The caller frees it.
int bfp8_decode_to(Ctx *ctx, const Buffer *src, int elem, mi_id *id, Buffer **out);
// What a one-sequence decode step's fused attention launch (attention.hip)
// leaves for its combine: the key chunks' partials ([KVH][S], laid out as
// combine.hpp states), the rotated queries [H, 64] and the new key and value
// rows [KVH][2][64], F32; H query heads, G a kv head, 64-wide.
struct AttnCombine {
  const float *part, *q, *kvn;
  int H, G, S;
  float scale;
};
// Whether attention_o_launch takes H heads over S chunks (the row's LDS).
bool attention_o_fits(int64_t H, int64_t S);
// out [1, N] = resid + attention row w^T, the attention row the combine of
// `c` (bit for bit attention.hip's combine_new_kernel) and w [N, H 64] BF16
// or BFP8: the combine and the o projection in one launch.  Returns the
// launch's status.
int attention_o_launch(Ctx *ctx, const AttnCombine &c, const Buffer *w, const float *resid, float *out);
// MI_E_UNSUPPORTED if a trace is being captured (host transfers and waits
// cannot be part of one).
int refuse_if_capturing(Ctx *ctx, const char *what);

// Kernel-side flag word for the context.
inline uint32_t *flags(Ctx *ctx) { return ctx->dev_flags; }

// Grid sizing: blocks to cover `n` items at `per_block`, capped.
inline unsigned grid_for(int64_t n, int64_t per_block, int64_t cap = 1 << 20) {
  int64_t g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

}  // namespace mi

struct mi_ctx : mi::Ctx {};

// Take the context's lock and validate it.
#define MI_ENTER(ctx)                                                  \
  if ((ctx) == nullptr) return MI_E_ARG;                               \
  std::lock_guard<std::recursive_mutex> mi_guard_((ctx)->mu)

// Look up id `id` into `Buffer *var`, failing with MI_E_ID.
#define MI_BUF(ctx, var, id)                                           \
  mi::Buffer *var = mi::lookup((ctx), (id));                           \
  if (var == nullptr)                                                  \
    return mi::fail((ctx), MI_E_ID, "unknown or freed buffer id %llu", \
                    (unsigned long long)(id))

// Ops that read a buffer's datums as plain slots refuse BFP8 storage.
#define MI_NO_BFP8(ctx, var, what)                                                                     \
  if ((var)->elem == MI_BFP8)                                                                          \
  return mi::fail((ctx), MI_E_ARG, "%s does not take a BFP8 buffer (mi_cast_bfp decodes it)", (what))
