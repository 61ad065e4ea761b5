// Seeded device random draws.
//
// Reference: Engine::random_dram (crates/burn-tt/src/server.rs:768), the draw
// kinds of crates/burn-tt/src/random.rs:73-126 and the per-call 64-bit base
// `splitmix64(seed ^ splitmix64(draws))` (random.rs:42-56).  Matching the CPU
// backend's sequence is not part of the contract (crates/burn-tt/README.md:
// 348-352); a draw is a pure function of (base, element index).
//
// Generator: element e takes the SplitMix64 output of `base + (e + 1) * golden`
// (Steele, Lea and Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014); uniforms use its top 24 bits; normals use Box-Muller over the
// two 32-bit halves of one draw.
#include "common.hpp"

namespace mi {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

__global__ void random_kernel(void *out, int64_t n, int draw, float p1, float p2, uint64_t base) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const uint64_t z = splitmix64(base + static_cast<uint64_t>(e) * 0x9e3779b97f4a7c15ull);
    const float u = static_cast<float>(z >> 40) * (1.0f / 16777216.0f);  // [0, 1)
    switch (draw) {
      case MI_DRAW_UNIT: static_cast<float *>(out)[e] = u; break;
      case MI_DRAW_UNIFORM: {
        float v = p1 + (p2 - p1) * u;
        static_cast<float *>(out)[e] = v < p2 ? v : p1;  // keep the half-open range
        break;
      }
      case MI_DRAW_NORMAL: {
        const float u1 = (static_cast<float>(z >> 40) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1)
        const float u2 = static_cast<float>((z >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        static_cast<float *>(out)[e] = p1 + p2 * (r * cospif(2.0f * u2));
        break;
      }
      case MI_DRAW_BERNOULLI: static_cast<float *>(out)[e] = u < p1 ? 1.0f : 0.0f; break;
      default: {  // MI_DRAW_INT_RANGE: [lo, hi)
        const int64_t lo = static_cast<int64_t>(p1), hi = static_cast<int64_t>(p2);
        const uint64_t span = static_cast<uint64_t>(hi - lo);
        static_cast<int32_t *>(out)[e] = static_cast<int32_t>(lo + static_cast<int64_t>((z >> 32) * span >> 32));
      }
    }
  }
}

}  // namespace mi

using namespace mi;

extern "C" int mi_random(mi_ctx *ctx, int64_t rows, int64_t cols, int draw, float p1, float p2, uint64_t base,
                         mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  if (draw < MI_DRAW_UNIT || draw > MI_DRAW_INT_RANGE) return fail(ctx, MI_E_ARG, "draw kind %d", draw);
  if (draw == MI_DRAW_UNIFORM && !(p1 < p2)) return fail(ctx, MI_E_ARG, "uniform range [%g, %g)", p1, p2);
  if (draw == MI_DRAW_INT_RANGE) {
    if (!(p1 < p2) || p1 != static_cast<float>(static_cast<int64_t>(p1)) || p2 != static_cast<float>(static_cast<int64_t>(p2)))
      return fail(ctx, MI_E_ARG, "integer range [%g, %g)", p1, p2);
  }
  const int elem = draw == MI_DRAW_INT_RANGE ? MI_I32 : MI_F32;
  mi_id id; Buffer *b;
  int s = new_buffer(ctx, rows, cols, elem, &id, &b);
  if (s) return s;
  const int64_t n = rows * cols;
  if (n > 0) {
    random_kernel<<<grid_for(n, 256 * 4, 256 * 32), 256, 0, ctx->stream>>>(b->ptr, n, draw, p1, p2, base);
    s = check_launch(ctx, "random");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}
