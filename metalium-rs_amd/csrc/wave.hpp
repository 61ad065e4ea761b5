// Wavefront (64-lane) folds shared by the row kernels.  Every fold is a
// fixed xor butterfly, so a result does not depend on scheduling.
#pragma once
#include <hip/hip_runtime.h>

namespace mi {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// NaN ranks above every number, so it propagates (a NaN `a` first, then a NaN
// `b`); of two equal numbers `a` is kept.  Written as selects: early returns
// compile to a divergent branch per call.
__device__ __forceinline__ float max_nan(float a, float b) {
  const float m = b > a ? b : a;
  return isnan(a) ? a : (isnan(b) ? b : m);
}
__device__ __forceinline__ float min_nan(float a, float b) {
  const float m = b < a ? b : a;
  return isnan(a) ? a : (isnan(b) ? b : m);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max_nan(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min_nan(v, __shfl_xor(v, o, 64));
  return v;
}

// Folds on the VALU lane paths of gfx950 -- DPP moves within 16-lane rows,
// v_permlane16_swap / v_permlane32_swap across them -- instead of __shfl_xor,
// which compiles to an LDS-crossbar ds_bpermute of ~100 cycles a step: a
// 64-lane sum is 6 VALU adds.  fold_sum<N> / fold_max<N>: over each aligned
// group of N (2 .. 64, a power of two) lanes, every lane ending with its
// group's value; the pairs combine in a fixed order (the lower lane or row
// first), so a result does not depend on scheduling.  Call with all 64 lanes
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// The pair (even row, odd row) of 16-lane rows -- or (lower half, upper
// half) -- of v at this lane's position.  The vector's elements go to named
// scalars before the casts: a bit cast of the element expression itself
// reads element 0 for both.
__device__ __forceinline__ void swap16_pair(float v, float &a, float &b) {
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  const unsigned x = q[0], y = q[1];
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ __forceinline__ void swap32_pair(float v, float &a, float &b) {
  const auto q = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  const unsigned x = q[0], y = q[1];
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
struct FoldAdd {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct FoldMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return max_nan(a, b); }
};
template <int N, typename Op>
__device__ __forceinline__ float fold(float v, Op op) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1 to 64 lanes, a power of two");
  if constexpr (N >= 2) v = op(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v = op(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v = op(v, dpp_f32<0x141>(v));  // row_half_mirror
  if constexpr (N >= 16) v = op(v, dpp_f32<0x140>(v)); // row_mirror
  if constexpr (N >= 32) {
    float a, b;
    swap16_pair(v, a, b);
    v = op(a, b);
  }
  if constexpr (N >= 64) {
    float a, b;
    swap32_pair(v, a, b);
    v = op(a, b);
  }
  return v;
}
template <int N>
__device__ __forceinline__ float fold_sum(float v) { return fold<N>(v, FoldAdd{}); }
template <int N>
__device__ __forceinline__ float fold_max(float v) { return fold<N>(v, FoldMax{}); }
// Sum over the lanes l' == l (mod C), C = 16 or 32 (the rows of a wavefront's
// column groups), every such lane ending with it; other C fall back to
// xor shuffles.
template <int C>
__device__ __forceinline__ float fold_columns(float v) {
  if constexpr (C == 16 || C == 32) {
    float a, b;
    if constexpr (C == 16) {
      swap16_pair(v, a, b);
      v = a + b;
    }
    swap32_pair(v, a, b);
    return a + b;
  } else {
#pragma unroll
    for (int o = C; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
  }
}

}  // namespace mi
