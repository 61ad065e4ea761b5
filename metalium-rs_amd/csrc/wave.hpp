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

}  // namespace mi
