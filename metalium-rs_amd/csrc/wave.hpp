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
__device__ __forceinline__ float max_nan(float a, float b) {
  // NaN ranks above every number, so it propagates.
  if (isnan(a)) return a;
  if (isnan(b)) return b;
  return b > a ? b : a;
}
__device__ __forceinline__ float min_nan(float a, float b) {
  if (isnan(a)) return a;
  if (isnan(b)) return b;
  return b < a ? b : a;
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
