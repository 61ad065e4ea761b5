// The combine of a fused decode step's key-chunk partials with the new key,
// shared by attention.hip's combine kernel and decode.hip's fused o
// projection, so the two give the same bits.
#pragma once

#include <cfloat>

#include "common.hpp"
#include "wave.hpp"

namespace mi {

// The fused decode step's partials, chunk s of item bj (a sequence's kv
// head) at part + (bj S + s) dqa_part_stride(G): the G query heads' score
// maxima, their sums of exponentials, zeros up to a multiple of 4 floats,
// then each head's 64 sums of weighted values (16-byte aligned).
__host__ __device__ constexpr int64_t dqa_part_acc0(int64_t G) { return (2 * G + 3) / 4 * 4; }
__host__ __device__ constexpr int64_t dqa_part_stride(int64_t G) { return dqa_part_acc0(G) + 64 * G; }

// One query head's attention output at the new position, on a row of 16
// lanes (lane r: elements 4 r .. 4 r + 3 of the head's 64): the chunks'
// partials weighted by exp(max_s - M), M the maximum over the chunks and the
// new key's score, plus the new key's value, over the weighted sums.  load()
// issues every load of the first CS chunks (later slots repeat the last
// chunk) and the lane's own chunk statistics (chunk r), so a caller issues
// them with its own before any wait; finish() does the arithmetic: the new
// key's score folded over the row, the maximum and the weights one chunk a
// lane, the row's weights passed through wl (S floats of LDS a row).
// Chunks past CS, and statistics past 16, are read in finish() (long
// contexts only).
template <int CS>
struct ChunkCombine {
  float4 ov[CS];
  float m, l;
  float4 q, k, v;

  __device__ __forceinline__ void load(const float *pitem, int G, int gg, int S, int r, const float *qh,
                                       const float *kn, const float *vn) {
    const int64_t PS = dqa_part_stride(G);
    const int sr = r < S ? r : S - 1;
    m = pitem[sr * PS + gg];
    l = pitem[sr * PS + G + gg];
    const float *pv = pitem + dqa_part_acc0(G) + gg * 64 + 4 * r;
#pragma unroll
    for (int s = 0; s < CS; ++s) ov[s] = *reinterpret_cast<const float4 *>(pv + (s < S ? s : S - 1) * PS);
    q = *reinterpret_cast<const float4 *>(qh + 4 * r);
    k = *reinterpret_cast<const float4 *>(kn + 4 * r);
    v = *reinterpret_cast<const float4 *>(vn + 4 * r);
  }

  __device__ __forceinline__ float4 finish(const float *pitem, int G, int gg, int S, int r, float scale,
                                           float *wl) const {
    const int64_t PS = dqa_part_stride(G);
    float sp = q.x * k.x;
    sp += q.y * k.y;
    sp += q.z * k.z;
    sp += q.w * k.w;
    const float snew = fold_sum<16>(sp) * scale;
    float mr = r < S ? m : -INFINITY;
    for (int s = r + 16; s < S; s += 16) mr = max_nan(mr, pitem[s * PS + gg]);
    const float M = max_nan(fold_max<16>(mr), snew);
    float lr = 0.0f;
    if (r < S) {
      const float w = expf(m - M);
      wl[r] = w;
      lr = w * l;
    }
    for (int s = r + 16; s < S; s += 16) {
      const float w = expf(pitem[s * PS + gg] - M);
      wl[s] = w;
      lr += w * pitem[s * PS + G + gg];
    }
    const float wn = expf(snew - M);
    float den = fold_sum<16>(lr) + wn;
    den = isnan(den) ? den : (den > FLT_MIN ? den : FLT_MIN);
    // The row's weights: written above by this wavefront's lanes, read
    // below by the same wavefront (its LDS accesses run in order).
    __builtin_amdgcn_wave_barrier();
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      const float w = wl[s < S ? s : S - 1];
      const bool in = s < S;
      num.x = in ? num.x + w * ov[s].x : num.x;
      num.y = in ? num.y + w * ov[s].y : num.y;
      num.z = in ? num.z + w * ov[s].z : num.z;
      num.w = in ? num.w + w * ov[s].w : num.w;
    }
    const float *pv = pitem + dqa_part_acc0(G) + gg * 64 + 4 * r;
    for (int s = CS; s < S; ++s) {
      const float w = wl[s];
      const float4 o = *reinterpret_cast<const float4 *>(pv + s * PS);
      num.x += w * o.x;
      num.y += w * o.y;
      num.z += w * o.z;
      num.w += w * o.w;
    }
    num.x += wn * v.x;
    num.y += wn * v.y;
    num.z += wn * v.z;
    num.w += wn * v.w;
    return make_float4(num.x / den, num.y / den, num.z / den, num.w / den);
  }
};

// The chunks a combine holds in registers for S chunks: 4, 8, 12 or 16.
inline int combine_cs(int64_t S) { return S <= 4 ? 4 : S <= 8 ? 8 : S <= 12 ? 12 : 16; }

}  // namespace mi
