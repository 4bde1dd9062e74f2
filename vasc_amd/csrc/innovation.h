// Canonical pair innovation shared by the pooling and selection kernels.
#pragma once

#include "common.h"

namespace vasc {

// nan_to_num(nan=0) of a pooled value (sparse_wrapper.py:3690-3694).
__device__ __forceinline__ float clean_value(float x) {
  if (x != x) return 0.f;
  if (x == INFINITY) return 3.402823466e38f;
  if (x == -INFINITY) return -3.402823466e38f;
  return x;
}

// One wave, head dim 64, lane d holds V[2p][d] (lv) and V[2p+1][d] (rv; the
// odd tail passes rv = lv). Returns 0.5*sqrt(mean_d (lv-rv)^2) in every lane
// (sparse_wrapper.py:3733-3740) with the mean's sum taken by the canonical
// float64 butterfly and every float32 operation rounded separately.
__device__ __forceinline__ float pair_innovation_wave(float lv, float rv) {
#pragma clang fp contract(off)
  const float diff = clean_value(lv) - clean_value(rv);
  const float sq = diff * diff;
  const double s = wave_butterfly(0.0 + static_cast<double>(sq));
  const float mean = static_cast<float>(s / 64.0);
  return sqrtf(mean) * 0.5f;
}

}  // namespace vasc
