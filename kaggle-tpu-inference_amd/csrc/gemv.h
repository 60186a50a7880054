// Row-streaming GEMV helpers shared by the decode kernels (layer.hip).
#pragma once

#include "common.h"

namespace g4mi {

// S lanes per row, IT 16-byte chunks per lane (K = 8*S*IT).
template <int S, int IT>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int sub, u32x4* w) {
#pragma unroll
  for (int i = 0; i < IT; ++i) w[i] = ld_stream((const u32x4*)row + sub + S * i);
}
template <int S, int IT>
__device__ __forceinline__ float dot_row(const u32x4* w, const u32x4* __restrict__ xs, int sub) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < IT; ++i) acc = dot8(w[i], xs[sub + S * i], acc);
  return group_sum<S>(acc);
}

}  // namespace g4mi
