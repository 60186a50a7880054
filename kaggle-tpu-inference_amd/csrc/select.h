// Router softmax + top-k selection shared by the MoE kernels (moe.hip) and
// the fused FFN-input kernel (layer.hip), model.py:228-231.
#pragma once

#include "common.h"

namespace g4mi {

constexpr int kMaxE = 256;  // one selection thread per expert in a 256-thread block
constexpr int kMaxK = 32;

template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
  return fmaxf(v, dpp_f<CTRL>(v));
}
// max over all 64 lanes (every lane gets it)
__device__ __forceinline__ float wave_max(float v) {
  v = dpp_max_step<kDppXor1>(v);
  v = dpp_max_step<kDppXor2>(v);
  v = dpp_max_step<kDppHalfMirror>(v);
  v = dpp_max_step<kDppMirror>(v);
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// Selection shared state (LDS) of one 256-thread block.
struct SelectLds {
  unsigned long long key[kMaxE];
  float pes[kMaxE];
  int rank_part[256];
  float topp[kMaxK];
  float topw[kMaxK];
  int topi[kMaxK];
  float redf[4];
  double redd[4];
};

// Softmax over the E scores of one token (f32; exp evaluated in f64 and
// rounded to f32; exact sums), stable top-k (value desc, index asc, as
// jax.lax.top_k), renormalised over the k picks and scaled by
// per_expert_scale (model.py:228-231).  Block-wide (256 threads, E <= 256);
// leaves topi/topw in LDS.
//
// Ranking: probabilities are >= 0, so their f32 bit patterns order like the
// values; key = (bits(p) << 32) | ~index makes every key distinct and orders
// ties by lower index, so rank(t) = #{e : key[e] > key[t]}.  The E*E key
// comparisons are spread over all 256 threads (256/E threads per expert).
// `s` is thread t's score (t < E), -inf for t >= E.
__device__ void block_select_values(float s, const uint16_t* __restrict__ pes, int E, int K, SelectLds& L) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t < E) L.pes[t] = bf2f(pes[t]);
  const float wm = wave_max(s);
  if (lane == 0) L.redf[w] = wm;
  __syncthreads();
  const float m = fmaxf(fmaxf(L.redf[0], L.redf[1]), fmaxf(L.redf[2], L.redf[3]));
  const float ex = (t < E) ? (float)exp((double)(s - m)) : 0.0f;
  const double ws = group_sum_f64<64>((double)ex);
  if (lane == 0) L.redd[w] = ws;
  __syncthreads();
  const float total = (float)(L.redd[0] + L.redd[1] + L.redd[2] + L.redd[3]);
  const float p = (t < E) ? ex / total : 0.0f;
  if (t < E) L.key[t] = ((unsigned long long)__float_as_uint(p) << 32) | (unsigned)(~t);
  __syncthreads();
  const int parts = max(1, 256 / E);
  const int chunk = (E + parts - 1) / parts;
  const int part = t / E, et = t - part * E;
  if (part < parts) {
    const unsigned long long mine = L.key[et];
    const int e0 = part * chunk, e1 = min(E, e0 + chunk);
    int r0 = 0, r1 = 0;
    int e = e0;
#pragma unroll 4
    for (; e + 1 < e1; e += 2) {
      r0 += L.key[e] > mine;
      r1 += L.key[e + 1] > mine;
    }
    if (e < e1) r0 += L.key[e] > mine;
    L.rank_part[t] = r0 + r1;
  }
  __syncthreads();
  if (t < E) {
    int rank = 0;
    for (int q = 0; q < parts; ++q) rank += L.rank_part[q * E + t];
    if (rank < K) {
      L.topp[rank] = p;
      L.topi[rank] = t;
    }
  }
  __syncthreads();
  if (t < 32) {
    const double v = (t < K) ? (double)L.topp[t] : 0.0;
    const float sk = (float)group_sum_f64<32>(v);
    if (t < K) L.topw[t] = (L.topp[t] / sk) * L.pes[L.topi[t]];
  }
  __syncthreads();
}

__device__ __forceinline__ void block_select(const float* __restrict__ srow, const uint16_t* __restrict__ pes, int E,
                                             int K, SelectLds& L) {
  block_select_values(((int)threadIdx.x < E) ? srow[threadIdx.x] : -INFINITY, pes, E, K, L);
}


}  // namespace g4mi
