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

template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned int)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned int)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((unsigned long long)(unsigned int)hi << 32) | (unsigned int)lo;
}
__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// Selection shared state (LDS) of one 256-thread block.
struct SelectLds {
  alignas(16) unsigned long long key[kMaxE];  // candidate keys, compacted
  unsigned long long rowmax[16];
  unsigned long long thresh;
  int wcnt[4];
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
// ties by lower index, so rank(t) = #{e : key[e] > key[t]}; only the keys
// that can be among the K largest are ranked (see below).
// `s` is thread t's score (t < E), -inf for t >= E; `pes_t` is thread t's
// per_expert_scale value (requested early by callers on a latency-bound
// path: a global load here would put its round trip on the critical path).
__device__ void block_select_values_pes(float s, float pes_t, int E, int K, SelectLds& L) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t < E) L.pes[t] = pes_t;
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
  // Ranking by key = (bits(p) << 32) | ~index (distinct; ties go to the
  // lower index).  Only keys >= T can be among the K largest, where T is the
  // K-th largest of the 16-lane row maxima (K distinct keys are >= T) or 0
  // with fewer than K rows; those candidates are compacted into LDS and
  // ranked among themselves, which gives their global ranks, since every
  // key above a top-K key is >= T as well.
  const unsigned long long key = (t < E) ? ((unsigned long long)__float_as_uint(p) << 32) | (unsigned)(~t) : 0ull;
  unsigned long long rm = key;
  rm = max_u64(rm, dpp_u64<kDppXor1>(rm));
  rm = max_u64(rm, dpp_u64<kDppXor2>(rm));
  rm = max_u64(rm, dpp_u64<kDppHalfMirror>(rm));
  rm = max_u64(rm, dpp_u64<kDppMirror>(rm));
  if ((lane & 15) == 0) L.rowmax[t >> 4] = rm;
  __syncthreads();
  const int nrows = (E + 15) / 16;
  if (nrows < K) {
    if (t == 0) L.thresh = 1ull;  // every real key (nonzero) is a candidate
  } else if (t < nrows) {
    const unsigned long long mine = L.rowmax[t];
    int r = 0;
    for (int q = 0; q < nrows; ++q) r += (L.rowmax[q] > mine) ? 1 : 0;
    if (r == K - 1) L.thresh = mine;
  }
  __syncthreads();
  const bool cand = key >= L.thresh && t < E;
  const unsigned long long bal = __ballot(cand);
  const int before = __builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0));
  if (lane == 0) L.wcnt[w] = __popcll(bal);
  __syncthreads();
  int off = 0;
  for (int q = 0; q < w; ++q) off += L.wcnt[q];
  const int C = L.wcnt[0] + L.wcnt[1] + L.wcnt[2] + L.wcnt[3];
  if (cand) L.key[off + before] = key;
  __syncthreads();
  if (t < C) {
    const unsigned long long mine = L.key[t];
    int rank = 0;
    for (int j = 0; j < C; ++j) rank += (L.key[j] > mine) ? 1 : 0;
    if (rank < K) {
      L.topp[rank] = __uint_as_float((unsigned int)(mine >> 32));
      L.topi[rank] = (int)(~(unsigned int)mine);
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

__device__ __forceinline__ void block_select_values(float s, const uint16_t* __restrict__ pes, int E, int K,
                                                    SelectLds& L) {
  const int t = threadIdx.x;
  block_select_values_pes(s, (t < E) ? bf2f(pes[t]) : 0.0f, E, K, L);
}

__device__ __forceinline__ void block_select(const float* __restrict__ srow, const uint16_t* __restrict__ pes, int E,
                                             int K, SelectLds& L) {
  block_select_values(((int)threadIdx.x < E) ? srow[threadIdx.x] : -INFINITY, pes, E, K, L);
}


}  // namespace g4mi
