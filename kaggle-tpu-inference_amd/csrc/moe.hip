// MoE decode block: router scores (K1), top-k selection, per-expert gate/up
// GEMV with the gated-GELU activation (K2), per-expert down GEMV with the
// weighted combine (K3).  Follows model.py _router / _moe (model.py:224-232,
// model.py:262-294).
//
// Only the rows of the selected experts are read from HBM: K2 reads
// gate_up[e] (2*F rows of H) and K3 reads down[e] (H rows of F) for the k
// experts each token picked -- the job the reference's per-expert
// dynamic_slice does on TPU.
//
// Schedule: the router kernel writes the bf16-rounded scores; every block of
// the gate/up kernel then redoes the (tiny) softmax + top-k selection for its
// token in LDS before issuing its weight loads.  That costs ~1 us of block
// latency instead of a device-wide fence and a second pass.
#include <string.h>

#include "capi_util.h"
#include "common.h"
#include "select.h"

namespace g4mi {

constexpr int kMaxH = 16384;

#define G4MI_IT_CASES(M) M(1) M(2) M(3) M(4) M(5) M(6) M(7) M(8) M(9) M(10) M(11) M(12) M(13) M(14) M(15) M(16)

// ============================================================== K1: router scores
//
// scores[n, e] = f32(bf16(x2 . proj[e])) where (model.py:225-227)
//     xe = rms_norm(x, pre_w)                  (only when pre_w != null)
//     x2 = bf16(bf16(rms_norm(xe) * scale) * bf16(H^-0.5))
// The dot is exact (f64, bf16*bf16 products are exact) and rounded once, so
// the scores -- and the top-k they induce -- do not depend on reduction order.
//
// More tokens, H = 256*IT: grid (ceil(E/8), N), 4 waves x 2 rows (the rows
// then come from the caches, and the prologue is shared by 8 rows).  Each half-wave
// issues its row's IT 16-byte loads first; meanwhile the block builds x2 once
// in LDS (each thread owns at most two 8-value chunks), then every half-wave
// dots its row against it.
template <int IT>
__global__ __launch_bounds__(256) void router_scores_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_w, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ proj, int E, float eps, float inv_sqrt_h_bf, float* __restrict__ scores) {
  constexpr int H = IT * 256;
  constexpr int CH = H / 8;  // 16-byte chunks per row
  __shared__ u32x4 xs[CH];
  __shared__ double red[4];
  const int tid = threadIdx.x;
  const int lane = tid & 63, half = lane >> 5, l = lane & 31, wave = wave_id();
  const int n = blockIdx.y;
  const int e = blockIdx.x * 8 + wave * 2 + half;
  u32x4 w[IT];
  if (e < E) {
    const u32x4* row = (const u32x4*)(proj + (size_t)e * H);
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 32 * i);
  }
  // thread tid owns chunks tid and tid+256 (CH <= 512 for IT <= 16)
  constexpr int PER = (CH + 255) / 256;
  const u32x4* xr = (const u32x4*)(x + (size_t)n * H);
  u32x4 v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = tid + 256 * j;
    v[j] = (c < CH) ? ld16(xr + c) : u32x4{0u, 0u, 0u, 0u};
  }
  if (pre_w != nullptr) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss = sumsq8_f64(v[j], ss);
    const float r = rms_scale(block_sum_f64(ss, red), H, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = tid + 256 * j;
      if (c < CH) {
        const u32x4 pw = ld16((const u32x4*)pre_w + c);
        v[j] = scale8(v[j], r, &pw);
      }
    }
  }
  {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss = sumsq8_f64(v[j], ss);
    const float r = rms_scale(block_sum_f64(ss, red), H, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = tid + 256 * j;
      if (c < CH) {
        const u32x4 sc = ld16((const u32x4*)scale + c);
        float f[8], g[8];
        unpack8(v[j], f);
        unpack8(sc, g);
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = rbf(rbf(rbf(f[q] * r) * g[q]) * inv_sqrt_h_bf);
        u32x4 o;
        o.x = pack2(f[0], f[1]); o.y = pack2(f[2], f[3]); o.z = pack2(f[4], f[5]); o.w = pack2(f[6], f[7]);
        xs[c] = o;
      }
    }
  }
  __syncthreads();
  if (e < E) {
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      if (i & 1) a1 = dot8_f64(w[i], xs[l + 32 * i], a1);
      else a0 = dot8_f64(w[i], xs[l + 32 * i], a0);
    }
    const double acc = group_sum_f64<32>(a0 + a1);
    if (l == 0) scores[(size_t)n * E + e] = rbf(f32_of(acc));
  }
}

// Few tokens (N <= 16), H = 256*IT: grid (ceil(E/2), N), one wave per block,
// a half-wave per expert row.  Every operand (the row's IT 16-byte chunks per lane, the
// token's activations and both norm weights) is requested before the first
// reduction, so a block waits on one memory round trip; the two norms are
// wave reductions, and x2 passes through LDS to the dots.  (With 8 rows per
// 4-wave block the weights were loaded after each block reduction: three
// dependent round trips, 16 blocks for the 26B router's 0.72 MB.)
template <int IT>
__global__ __launch_bounds__(64) void router_scores_wave_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_w, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ proj, int E, float eps, float inv_sqrt_h_bf, float* __restrict__ scores) {
  constexpr int H = IT * 256;
  constexpr int CH = H / 8;                // 16-byte chunks per row
  constexpr int PER = (CH + 63) / 64;      // chunks per lane
  __shared__ u32x4 xs[CH];
  const int lane = threadIdx.x, half = lane >> 5, l = lane & 31;
  const int n = blockIdx.y;
  const int e = blockIdx.x * 2 + half;
  u32x4 w[IT];
  const u32x4* row = (const u32x4*)(proj + (size_t)min(e, E - 1) * H);
#pragma unroll
  for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 32 * i);
  const u32x4* xr = (const u32x4*)(x + (size_t)n * H);
  const u32x4* pwr = (const u32x4*)(pre_w != nullptr ? pre_w : scale);
  u32x4 v[PER], pw[PER], sc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = min(lane + 64 * j, CH - 1);
    v[j] = ld16(xr + c);
    pw[j] = ld16(pwr + c);
    sc[j] = ld16((const u32x4*)scale + c);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (lane + 64 * j >= CH) v[j] = u32x4{0u, 0u, 0u, 0u};
  if (pre_w != nullptr) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss = sumsq8_f64(v[j], ss);
    const float r = rms_scale(group_sum_f64<64>(ss), H, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = scale8(v[j], r, &pw[j]);
  }
  {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss = sumsq8_f64(v[j], ss);
    const float r = rms_scale(group_sum_f64<64>(ss), H, eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = lane + 64 * j;
      if (c < CH) {
        float f[8], g[8];
        unpack8(v[j], f);
        unpack8(sc[j], g);
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = rbf(rbf(rbf(f[q] * r) * g[q]) * inv_sqrt_h_bf);
        u32x4 o;
        o.x = pack2(f[0], f[1]); o.y = pack2(f[2], f[3]); o.z = pack2(f[4], f[5]); o.w = pack2(f[6], f[7]);
        xs[c] = o;
      }
    }
  }
  __syncthreads();
  double a0 = 0.0, a1 = 0.0;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    if (i & 1) a1 = dot8_f64(w[i], xs[l + 32 * i], a1);
    else a0 = dot8_f64(w[i], xs[l + 32 * i], a0);
  }
  const double acc = group_sum_f64<32>(a0 + a1);
  if (e < E && l == 0) scores[(size_t)n * E + e] = rbf(f32_of(acc));
}

constexpr int kRouterWaveRows = 16;  // tokens up to which router_scores_wave_kernel runs

// Generic-H router scores: one block per (8 experts, token); the router input
// is rebuilt in LDS with block reductions.
__global__ __launch_bounds__(256) void router_scores_generic_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_w, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ proj, int H, int E, float eps, float inv_sqrt_h_bf, float* __restrict__ scores) {
  __shared__ uint16_t xs[kMaxH];
  __shared__ double red[4];
  const int n = blockIdx.y, tid = threadIdx.x;
  const uint16_t* xrow = x + (size_t)n * H;
  for (int i = tid; i < H; i += blockDim.x) xs[i] = xrow[i];
  __syncthreads();
  if (pre_w != nullptr) {
    double ss = 0.0;
    for (int i = tid; i < H; i += blockDim.x) { const double v = bf2f(xs[i]); ss = fma(v, v, ss); }
    const float r = rms_scale(block_sum_f64(ss, red), H, eps);
    __syncthreads();
    for (int i = tid; i < H; i += blockDim.x) xs[i] = f2bf(bf2f(xs[i]) * r * bf2f(pre_w[i]));
    __syncthreads();
  }
  {
    double ss = 0.0;
    for (int i = tid; i < H; i += blockDim.x) { const double v = bf2f(xs[i]); ss = fma(v, v, ss); }
    const float r = rms_scale(block_sum_f64(ss, red), H, eps);
    __syncthreads();
    for (int i = tid; i < H; i += blockDim.x)
      xs[i] = f2bf(rbf(rbf(bf2f(xs[i]) * r) * bf2f(scale[i])) * inv_sqrt_h_bf);
    __syncthreads();
  }
  const int lane = tid & 63, l = lane & 31, wave = wave_id();
  const int e = blockIdx.x * 8 + wave * 2 + (lane >> 5);
  if (e < E) {
    const u32x4* row = (const u32x4*)(proj + (size_t)e * H);
    double acc = 0.0;
    for (int c = l; c < (H >> 3); c += 32) acc = dot8_f64(ld16(row + c), ld16(xs + 8 * c), acc);
    acc = group_sum_f64<32>(acc);
    if (l == 0) scores[(size_t)n * E + e] = rbf(f32_of(acc));
  }
}

// One block per token: selection only (the standalone top-k entry point).
__global__ __launch_bounds__(256) void router_select_kernel(const float* __restrict__ scores,
                                                            const uint16_t* __restrict__ pes, int E, int K,
                                                            float* __restrict__ out_w, int32_t* __restrict__ out_i) {
  __shared__ SelectLds L;
  const int n = blockIdx.x;
  block_select(scores + (size_t)n * E, pes, E, K, L);
  if (threadIdx.x < K) {
    out_w[(size_t)n * K + threadIdx.x] = L.topw[threadIdx.x];
    out_i[(size_t)n * K + threadIdx.x] = L.topi[threadIdx.x];
  }
}

// ============================================================== K2: gate/up
//
// One wave per (token, slot, f): lanes 0-31 dot x with gate row f of expert
// e = top_i[slot], lanes 32-63 with up row f; IT = H/256 16-byte chunks per lane.
//     act = bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(top_w))   (model.py:270-271)
// Routing comes either from top_w/top_i (global) or, when `scores` is given,
// from a per-block selection; block x == 0 of each token then also stores
// top_w/top_i for later kernels.  With the routing given and several tokens
// (N * K <= 64 pairs), an expert chosen by more than one (token, slot) pair
// has its rows read once: the first such pair's wave computes row f for
// every pair that chose the expert (the other tokens' x from global memory,
// the same dot products), and the later pairs' waves return.
template <int IT>
__global__ __launch_bounds__(256) void moe_gateup_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate_up, const float* __restrict__ scores,
    const uint16_t* __restrict__ pes, float* __restrict__ top_w, int32_t* __restrict__ top_i, int F, int E, int K,
    uint16_t* __restrict__ act) {
  constexpr int H = IT * 256;
  constexpr int XPT = (H / 8 + 127) / 128;  // x chunks per thread (blocks of >= 128 threads)
  __shared__ SelectLds L;
  __shared__ u32x4 xs[H / 8];
  const int lane = threadIdx.x & 63, half = lane >> 5, l = lane & 31;
  const int task = blockIdx.x * (blockDim.x >> 6) + wave_id();
  const int n = blockIdx.y;
  // x is staged in LDS once per block: each wave loading it itself took as
  // many vector memory slots as its expert rows
  const u32x4* xv = (const u32x4*)(x + (size_t)n * H);
  u32x4 xr[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) xr[j] = ld16(xv + min((int)threadIdx.x + (int)blockDim.x * j, H / 8 - 1));
  if (scores != nullptr) {
    block_select(scores + (size_t)n * E, pes, E, K, L);
    if (blockIdx.x == 0 && threadIdx.x < K) {
      top_w[(size_t)n * K + threadIdx.x] = L.topw[threadIdx.x];
      top_i[(size_t)n * K + threadIdx.x] = L.topi[threadIdx.x];
    }
  }
  const int tc = min(task, K * F - 1);  // clamped: loads stay unconditional
  const int slot = tc / F, f = tc - slot * F;
  const int ei = (scores != nullptr) ? L.topi[slot] : top_i[n * K + slot];
  const bool ok = task < K * F && ei >= 0 && ei < E;  // else: contribute nothing
  const int NK = (int)gridDim.y * K;
  const bool dedup = scores == nullptr && gridDim.y > 1 && NK <= 64;  // block-uniform
  const int pe_raw = top_i[min(lane, NK - 1)];  // every pair's expert, one per lane (unconditional load)
  const int pe = (dedup && lane < NK) ? pe_raw : -1;
  const int p = n * K + slot;
  // the pairs that chose this expert (includes p); a wave whose expert an
  // earlier pair also chose requests no rows: that pair's wave computes
  // row f for them all (the row address waits for the routing anyway)
  const unsigned long long same = __ballot(pe == ei);
  const bool dup = dedup && ok && task < K * F && (same & ((1ull << p) - 1ull)) != 0ull;
  const u32x4* row = (const u32x4*)(gate_up + ((size_t)(max(min(ei, E - 1), 0) * 2 + half) * F + f) * H);
  u32x4 w[IT];
  if (!dup) {
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 32 * i);
  }
#pragma unroll
  for (int j = 0; j < XPT; ++j)
    if ((int)threadIdx.x + (int)blockDim.x * j < H / 8) xs[threadIdx.x + blockDim.x * j] = xr[j];
  lds_barrier();
  // act of pair q = (token nq, slot q % K) from row f of its expert (in w)
  auto emit = [&](int q, int nq) __attribute__((always_inline)) {
    float acc = 0.0f;
    if (nq == n) {
#pragma unroll
      for (int i = 0; i < IT; ++i) acc = dot8(w[i], xs[l + 32 * i], acc);
    } else {
      const u32x4* xq = (const u32x4*)(x + (size_t)nq * H);
      u32x4 xv[IT];
#pragma unroll
      for (int i = 0; i < IT; ++i) xv[i] = ld16(xq + l + 32 * i);
#pragma unroll
      for (int i = 0; i < IT; ++i) acc = dot8(w[i], xv[i], acc);
    }
    acc = group_sum<32>(acc);
    const float up = __shfl(acc, 32, kWave);
    if (lane == 0) {
      const float tw = (scores != nullptr) ? L.topw[q % K] : top_w[q];
      const float g = rbf(acc), u = rbf(up);
      const float a = rbf(rbf(rbf(gelu_tanh(g)) * u) * rbf(tw));
      act[(size_t)q * F + f] = ok ? f2bf(a) : (uint16_t)0;
    }
  };
  if (task >= K * F) return;
  if (!dedup || !ok) {
    emit(p, n);
    return;
  }
  if (dup) return;
  unsigned long long rest = same;
  while (rest != 0ull) {
    const int q = (int)__builtin_ctzll(rest);
    rest &= rest - 1ull;
    emit(q, q / K);
  }
}

// ============================================================== K3: down + combine
//
// One wave per (token, output row h).  Lane group g (8 lanes) dots slot g's
// row down[e_g][h] (F values) with act[g]; IT = F/64 chunks per lane; slots
// beyond 8 take further passes.  Combine:
//   bf16_running = 1: bf16 running sum of bf16(part) in slot order (model.py:289-293)
//   bf16_running = 0: bf16 of the f32 sum of parts (the dense contraction, model.py:250)
// The token's K * F activations are staged in LDS once per block (each wave
// loading them itself took as many vector memory slots as its expert rows),
// and a block is kDownWaves rows: the 26B layer's 2,816 rows are then one
// block per CU.
constexpr int kDownWaves = 11;

template <int IT>
__global__ __launch_bounds__(64 * kDownWaves) void moe_down_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ down, const int32_t* __restrict__ top_i,
    int H, int E, int K, int bf16_running, uint16_t* __restrict__ out) {
  constexpr int F = IT * 64;
  constexpr int NT = 64 * kDownWaves;
  extern __shared__ u32x4 act_lds[];  // K * F/8 chunks of token n
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 3, l = lane & 7;
  const int h = blockIdx.x * kDownWaves + wave_id();
  const int n = blockIdx.y;
  const int hc = min(h, H - 1);
  const int mch = K * (F / 8);
  const u32x4* actn = (const u32x4*)(act + (size_t)n * K * F);
  // the first 8 slots' experts and this thread's first activation chunk,
  // then the rows, then the staging store
  const int e0 = (g < K) ? top_i[n * K + g] : -1;
  const u32x4 a0 = ld16(actn + min(tid, mch - 1));
  float run = 0.0f;
  bool first = true;
  for (int s0 = 0; s0 < K; s0 += 8) {
    const int slot = s0 + g;
    const int e = (s0 == 0) ? e0 : ((slot < K) ? top_i[n * K + slot] : -1);
    const bool ok = slot < K && e >= 0 && e < E;
    const u32x4* row = (const u32x4*)(down + ((size_t)(ok ? e : 0) * H + hc) * F);
    u32x4 w[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 8 * i);
    if (s0 == 0) {
      if (tid < mch) act_lds[tid] = a0;
      for (int c = tid + NT; c < mch; c += NT) act_lds[c] = ld16(actn + c);
      lds_barrier();
    }
    float part = 0.0f;
    if (ok) {
      const u32x4* av = act_lds + slot * (F / 8);
#pragma unroll
      for (int i = 0; i < IT; ++i) part = dot8(w[i], av[l + 8 * i], part);
    }
    part = group_sum<8>(part);
    const int cnt = min(8, K - s0);
    for (int q = 0; q < cnt; ++q) {
      const float pq = __shfl(part, 8 * q, kWave);
      if (bf16_running) {
        const float b = rbf(pq);
        run = first ? b : rbf(run + b);
      } else {
        run = first ? pq : run + pq;
      }
      first = false;
    }
  }
  if (lane == 0 && h < H) out[(size_t)n * H + h] = f2bf(run);
}

// Several tokens (2 <= N <= 8, K <= 8), routing given: one wave per output
// row h for all N tokens, so the row h of an expert that several tokens chose
// is read once (moe_down_kernel reads it once per token, the repeats coming
// from the MALL).  Each wave lists the distinct valid experts of the N * K
// (token, slot) pairs in order of first occurrence, with the mask of pairs
// that chose each; in pass r lane group g reads the row of distinct expert
// 8r + g (the next pass's rows are requested before this pass's products)
// and dots it with the activations of each of its pairs exactly as
// moe_down_kernel's lane group for that pair does (the same chunks per lane
// in the same order, the same 8-lane sum), into the wave's part of that pair;
// lane n then combines token n's parts in slot order.  A pair whose expert is
// outside [0, E) keeps part 0, as there.  Bit-identical to moe_down_kernel.
constexpr int kDownShMaxN = 8, kDownShMaxK = 8;
constexpr int kDownShPairs = kDownShMaxN * kDownShMaxK;

template <int IT>
__global__ __launch_bounds__(64 * kDownWaves) void moe_down_shared_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ down, const int32_t* __restrict__ top_i, int N,
    int H, int E, int K, int bf16_running, uint16_t* __restrict__ out) {
  constexpr int F = IT * 64;
  constexpr int NT = 64 * kDownWaves;
  constexpr int APT = (kDownShPairs * (F / 8) + NT - 1) / NT;  // activation chunks per thread, at most
  __shared__ u32x4 act_lds[kDownShPairs * (F / 8)];
  __shared__ int dexp[kDownWaves][kDownShPairs];                  // distinct expert d of each wave
  __shared__ unsigned long long dmask[kDownWaves][kDownShPairs];  // the pairs that chose it
  __shared__ float parts[kDownWaves][kDownShPairs];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 3, l8 = lane & 7, wave = wave_id();
  const int h = blockIdx.x * kDownWaves + wave;
  const int hc = min(h, H - 1);
  const int NK = N * K, mch = NK * (F / 8);
  // every pair's expert (one per lane), then this thread's activation chunks
  const int pe_raw = top_i[min(lane, NK - 1)];
  u32x4 av[APT];
#pragma unroll
  for (int j = 0; j < APT; ++j) av[j] = ld16((const u32x4*)act + min(tid + NT * j, mch - 1));
  const int pe = (lane < NK && pe_raw >= 0 && pe_raw < E) ? pe_raw : -1;
  parts[wave][lane] = 0.0f;
  // distinct experts in order of first occurrence; lane group g keeps the
  // expert of its first pass in a register
  unsigned long long rem = __ballot(pe >= 0);
  int nd = 0, e0 = 0;
  while (rem != 0ull) {
    const int q0 = (int)__builtin_ctzll(rem);
    const int v = __builtin_amdgcn_readlane(pe, q0);
    const unsigned long long m = __ballot(pe == v);
    if (lane == 0) {
      dexp[wave][nd] = v;
      dmask[wave][nd] = m;
    }
    if (nd == g) e0 = v;
    rem &= ~m;
    ++nd;
  }
  const int npass = (nd + 7) / 8;
  auto load_rows = [&](int e, u32x4 (&w)[IT]) __attribute__((always_inline)) {
    const u32x4* row = (const u32x4*)(down + ((size_t)e * H + hc) * F);
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l8 + 8 * i);
  };
  u32x4 wa[IT], wb[IT];
  load_rows(e0, wa);
#pragma unroll
  for (int j = 0; j < APT; ++j)
    if (tid + NT * j < mch) act_lds[tid + NT * j] = av[j];
  lds_barrier();
  // pass r: rows in `cur`; the next pass's rows requested into `nxt` first
  auto pass = [&](int r, u32x4 (&cur)[IT], u32x4 (&nxt)[IT]) __attribute__((always_inline)) {
    if (r + 1 < npass) {
      const int dn = min(8 * (r + 1) + g, nd - 1);
      load_rows(dexp[wave][dn], nxt);
    }
    const int d = 8 * r + g;
    unsigned long long pm = (d < nd) ? dmask[wave][d] : 0ull;
    while (pm != 0ull) {  // uniform per lane group
      const int q = (int)__builtin_ctzll(pm);
      pm &= pm - 1ull;
      const u32x4* am = act_lds + q * (F / 8);
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < IT; ++i) part = dot8(cur[i], am[l8 + 8 * i], part);
      part = group_sum<8>(part);
      if (l8 == 0) parts[wave][q] = part;
    }
  };
  for (int r = 0; r < npass; r += 2) {
    pass(r, wa, wb);
    if (r + 1 < npass) pass(r + 1, wb, wa);
  }
  if (lane < N && h < H) {
    float run = 0.0f;
    for (int s = 0; s < K; ++s) {
      const float pq = parts[wave][lane * K + s];
      if (bf16_running) {
        const float b = rbf(pq);
        run = (s == 0) ? b : rbf(run + b);
      } else {
        run = (s == 0) ? pq : run + pq;
      }
    }
    out[(size_t)lane * H + h] = f2bf(run);
  }
}

// ------------------------------------------------------------------ launchers
static float bf16_inv_sqrt(int64_t H) {
  // bf16(H^-0.5): the constant the reference multiplies in bf16 (model.py:226)
  const float c = (float)(1.0 / sqrt((double)H));
  uint32_t u;
  memcpy(&u, &c, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

// Many rows (prefill) on f64 MFMA (v_mfma_f64_16x16x4_f64: lane l supplies
// A[l%16][l/16] and B[l/16][l%16] and holds D[4r + l/16][l%16], r < 4).  A
// block takes kRouterMRows = 16 token rows and 64 experts: the rows are
// normalised into LDS (the same rounding steps as router_scores_kernel),
// then wave w accumulates the 16 x 16 dots of experts 64*blockIdx.y + 16w ..
// +15 in f64 (the bf16 x bf16 products are exact; the sum is f64 as in the
// per-row kernels, in another order).  Per 32-wide k chunk lane l reads 8
// consecutive k of row l%16 (LDS) and of expert l%16 (router row, 16 bytes)
// at chunk offset 8*(l/16), and MFMA s of the chunk takes k = 8*(l/16) + s:
// the four k slots of the MFMA cover the chunk over s = 0..7.  H % 32 == 0,
// H <= kRouterMaxH.
constexpr int kRouterMRows = 16;
constexpr int kRouterMExperts = 64;
constexpr int kRouterMaxH = 4096;
typedef double f64x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void router_scores_mfma_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ pre_w,
                                                                 const uint16_t* __restrict__ scale,
                                                                 const uint16_t* __restrict__ proj, int N, int H,
                                                                 int E, float eps, float inv_sqrt_h_bf,
                                                                 float* __restrict__ scores) {
  __shared__ u32x4 xs_rows[kRouterMRows * kRouterMaxH / 8];  // 16 x H/8 chunks
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int CH = H / 8;
  const int r0 = blockIdx.x * kRouterMRows;
  const int e0 = blockIdx.y * kRouterMExperts + wave * 16;
  const u32x4* pw = (const u32x4*)pre_w;
  const u32x4* sw = (const u32x4*)scale;
  // this wave's first router rows, requested before the normalisation
  const int er = min(e0 + (lane & 15), E - 1);
  const u32x4* wrow = (const u32x4*)(proj + (size_t)er * H) + (lane >> 4);
  constexpr int PF = 8;  // router chunks in flight per lane
  u32x4 wq[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) wq[u] = ld16(wrow + 4 * min(u, CH / 4 - 1));
  // the wave's 4 token rows and both norm weights, all requested at once
  // (one round trip, not three per row), then normalised from registers
  constexpr int RW = kRouterMRows / 4;                 // rows per wave
  constexpr int XPL = (kRouterMaxH / 8 + 63) / 64;     // 16-byte chunks per lane and row
  u32x4 xv[RW][XPL], pwv[XPL], scv[XPL];
#pragma unroll
  for (int j = 0; j < XPL; ++j) {
    const int cc = min(lane + 64 * j, CH - 1);
    pwv[j] = ld16((pre_w != nullptr ? pw : sw) + cc);
    scv[j] = ld16(sw + cc);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
      const int r = wave * RW + rr;
      xv[rr][j] = ld16((const u32x4*)(x + (size_t)min(r0 + r, N - 1) * H) + cc);
    }
  }
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int r = wave * RW + rr;
    float rp = 1.0f;
    if (pre_w != nullptr) {  // pre_feedforward_layernorm_2 (model.py:315)
      double s0 = 0.0;
#pragma unroll
      for (int j = 0; j < XPL; ++j)
        if (lane + 64 * j < CH) s0 = sumsq8_f64(xv[rr][j], s0);
      rp = rms_scale(group_sum_f64<64>(s0), H, eps);
#pragma unroll
      for (int j = 0; j < XPL; ++j) xv[rr][j] = scale8(xv[rr][j], rp, &pwv[j]);
    }
    double s1 = 0.0;
#pragma unroll
    for (int j = 0; j < XPL; ++j)
      if (lane + 64 * j < CH) s1 = sumsq8_f64(xv[rr][j], s1);
    const float r1 = rms_scale(group_sum_f64<64>(s1), H, eps);
#pragma unroll
    for (int j = 0; j < XPL; ++j) {
      const int c8 = lane + 64 * j;
      if (c8 < CH) {
        float f[8], g[8];
        unpack8(xv[rr][j], f);
        unpack8(scv[j], g);
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = rbf(rbf(rbf(f[q] * r1) * g[q]) * inv_sqrt_h_bf);
        u32x4 o;
        o.x = pack2(f[0], f[1]); o.y = pack2(f[2], f[3]); o.z = pack2(f[4], f[5]); o.w = pack2(f[6], f[7]);
        xs_rows[r * CH + c8] = o;
      }
    }
  }
  __syncthreads();
  if (e0 >= E) return;  // no barrier below
  const u32x4* xrow = xs_rows + (lane & 15) * CH + (lane >> 4);
  // two accumulator chains (even and odd k slots of each MFMA group), so
  // consecutive MFMAs do not wait for each other's result; summed at the end
  f64x4 acc[2] = {{0.0, 0.0, 0.0, 0.0}, {0.0, 0.0, 0.0, 0.0}};
  const int nch = CH / 4;  // 32-wide k chunks
  for (int c0 = 0; c0 < nch; c0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int c = c0 + u;
      if (c < nch) {
        const u32x4 wv = wq[u];
        wq[u] = ld16(wrow + 4 * min(c + PF, nch - 1));  // chunk c + PF (clamped: a cache hit at the end)
        const u32x4 xv = xrow[4 * c];
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const double a = (double)((s & 1) ? bf_hi(xw[s >> 1]) : bf_lo(xw[s >> 1]));
          const double b = (double)((s & 1) ? bf_hi(ww[s >> 1]) : bf_lo(ww[s >> 1]));
          acc[s & 1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[s & 1], 0, 0, 0);
        }
      }
    }
  }
  const int e = e0 + (lane & 15);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = r0 + 4 * r + (lane >> 4);
    if (n < N && e < E) scores[(size_t)n * E + e] = rbf(f32_of(acc[0][r] + acc[1][r]));
  }
}

static void launch_scores(const uint16_t* x, const uint16_t* pre_w, const uint16_t* scale, const uint16_t* proj,
                          int N, int H, int E, float eps, float* scores, hipStream_t st) {
  dim3 grid((unsigned)((E + 7) / 8), (unsigned)N);
  const float c = bf16_inv_sqrt(H);
  // many rows: 16-row tiles on f64 MFMA; the per-row kernel grows with N
  // (~5 us at 54 rows, ~200 us at 2,048)
  if (N >= 128 && H % 32 == 0 && H <= kRouterMaxH && ((uintptr_t)scale & 15u) == 0 &&
      ((uintptr_t)pre_w & 15u) == 0) {
    const dim3 tgrid((unsigned)((N + kRouterMRows - 1) / kRouterMRows),
                     (unsigned)((E + kRouterMExperts - 1) / kRouterMExperts));
    hipLaunchKernelGGL(router_scores_mfma_kernel, tgrid, dim3(256), 0, st, x, pre_w, scale, proj, N, H, E, eps, c,
                       scores);
    return;
  }
  const bool aligned = ((uintptr_t)scale & 15u) == 0 && ((uintptr_t)pre_w & 15u) == 0;
  if (H % 256 == 0 && H / 256 <= 16 && aligned) {
    switch (H / 256) {
#define G4MI_CASE(I)                                                                                       \
  case I:                                                                                                  \
    if (N <= kRouterWaveRows)                                                                              \
      hipLaunchKernelGGL(router_scores_wave_kernel<I>, dim3((unsigned)((E + 1) / 2), (unsigned)N), dim3(64), 0, \
                         st, x, pre_w, scale, proj, E, eps, c, scores);                                    \
    else                                                                                                   \
      hipLaunchKernelGGL(router_scores_kernel<I>, grid, dim3(256), 0, st, x, pre_w, scale, proj, E, eps, c, \
                         scores);                                                                          \
    return;
      G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
    }
  }
  hipLaunchKernelGGL(router_scores_generic_kernel, grid, dim3(256), 0, st, x, pre_w, scale, proj, H, E, eps, c,
                     scores);
}

static void launch_gateup(int it, const uint16_t* x, const uint16_t* gu, const float* scores, const uint16_t* pes,
                          float* tw, int32_t* ti, int N, int F, int E, int K, uint16_t* act, hipStream_t st) {
  // the in-block selection needs 4 waves; with the routing given, 2-wave
  // blocks spread the 8 x 704 tasks of a 26B token evenly (11 blocks per CU)
  const int waves = (scores != nullptr) ? 4 : 2;
  dim3 grid((unsigned)((K * F + waves - 1) / waves), (unsigned)N);
  switch (it) {
#define G4MI_CASE(I)                                                                                           \
  case I:                                                                                                      \
    hipLaunchKernelGGL(moe_gateup_kernel<I>, grid, dim3(64 * waves), 0, st, x, gu, scores, pes, tw, ti, F, E, K, \
                       act);                                                                                   \
    return;
    G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
  }
}

// The shared-row down at 8 tokens of at most 8 slots each: 26B shapes,
// uniform routing (50.9 of 64 experts distinct), 37.9 against 40.1 us for the
// token rows; at 2 and 4 tokens (15.8 and 28.5 distinct) the token rows,
// whose repeats come from the MALL, are faster (12.0 / 20.9 against
// 13.5 / 22.6 us), and at 6 as well.  G4MI_MOE_DOWN_SHARED=0 keeps the token
// rows at 8, =1 forces the shared rows from 2 tokens.
static bool down_shared(int N, int K) {
  if (N < 2 || N > kDownShMaxN || K > kDownShMaxK) return false;
  const char* e = getenv("G4MI_MOE_DOWN_SHARED");
  if (e != nullptr) return atoi(e) != 0;
  return N == kDownShMaxN;
}

static void launch_down(int it, const uint16_t* act, const uint16_t* dn, const int32_t* ti, int N, int H, int E,
                        int K, int running, uint16_t* out, hipStream_t st) {
  if (down_shared(N, K)) {
    const dim3 sgrid((unsigned)((H + kDownWaves - 1) / kDownWaves));
    switch (it) {
#define G4MI_CASE(I)                                                                                          \
  case I:                                                                                                     \
    hipLaunchKernelGGL(moe_down_shared_kernel<I>, sgrid, dim3(64 * kDownWaves), 0, st, act, dn, ti, N, H, E, K, \
                       running, out);                                                                         \
    return;
      G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
    }
  }
  dim3 grid((unsigned)((H + kDownWaves - 1) / kDownWaves), (unsigned)N);
  const size_t lds = (size_t)K * it * 64 * 2;  // K * F bf16 activations
  switch (it) {
#define G4MI_CASE(I)                                                                                         \
  case I:                                                                                                    \
    hipLaunchKernelGGL(moe_down_kernel<I>, grid, dim3(64 * kDownWaves), lds, st, act, dn, ti, H, E, K, running, \
                       out);                                                                                 \
    return;
    G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
  }
}

static int check_router(const char* what, int64_t N, int64_t H, int64_t E) {
  G4MI_REQUIRE(N >= 1 && N <= 65535, G4MI_EINVAL, "%s: N=%lld out of range", what, (long long)N);
  G4MI_REQUIRE(H >= 8 && H % 8 == 0 && H <= kMaxH, G4MI_EINVAL, "%s: H=%lld must be a multiple of 8 in [8, %d]",
               what, (long long)H, kMaxH);
  G4MI_REQUIRE(E >= 1 && E <= kMaxE, G4MI_EINVAL, "%s: E=%lld out of range [1, %d]", what, (long long)E, kMaxE);
  return 0;
}

static int check_experts(const char* what, int64_t N, int64_t H, int64_t F, int64_t E, int64_t k) {
  G4MI_REQUIRE(N >= 1 && N <= 65535, G4MI_EINVAL, "%s: N=%lld out of range", what, (long long)N);
  G4MI_REQUIRE(E >= 1 && E <= kMaxE && k >= 1 && k <= E && k <= kMaxK, G4MI_EINVAL, "%s: bad E=%lld k=%lld", what,
               (long long)E, (long long)k);
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "%s: H=%lld must be 256*i with i in [1,16]", what, (long long)H);
  G4MI_REQUIRE(F % 64 == 0 && F / 64 >= 1 && F / 64 <= 16, G4MI_EUNSUPPORTED,
               "%s: F=%lld must be 64*i with i in [1,16]", what, (long long)F);
  return 0;
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int g4mi_moe_router_scores(const uint16_t* x, const uint16_t* pre_norm_w, const uint16_t* router_scale,
                           const uint16_t* router_proj, int64_t N, int64_t H, int64_t E, float eps, float* scores,
                           void* stream) {
  G4MI_REQUIRE(x && router_scale && router_proj && scores, G4MI_EINVAL, "moe_router_scores: null pointer argument");
  int rc = check_router("moe_router_scores", N, H, E);
  if (rc) return rc;
  G4MI_REQUIRE(al16(x) && al16(router_proj), G4MI_EALIGN,
               "moe_router_scores: x and router_proj must be 16-byte aligned");
  launch_scores(x, pre_norm_w, router_scale, router_proj, (int)N, (int)H, (int)E, eps, scores, as_stream(stream));
  return check_launch("moe_router_scores");
}

int64_t g4mi_moe_router_workspace_bytes(int64_t N, int64_t E) { return ((N * E * 4 + 255) / 256) * 256; }

int g4mi_moe_router_topk(const uint16_t* x, const uint16_t* pre_norm_w, const uint16_t* router_scale,
                         const uint16_t* router_proj, const uint16_t* per_expert_scale, int64_t N, int64_t H,
                         int64_t E, int64_t k, float eps, float* out_w, int32_t* out_i, void* ws,
                         int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(per_expert_scale && out_w && out_i && ws, G4MI_EINVAL, "moe_router_topk: null pointer argument");
  int rc = check_router("moe_router_topk", N, H, E);
  if (rc) return rc;
  G4MI_REQUIRE(k >= 1 && k <= E && k <= kMaxK, G4MI_EINVAL, "moe_router_topk: k=%lld out of range", (long long)k);
  G4MI_REQUIRE(ws_bytes >= g4mi_moe_router_workspace_bytes(N, E), G4MI_EWORKSPACE,
               "moe_router_topk: workspace %lld < %lld bytes", (long long)ws_bytes,
               (long long)g4mi_moe_router_workspace_bytes(N, E));
  float* scores = (float*)ws;
  rc = g4mi_moe_router_scores(x, pre_norm_w, router_scale, router_proj, N, H, E, eps, scores, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(router_select_kernel, dim3((unsigned)N), dim3(256), 0, as_stream(stream), scores,
                     per_expert_scale, (int)E, (int)k, out_w, out_i);
  return check_launch("moe_router_topk/select");
}

int g4mi_moe_gateup(const uint16_t* xn, const uint16_t* gate_up, const float* top_w, const int32_t* top_i,
                    int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, uint16_t* act, void* stream) {
  G4MI_REQUIRE(xn && gate_up && top_w && top_i && act, G4MI_EINVAL, "moe_gateup: null pointer argument");
  int rc = check_experts("moe_gateup", N, H, F, E, k);
  if (rc) return rc;
  G4MI_REQUIRE(al16(xn) && al16(gate_up), G4MI_EALIGN, "moe_gateup: xn and gate_up must be 16-byte aligned");
  launch_gateup((int)(H / 256), xn, gate_up, nullptr, nullptr, const_cast<float*>(top_w),
                const_cast<int32_t*>(top_i), (int)N, (int)F, (int)E, (int)k, act, as_stream(stream));
  return check_launch("moe_gateup");
}

int g4mi_moe_gateup_routed(const uint16_t* xn, const float* scores, const uint16_t* per_expert_scale,
                           const uint16_t* gate_up, int64_t N, int64_t H, int64_t F, int64_t E, int64_t k,
                           uint16_t* act, float* top_w, int32_t* top_i, void* stream) {
  G4MI_REQUIRE(xn && scores && per_expert_scale && gate_up && act && top_w && top_i, G4MI_EINVAL,
               "moe_gateup_routed: null pointer argument");
  int rc = check_experts("moe_gateup_routed", N, H, F, E, k);
  if (rc) return rc;
  G4MI_REQUIRE(al16(xn) && al16(gate_up), G4MI_EALIGN, "moe_gateup_routed: xn and gate_up must be 16-byte aligned");
  launch_gateup((int)(H / 256), xn, gate_up, scores, per_expert_scale, top_w, top_i, (int)N, (int)F, (int)E, (int)k,
                act, as_stream(stream));
  return check_launch("moe_gateup_routed");
}

int g4mi_moe_down(const uint16_t* act, const uint16_t* down, const int32_t* top_i, int64_t N, int64_t H,
                  int64_t F, int64_t E, int64_t k, int32_t combine, uint16_t* out, void* stream) {
  G4MI_REQUIRE(act && down && top_i && out, G4MI_EINVAL, "moe_down: null pointer argument");
  int rc = check_experts("moe_down", N, H, F, E, k);
  if (rc) return rc;
  G4MI_REQUIRE(combine == G4MI_COMBINE_BF16_RUNNING || combine == G4MI_COMBINE_F32, G4MI_EINVAL,
               "moe_down: unknown combine mode %d", combine);
  G4MI_REQUIRE(al16(act) && al16(down), G4MI_EALIGN, "moe_down: act and down must be 16-byte aligned");
  launch_down((int)(F / 64), act, down, top_i, (int)N, (int)H, (int)E, (int)k,
              combine == G4MI_COMBINE_BF16_RUNNING ? 1 : 0, out, as_stream(stream));
  return check_launch("moe_down");
}

int64_t g4mi_moe_experts_workspace_bytes(int64_t N, int64_t F, int64_t k) {
  return ((N * k * F * 2 + 255) / 256) * 256;
}

int g4mi_moe_experts_decode(const uint16_t* xn, const uint16_t* gate_up, const uint16_t* down,
                            const float* top_w, const int32_t* top_i, int64_t N, int64_t H, int64_t F,
                            int64_t E, int64_t k, int32_t combine, uint16_t* out, void* ws, int64_t ws_bytes,
                            void* stream) {
  G4MI_REQUIRE(ws != nullptr, G4MI_EINVAL, "moe_experts_decode: null workspace");
  G4MI_REQUIRE(N >= 1 && k >= 1 && ws_bytes >= g4mi_moe_experts_workspace_bytes(N, F, k), G4MI_EWORKSPACE,
               "moe_experts_decode: workspace too small");
  G4MI_REQUIRE(al16(ws), G4MI_EALIGN, "moe_experts_decode: workspace must be 16-byte aligned");
  uint16_t* act = (uint16_t*)ws;
  int rc = g4mi_moe_gateup(xn, gate_up, top_w, top_i, N, H, F, E, k, act, stream);
  if (rc) return rc;
  return g4mi_moe_down(act, down, top_i, N, H, F, E, k, combine, out, stream);
}

int64_t g4mi_moe_block_workspace_bytes(int64_t N, int64_t E, int64_t F, int64_t k) {
  return g4mi_moe_router_workspace_bytes(N, E) + g4mi_moe_experts_workspace_bytes(N, F, k);
}

int g4mi_moe_block_decode(const uint16_t* xn, const uint16_t* router_scale, const uint16_t* router_proj,
                          const uint16_t* per_expert_scale, const uint16_t* gate_up, const uint16_t* down,
                          int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, float eps, int32_t combine,
                          uint16_t* out, float* top_w, int32_t* top_i, void* ws, int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(ws != nullptr, G4MI_EINVAL, "moe_block_decode: null workspace");
  G4MI_REQUIRE(N >= 1 && k >= 1 && ws_bytes >= g4mi_moe_block_workspace_bytes(N, E, F, k), G4MI_EWORKSPACE,
               "moe_block_decode: workspace too small");
  G4MI_REQUIRE(al16(ws), G4MI_EALIGN, "moe_block_decode: workspace must be 16-byte aligned");
  float* scores = (float*)ws;
  uint16_t* act = (uint16_t*)((char*)ws + g4mi_moe_router_workspace_bytes(N, E));
  int rc;
  if (N > 1 && N * k <= 64) {
    // several tokens: one selection launch, then the gate/up with the routing
    // given, which reads an expert chosen by several tokens once
    rc = g4mi_moe_router_topk(xn, nullptr, router_scale, router_proj, per_expert_scale, N, H, E, k, eps, top_w,
                              top_i, ws, g4mi_moe_router_workspace_bytes(N, E), stream);
    if (rc) return rc;
    rc = g4mi_moe_gateup(xn, gate_up, top_w, top_i, N, H, F, E, k, act, stream);
  } else {
    // one token: the selection runs in every gate/up block (no launch between)
    rc = g4mi_moe_router_scores(xn, nullptr, router_scale, router_proj, N, H, E, eps, scores, stream);
    if (rc) return rc;
    rc = g4mi_moe_gateup_routed(xn, scores, per_expert_scale, gate_up, N, H, F, E, k, act, top_w, top_i, stream);
  }
  if (rc) return rc;
  return g4mi_moe_down(act, down, top_i, N, H, F, E, k, combine, out, stream);
}

}  // extern "C"
