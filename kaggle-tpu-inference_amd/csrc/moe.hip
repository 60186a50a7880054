// MoE decode block: router + top-k (K1), per-expert gate/up GEMV with the
// gated-GELU activation (K2), per-expert down GEMV with the weighted combine
// (K3).  Follows model.py _router / _moe (model.py:224-232, model.py:262-294).
//
// Only the rows of the selected experts are read from HBM: K2 reads
// gate_up[e] (2*F rows of H) and K3 reads down[e] (H rows of F) for the k
// experts each token picked, which is the job the reference's per-expert
// dynamic_slice does on TPU.
#include <string.h>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

constexpr int kMaxH = 16384;   // router prologue keeps one token row in LDS
constexpr int kMaxE = 256;
constexpr int kMaxK = 32;

#define G4MI_IT_CASES(M) M(1) M(2) M(3) M(4) M(5) M(6) M(7) M(8) M(9) M(10) M(11) M(12) M(13) M(14) M(15) M(16)

// Softmax over E scores per token (f32; exp in f64 rounded to f32; exact
// sums), stable top-k (value desc, index asc), renormalise over the k picks,
// scale by per_expert_scale.  Run by the one block that finished last.
__device__ void router_select(const float* __restrict__ scores, const uint16_t* __restrict__ pes, int N, int E,
                              int K, float* __restrict__ out_w, int32_t* __restrict__ out_i) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  for (int t = wave; t < N; t += nw) {
    const float* s = scores + (size_t)t * E;
    float sv[kMaxE / 64];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxE / 64; ++j) {
      const int ee = lane + 64 * j;
      sv[j] = (ee < E) ? s[ee] : -INFINITY;
      m = fmaxf(m, sv[j]);
    }
    m = group_max<64>(m);
    float ex[kMaxE / 64];
    double se = 0.0;
#pragma unroll
    for (int j = 0; j < kMaxE / 64; ++j) {
      const int ee = lane + 64 * j;
      ex[j] = (ee < E) ? (float)exp((double)(sv[j] - m)) : 0.0f;
      se += (double)ex[j];
    }
    const float sum = (float)group_sum_f64<64>(se);
    float p[kMaxE / 64];
#pragma unroll
    for (int j = 0; j < kMaxE / 64; ++j) p[j] = (lane + 64 * j < E) ? ex[j] / sum : -INFINITY;

    float topv = 0.0f;  // lane j < K keeps the j-th selected probability
    int topi = 0;
    for (int kk = 0; kk < K; ++kk) {
      // lane-local best (value desc, index asc)
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < kMaxE / 64; ++j) {
        const int ee = lane + 64 * j;
        if (ee < E && (p[j] > bv || (p[j] == bv && ee < bi))) { bv = p[j]; bi = ee; }
      }
#pragma unroll
      for (int msk = 32; msk >= 1; msk >>= 1) {
        const float ov = __shfl_xor(bv, msk, kWave);
        const int oi = __shfl_xor(bi, msk, kWave);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (lane == kk) { topv = bv; topi = bi; }
#pragma unroll
      for (int j = 0; j < kMaxE / 64; ++j)
        if (lane + 64 * j == bi) p[j] = -INFINITY;
    }
    double sk = (lane < K) ? (double)topv : 0.0;
    const float ssum = (float)group_sum_f64<64>(sk);
    if (lane < K) {
      const float w = (topv / ssum) * bf2f(pes[topi]);
      out_w[(size_t)t * K + lane] = w;
      out_i[(size_t)t * K + lane] = topi;
    }
  }
}

// ============================================================== K1: router
//
// grid (ceil(E / rows_per_block), N), 256 threads.  Every block rebuilds the
// router input of its token in LDS:
//     xe = rms_norm(x, pre_w)             (only when pre_w != null)
//     xn = rms_norm(xe, None)
//     x2 = bf16(bf16(xn * scale) * bf16(H^-0.5))
// and writes the bf16-rounded scores of its experts.  The last block to
// finish turns the scores of every token into (top_w, top_i).
__global__ __launch_bounds__(256) void router_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_w, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ proj, const uint16_t* __restrict__ pes, int N, int H, int E, int K,
    float eps, float inv_sqrt_h_bf, float* __restrict__ scores, unsigned int* __restrict__ counter,
    float* __restrict__ out_w, int32_t* __restrict__ out_i) {
  __shared__ uint16_t xs[kMaxH];
  __shared__ double red[4];
  __shared__ int flag;
  const int n = blockIdx.y;
  const int tid = threadIdx.x;
  const uint16_t* xrow = x + (size_t)n * H;

  // ---- prologue: router input in LDS
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
    for (int i = tid; i < H; i += blockDim.x) {
      const float xn = rbf(bf2f(xs[i]) * r);
      const float t = rbf(xn * bf2f(scale[i]));
      xs[i] = f2bf(t * inv_sqrt_h_bf);
    }
    __syncthreads();
  }

  // ---- scores: 32 lanes per expert row, exact f64 dot, one rounding to bf16
  const int lane = tid & 63, half = lane >> 5, l = lane & 31, wave = tid >> 6;
  const int rows_per_block = (blockDim.x >> 6) * 2;
  const int e = blockIdx.x * rows_per_block + wave * 2 + half;
  const int nch = H >> 3;
  if (e < E) {
    const u32x4* row = (const u32x4*)(proj + (size_t)e * H);
    double acc = 0.0;
    for (int c = l; c < nch; c += 32) acc = dot8_f64(ld16(row + c), ld16(xs + 8 * c), acc);
    acc = group_sum_f64<32>(acc);
    if (l == 0) scores[(size_t)n * E + e] = rbf((float)acc);
  }

  // ---- last block: softmax (f32, exp in f64), stable top-k, renormalise
  if (!arrive_last(counter, gridDim.x * gridDim.y, &flag)) return;
  router_select(scores, pes, N, E, K, out_w, out_i);
}

// K1 fast path for H = 256*IT: grid (ceil(E/8), N), 4 waves of 2 rows.  Each
// half-wave issues its expert row's IT 16-byte loads first, then rebuilds the
// router input in registers (every half-wave holds the whole token row, so
// the RMSNorm reductions are half-wave shuffles with no block barrier).
template <int IT>
__global__ __launch_bounds__(256) void router_fast_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_w, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ proj, const uint16_t* __restrict__ pes, int N, int E, int K, float eps,
    float inv_sqrt_h_bf, float* __restrict__ scores, unsigned int* __restrict__ counter,
    float* __restrict__ out_w, int32_t* __restrict__ out_i) {
  constexpr int H = IT * 256;
  __shared__ int flag;
  const int lane = threadIdx.x & 63, half = lane >> 5, l = lane & 31, wave = threadIdx.x >> 6;
  const int n = blockIdx.y;
  const int e = blockIdx.x * 8 + wave * 2 + half;
  u32x4 w[IT];
  if (e < E) {
    const u32x4* row = (const u32x4*)(proj + (size_t)e * H);
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 32 * i);
  }
  const u32x4* xr = (const u32x4*)(x + (size_t)n * H);
  u32x4 xv[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) xv[i] = ld16(xr + l + 32 * i);
  if (pre_w != nullptr) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < IT; ++i) ss = sumsq8_f64(xv[i], ss);
    const float r = rms_scale(group_sum_f64<32>(ss), H, eps);
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const u32x4 pw = ld16((const u32x4*)pre_w + l + 32 * i);
      xv[i] = scale8(xv[i], r, &pw);
    }
  }
  {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < IT; ++i) ss = sumsq8_f64(xv[i], ss);
    const float r = rms_scale(group_sum_f64<32>(ss), H, eps);
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const u32x4 sc = ld16((const u32x4*)scale + l + 32 * i);
      float f[8], g[8];
      unpack8(xv[i], f);
      unpack8(sc, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = rbf(rbf(rbf(f[j] * r) * g[j]) * inv_sqrt_h_bf);
      xv[i].x = pack2(f[0], f[1]); xv[i].y = pack2(f[2], f[3]);
      xv[i].z = pack2(f[4], f[5]); xv[i].w = pack2(f[6], f[7]);
    }
  }
  if (e < E) {
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < IT; ++i) acc = dot8_f64(w[i], xv[i], acc);
    acc = group_sum_f64<32>(acc);
    if (l == 0) scores[(size_t)n * E + e] = rbf((float)acc);
  }
  if (!arrive_last(counter, gridDim.x * gridDim.y, &flag)) return;
  router_select(scores, pes, N, E, K, out_w, out_i);
}

// ============================================================== K2: gate/up
//
// One wave per (token, slot, f): lanes 0-31 dot x with gate row f of expert
// top_i[slot], lanes 32-63 with up row f.  IT = H/256 16-byte chunks per lane.
//     act = bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(top_w))
template <int IT>
__global__ __launch_bounds__(256) void moe_gateup_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate_up, const float* __restrict__ top_w,
    const int32_t* __restrict__ top_i, int F, int E, int K, uint16_t* __restrict__ act) {
  constexpr int H = IT * 256;
  const int lane = threadIdx.x & 63, half = lane >> 5, l = lane & 31;
  const int task = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n = blockIdx.y;
  if (task >= K * F) return;
  const int slot = task / F, f = task - slot * F;
  const int e = top_i[n * K + slot];
  if (e < 0 || e >= E) {  // not an expert index: contribute nothing
    if (lane == 0) act[((size_t)n * K + slot) * F + f] = 0;
    return;
  }
  const u32x4* row = (const u32x4*)(gate_up + ((size_t)(e * 2 + half) * F + f) * H);
  u32x4 w[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 32 * i);
  const u32x4* xv = (const u32x4*)(x + (size_t)n * H);
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < IT; ++i) acc = dot8(w[i], ld16(xv + l + 32 * i), acc);
  acc = group_sum<32>(acc);
  const float up = __shfl(acc, 32, kWave);
  if (lane == 0) {
    const float g = rbf(acc), u = rbf(up);
    const float a = rbf(rbf(rbf(gelu_tanh(g)) * u) * rbf(top_w[n * K + slot]));
    act[((size_t)n * K + slot) * F + f] = f2bf(a);
  }
}

// ============================================================== K3: down + combine
//
// One wave per (token, output row h).  Lane group g (8 lanes) computes slot g's
// dot of down[e_g][h] (F values) with act[g]; IT = F/64 chunks per lane.
// Slots beyond 8 are processed in further passes.  Combine:
//   bf16_running = true : out = bf16 running sum of bf16(part_g) in slot order
//                          (the reference's decode path, model.py:289-293)
//   bf16_running = false: out = bf16(sum of f32 parts) (the dense/prefill
//                          contraction, model.py:250)
template <int IT>
__global__ __launch_bounds__(256) void moe_down_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ down, const int32_t* __restrict__ top_i,
    int H, int E, int K, int bf16_running, uint16_t* __restrict__ out) {
  constexpr int F = IT * 64;
  const int lane = threadIdx.x & 63, g = lane >> 3, l = lane & 7;
  const int h = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n = blockIdx.y;
  if (h >= H) return;
  float run = 0.0f;
  bool first = true;
  for (int s0 = 0; s0 < K; s0 += 8) {
    const int slot = s0 + g;
    float part = 0.0f;
    const int e = (slot < K) ? top_i[n * K + slot] : -1;
    if (e >= 0 && e < E) {
      const u32x4* row = (const u32x4*)(down + ((size_t)e * H + h) * F);
      const u32x4* av = (const u32x4*)(act + ((size_t)n * K + slot) * F);
      u32x4 w[IT];
#pragma unroll
      for (int i = 0; i < IT; ++i) w[i] = ld_stream(row + l + 8 * i);
#pragma unroll
      for (int i = 0; i < IT; ++i) part = dot8(w[i], ld16(av + l + 8 * i), part);
    }
    part = group_sum<8>(part);
    // lane 0 walks the slots of this pass in order
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
  if (lane == 0) out[(size_t)n * H + h] = f2bf(run);
}

template <int IT>
static void launch_gateup(const uint16_t* x, const uint16_t* gu, const float* tw, const int32_t* ti, int N,
                          int F, int E, int K, uint16_t* act, hipStream_t st) {
  const int waves = 4;
  const int tasks = K * F;
  dim3 grid((tasks + waves - 1) / waves, N);
  hipLaunchKernelGGL(moe_gateup_kernel<IT>, grid, dim3(64 * waves), 0, st, x, gu, tw, ti, F, E, K, act);
}

template <int IT>
static void launch_down(const uint16_t* act, const uint16_t* dn, const int32_t* ti, int N, int H, int E,
                        int K, int running, uint16_t* out, hipStream_t st) {
  const int waves = 4;
  dim3 grid((H + waves - 1) / waves, N);
  hipLaunchKernelGGL(moe_down_kernel<IT>, grid, dim3(64 * waves), 0, st, act, dn, ti, H, E, K, running, out);
}


static int dispatch_gateup(int it, const uint16_t* x, const uint16_t* gu, const float* tw, const int32_t* ti,
                           int N, int F, int E, int K, uint16_t* act, hipStream_t st) {
  switch (it) {
#define G4MI_CASE(I) case I: launch_gateup<I>(x, gu, tw, ti, N, F, E, K, act, st); return 0;
    G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
    default: return -1;
  }
}

static int dispatch_down(int it, const uint16_t* act, const uint16_t* dn, const int32_t* ti, int N, int H, int E,
                         int K, int running, uint16_t* out, hipStream_t st) {
  switch (it) {
#define G4MI_CASE(I) case I: launch_down<I>(act, dn, ti, N, H, E, K, running, out, st); return 0;
    G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
    default: return -1;
  }
}

}  // namespace g4mi

extern "C" {

int64_t g4mi_moe_router_workspace_bytes(int64_t N, int64_t E) {
  // [0, 256): completion counter (at a fixed offset, so a workspace sized for
  // one N stays valid for any other); then scores [N, E] f32.
  return 256 + ((N * E * 4 + 255) / 256) * 256;
}

int g4mi_moe_router_topk(const uint16_t* x, const uint16_t* pre_norm_w, const uint16_t* router_scale,
                         const uint16_t* router_proj, const uint16_t* per_expert_scale, int64_t N, int64_t H,
                         int64_t E, int64_t k, float eps, float* out_w, int32_t* out_i, void* ws,
                         int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(x && router_scale && router_proj && per_expert_scale && out_w && out_i && ws, G4MI_EINVAL,
               "moe_router_topk: null pointer argument");
  G4MI_REQUIRE(N >= 1 && N <= 65535, G4MI_EINVAL, "moe_router_topk: N=%lld out of range", (long long)N);
  G4MI_REQUIRE(H >= 8 && H % 8 == 0 && H <= g4mi::kMaxH, G4MI_EINVAL,
               "moe_router_topk: H=%lld must be a multiple of 8 in [8, %d]", (long long)H, g4mi::kMaxH);
  G4MI_REQUIRE(E >= 1 && E <= g4mi::kMaxE, G4MI_EINVAL, "moe_router_topk: E=%lld out of range", (long long)E);
  G4MI_REQUIRE(k >= 1 && k <= E && k <= g4mi::kMaxK, G4MI_EINVAL, "moe_router_topk: k=%lld out of range",
               (long long)k);
  G4MI_REQUIRE(ws_bytes >= g4mi_moe_router_workspace_bytes(N, E), G4MI_EWORKSPACE,
               "moe_router_topk: workspace %lld < %lld bytes", (long long)ws_bytes,
               (long long)g4mi_moe_router_workspace_bytes(N, E));
  G4MI_REQUIRE(((uintptr_t)router_proj & 15u) == 0 && ((uintptr_t)x & 15u) == 0, G4MI_EALIGN,
               "moe_router_topk: x and router_proj must be 16-byte aligned");
  unsigned int* counter = (unsigned int*)ws;
  float* scores = (float*)((char*)ws + 256);
  // bf16(H^-0.5), the constant the reference multiplies in bf16 (model.py:226)
  const float c = (float)(1.0 / sqrt((double)H));
  uint32_t u;
  memcpy(&u, &c, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float cbf;
  memcpy(&cbf, &u, 4);
  const int rows_per_block = 8;
  dim3 grid((unsigned)((E + rows_per_block - 1) / rows_per_block), (unsigned)N);
  hipStream_t st = g4mi::as_stream(stream);
  const bool aligned = ((uintptr_t)router_scale & 15u) == 0 && (pre_norm_w == nullptr || ((uintptr_t)pre_norm_w & 15u) == 0);
  if (H % 256 == 0 && H / 256 <= 16 && aligned) {
    switch (H / 256) {
#define G4MI_CASE(I)                                                                                          \
  case I:                                                                                                     \
    hipLaunchKernelGGL(g4mi::router_fast_kernel<I>, grid, dim3(256), 0, st, x, pre_norm_w, router_scale,     \
                       router_proj, per_expert_scale, (int)N, (int)E, (int)k, eps, cbf, scores, counter, out_w, \
                       out_i);                                                                                \
    break;
      G4MI_IT_CASES(G4MI_CASE)
#undef G4MI_CASE
    }
  } else {
    hipLaunchKernelGGL(g4mi::router_kernel, grid, dim3(256), 0, st, x, pre_norm_w, router_scale, router_proj,
                       per_expert_scale, (int)N, (int)H, (int)E, (int)k, eps, cbf, scores, counter, out_w, out_i);
  }
  return g4mi::check_launch("moe_router_topk");
}

static int check_expert_shapes(const char* what, int64_t N, int64_t H, int64_t F, int64_t E, int64_t k) {
  G4MI_REQUIRE(N >= 1 && N <= 65535, G4MI_EINVAL, "%s: N=%lld out of range", what, (long long)N);
  G4MI_REQUIRE(E >= 1 && k >= 1 && k <= E && k <= g4mi::kMaxK, G4MI_EINVAL, "%s: bad E=%lld k=%lld", what,
               (long long)E, (long long)k);
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "%s: H=%lld must be 256*i with i in [1,16]", what, (long long)H);
  G4MI_REQUIRE(F % 64 == 0 && F / 64 >= 1 && F / 64 <= 16, G4MI_EUNSUPPORTED,
               "%s: F=%lld must be 64*i with i in [1,16]", what, (long long)F);
  return 0;
}

int g4mi_moe_gateup(const uint16_t* xn, const uint16_t* gate_up, const float* top_w, const int32_t* top_i,
                    int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, uint16_t* act, void* stream) {
  G4MI_REQUIRE(xn && gate_up && top_w && top_i && act, G4MI_EINVAL, "moe_gateup: null pointer argument");
  int rc = check_expert_shapes("moe_gateup", N, H, F, E, k);
  if (rc) return rc;
  G4MI_REQUIRE(((uintptr_t)xn & 15u) == 0 && ((uintptr_t)gate_up & 15u) == 0, G4MI_EALIGN,
               "moe_gateup: xn and gate_up must be 16-byte aligned");
  g4mi::dispatch_gateup((int)(H / 256), xn, gate_up, top_w, top_i, (int)N, (int)F, (int)E, (int)k, act,
                        g4mi::as_stream(stream));
  return g4mi::check_launch("moe_gateup");
}

int g4mi_moe_down(const uint16_t* act, const uint16_t* down, const int32_t* top_i, int64_t N, int64_t H,
                  int64_t F, int64_t E, int64_t k, int32_t combine, uint16_t* out, void* stream) {
  G4MI_REQUIRE(act && down && top_i && out, G4MI_EINVAL, "moe_down: null pointer argument");
  int rc = check_expert_shapes("moe_down", N, H, F, E, k);
  if (rc) return rc;
  G4MI_REQUIRE(combine == G4MI_COMBINE_BF16_RUNNING || combine == G4MI_COMBINE_F32, G4MI_EINVAL,
               "moe_down: unknown combine mode %d", combine);
  G4MI_REQUIRE(((uintptr_t)act & 15u) == 0 && ((uintptr_t)down & 15u) == 0, G4MI_EALIGN,
               "moe_down: act and down must be 16-byte aligned");
  g4mi::dispatch_down((int)(F / 64), act, down, top_i, (int)N, (int)H, (int)E, (int)k,
                      combine == G4MI_COMBINE_BF16_RUNNING ? 1 : 0, out, g4mi::as_stream(stream));
  return g4mi::check_launch("moe_down");
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
  G4MI_REQUIRE(((uintptr_t)ws & 15u) == 0, G4MI_EALIGN, "moe_experts_decode: workspace must be 16-byte aligned");
  uint16_t* act = (uint16_t*)ws;
  int rc = g4mi_moe_gateup(xn, gate_up, top_w, top_i, N, H, F, E, k, act, stream);
  if (rc) return rc;
  return g4mi_moe_down(act, down, top_i, N, H, F, E, k, combine, out, stream);
}

}  // extern "C"
