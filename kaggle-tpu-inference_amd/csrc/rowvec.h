// Length-H bf16 vectors held by one thread block, and the RMSNorm / layer
// tail arithmetic on them (model.py:42-47, model.py:312-322).  Shared by the
// decode GEMV kernels (one vector per block) and the prefill row kernels
// (one token row per block).
#pragma once

#include "common.h"

namespace g4mi {

// A length-H bf16 vector spread over an NT-thread block (H <= 4096): thread
// t owns the 16-byte chunks t + NT*j, j < NC.  Chunks past H/8 are zero, so
// the arithmetic helpers need no bounds checks (a zero chunk stays zero and
// adds nothing to a sum of squares); only stores are masked.
template <int NT>
struct VecT {
  static constexpr int NC = (512 + NT - 1) / NT;
  u32x4 c[NC];
};
using Vec = VecT<256>;

// Branch-free: every lane loads (a clamped chunk past the end) and zeroes
// afterwards.  A load under a branch makes the compiler's s_waitcnt placement
// conservative: it then waits for loads issued after the vector (the weight
// rows) before using it.
template <int NT>
__device__ __forceinline__ void vload(VecT<NT>& v, const uint16_t* __restrict__ p, int nch) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    const int c = threadIdx.x + NT * j;
    const u32x4 t = ld16((const u32x4*)p + min(c, nch - 1));
    v.c[j] = (c < nch) ? t : u32x4{0u, 0u, 0u, 0u};
  }
}
// vload of a vector other blocks of this kernel wrote with coherent stores
template <int NT>
__device__ __forceinline__ void vload_coherent(VecT<NT>& v, const uint16_t* p, int nch) {
  const __amdgpu_buffer_rsrc_t r = buffer_rsrc(p, (uint32_t)nch * 16u);
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    const int c = threadIdx.x + NT * j;
    v.c[j] = coherent_load16(r, (uint32_t)c * 16u);  // out of range reads zero
  }
}
template <int NT>
__device__ __forceinline__ double vsumsq(const VecT<NT>& v) {
  // two accumulators per chunk halve the dependent f64 chain
  double s0 = 0.0, s1 = 0.0;
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    float f[8];
    unpack8(v.c[j], f);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      s0 = fma((double)f[i], (double)f[i], s0);
      s1 = fma((double)f[i + 1], (double)f[i + 1], s1);
    }
  }
  return s0 + s1;
}
// v = bf16(v * r * w)  (w may be null)
template <int NT>
__device__ __forceinline__ void vscale(VecT<NT>& v, float r, const uint16_t* __restrict__ w, int nch) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    if (w != nullptr) {
      const u32x4 wc = ld16((const u32x4*)w + min((int)threadIdx.x + NT * j, nch - 1));
      v.c[j] = scale8(v.c[j], r, &wc);
    } else {
      v.c[j] = scale8(v.c[j], r, nullptr);
    }
  }
}
// a = bf16(a + b)
template <int NT>
__device__ __forceinline__ void vadd(VecT<NT>& a, const VecT<NT>& b) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    float x[8], y[8];
    unpack8(a.c[j], x);
    unpack8(b.c[j], y);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = x[i] + y[i];
    a.c[j].x = pack2(x[0], x[1]); a.c[j].y = pack2(x[2], x[3]);
    a.c[j].z = pack2(x[4], x[5]); a.c[j].w = pack2(x[6], x[7]);
  }
}
// a = bf16(a * s)
template <int NT>
__device__ __forceinline__ void vmul(VecT<NT>& a, float s) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) a.c[j] = scale8(a.c[j], s, nullptr);
}
template <int NT>
__device__ __forceinline__ void vstore(const VecT<NT>& v, u32x4* dst, int nch) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) {
    const int c = threadIdx.x + NT * j;
    if (c < nch) dst[c] = v.c[j];
  }
}
// `red` holds NT/64 doubles.  FRESH: no thread of the block reads `red`
// any more (a region not used before in the kernel), so the barrier that
// orders this round's stores after an earlier round's reads is left out.
template <int NT, bool FRESH = false>
__device__ __forceinline__ double block_sum_nt(double v, double* red) {
  constexpr int NW = NT / 64;
  v = group_sum_f64<kWave>(v);
  if constexpr (!FRESH) __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t += red[i];
  return t;
}
template <int NT, bool FRESH = false>
__device__ __forceinline__ float vrms(const VecT<NT>& v, int H, float eps, double* red) {
  return rms_scale(block_sum_nt<NT, FRESH>(vsumsq(v), red), H, eps);
}

// v = bf16(v * r * w) with the weight already in registers
template <int NT>
__device__ __forceinline__ void vscale_w(VecT<NT>& v, float r, const VecT<NT>& w) {
#pragma unroll
  for (int j = 0; j < VecT<NT>::NC; ++j) v.c[j] = scale8(v.c[j], r, &w.c[j]);
}
// Two block sums in one reduction round (`red`: 2*NT/64 doubles; FRESH as
// in block_sum_nt).
template <int NT, bool FRESH = false>
__device__ __forceinline__ void block_sum2_f64(double& a, double& b, double* red) {
  constexpr int NW = NT / 64;
  a = group_sum_f64<kWave>(a);
  b = group_sum_f64<kWave>(b);
  const int w = threadIdx.x >> 6;
  if constexpr (!FRESH) __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[w] = a;
    red[NW + w] = b;
  }
  __syncthreads();
  double ta = red[0], tb = red[NW];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    ta += red[i];
    tb += red[NW + i];
  }
  a = ta;
  b = tb;
}

// Tail of the previous layer: x = bf16(bf16(x1 + rms(hs, post_ff)) * ls),
// hs = bf16(rms(mlp, post_ff_1) + rms(moe, post_ff_2)), or hs = mlp without MoE.
// All operands are loaded up front (one memory round trip), then two
// dependent reduction rounds follow.  `red`: 3*NT/64 doubles the block has
// not used before (callers keep red[3*NT/64, 4*NT/64) for their next norm).
struct TailArgs {
  const uint16_t *x1, *mlp, *moe, *w_pf1, *w_pf2, *w_pf, *ls;
};
template <int NT>
struct TailRegs {
  VecT<NT> a, b, x1, w1, w2, w3;
  uint16_t ls;
};
// Unconditional loads (see vload): without the MoE block the MoE operands
// are read from the dense ones and ignored.
template <int NT>
__device__ __forceinline__ void tail_load(TailRegs<NT>& T, const TailArgs& t, int nch) {
  const bool moe = t.moe != nullptr;
  vload(T.a, t.mlp, nch);
  vload(T.x1, t.x1, nch);
  vload(T.w3, t.w_pf, nch);
  vload(T.b, moe ? t.moe : t.mlp, nch);
  vload(T.w1, moe ? t.w_pf1 : t.w_pf, nch);
  vload(T.w2, moe ? t.w_pf2 : t.w_pf, nch);
  T.ls = t.ls[0];
}
template <int NT>
__device__ __forceinline__ void tail_compute(VecT<NT>& x, TailRegs<NT>& T, bool moe, int H, float eps, double* red) {
  // each reduction round in a region of its own (red[0, 3*NT/64), fresh):
  // one barrier per round
  constexpr int NW = NT / 64;
  if (moe) {
    double s1 = vsumsq(T.a), s2 = vsumsq(T.b);
    block_sum2_f64<NT, true>(s1, s2, red);
    vscale_w(T.a, rms_scale(s1, H, eps), T.w1);
    vscale_w(T.b, rms_scale(s2, H, eps), T.w2);
    vadd(T.a, T.b);
  }
  vscale_w(T.a, vrms<NT, true>(T.a, H, eps, red + 2 * NW), T.w3);
  x = T.x1;
  vadd(x, T.a);
  vmul(x, bf2f(T.ls));
}

}  // namespace g4mi
