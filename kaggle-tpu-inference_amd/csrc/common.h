// Shared device helpers for the gfx950 kernels of libg4mi.
//
// bf16 values travel as raw uint16_t (the upper half of an IEEE f32).  All
// arithmetic happens in f32 (or f64 where a result must be independent of the
// reduction order) and is rounded back to bf16 round-to-nearest-even at the
// points where the JAX reference materialises a bf16 tensor.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>
#include <stdint.h>

namespace g4mi {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));  // MFMA bf16 operand (16 bytes)
typedef float f32x4 __attribute__((ext_vector_type(4)));    // MFMA 16x16 accumulator per lane

constexpr int kWave = 64;

// ------------------------------------------------------------------ bf16 <-> f32
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }

// f32 -> bf16, round to nearest even (gfx950's v_cvt_pk_bf16_f32; NaN stays
// a quiet NaN).  One instruction converts a pair.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// Round an f32 to the nearest bf16 and return it as f32.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// exp(x) for x <= 0 with expf's rounding on [-103.97, 0]: x * log2(e) as the
// unevaluated sum hi + lo (hi = RN(x * L2E), lo = fma(x, L2E, -hi) +
// x * L2E_LO, where L2E + L2E_LO = log2(e) to 48 bits), n = rne(hi), then
// 2^(hi - n + lo) on the hardware exp2, scaled by 2^n.  expf's range checks
// are left out: x <= 0 cannot overflow, and below -103.97 this returns at
// most 2^-149 where expf returns 0 (the softmax callers round probabilities
// to bf16, whose smallest value is 2^-133, and add exps to sums that hold
// exp(0) = 1).  -inf gives NaN: callers select 0 for masked scores.
__device__ __forceinline__ float exp_nonpos(float x) {
#pragma clang fp contract(off)  // hi - n must not become fma(x, L2E, -n)
  constexpr float kL2E = 0x1.715476p+0f, kL2ELo = 0x1.4ae0bep-26f;
  const float hi = x * kL2E;
  const float lo = __builtin_fmaf(x, kL2ELo, __builtin_fmaf(x, kL2E, -hi));
  const float n = __builtin_rintf(hi);
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((hi - n) + lo), (int)n);
}
// f64 -> f32, kept opaque: the reference rounds f64 results to f32 first, and
// without the barrier the compiler fuses f64 -> f32 -> bf16 into a single
// f64 -> bf16 rounding, which differs in rare halfway cases.
__device__ __forceinline__ float f32_of(double d) {
  float f = (float)d;
  asm volatile("" : "+v"(f));
  return f;
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 in a 16-byte vector -> 8 f32.
__device__ __forceinline__ void unpack8(const u32x4 v, float* f) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

// f32 dot of 8 bf16 pairs, accumulated into acc pairwise in element order
// with v_dot2c_f32_bf16: each step adds two exact bf16 products to acc (one
// instruction per 4 bytes of each operand instead of unpacking and two FMAs;
// measured on gfx950: within 2^-23 of the sum of magnitudes of the exact
// result, round to nearest, like two chained FMAs).
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc, false);
}
__device__ __forceinline__ float dot8(const u32x4 a, const u32x4 b, float acc) {
  acc = dot2bf(a.x, b.x, acc);
  acc = dot2bf(a.y, b.y, acc);
  acc = dot2bf(a.z, b.z, acc);
  acc = dot2bf(a.w, b.w, acc);
  return acc;
}

// f64 dot of 8 bf16 pairs.  Every bf16*bf16 product is exact in f64 and, for
// operands within ~2^37 of each other in magnitude, so is every partial sum:
// the result does not depend on the order in which lanes are combined.
__device__ __forceinline__ double dot8_f64(const u32x4 a, const u32x4 b, double acc) {
  acc = fma((double)bf_lo(a.x), (double)bf_lo(b.x), acc); acc = fma((double)bf_hi(a.x), (double)bf_hi(b.x), acc);
  acc = fma((double)bf_lo(a.y), (double)bf_lo(b.y), acc); acc = fma((double)bf_hi(a.y), (double)bf_hi(b.y), acc);
  acc = fma((double)bf_lo(a.z), (double)bf_lo(b.z), acc); acc = fma((double)bf_hi(a.z), (double)bf_hi(b.z), acc);
  acc = fma((double)bf_lo(a.w), (double)bf_lo(b.w), acc); acc = fma((double)bf_hi(a.w), (double)bf_hi(b.w), acc);
  return acc;
}

__device__ __forceinline__ double sumsq8_f64(const u32x4 a, double acc) {
  float f[8];
  unpack8(a, f);
#pragma unroll
  for (int i = 0; i < 8; ++i) acc = fma((double)f[i], (double)f[i], acc);
  return acc;
}

// ------------------------------------------------------------------ loads
// Weights are streamed once per token: mark them non-temporal so they do not
// evict the activations and KV pages that are re-read.
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }

// The wave's index in its block as a scalar: every lane of a wave has the
// same threadIdx.x >> 6, and saying so keeps loops and branches on it
// uniform (scalar branches; no exec-masked loops whose loads the compiler
// sinks into divergent blocks behind a full vmcnt(0) wait).
// f(integral_constant<int, i>) for i = 0 .. N-1
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// A block barrier for data exchanged through LDS alone.  __syncthreads()
// also waits for every global load the wave has in flight (its workgroup
// fence drains vmcnt), so rows requested ahead of it would all have to
// arrive before any wave passes; this waits only for the wave's LDS
// operations, and each load in flight is waited for where its registers are
// first used.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// The XCD (0..7) running the calling wave (hardware register XCC_ID).
__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 15; }

// Whether every launch on this device runs block b on the XCD of block
// b % 8, 8 consecutive blocks on 8 different XCDs (checked once per device,
// outside graph capture; xcd.hip).  Blocks b, b + 8, b + 16, ... of such a
// launch share one L2 and may pass data through it with plain stores and
// loads.
bool xcc_round_robin(hipStream_t st);
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }

// ------------------------------------------------------------------ reductions
// Cross-lane sums: DPP quad/mirror moves inside a row of 16 lanes (no LDS
// round trip), then one ds_bpermute per step across rows.  Every lane of a
// group ends with the same, bitwise identical, total (IEEE add commutes).
// (The gfx950 permlane16/32_swap builtins are avoided: with both operands the
// same value the compiler drops the swapped-out second result.)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
constexpr int kDppXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// Sum over aligned groups of W consecutive lanes (W in {1,2,4,...,64}).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 2) v += dpp_f<kDppXor1>(v);
  if constexpr (W >= 4) v += dpp_f<kDppXor2>(v);
  if constexpr (W >= 8) v += dpp_f<kDppHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_f<kDppMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}
template <int W>
__device__ __forceinline__ double group_sum_f64(double v) {
  if constexpr (W >= 2) v += dpp_d<kDppXor1>(v);
  if constexpr (W >= 4) v += dpp_d<kDppXor2>(v);
  if constexpr (W >= 8) v += dpp_d<kDppHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_d<kDppMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = W / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Block-wide f64 sum (exact inputs => order-independent result).  `red` must
// hold blockDim.x/64 doubles of LDS.  All threads receive the total.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = group_sum_f64<kWave>(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// ------------------------------------------------------------------ RMSNorm
// The RMSNorm scale of the reference (model.py rms_norm): x * rsqrt(mean(x^2)+eps)
// with mean/eps in f32.  The sum of squares is exact (f64) and the reciprocal
// square root is taken in f64 and rounded once, so the CPU oracle and every
// wave that recomputes it agree bit for bit.
__device__ __forceinline__ float rms_scale(double sumsq, int n, float eps) {
  float mean = (float)sumsq / (float)n;
  float a = mean + eps;
  return (float)(1.0 / sqrt((double)a));
}

// out = bf16(x * r * w) elementwise on 8 packed bf16 (w may be null: weight 1).
__device__ __forceinline__ u32x4 scale8(const u32x4 x, float r, const u32x4* w) {
  float f[8];
  unpack8(x, f);
  if (w != nullptr) {
    float g[8];
    unpack8(*w, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = f[i] * r * g[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = f[i] * r;
  }
  u32x4 o;
  o.x = pack2(f[0], f[1]); o.y = pack2(f[2], f[3]); o.z = pack2(f[4], f[5]); o.w = pack2(f[6], f[7]);
  return o;
}

// ------------------------------------------------------------------ activations
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float x3 = x * x * x;
  const float cdf = 0.5f * (1.0f + tanhf(k0 * (x + 0.044715f * x3)));
  return x * cdf;
}

// Cross-block hand-off inside one kernel without flushing the L2 caches.
// On gfx950 each XCD has its own L2; a __threadfence() writes back and
// invalidates the whole L2 of the calling XCD, which costs microseconds.
// Data that another block will read is instead written and read with
// device-scope (sc1) buffer stores and loads, coherent across the XCD L2s by
// themselves (the gfx94x/gfx950 memory model emits the same sc1 accesses for
// agent-scope atomics).  arrive_last() waits until the block's own stores
// have completed (s_waitcnt vmcnt(0)), then counts the block in; the block
// that brings the count to `total` gets true, resets the counter for the
// next launch or graph replay, and may then read every block's coherent
// stores with coherent_load4.  Buffer accesses outside the resource's range
// read zero and write nothing.
constexpr int kCPolSC1 = 16;  // cache-policy bit: device scope
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void coherent_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
  u32x4 w;
  w.x = __float_as_uint(v.x); w.y = __float_as_uint(v.y); w.z = __float_as_uint(v.z); w.w = __float_as_uint(v.w);
  __builtin_amdgcn_raw_buffer_store_b128(w, r, byte_off, 0, kCPolSC1);
}
// An ordinary (L2 write-back) 16-byte buffer store, for data read only by
// later launches.
__device__ __forceinline__ void store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
  u32x4 w;
  w.x = __float_as_uint(v.x); w.y = __float_as_uint(v.y); w.z = __float_as_uint(v.z); w.w = __float_as_uint(v.w);
  __builtin_amdgcn_raw_buffer_store_b128(w, r, byte_off, 0, 0);
}
__device__ __forceinline__ u32x4 coherent_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCPolSC1);
}
__device__ __forceinline__ void coherent_store_bf16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 coherent_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCPolSC1);
  return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
}
__device__ __forceinline__ bool arrive_last(unsigned int* counter, unsigned int total, int* flag_lds) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev = atomicAdd(counter, 1u);
    const int last = (prev == total - 1);
    if (last) atomicExch(counter, 0u);
    *flag_lds = last;
  }
  __syncthreads();
  return *flag_lds != 0;
}

// arrive_last for a large grid: device-scope atomics on one address
// serialise (~20 ns each), so blocks first arrive on their group's counter
// (kArriveGroup consecutive blocks, counters 128 bytes apart) and the last of
// each group on the top counter.  counters: 1 + 32 * ceil(gridDim.x / 32)
// words, zero between launches (each launch leaves them at zero).
constexpr int kArriveGroup = 32;
constexpr int kArriveStride = 32;  // words between group counters
__device__ __forceinline__ bool arrive_last_grid(unsigned int* counters, int* flag_lds) {
  const unsigned int nb = gridDim.x, grp = blockIdx.x / kArriveGroup;
  const unsigned int ng = (nb + kArriveGroup - 1) / kArriveGroup;
  const unsigned int gsz = min((unsigned int)kArriveGroup, nb - grp * kArriveGroup);
  if (!arrive_last(counters + kArriveStride * (1 + grp), gsz, flag_lds)) return false;
  return arrive_last(counters, ng, flag_lds);
}

}  // namespace g4mi
