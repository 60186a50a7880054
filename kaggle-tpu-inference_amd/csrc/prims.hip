// The reference model's standalone primitives (model.py:42-78): rms_norm,
// gelu, rope_tables and apply_rope, for callers that use them outside a
// decode step.  The decode and prefill kernels fuse the same arithmetic into
// their prologues; these follow the same rounding recipe:
//   rms_norm:   out = cast(f32(x) * r * f32(w)), r = f32(1/sqrt(f64(mean + eps))),
//               mean = f32(sum of squares, exact in f64) / dim;
//   gelu:       the tanh approximation in f32, one rounding to x's dtype;
//   rope_tables: angle = f32(pos) * inv_freq (an f32 product), cos/sin of that
//               f32 angle evaluated in f64 and rounded to f32, halves duplicated;
//   apply_rope: c = cast(cos), s = cast(sin) to x's dtype; x*c and rot*s
//               rounded to x's dtype, then their sum (bf16 elementwise ops).
// Tensors are bf16 (dtype code 0) or f32 (dtype code 1).  Not on the decode
// path: these are simple grid-stride kernels.
#include "capi_util.h"
#include "common.h"

namespace g4mi {

__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int is_f32) {
  return is_f32 ? ((const float*)p)[i] : bf2f(((const uint16_t*)p)[i]);
}
__device__ __forceinline__ float round_to(float v, int is_f32) { return is_f32 ? v : rbf(v); }
__device__ __forceinline__ void store_as(void* p, int64_t i, float v, int is_f32) {
  if (is_f32)
    ((float*)p)[i] = v;
  else
    ((uint16_t*)p)[i] = f2bf(v);
}

// One block per row: exact f64 sum of squares, then the scaled row.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const void* __restrict__ x, int x_f32,
                                                            const void* __restrict__ w, int w_f32, int dim,
                                                            float eps, void* __restrict__ out) {
  __shared__ double red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * (int64_t)dim;
  double ss = 0.0;
  for (int i = threadIdx.x; i < dim; i += 256) {
    const double v = (double)load_as_f32(x, base + i, x_f32);
    ss = fma(v, v, ss);
  }
  const float r = rms_scale(block_sum_f64(ss, red), dim, eps);
  for (int i = threadIdx.x; i < dim; i += 256) {
    float v = load_as_f32(x, base + i, x_f32) * r;
    if (w != nullptr) v = v * load_as_f32(w, i, w_f32);
    store_as(out, base + i, v, x_f32);
  }
}

__global__ __launch_bounds__(256) void gelu_kernel(const void* __restrict__ x, int x_f32, int64_t n,
                                                   void* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    store_as(out, i, gelu_tanh(load_as_f32(x, i, x_f32)), x_f32);
}

// cos/sin [T, 2*half]: entry (t, j) and (t, j + half) hold the value of pair j.
__global__ __launch_bounds__(256) void rope_tables_kernel(const int32_t* __restrict__ pos, int64_t T,
                                                          const float* __restrict__ inv_freq, int half,
                                                          float* __restrict__ cos_out, float* __restrict__ sin_out) {
  const int64_t n = T * half;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / half;
    const int j = (int)(i % half);
    const float ang = (float)pos[t] * inv_freq[j];
    const float c = f32_of(cos((double)ang)), s = f32_of(sin((double)ang));
    const int64_t o = t * 2 * half + j;
    cos_out[o] = c;
    cos_out[o + half] = c;
    sin_out[o] = s;
    sin_out[o + half] = s;
  }
}

// x [B, T, inner, D] (inner = the product of the head axes); cos/sin [T, D] f32.
__global__ __launch_bounds__(256) void apply_rope_kernel(const void* __restrict__ x, int x_f32, int64_t T,
                                                         int64_t inner, int D, const float* __restrict__ cs,
                                                         const float* __restrict__ sn, int64_t n,
                                                         void* __restrict__ out) {
  const int half = D / 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int d = (int)(i % D);
    const int64_t t = (i / ((int64_t)D * inner)) % T;
    const float xv = load_as_f32(x, i, x_f32);
    const float partner = load_as_f32(x, d < half ? i + half : i - half, x_f32);
    const float rot = d < half ? -partner : partner;
    const float c = round_to(cs[t * D + d], x_f32), s = round_to(sn[t * D + d], x_f32);
    const float a = round_to(xv * c, x_f32), b = round_to(rot * s, x_f32);
    store_as(out, i, a + b, x_f32);
  }
}

static unsigned grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int g4mi_rms_norm(const void* x, int32_t x_f32, const void* w, int32_t w_f32, int64_t rows, int64_t dim, float eps,
                  void* out, void* stream) {
  G4MI_REQUIRE(x && out, G4MI_EINVAL, "rms_norm: null pointer argument");
  G4MI_REQUIRE(rows >= 0 && rows <= 0x7fffffff && dim >= 1 && dim <= (1 << 24), G4MI_EINVAL,
               "rms_norm: bad rows=%lld dim=%lld", (long long)rows, (long long)dim);
  if (rows == 0) return 0;
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), x, x_f32 ? 1 : 0,
                     w, w_f32 ? 1 : 0, (int)dim, eps, out);
  return check_launch("rms_norm");
}

int g4mi_gelu_tanh(const void* x, int32_t x_f32, int64_t n, void* out, void* stream) {
  G4MI_REQUIRE(x && out, G4MI_EINVAL, "gelu_tanh: null pointer argument");
  G4MI_REQUIRE(n >= 0, G4MI_EINVAL, "gelu_tanh: negative size");
  if (n == 0) return 0;
  hipLaunchKernelGGL(gelu_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), x, x_f32 ? 1 : 0, n, out);
  return check_launch("gelu_tanh");
}

int g4mi_rope_tables(const int32_t* positions, int64_t T, const float* inv_freq, int64_t half, float* cos_out,
                     float* sin_out, void* stream) {
  G4MI_REQUIRE(positions && inv_freq && cos_out && sin_out, G4MI_EINVAL, "rope_tables: null pointer argument");
  G4MI_REQUIRE(T >= 0 && half >= 1 && half <= (1 << 20), G4MI_EINVAL, "rope_tables: bad T/half");
  if (T == 0) return 0;
  hipLaunchKernelGGL(rope_tables_kernel, dim3(grid_for(T * half)), dim3(256), 0, as_stream(stream), positions, T,
                     inv_freq, (int)half, cos_out, sin_out);
  return check_launch("rope_tables");
}

int g4mi_apply_rope(const void* x, int32_t x_f32, const float* rope_cos, const float* rope_sin, int64_t B, int64_t T,
                    int64_t inner, int64_t D, void* out, void* stream) {
  G4MI_REQUIRE(x && rope_cos && rope_sin && out, G4MI_EINVAL, "apply_rope: null pointer argument");
  G4MI_REQUIRE(B >= 0 && T >= 0 && inner >= 1 && D >= 2 && D % 2 == 0 && D <= (1 << 20), G4MI_EINVAL,
               "apply_rope: bad B/T/inner/D");
  const int64_t n = B * T * inner * D;
  if (n == 0) return 0;
  G4MI_REQUIRE(x != out, G4MI_EINVAL, "apply_rope: out must not alias x");
  hipLaunchKernelGGL(apply_rope_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), x, x_f32 ? 1 : 0, T,
                     inner, (int)D, rope_cos, rope_sin, n, out);
  return check_launch("apply_rope");
}

}  // extern "C"
