// Deterministic N(0, std) bf16 initialisation of weight tensors on the GPU.
//
// Element i of a tensor is drawn from the Philox4x32-10 block at counter
// (i/2 lo, i/2 hi, 0, 0) under the tensor's 64-bit key; words 0 and 1 feed a
// Box-Muller transform evaluated in f64, whose cosine branch gives the even
// element and whose sine branch gives the odd one.  The value std*z is
// rounded f64 -> f32 -> bf16 (nearest even).  The CPU oracle restates the
// same generator in numpy, so small models can be checked element by element.
#include "capi_util.h"
#include "common.h"
#include "philox.h"

namespace g4mi {

__global__ __launch_bounds__(256) void fill_normal_bf16_kernel(uint16_t* __restrict__ out, int64_t n,
                                                               uint32_t k0, uint32_t k1, double stdv) {
  const int64_t npairs = (n + 1) >> 1;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < npairs;
       j += (int64_t)gridDim.x * blockDim.x) {
    Philox4 r = philox4x32_10((uint32_t)j, (uint32_t)((uint64_t)j >> 32), 0u, 0u, k0, k1);
    const double two32 = 4294967296.0;
    const double u1 = ((double)r.v[0] + 1.0) / two32;  // (0, 1]
    const double u2 = (double)r.v[1] / two32;          // [0, 1)
    const double rad = sqrt(-2.0 * log(u1));
    const double ang = 6.283185307179586476925286766559 * u2;
    const double z0 = rad * cos(ang), z1 = rad * sin(ang);
    const uint16_t b0 = f2bf(f32_of(stdv * z0));
    const uint16_t b1 = f2bf(f32_of(stdv * z1));
    const int64_t i = 2 * j;
    if (i + 1 < n) {
      // i is even: the pair is 4-byte aligned when `out` is.
      *(uint32_t*)(out + i) = (uint32_t)b0 | ((uint32_t)b1 << 16);
    } else {
      out[i] = b0;
    }
  }
}

__global__ void philox_block_kernel(const uint32_t* __restrict__ ctr, uint32_t k0, uint32_t k1,
                                    uint32_t* __restrict__ out, int64_t nblocks) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= nblocks) return;
  Philox4 r = philox4x32_10(ctr[4 * j], ctr[4 * j + 1], ctr[4 * j + 2], ctr[4 * j + 3], k0, k1);
  for (int q = 0; q < 4; ++q) out[4 * j + q] = r.v[q];
}

}  // namespace g4mi

extern "C" {

int g4mi_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t key, double stdv, void* stream) {
  G4MI_REQUIRE(out != nullptr || n == 0, G4MI_EINVAL, "fill_normal_bf16: null output");
  G4MI_REQUIRE(n >= 0, G4MI_EINVAL, "fill_normal_bf16: negative length %lld", (long long)n);
  G4MI_REQUIRE(((uintptr_t)out & 3u) == 0, G4MI_EALIGN, "fill_normal_bf16: output not 4-byte aligned");
  if (n == 0) return 0;
  const int64_t npairs = (n + 1) >> 1;
  int64_t blocks = (npairs + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(g4mi::fill_normal_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     g4mi::as_stream(stream), out, n, (uint32_t)key, (uint32_t)(key >> 32), stdv);
  return g4mi::check_launch("fill_normal_bf16");
}

int g4mi_philox4x32_10(const uint32_t* ctr, uint64_t key, uint32_t* out, int64_t nblocks, void* stream) {
  G4MI_REQUIRE(nblocks >= 0, G4MI_EINVAL, "philox4x32_10: negative count");
  if (nblocks == 0) return 0;
  G4MI_REQUIRE(ctr && out, G4MI_EINVAL, "philox4x32_10: null pointer");
  const int64_t blocks = (nblocks + 255) / 256;
  hipLaunchKernelGGL(g4mi::philox_block_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     g4mi::as_stream(stream), ctr, (uint32_t)key, (uint32_t)(key >> 32), out, nblocks);
  return g4mi::check_launch("philox4x32_10");
}

}  // extern "C"
