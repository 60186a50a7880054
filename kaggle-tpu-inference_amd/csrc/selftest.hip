// Diagnostics: exercises the cross-lane reduction helpers every kernel relies
// on, so a test can check their lane layout against a host computation.
#include "capi_util.h"
#include "common.h"

namespace g4mi {

// in: 64*nw floats; out: for each wave and each W in {2,4,8,16,32,64} the
// per-lane group sum (f32 and f64) -> out[(w*6 + j)*64 + lane], out_d likewise.
__global__ void selftest_reduce_kernel(const float* __restrict__ in, float* __restrict__ out,
                                       double* __restrict__ out_d) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const float v = in[threadIdx.x];
  const double d = (double)v;
  float r[6];
  double rd[6];
  r[0] = group_sum<2>(v); r[1] = group_sum<4>(v); r[2] = group_sum<8>(v);
  r[3] = group_sum<16>(v); r[4] = group_sum<32>(v); r[5] = group_sum<64>(v);
  rd[0] = group_sum_f64<2>(d); rd[1] = group_sum_f64<4>(d); rd[2] = group_sum_f64<8>(d);
  rd[3] = group_sum_f64<16>(d); rd[4] = group_sum_f64<32>(d); rd[5] = group_sum_f64<64>(d);
  for (int j = 0; j < 6; ++j) {
    out[(w * 6 + j) * 64 + lane] = r[j];
    out_d[(w * 6 + j) * 64 + lane] = rd[j];
  }
}

// exp_nonpos(x) against expf(x) for x = -(the float with bits lo + k),
// k < count: counts the x whose results differ, where below -103.97 (expf's
// zero) a result of at most 2^-149 counts as equal.
__global__ __launch_bounds__(256) void selftest_exp_kernel(uint32_t lo, uint32_t count,
                                                           unsigned long long* __restrict__ mismatches) {
  unsigned long long bad = 0;
  for (uint32_t k = blockIdx.x * 256u + threadIdx.x; k < count; k += gridDim.x * 256u) {
    const float x = -__uint_as_float(lo + k);
    const float a = exp_nonpos(x), b = expf(x);
    bad += !(__float_as_uint(a) == __float_as_uint(b) || (b == 0.0f && a <= 0x1p-149f));
  }
  if (bad != 0) atomicAdd(mismatches, bad);
}

}  // namespace g4mi

extern "C" int g4mi_selftest_exp_nonpositive(int64_t lo, int64_t count, uint64_t* mismatches, void* stream) {
  G4MI_REQUIRE(mismatches, G4MI_EINVAL, "selftest_exp_nonpositive: null pointer");
  G4MI_REQUIRE(lo >= 0 && count >= 1 && lo + count <= 0x7f800000LL, G4MI_EINVAL,
               "selftest_exp_nonpositive: bits [%lld, %lld) are not finite floats", (long long)lo,
               (long long)(lo + count));
  hipLaunchKernelGGL(g4mi::selftest_exp_kernel, dim3(4096), dim3(256), 0, g4mi::as_stream(stream), (uint32_t)lo,
                     (uint32_t)count, (unsigned long long*)mismatches);
  return g4mi::check_launch("selftest_exp_nonpositive");
}

extern "C" int g4mi_selftest_lane_reductions(const float* in, float* out, double* out_d, int32_t waves,
                                             void* stream) {
  G4MI_REQUIRE(in && out && out_d, G4MI_EINVAL, "selftest_lane_reductions: null pointer");
  G4MI_REQUIRE(waves >= 1 && waves <= 16, G4MI_EINVAL, "selftest_lane_reductions: waves in [1,16]");
  hipLaunchKernelGGL(g4mi::selftest_reduce_kernel, dim3(1), dim3(64 * waves), 0, g4mi::as_stream(stream), in, out,
                     out_d);
  return g4mi::check_launch("selftest_lane_reductions");
}
