// Plain dense products of the batched prefill through the ROCm library GEMM
// (rocBLAS, bf16 in, f32 accumulate), and the gated activation that follows
// the separate gate and up products.  The fused, grouped and skinny products
// stay on the hand-written MFMA kernels (gemm.hip); these are the unfused
// q/k/v/o/down projections and the dense MLP's gate and up rows, where the
// library's tuned tiles and stream-K scheduling beat a fixed 128x128 tiling
// on the 256-CU grid.
#include <rocblas/rocblas.h>

#include <mutex>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

constexpr int kMaxDevices = 64;
static std::mutex g_blas_mu;
static rocblas_handle g_blas[kMaxDevices];

// One handle per device, created on first use with atomics disallowed (the
// library then picks only solutions whose result does not depend on the
// order in which blocks finish).
static rocblas_handle blas_handle(int dev) {
  std::lock_guard<std::mutex> lk(g_blas_mu);
  if (g_blas[dev] == nullptr) {
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
    if (rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed) != rocblas_status_success) {
      rocblas_destroy_handle(h);
      return nullptr;
    }
    g_blas[dev] = h;
  }
  return g_blas[dev];
}

// act = bf16(bf16(gelu_tanh(g)) * u) for bf16 g, u (model.py:220): the gated
// GEMM epilogue's arithmetic on products already rounded to bf16.
__global__ __launch_bounds__(256) void gated_act_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                        int64_t n8, uint16_t* __restrict__ act) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const u32x4 gv = ((const u32x4*)g)[i], uv = ((const u32x4*)u)[i];
  float gf[8], uf[8];
  unpack8(gv, gf);
  unpack8(uv, uf);
#pragma unroll
  for (int q = 0; q < 8; ++q) gf[q] = rbf(rbf(gelu_tanh(gf[q])) * uf[q]);
  u32x4 o;
  o.x = pack2(gf[0], gf[1]); o.y = pack2(gf[2], gf[3]); o.z = pack2(gf[4], gf[5]); o.w = pack2(gf[6], gf[7]);
  ((u32x4*)act)[i] = o;
}

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int g4mi_gemm_bf16_library(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t M, int64_t N,
                           int64_t K, int32_t f32_out, void* c, int64_t ldc, void* stream) {
  G4MI_REQUIRE(a && b && c && M >= 1 && N >= 1 && K >= 1, G4MI_EINVAL, "gemm_library: missing argument");
  G4MI_REQUIRE(M <= 2147483647 && N <= 2147483647 && K <= 2147483647 && lda >= K && ldb >= K && ldc >= N,
               G4MI_EINVAL, "gemm_library: bad sizes or strides");
  int dev = 0;
  G4MI_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, G4MI_EINVAL,
               "gemm_library: no current device");
  rocblas_handle h = blas_handle(dev);
  G4MI_REQUIRE(h != nullptr, G4MI_EUNSUPPORTED, "gemm_library: rocBLAS handle creation failed");
  G4MI_REQUIRE(rocblas_set_stream(h, as_stream(stream)) == rocblas_status_success, G4MI_EINVAL,
               "gemm_library: rocblas_set_stream failed");
  const float alpha = 1.0f, beta = 0.0f;
  const rocblas_datatype ct = f32_out ? rocblas_datatype_f32_r : rocblas_datatype_bf16_r;
  // row-major C[M,N] = A[M,K] . B[N,K]^T is column-major C^T = op(B^T)^T . A^T
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)N, (rocblas_int)M, (rocblas_int)K, &alpha,
      b, rocblas_datatype_bf16_r, (rocblas_int)ldb, a, rocblas_datatype_bf16_r, (rocblas_int)lda, &beta, c, ct,
      (rocblas_int)ldc, c, ct, (rocblas_int)ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  G4MI_REQUIRE(st == rocblas_status_success, G4MI_EUNSUPPORTED, "gemm_library: rocblas_gemm_ex returned %d", (int)st);
  return check_launch("gemm_library");
}

int g4mi_gated_act(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* act, void* stream) {
  G4MI_REQUIRE(g && u && act && n >= 8 && n % 8 == 0, G4MI_EINVAL, "gated_act: n=%lld must be a positive multiple of 8",
               (long long)n);
  G4MI_REQUIRE(((uintptr_t)g & 15u) == 0 && ((uintptr_t)u & 15u) == 0 && ((uintptr_t)act & 15u) == 0, G4MI_EALIGN,
               "gated_act: operands must be 16-byte aligned");
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(gated_act_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, as_stream(stream), g, u, n8,
                     act);
  return check_launch("gated_act");
}

}  // extern "C"
