// The dispatcher's block -> XCD map (gfx950: 8 XCDs, each with its own L2).
// Kernels whose blocks pass data through one XCD's L2 (plain stores and
// loads instead of device-scope ones) rely on block b running on the XCD of
// block b % 8; xcc_round_robin() checks that once per device.
#include <mutex>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

// The blocks of the check record their XCD in a file-scope array (no
// allocation).
constexpr int kXccProbeBlocks = 1024;
__device__ int xcc_probe[kXccProbeBlocks];
static __global__ void xcc_map_kernel(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// Whether this device runs block b of every launch on the XCD of block b % 8,
// with 8 consecutive blocks on 8 different XCDs (the dispatcher's round
// robin), checked once per device by recording each block's XCD for two
// launches (the first of 13 blocks, so a dispatcher that continued its
// round robin across launches would show).  Not checked while `st` is being
// captured into a graph (the check copies to the host): the caller then takes
// its path without the L2 hand-off, and the check runs at the next call
// outside a capture.
static std::mutex g_xcc_mu;
static int g_xcc_state[64];  // 0 unknown, 1 round robin, -1 not
bool xcc_round_robin(hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lock(g_xcc_mu);
  if (g_xcc_state[dev] != 0) return g_xcc_state[dev] > 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  constexpr int n = kXccProbeBlocks;
  int* d = nullptr;
  if (hipGetSymbolAddress((void**)&d, HIP_SYMBOL(xcc_probe)) != hipSuccess || d == nullptr) {
    (void)hipGetLastError();
    return false;
  }
  int h[n];
  bool ok = true;
  for (int rep = 0; rep < 2 && ok; ++rep) {
    const int nb = rep == 0 ? 13 : n;
    hipLaunchKernelGGL(xcc_map_kernel, dim3((unsigned)nb), dim3(64), 0, st, d);
    ok = hipMemcpyAsync(h, d, nb * sizeof(int), hipMemcpyDeviceToHost, st) == hipSuccess &&
         hipStreamSynchronize(st) == hipSuccess;
    bool seen[16] = {};
    for (int b = 0; ok && b < nb; ++b) {
      ok = h[b] >= 0 && h[b] < 8 && h[b] == h[b % 8];
      if (ok && b < 8) {
        ok = !seen[h[b]];
        seen[h[b]] = true;
      }
    }
    ok = ok && nb >= 8;
    if (rep == 0) ok = true;  // the 13-block launch only shifts a round robin that carries over
  }
  (void)hipGetLastError();
  g_xcc_state[dev] = ok ? 1 : -1;
  return ok;
}

}  // namespace g4mi
