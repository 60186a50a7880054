// Top-k / nucleus sampling of one logits row on the device (model.py:414-424).
//
// The reference: greedy = argmax(logits) (first index of the maximum) when
// temperature <= 0; otherwise v = logits / max(T, 1e-6), keep the top_k
// largest v (jax.lax.top_k: descending, ties to the lower index), p =
// softmax(v), keep entries whose exclusive prefix sum (csum - p) < top_p,
// renormalise and draw one.
//
// Candidates are ranked by a 64-bit key: the order-preserving bits of v in
// the high word and the complement of the index in the low word, so "larger
// key" means "larger value, then lower index", exactly top_k's order, and all
// keys are distinct.  Two reduction kernels keep each block's 64 largest keys
// (every element of the global top-64 is among its block's top-64) until at
// most 1024 remain; a final block sorts those, and one lane does the 64-entry
// softmax, the nucleus cut and the draw.  The uniform comes from
// Philox4x32-10 under the caller's 64-bit seed at counter (step, 0x53414D50,
// 0, 0), where step is the decode position (the reference folds the position
// into its key, engine.py:80) or 0 for the sample after a prefill
// (engine.py:66).  The stream is this library's own, not JAX's.
//
// Like the greedy argmax kernel, the final kernel writes the token and, when
// `pos` is given, advances the device position and records the token in the
// history, so a captured decode step needs no host round trip.
#include "capi_util.h"
#include "common.h"
#include "philox.h"

namespace g4mi {

constexpr int kSortN = 1024;   // keys sorted per block
constexpr int kKeep = 64;      // keys a reduction block keeps (>= top_k)
constexpr uint32_t kSampleTag = 0x53414D50u;

struct SampleParams {
  float temperature;
  float top_p;
  uint64_t seed;
};

__device__ __forceinline__ uint32_t ord_bits(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_ord(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint64_t make_key(float v, int i) {
  if (v != v) return 0ull;  // NaN ranks last
  return ((uint64_t)ord_bits(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}
__device__ __forceinline__ int key_index(uint64_t k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }
__device__ __forceinline__ float key_value(uint64_t k) { return from_ord((uint32_t)(k >> 32)); }

// Descending bitonic sort of kSortN keys in LDS by 256 threads.
__device__ __forceinline__ void sort_desc(uint64_t* s) {
  for (int k = 2; k <= kSortN; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int h = 0; h < kSortN / 2 / 256; ++h) {
        const int q = threadIdx.x + 256 * h;        // pair index
        const int i = 2 * j * (q / j) + (q % j);    // lower element of the pair
        const int l = i + j;
        const uint64_t a = s[i], b = s[l];
        const bool desc = (i & k) == 0;
        if (desc ? (a < b) : (a > b)) {
          s[i] = b;
          s[l] = a;
        }
      }
      __syncthreads();
    }
  }
}

// One reduction stage: block b sorts keys [b*1024, (b+1)*1024) and writes its
// 64 largest to out[b*64 ..].  FROM_LOGITS: the keys are built from logits / t.
template <bool FROM_LOGITS>
__global__ __launch_bounds__(256) void topk_stage_kernel(const float* __restrict__ logits,
                                                         const uint64_t* __restrict__ in, int n,
                                                         const SampleParams* __restrict__ prm,
                                                         uint64_t* __restrict__ out) {
  __shared__ uint64_t s[kSortN];
  const int base = blockIdx.x * kSortN;
  // greedy (temperature <= 0) ranks the raw logits: dividing by 1e-6 could
  // merge neighbouring floats and move the first-index argmax
  const float T = FROM_LOGITS ? prm->temperature : 0.0f;
  const float t = (T > 0.0f) ? fmaxf(T, 1e-6f) : 1.0f;
#pragma unroll
  for (int h = 0; h < kSortN / 256; ++h) {
    const int j = threadIdx.x + 256 * h;
    const int i = base + j;
    uint64_t key = 0ull;
    if (i < n) {
      if constexpr (FROM_LOGITS) key = make_key(logits[i] / t, i);
      else key = in[i];
    }
    s[j] = key;
  }
  __syncthreads();
  sort_desc(s);
  if (threadIdx.x < kKeep) out[(size_t)blockIdx.x * kKeep + threadIdx.x] = s[threadIdx.x];
}

// Final stage: n <= 1024 candidate keys -> token.
__global__ __launch_bounds__(256) void sample_final_kernel(const uint64_t* __restrict__ in, int n, int V, int top_k,
                                                           const SampleParams* __restrict__ prm, int counter_mode,
                                                           int32_t* __restrict__ tok, int32_t* __restrict__ pos,
                                                           int32_t* __restrict__ hist, int hist_len) {
  __shared__ uint64_t s[kSortN];
#pragma unroll
  for (int h = 0; h < kSortN / 256; ++h) {
    const int j = threadIdx.x + 256 * h;
    s[j] = (j < n) ? in[j] : 0ull;
  }
  __syncthreads();
  sort_desc(s);
  if (threadIdx.x != 0) return;
  const SampleParams P = *prm;
  const int K = min(top_k, min(n, V));
  int choice = key_index(s[0]);  // greedy: the largest logit, lowest index on ties
  if (P.temperature > 0.0f && K > 1) {
    float p[kKeep];
    const float m = key_value(s[0]);
    float z = 0.0f;
    for (int i = 0; i < K; ++i) {
      p[i] = expf(key_value(s[i]) - m);
      z += p[i];
    }
    float csum = 0.0f, kept = 0.0f;
    for (int i = 0; i < K; ++i) {
      p[i] /= z;
      csum += p[i];
      if (!(csum - p[i] < P.top_p)) p[i] = 0.0f;  // nucleus cut on the exclusive prefix sum
      kept += p[i];
    }
    const int p0 = (pos != nullptr) ? pos[0] : 0;
    const uint32_t step = counter_mode ? (uint32_t)p0 : 0u;
    const Philox4 r = philox4x32_10(step, kSampleTag, 0u, 0u, (uint32_t)P.seed, (uint32_t)(P.seed >> 32));
    const float u = (float)(r.v[0] >> 8) * (1.0f / 16777216.0f);  // [0, 1)
    const float target = u * kept;
    float acc = 0.0f;
    int last = 0;
    for (int i = 0; i < K; ++i) {
      if (p[i] > 0.0f) {
        last = i;
        acc += p[i];
        if (acc > target) break;
      }
    }
    choice = key_index(s[last]);
  }
  tok[0] = choice;
  if (pos != nullptr) {
    const int np = pos[0] + 1;
    pos[0] = np;
    if (hist != nullptr && np >= 0 && np < hist_len) hist[np] = choice;
  }
}

static int64_t stage_keys(int64_t n) { return ((n + kSortN - 1) / kSortN) * kKeep; }

}  // namespace g4mi

using namespace g4mi;

// ------------------------------------------------------------------ batched head
// Rows b of bf16 logits [B, V] (x . embed^T rounded to bf16, model.py:381):
// v = f32 logit, softcap c*tanh(v/c) when c > 0 (model.py:382-385), optional
// f32 copy, then the first index of the maximum (model.py:416 greedy).  Stage
// 1: grid (kArgParts, B), each block the best (value, index) of its slice of
// the row; stage 2: one block per row reduces the slices and writes tok[b] =
// it; pos[b] += 1; hist[b][pos[b]] = it.
constexpr int kArgParts = 64;

__device__ __forceinline__ void better_vi(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ __launch_bounds__(256) void argmax_rows_part_kernel(const uint16_t* __restrict__ logits, int V, float cap,
                                                               float* __restrict__ out_f32, float* __restrict__ pv,
                                                               int* __restrict__ pi) {
  __shared__ float vs[4];
  __shared__ int is[4];
  const int part = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int span = (V + kArgParts - 1) / kArgParts;
  const int j0 = part * span, j1 = min(V, j0 + span);
  const uint16_t* row = logits + (size_t)b * V;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = j0 + tid; j < j1; j += 256) {
    float v = bf2f(row[j]);
    if (cap > 0.0f) v = tanhf(v / cap) * cap;
    if (out_f32 != nullptr) out_f32[(size_t)b * V + j] = v;
    better_vi(bv, bi, v, j);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) better_vi(bv, bi, __shfl_xor(bv, m, kWave), __shfl_xor(bi, m, kWave));
  if (lane == 0) {
    vs[wave] = bv;
    is[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) better_vi(bv, bi, vs[w], is[w]);
    pv[b * kArgParts + part] = bv;
    pi[b * kArgParts + part] = bi;
  }
}

__global__ __launch_bounds__(64) void argmax_rows_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                               int32_t* tok, int32_t* pos, int32_t* hist,
                                                               int hist_len) {
  const int b = blockIdx.x, lane = threadIdx.x;
  float bv = pv[b * kArgParts + lane];
  int bi = pi[b * kArgParts + lane];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) better_vi(bv, bi, __shfl_xor(bv, m, kWave), __shfl_xor(bi, m, kWave));
  if (lane == 0) {
    bi = (bi == 0x7fffffff) ? 0 : bi;
    tok[b] = bi;
    if (pos != nullptr) {
      const int p = pos[b] + 1;
      pos[b] = p;
      if (hist != nullptr && p >= 0 && p < hist_len) hist[(size_t)b * hist_len + p] = bi;
    }
  }
}

extern "C" {

int64_t g4mi_argmax_rows_workspace_bytes(int64_t B) { return B * kArgParts * 8; }

int g4mi_argmax_rows(const uint16_t* logits, int64_t B, int64_t V, float softcap, float* logits_f32, int32_t* tok,
                     int32_t* pos, int32_t* hist, int64_t hist_len, void* ws, int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(logits && tok && B >= 1 && B <= 65535 && V >= 1 && V <= 2147483647, G4MI_EINVAL,
               "argmax_rows: bad arguments (B=%lld V=%lld)", (long long)B, (long long)V);
  G4MI_REQUIRE(hist == nullptr || (pos && hist_len >= 1), G4MI_EINVAL, "argmax_rows: hist needs pos and hist_len");
  G4MI_REQUIRE(ws && ws_bytes >= g4mi_argmax_rows_workspace_bytes(B), G4MI_EWORKSPACE,
               "argmax_rows: workspace too small");
  float* pv = (float*)ws;
  int* pi = (int*)((char*)ws + B * kArgParts * 4);
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(argmax_rows_part_kernel, dim3(kArgParts, (unsigned)B), dim3(256), 0, st, logits, (int)V,
                     softcap, logits_f32, pv, pi);
  int rc = check_launch("argmax_rows (slices)");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_rows_final_kernel, dim3((unsigned)B), dim3(64), 0, st, pv, pi, tok, pos, hist,
                     (int)hist_len);
  return check_launch("argmax_rows");
}


int64_t g4mi_sample_workspace_bytes(int64_t V) {
  const int64_t a = stage_keys(V);
  return 2 * ((a * 8 + 255) / 256) * 256;
}

int g4mi_sample(const float* logits, int64_t V, int64_t top_k, const void* params, int32_t counter_mode,
                int32_t* tok, int32_t* pos, int32_t* hist, int64_t hist_len, void* ws, int64_t ws_bytes,
                void* stream) {
  G4MI_REQUIRE(logits && params && tok && ws, G4MI_EINVAL, "sample: null pointer argument");
  G4MI_REQUIRE(V >= 1 && V <= ((int64_t)1 << 30), G4MI_EINVAL, "sample: bad vocab %lld", (long long)V);
  G4MI_REQUIRE(top_k >= 1 && top_k <= kKeep, G4MI_EUNSUPPORTED, "sample: top_k %lld not in [1, %d]",
               (long long)top_k, kKeep);
  G4MI_REQUIRE(ws_bytes >= g4mi_sample_workspace_bytes(V), G4MI_EWORKSPACE, "sample: workspace too small");
  G4MI_REQUIRE(((uintptr_t)params & 7u) == 0 && ((uintptr_t)ws & 7u) == 0, G4MI_EALIGN,
               "sample: params and workspace must be 8-byte aligned");
  hipStream_t st = as_stream(stream);
  const SampleParams* prm = (const SampleParams*)params;
  uint64_t* buf[2];
  buf[0] = (uint64_t*)ws;
  buf[1] = (uint64_t*)((char*)ws + g4mi_sample_workspace_bytes(V) / 2);
  int64_t n = V;
  int cur = 0;
  bool from_logits = true;
  // reduce until the candidates fit one final block
  while (from_logits || n > kSortN) {
    const int64_t blocks = (n + kSortN - 1) / kSortN;
    if (from_logits)
      hipLaunchKernelGGL((topk_stage_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, st, logits, nullptr,
                         (int)n, prm, buf[cur]);
    else
      hipLaunchKernelGGL((topk_stage_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, st, nullptr,
                         buf[cur ^ 1], (int)n, prm, buf[cur]);
    n = blocks * kKeep;
    cur ^= 1;
    from_logits = false;
  }
  hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(256), 0, st, buf[cur ^ 1], (int)n, (int)V, (int)top_k, prm,
                     counter_mode, tok, pos, hist, (int)hist_len);
  return check_launch("sample");
}

}  // extern "C"
