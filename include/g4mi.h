/*
 * libg4mi — MI355X (gfx950) kernels for the Gemma-4 MoE decode hot path.
 *
 * Plain C ABI: raw device pointers, int64 sizes, an explicit HIP stream passed
 * as void* (NULL = the default stream).  bf16 tensors are passed as uint16_t*
 * holding the upper 16 bits of an IEEE f32.  No entry point allocates or frees
 * memory: scratch space is a caller-owned device buffer whose size the
 * matching *_workspace_bytes() function returns, zero-filled once by the
 * caller before its first use (every kernel leaves it reusable).
 *
 * Return value: 0 on success, a negative G4MI_E* code when an argument is
 * rejected (nothing is launched), or the positive hipError_t of a failed
 * launch.  g4mi_last_error_string() describes the last failure of the
 * calling thread.  Work is stream-ordered; entry points keep no state between
 * calls, and calls that share a workspace must be ordered on one stream.
 *
 * Every entry point names the reference function (YLiu95/kaggle-tpu-inference,
 * JAX) whose semantics it reproduces.
 */
#ifndef G4MI_H_
#define G4MI_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4MI_ABI_VERSION 1

#define G4MI_EINVAL (-1)      /* bad argument (null pointer, size out of range) */
#define G4MI_EALIGN (-2)      /* a pointer is not aligned as the kernel requires */
#define G4MI_EWORKSPACE (-3)  /* workspace smaller than *_workspace_bytes() */
#define G4MI_EUNSUPPORTED (-4) /* shape has no kernel instance */

/* Expert-combine modes of g4mi_moe_experts_decode. */
#define G4MI_COMBINE_BF16_RUNNING 0 /* bf16 running sum in top-k order: model.py:289-293 (decode) */
#define G4MI_COMBINE_F32 1          /* one f32 contraction over experts: model.py:250 (dense prefill) */

int g4mi_version(void);
const char* g4mi_last_error_string(void);

/* Diagnostics (no counterpart in the reference): per-lane group sums over
 * aligned groups of 2..64 lanes of `waves` wave64s, in f32 and f64, written as
 * out[(w*6 + j)*64 + lane] for group width 2^(j+1).  Lets a test pin the lane
 * layout of the cross-lane reductions every kernel uses. */
int g4mi_selftest_lane_reductions(const float* in, float* out, double* out_d, int32_t waves, void* stream);

/* ---------------------------------------------------------------- init
 * Fills out[0:n) with bf16(std * z), z ~ N(0,1) from Philox4x32-10 keyed by
 * `key` (element i uses counter i/2) and a Box-Muller transform in f64.
 * Replaces the host-side random init of the parity test
 * (tests/test_parity.py:70-73, normal_ on every parameter); `out` 4-byte aligned. */
int g4mi_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t key, double stdv, void* stream);

/* Raw Philox4x32-10 blocks (counter words ctr[4*j .. 4*j+3] -> out[4*j ..]);
 * exposed so the generator can be checked against published known answers. */
int g4mi_philox4x32_10(const uint32_t* ctr, uint64_t key, uint32_t* out, int64_t nblocks, void* stream);

/* ---------------------------------------------------------------- MoE (K1-K3)
 * Router scores: model.py:225-227 (_router up to the f32 cast), fused with the
 * pre_feedforward_layernorm_2 RMSNorm of model.py:315 when pre_norm_w != NULL.
 *   x [N,H] bf16 (residual if pre_norm_w given, else already normalised),
 *   router_scale [H], router_proj [E,H] bf16 -> scores [N,E] f32 holding the
 *   bf16-rounded logits.  x and router_proj 16-byte aligned; H % 8 == 0,
 *   H <= 16384, E <= 256. */
int g4mi_moe_router_scores(const uint16_t* x, const uint16_t* pre_norm_w, const uint16_t* router_scale,
                           const uint16_t* router_proj, int64_t N, int64_t H, int64_t E, float eps, float* scores,
                           void* stream);

/* Router + top-k: model.py:224-232 (_router).  As g4mi_moe_router_scores, then
 * f32 softmax, top-k (descending probability, ties to the lower expert index
 * as jax.lax.top_k), renormalisation and per_expert_scale [E]:
 *   out_w [N,k] f32, out_i [N,k] int32.  k <= 32. */
int64_t g4mi_moe_router_workspace_bytes(int64_t N, int64_t E);
int g4mi_moe_router_topk(const uint16_t* x, const uint16_t* pre_norm_w, const uint16_t* router_scale,
                         const uint16_t* router_proj, const uint16_t* per_expert_scale, int64_t N, int64_t H,
                         int64_t E, int64_t k, float eps, float* out_w, int32_t* out_i, void* ws,
                         int64_t ws_bytes, void* stream);

/* Selected-expert gate/up GEMV + activation, model.py:267-271:
 *   act[N,k,F] bf16 = bf16(bf16(bf16(gelu(g)) * u) * bf16(top_w)) where (g, u)
 *   are the gate/up rows of expert top_i[n,slot] applied to xn [N,H].
 * gate_up [E,2,F,H] bf16 (gate rows then up rows).  Reads only the selected
 * experts' rows.  H = 256*i, F = 64*i (1 <= i <= 16), k <= 32. */
int g4mi_moe_gateup(const uint16_t* xn, const uint16_t* gate_up, const float* top_w, const int32_t* top_i,
                    int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, uint16_t* act, void* stream);

/* The same with the routing taken from router scores [N,E] (softmax + top-k of
 * model.py:228-231 done inside); also stores top_w [N,k] / top_i [N,k]. */
int g4mi_moe_gateup_routed(const uint16_t* xn, const float* scores, const uint16_t* per_expert_scale,
                           const uint16_t* gate_up, int64_t N, int64_t H, int64_t F, int64_t E, int64_t k,
                           uint16_t* act, float* top_w, int32_t* top_i, void* stream);

/* Selected-expert down GEMV (model.py:272-273) and combine:
 * G4MI_COMBINE_BF16_RUNNING = the decode path's bf16 running sum in top-k
 * order (model.py:289-293); G4MI_COMBINE_F32 = one f32 contraction over the
 * experts (the dense prefill path, model.py:250).  down [E,H,F] bf16. */
int g4mi_moe_down(const uint16_t* act, const uint16_t* down, const int32_t* top_i, int64_t N, int64_t H,
                  int64_t F, int64_t E, int64_t k, int32_t combine, uint16_t* out, void* stream);

/* gate/up + down for given routing: model.py:262-294 (decode) or 241-250 (dense). */
int64_t g4mi_moe_experts_workspace_bytes(int64_t N, int64_t F, int64_t k);
int g4mi_moe_experts_decode(const uint16_t* xn, const uint16_t* gate_up, const uint16_t* down,
                            const float* top_w, const int32_t* top_i, int64_t N, int64_t H, int64_t F,
                            int64_t E, int64_t k, int32_t combine, uint16_t* out, void* ws, int64_t ws_bytes,
                            void* stream);

/* The whole MoE decode block of model.py:235-294 on xn [N,H] (the
 * pre_feedforward_layernorm_2 output): router scores, then gate/up with the
 * selection fused in, then down + combine.  Three kernels, no host sync. */
int64_t g4mi_moe_block_workspace_bytes(int64_t N, int64_t E, int64_t F, int64_t k);
int g4mi_moe_block_decode(const uint16_t* xn, const uint16_t* router_scale, const uint16_t* router_proj,
                          const uint16_t* per_expert_scale, const uint16_t* gate_up, const uint16_t* down,
                          int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, float eps, int32_t combine,
                          uint16_t* out, float* top_w, int32_t* top_i, void* ws, int64_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* G4MI_H_ */
