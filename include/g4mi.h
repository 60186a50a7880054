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

/* Diagnostics (no counterpart in the reference): adds to *mismatches (device
 * memory, zeroed by the caller) the number of floats x = -(bits lo + k),
 * k < count, where the softmax's exp for x <= 0 differs from expf (below
 * -103.97, where expf gives 0, a result of at most 2^-149 counts as equal).
 * lo + count <= 0x7f800000 (finite floats). */
int g4mi_selftest_exp_nonpositive(int64_t lo, int64_t count, uint64_t* mismatches, void* stream);

/* Diagnostics (no counterpart in the reference; runs on the host, no GPU
 * needed): the MFMA GEMM's block -> tile map.  For a grid sized for max_tiles
 * row tiles x ncol_tiles column tiles with mtiles row tiles live (grouped
 * tiles come from a device list whose live count is known only on the GPU),
 * out[2b], out[2b+1] = the (row tile, column tile) block b computes, or -1, -1
 * for a block that exits.  out_len >= 2 * 8 * ceil(max_tiles*ncol_tiles/8). */
int g4mi_selftest_tile_order(int32_t mtiles, int32_t max_tiles, int32_t ncol_tiles, int32_t grouped,
                             int32_t* out, int64_t out_len);

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
 * experts' rows; with N > 1 and N*k <= 64 an expert chosen by several
 * (token, slot) pairs has its rows read once for all of them (same results).
 * H = 256*i, F = 64*i (1 <= i <= 16), k <= 32. */
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
 * selection fused in, then down + combine (three kernels); with N > 1 and
 * N*k <= 64 the selection is its own kernel and the gate/up reads a shared
 * expert once (four kernels).  No host sync. */
int64_t g4mi_moe_block_workspace_bytes(int64_t N, int64_t E, int64_t F, int64_t k);
int g4mi_moe_block_decode(const uint16_t* xn, const uint16_t* router_scale, const uint16_t* router_proj,
                          const uint16_t* per_expert_scale, const uint16_t* gate_up, const uint16_t* down,
                          int64_t N, int64_t H, int64_t F, int64_t E, int64_t k, float eps, int32_t combine,
                          uint16_t* out, float* top_w, int32_t* top_i, void* ws, int64_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- attention (K5)
 * Split-K decode attention over a paged bf16 KV cache, model.py:197-213 with
 * the decode masks of model.py:402-408 (sliding: pos-window < kv <= pos, full:
 * kv <= pos), scale 1.0, optional logit softcap (0 = off, the reference).
 *   q_raw [B,NH,D], k_raw/v_raw [B,KV,D] bf16: the raw projections of the new
 *   token (v_raw NULL on k==v layers: V = rms_norm(k_raw)); q_norm/k_norm [D];
 *   rope_cos/rope_sin [>=lmax, D/2] bf16; k_pages/v_pages [num_pages,KV,PAGE,D];
 *   page_table [B,max_pages] int32, or NULL when sequence b owns pages
 *   [b*max_pages, (b+1)*max_pages) in order (B*max_pages <= num_pages; the
 *   kernels then compute page indices instead of loading them); pos [B]
 *   int32 (device).
 * With append != 0 the new K/V are normalised, roped and written at pos.
 * ctx [B,NH,D] bf16.  D in {64,128,256,512}; NH/KV in {1,2,4,8};
 * g4mi_attention_min_splits(span) <= n_split_max <= 256, span = window (when
 * 0 < window < lmax) else lmax (a split holds <= 256 positions, so span <=
 * 65536).  A position outside [0, lmax) attends to nothing (ctx = 0).  The
 * workspace starts with arrival counters: zero-fill it once before first use
 * (each call leaves the counters at zero).  Calls may share a workspace when
 * they have the same B and NH (their counters coincide; the rest is scratch),
 * e.g. the sliding and full layers of one decode step; concurrent calls need
 * separate workspaces. */
int64_t g4mi_attention_min_splits(int64_t lmax);
int64_t g4mi_decode_attention_workspace_bytes(int64_t B, int64_t NH, int64_t D, int64_t lmax, int64_t n_split_max);
int g4mi_decode_attention(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                          const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                          const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                          const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B, int64_t NH,
                          int64_t KV, int64_t D, int64_t page_size, int64_t window, float softcap, float eps,
                          int32_t append, int64_t lmax, int64_t n_split_max, uint16_t* ctx, void* ws,
                          int64_t ws_bytes, void* stream);

/* g4mi_decode_attention without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * split-K scratch lives in a file-scope device array of
 * G4MI_NOALLOC_ATTENTION_SCRATCH_BYTES per GPU, loaded with the library and
 * held until the process ends; its address is looked up once per device on
 * the first call made with that device current.  A call whose
 * g4mi_decode_attention_workspace_bytes() exceeds that size is rejected with
 * G4MI_EWORKSPACE (nothing is launched); the 26B-A4B decode step at 32,768
 * positions needs 6.6 MiB.  Each call first zeroes its arrival counters with
 * a fill kernel on `stream`, then runs the same kernels as
 * g4mi_decode_attention.  Every call on one GPU shares that GPU's array:
 * calls that may overlap on one GPU (other streams, other host threads) race
 * and give wrong results; order them on one stream.  Nothing is allocated or
 * freed. */
#define G4MI_NOALLOC_ATTENTION_SCRATCH_BYTES (16ll << 20)
int g4mi_decode_attention_noalloc(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                  const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                                  const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                                  const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B,
                                  int64_t NH, int64_t KV, int64_t D, int64_t page_size, int64_t window,
                                  float softcap, float eps, int32_t append, int64_t lmax, int64_t n_split_max,
                                  uint16_t* ctx, void* stream);

/* Cache append of T tokens of one sequence (model.py:202-206, the
 * dynamic_update_slice of model.py:205-206): k = rope(rms_norm(k_raw, k_norm)),
 * v = rms_norm(v_raw) written at positions pos[T] through page_table_row. */
int g4mi_kv_append(const uint16_t* k_raw, const uint16_t* v_raw, const uint16_t* k_norm, const uint16_t* rope_cos,
                   const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                   const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t T, int64_t KV, int64_t D,
                   int64_t page_size, int64_t lmax, float eps, void* stream);

/* ---------------------------------------------------------------- decode layer (K4, K6, K7)
 * Batch-1 pieces of one decode step; all vectors are bf16 of length H unless
 * stated.  H = 256*i (i <= 16).
 *
 * g4mi_layer_in: the q/k/v projection rows (model.py:197-201) applied to
 * rms_norm(x, input_layernorm) (model.py:301), where x is
 *   mode 0: bf16(embed[tok[0]] * bf16(sqrt(H)))               (model.py:355-357)
 *   mode 1: the previous layer's tail bf16(bf16(x1 + rms_norm(hs, post_ff)) *
 *           layer_scalar), hs = bf16(rms_norm(mlp_out, post_ff_1) +
 *           rms_norm(moe_out, post_ff_2)) (hs = mlp_out when moe_out is NULL)
 *                                                              (model.py:312-322)
 *   mode 2: x_in.
 *   mode 3: x_in is already rms_norm(x, input_layernorm) (as g4mi_ffn_out's
 *           epilogue writes it); input_ln and x_out are not used.
 * Modes 0-2 also store x to x_out.  qkv_out = [q rows | k rows | v rows] bf16. */
int g4mi_layer_in(int32_t mode, const int32_t* tok, const uint16_t* embed, int64_t vocab, const uint16_t* x_in,
                  const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, const uint16_t* post_ff1_ln,
                  const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                  const uint16_t* input_ln, uint16_t* x_out, const uint16_t* wq, int64_t q_rows, const uint16_t* wk,
                  int64_t k_rows, const uint16_t* wv, int64_t v_rows, uint16_t* qkv_out, int64_t H, float eps,
                  void* stream);

/* out[rows] = ctx[K] . w[rows, K]: the o_proj of model.py:214.  K = 512*i or 256*i (i <= 16). */
int g4mi_oproj(const uint16_t* ctx, const uint16_t* w, int64_t rows, int64_t K, uint16_t* out, void* stream);

/* x1 = bf16(x + rms_norm(o, post_attention_layernorm)) (model.py:303-304);
 * act_mlp[I] = bf16(bf16(gelu(g)) * u) of the dense MLP on rms_norm(x1,
 * pre_feedforward_layernorm) (model.py:218-220, 310); with router_proj,
 * xe = rms_norm(x1, pre_feedforward_layernorm_2) (model.py:315) and the
 * router scores [E] on it (model.py:225-227).  With per_expert_scale also the
 * expert selection of model.py:228-231 (softmax, top-k, renormalisation,
 * per-expert scale) -> top_w [k] f32, top_i [k] int32, computed once by the
 * last router block to finish; E <= 256, k <= 32.  The workspace holds that
 * block's arrival counter: zero-fill it once (each call leaves it at zero). */
int64_t g4mi_ffn_in_workspace_bytes(void);
int g4mi_ffn_in(const uint16_t* x, const uint16_t* o, const uint16_t* post_attn_ln, const uint16_t* pre_ff_ln,
                const uint16_t* pre_ff2_ln, uint16_t* x1_out, uint16_t* xe_out, const uint16_t* gate,
                const uint16_t* up, int64_t I, uint16_t* act_mlp, const uint16_t* router_scale,
                const uint16_t* router_proj, int64_t E, float* scores, const uint16_t* per_expert_scale, int64_t k,
                float* top_w, int32_t* top_i, void* ws, int64_t ws_bytes, int64_t H, float eps, void* stream);

/* mlp_out[H] = act_mlp . down[H, I] (model.py:221) and, with experts_down,
 * moe_out[H] = the combine of the k selected experts' down rows applied to
 * act_moe [k, F] (model.py:272-293 / model.py:250 by `combine`).  k <= 8.
 * With next_ln, the last block to finish also applies the layer tail
 * (model.py:312-322: x_out = bf16(bf16(x1 + rms_norm(hs, post_ff)) *
 * layer_scalar), hs as in g4mi_layer_in mode 1) and the next norm
 * (model.py:298 or the final norm, model.py:373): xn_out = rms_norm(x_out,
 * next_ln).  H <= 4096 then.  The workspace holds that block's arrival
 * counter: zero-fill it once (each call leaves it at zero). */
int64_t g4mi_ffn_out_workspace_bytes(void);
int g4mi_ffn_out(const uint16_t* act_mlp, const uint16_t* down, int64_t I, uint16_t* mlp_out,
                 const uint16_t* act_moe, const uint16_t* experts_down, const int32_t* top_i, int64_t E, int64_t k,
                 int64_t F, int32_t combine, uint16_t* moe_out, const uint16_t* x1, const uint16_t* post_ff1_ln,
                 const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                 const uint16_t* next_ln, uint16_t* x_out, uint16_t* xn_out, float eps, void* ws, int64_t ws_bytes,
                 int64_t H, void* stream);

/* The last layer's tail (as g4mi_layer_in mode 1), the final norm
 * (model.py:373), logits[V] f32 = softcap(f32(bf16(x . embed[v])))
 * (model.py:381-385, softcap 0 = off), and the per-block maxima
 * blk_val/blk_idx [g4mi_lm_head_blocks(V)] for g4mi_argmax_finalize. */
int64_t g4mi_lm_head_blocks(int64_t V);
int g4mi_lm_head(const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, const uint16_t* post_ff1_ln,
                 const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                 const uint16_t* final_norm, const uint16_t* embed, int64_t V, int64_t H, float softcap, float eps,
                 float* logits, float* blk_val, int32_t* blk_idx, void* stream);

/* Greedy token (model.py:416: first index of the maximum) from the per-block
 * maxima -> tok[0].  With pos != NULL also pos[0] += 1 and hist[pos[0]] = token
 * (when within hist_len), so a captured decode step advances on its own. */
/* logits and per-block maxima as g4mi_lm_head from an input that is already
 * rms_norm(x, final_norm) (g4mi_ffn_out's epilogue writes it). */
int g4mi_lm_head_normed(const uint16_t* xn, const uint16_t* embed, int64_t V, int64_t H, float softcap,
                        float* logits, float* blk_val, int32_t* blk_idx, void* stream);

int g4mi_argmax_finalize(const float* blk_val, const int32_t* blk_idx, int64_t n, int32_t* tok, int32_t* pos,
                         int32_t* hist, int64_t hist_len, void* stream);

/* Prompt feeding of a token-at-a-time prefill (engine.py:57-67 runs the whole
 * prompt through forward; here each prompt token is one captured step):
 * pos[0] += 1, then, if pos < feed_cap, tok[0] = feed[pos] and hist[pos] =
 * tok[0] (when within hist_len).  feed holds the prompt at its positions. */
int g4mi_advance_feed(const int32_t* feed, int64_t feed_cap, int32_t* tok, int32_t* pos, int32_t* hist,
                      int64_t hist_len, void* stream);

/* ---------------------------------------------------------------- sampling (K7)
 * model.py:414-424 (sample): temperature <= 0 -> greedy (first index of the
 * maximum logit); else top_k of logits / max(T, 1e-6) (descending, ties to
 * the lower index), softmax, nucleus cut where the exclusive prefix sum
 * (csum - p) >= top_p, renormalise, one draw.  The uniform is Philox4x32-10
 * under params->seed at counter (step, 0x53414D50, 0, 0) with step = pos[0]
 * when counter_mode != 0 (decode, engine.py:80) else 0 (after a prefill,
 * engine.py:66); it is this library's stream, not JAX's.  `params` is a
 * device g4mi_sample_params, read when the kernels run, so a captured step
 * picks up new settings.  Writes tok[0]; with pos != NULL also advances it
 * and records hist as g4mi_argmax_finalize does.  logits [V] f32, top_k <= 64;
 * params and ws 8-byte aligned. */
typedef struct g4mi_sample_params {
  float temperature;
  float top_p;
  uint64_t seed;
} g4mi_sample_params;
int64_t g4mi_sample_workspace_bytes(int64_t V);
int g4mi_sample(const float* logits, int64_t V, int64_t top_k, const void* params, int32_t counter_mode,
                int32_t* tok, int32_t* pos, int32_t* hist, int64_t hist_len, void* ws, int64_t ws_bytes,
                void* stream);

/* ---------------------------------------------------------------- prefill (K8, K9)
 * bf16 GEMM on MFMA: C[m, n] = sum_k A[a_rows ? a_rows[m] : m, k] * B[n, k],
 * A [*, K] (row stride lda), B [N, K] (row stride ldb), f32 accumulation.
 * epilogue 0: C bf16 [M, N] (ldc); 1: C f32; 2 (gated): N gate rows from B
 * and the up rows at B + pair_offset, C[m, n] = bf16(bf16(bf16(gelu(bf16(g)))
 * * bf16(u)) * bf16(row_scale[m])) (model.py:220, 246-247; row_scale may be
 * NULL).  With tiles (device int32 triples (group, m0, m1), count *ntiles <=
 * max_tiles, m1 - m0 <= 128) each tile uses B + group * b_group_stride: the
 * grouped per-expert GEMM.  k_slices > 1 splits K over blocks (plain
 * epilogues 0/1 only) with a workspace of g4mi_gemm_workspace_bytes.
 * K % 64 == 0; rows 16-byte aligned.  M <= 16 without tiles or split-K
 * runs a skinny kernel (16 output columns per block, K split over its waves,
 * each wave's K range requested in one round trip).
 * No reference counterpart: XLA's dot. */
int64_t g4mi_gemm_workspace_bytes(int64_t M, int64_t N, int64_t k_slices);
int g4mi_gemm_bf16(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b, int64_t ldb,
                   int64_t b_group_stride, int64_t pair_offset, int64_t M, int64_t N, int64_t K,
                   const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles, int32_t epilogue, void* c,
                   int64_t ldc, const float* row_scale, int64_t k_slices, void* ws, int64_t ws_bytes,
                   void* stream);

/* Several products that share A in one skinny launch: C_s = A . B_s^T for
 * the nseg <= 4 segments, B_s [n[s], K] (row stride K), C_s [M, n[s]] bf16
 * (row stride n[s]); M <= 16, every n[s] a multiple of 16, K % 64 == 0.
 * For the batched decode step's q, k and v projections of the same
 * normalised rows (model.py:197-200), which read 46 MB of weights per
 * sliding layer in one launch instead of three. */
int g4mi_gemm_bf16_segments(const uint16_t* a, int64_t lda, int64_t M, int64_t K, int32_t nseg,
                            const uint16_t* const* b, const int64_t* n, uint16_t* const* c, void* stream);

/* The dense-MoE prefill of model.py:241-250 for n tokens: xn [n, H] (the
 * pre_feedforward_layernorm_2 output), routing top_w [n, K] f32 / top_i
 * [n, K] int32, gate_up [E, 2, F, H], down [E, H, F] -> out [n, H] bf16 = bf16
 * of one f32 sum over the selected experts.  Unselected experts contribute
 * exact zeros in the reference (masked weights), so only the selected
 * (token, expert) pairs are computed, as grouped MFMA GEMMs.  With out =
 * NULL the combine is left out and each (token, slot) pair's f32 output stays
 * in ws for g4mi_rows_tail_experts.  n <= 65535, E <= 256, K <= 32, H and F
 * multiples of 64. */
int64_t g4mi_moe_prefill_workspace_bytes(int64_t n, int64_t K, int64_t E, int64_t F, int64_t H);
int g4mi_moe_prefill(const uint16_t* xn, const float* top_w, const int32_t* top_i, const uint16_t* gate_up,
                     const uint16_t* down, int64_t n, int64_t H, int64_t F, int64_t E, int64_t K, uint16_t* out,
                     void* ws, int64_t ws_bytes, void* stream);

/* The experts of a batched decode step (model.py:262-294 for each of n <= 16
 * tokens): the routing's (token, slot) pairs are grouped by expert, and each
 * selected expert's gate/up and down rows stream from HBM once for every
 * token that chose it (GEMV row walks over the union of the routed experts);
 * then the per-token combine in slot order, G4MI_COMBINE_BF16_RUNNING (the
 * decode path) or G4MI_COMBINE_F32.  act and the down partials equal
 * g4mi_moe_gateup / g4mi_moe_down's.  xn [n, H], top_w/top_i [n, K],
 * gate_up [E, 2, F, H], down [E, H, F] -> out [n, H] bf16.  Workspace:
 * g4mi_moe_prefill_workspace_bytes(n, K, E, F, H).  H = 256*i (i <= 16),
 * F = 64*j (j <= 16). */
int g4mi_moe_decode_grouped(const uint16_t* xn, const float* top_w, const int32_t* top_i, const uint16_t* gate_up,
                            const uint16_t* down, int64_t n, int64_t H, int64_t F, int64_t E, int64_t K,
                            int32_t combine, uint16_t* out, void* ws, int64_t ws_bytes, void* stream);

/* Row kernels between the batched prefill GEMMs, one token row of H <= 4096
 * per block, with the decode kernels' rounding recipe:
 *  rows_embed:     x = bf16(embed[tok] * bf16(sqrt(H))) (model.py:355-357),
 *                  xn = rms_norm(x, input_layernorm) (model.py:298);
 *  rows_post_attn: x1 = bf16(x + rms_norm(o, post_attention_layernorm)),
 *                  xm = rms_norm(x1, pre_feedforward_layernorm), xe =
 *                  rms_norm(x1, pre_feedforward_layernorm_2) (model.py:301-315;
 *                  xe_out NULL without the MoE block);
 *  rows_tail:      x = the layer tail (model.py:312-322), xn = rms_norm(x,
 *                  next_ln) (the next layer's input norm). */
int g4mi_rows_embed(const int32_t* tok, int64_t n, const uint16_t* embed, int64_t vocab, const uint16_t* input_ln,
                    int64_t H, float eps, uint16_t* x_out, uint16_t* xn_out, void* stream);
int g4mi_rows_post_attn(const uint16_t* x, const uint16_t* o, int64_t n, const uint16_t* post_attn_ln,
                        const uint16_t* pre_ff_ln, const uint16_t* pre_ff2_ln, int64_t H, float eps, uint16_t* x1_out,
                        uint16_t* xm_out, uint16_t* xe_out, void* stream);
int g4mi_rows_tail(const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, int64_t n,
                   const uint16_t* post_ff1_ln, const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln,
                   const uint16_t* layer_scalar, const uint16_t* next_ln, int64_t H, float eps, uint16_t* x_out,
                   uint16_t* xn_out, void* stream);
/* g4mi_rows_tail with moe_out = the combine of the per-expert outputs that
 * g4mi_moe_prefill(out = NULL) left in its workspace moe_ws (the same n, K,
 * E, F, H): moe[t] = bf16(f32 sum over the token's K slots in order,
 * model.py:250), then the tail (model.py:312-322) and the next norm, in one
 * launch.  Identical to g4mi_moe_prefill with out followed by g4mi_rows_tail.
 * H = 64*i <= 4096. */
int g4mi_rows_tail_experts(const uint16_t* x1, const uint16_t* mlp_out, int64_t n, int64_t K, int64_t E, int64_t F,
                           const uint16_t* post_ff1_ln, const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln,
                           const uint16_t* layer_scalar, const uint16_t* next_ln, int64_t H, float eps,
                           uint16_t* x_out, uint16_t* xn_out, const void* moe_ws, int64_t moe_ws_bytes,
                           void* stream);

/* Prefill attention (model.py:195-215 at T > 1).  q_norm_rope: q = rope(
 * rms_norm(q, q_norm)) in place for T rows x NH heads at positions p0 + t
 * (model.py:198-199; rope tables [rope_len, D/2] as for decode attention).
 * prefill_attention: query row t (position p0 + t, q already normed and
 * rotated) attends the cached keys [max(0, p0 + t + 1 - window), p0 + t]
 * (window 0: all of [0, p0 + t]) -- the causal / sliding prefill mask of
 * model.py:392-399 -- with scale 1.0, optional softcap, probabilities rounded
 * to bf16 after normalisation; ctx [T, NH, D] bf16.  Two passes over the
 * keys on MFMA; page_size a multiple of 64; K/V of the T rows must already
 * be in the cache (g4mi_kv_append). */
int g4mi_q_norm_rope(uint16_t* q, const uint16_t* q_norm, const uint16_t* rope_cos, const uint16_t* rope_sin,
                     int64_t T, int64_t NH, int64_t D, int64_t p0, int64_t rope_len, float eps, void* stream);
int g4mi_prefill_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages, int64_t num_pages,
                           const int32_t* page_table, int64_t max_pages, int64_t page_size, int64_t T, int64_t p0,
                           int64_t NH, int64_t KV, int64_t D, int64_t window, float softcap, uint16_t* ctx,
                           void* stream);

/* Batched greedy head (model.py:381-385, 416 for B sequences): logits [B, V]
 * bf16 (x . embed^T, e.g. from g4mi_gemm_bf16) -> softcap in f32 (softcap 0:
 * off), optional f32 copy [B, V], first index of the maximum per row; tok[b] =
 * it, pos[b] += 1 and hist[b * hist_len + pos[b]] = it when pos / hist are
 * given.  Workspace: g4mi_argmax_rows_workspace_bytes(B). */
int64_t g4mi_argmax_rows_workspace_bytes(int64_t B);
int g4mi_argmax_rows(const uint16_t* logits, int64_t B, int64_t V, float softcap, float* logits_f32, int32_t* tok,
                     int32_t* pos, int32_t* hist, int64_t hist_len, void* ws, int64_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- model primitives
 * The reference model's standalone primitives (model.py:42-78), with the
 * rounding recipe of the fused kernels.  Tensor dtype codes: 0 = bf16,
 * 1 = f32 (the output has x's dtype).
 *   g4mi_rms_norm:    out[r, :] = cast(f32(x) * r * f32(w)), r = 1/sqrt(mean(x^2) + eps)
 *                     with the sum of squares exact (model.py:42-47); w may be NULL.
 *   g4mi_gelu_tanh:   tanh-approximation GELU in f32, one rounding (model.py:50-51).
 *   g4mi_rope_tables: cos/sin [T, 2*half] f32 of f32(pos) * inv_freq[j] with
 *                     the halves duplicated (model.py:64-67).
 *   g4mi_apply_rope:  x [B, T, inner, D] (inner = the head axes) with cos/sin
 *                     [T, D] cast to x's dtype: x*c + rotate_half(x)*s, each
 *                     product and the sum rounded to x's dtype (model.py:70-78);
 *                     out must not alias x. */
int g4mi_rms_norm(const void* x, int32_t x_f32, const void* w, int32_t w_f32, int64_t rows, int64_t dim, float eps,
                  void* out, void* stream);
int g4mi_gelu_tanh(const void* x, int32_t x_f32, int64_t n, void* out, void* stream);
int g4mi_rope_tables(const int32_t* positions, int64_t T, const float* inv_freq, int64_t half, float* cos_out,
                     float* sin_out, void* stream);
int g4mi_apply_rope(const void* x, int32_t x_f32, const float* rope_cos, const float* rope_sin, int64_t B, int64_t T,
                    int64_t inner, int64_t D, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* G4MI_H_ */
