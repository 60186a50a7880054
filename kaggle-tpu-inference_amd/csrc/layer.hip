// The dense parts of one decode layer and the lm_head (model.py:297-322,
// model.py:355-385), batch 1:
//
//   layer_in   prologue: layer 0 embeds the token (x = bf16(embed[tok] *
//              bf16(sqrt(H))), model.py:355-357); later layers finish the
//              previous layer (h1 = rms(mlp, post_ff_1), h2 = rms(moe,
//              post_ff_2), h = rms(bf16(h1+h2), post_ff), x = bf16(bf16(x1+h) *
//              layer_scalar), model.py:313-322); then rms(x, input_ln).
//              Body: the q/k/v projection rows (model.py:197-201).
//   oproj      ctx . o_proj (model.py:214).
//   ffn_in     prologue: x1 = bf16(x + rms(o, post_attention_ln)); xm =
//              rms(x1, pre_ff); xe = rms(x1, pre_ff_2) (model.py:303-315).
//              Body: dense gate/up rows with gelu*up (model.py:218-220) and
//              the router scores on xe (model.py:225-227).
//   ffn_out    per output row: the dense down row (model.py:221) and the
//              selected experts' down rows with the combine (model.py:272-293).
//   lm_head    prologue: the last layer's tail and the final norm
//              (model.py:373); body: tied-embedding rows, f32 softcap
//              (model.py:381-385); per-block argmax.
//   argmax     first index of the maximum over all blocks (model.py:416);
//              writes the token, advances the position, records history.
//
// Every block rebuilds its prologue vector in LDS (the vectors are ~6 KB and
// L2-resident) after issuing its weight loads, so the prologue latency hides
// under the HBM latency of its own rows.  RMSNorm scales use exact f64 sums.
#include <string.h>

#include <algorithm>

#include "capi_util.h"
#include <cstdlib>

#include "common.h"
#include "gemv.h"
#include "rowvec.h"
#include "select.h"

namespace g4mi {

// ------------------------------------------------------------------ layer_in
enum { kInEmbed = 0, kInTail = 1, kInPlain = 2, kInNormed = 3 };
struct InArgs {
  int mode;
  const int32_t* tok;
  const uint16_t* embed;
  int vocab;
  float embed_c;          // bf16(sqrt(H))
  const uint16_t* x_in;   // kInPlain
  TailArgs tail;          // kInTail
  const uint16_t* w_in;   // input_layernorm
  uint16_t* x_out;        // the residual x (written by block 0)
  const uint16_t* W[3];   // q, k, v projection rows [rows, H]
  int rows[3];
  uint16_t* out;          // [rows0 + rows1 + rows2]
  int pairs_per_block;
  int H;
  float eps;
};

// Row walk shared by the GEMV kernels: a block owns `ppb` consecutive row
// pairs; wave w handles pairs w, w+4, ... and half-wave h row 2*pair+h.  Each wave keeps the next pair's loads in flight while it
// reduces the current one, so a block per CU streams at full rate and the
// block's prologue is computed once per CU instead of once per 8 rows.
template <int IT>
struct PairWalk {
  int p, pend, plast;
  __device__ __forceinline__ PairWalk(int ppb, int npairs) {
    const int wave = wave_id();
    const int p0 = blockIdx.x * ppb;
    p = p0 + wave;
    pend = min(p0 + ppb, npairs);
    plast = max(pend - 1, 0);
  }
};

constexpr int kInPrefetch = 4;  // row pairs per wave in flight in layer_in

template <int IT, int MODE>
__global__ __launch_bounds__(256) void layer_in_kernel(InArgs a) {
  constexpr int H = IT * 256;
  constexpr int NCH = H / 8;
  __shared__ u32x4 xs[NCH];
  __shared__ double red[16];
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l = lane & 31;
  const int q_rows = a.rows[0], k_rows = a.rows[1];
  const int total = q_rows + k_rows + a.rows[2];
  auto rowptr = [&](int pair) {
    const int rc = min(2 * pair + half, total - 1);
    return (rc < q_rows) ? a.W[0] + (size_t)rc * H
           : (rc < q_rows + k_rows) ? a.W[1] + (size_t)(rc - q_rows) * H
                                    : a.W[2] + (size_t)(rc - q_rows - k_rows) * H;
  };
  // Loads are counted in issue order (s_waitcnt vmcnt), so the small
  // L2-resident prologue operands are requested before the weight rows and
  // the prologue runs while the rows stream in.  MODE is a template
  // parameter and the row loads are unconditional (clamped addresses), so no
  // branch merge forces an early full wait.
  Vec x, win;
  TailRegs<256> T;
  if constexpr (MODE != kInNormed) vload(win, a.w_in, NCH);
  if constexpr (MODE == kInEmbed) {
    int t = a.tok[0];
    t = (t < 0 || t >= a.vocab) ? 0 : t;
    vload(x, a.embed + (size_t)t * H, NCH);
  } else if constexpr (MODE == kInTail) {
    tail_load(T, a.tail, NCH);
  } else {
    vload(x, a.x_in, NCH);
  }
  // The compiler may not sink the prologue loads below the row loads (their
  // results would then wait for the rows).  One row batch of the wave is
  // requested before the prologue and the other NPF - 1 after it: a CU
  // queues only so many vector memory instructions, and a wave that
  // requested all its batches first would stall at issue, the prologue (the
  // layer tail is three dependent block reductions) behind the stalled
  // requests, until most of its rows had arrived.
  asm volatile("" ::: "memory");
  PairWalk<IT> pw(a.pairs_per_block, (total + 1) / 2);
  constexpr int NPF = kInPrefetch;
  u32x4 w[NPF][IT];
  load_row<32, IT>(rowptr(min(pw.p, pw.plast)), l, w[0]);
  if constexpr (MODE == kInEmbed) vmul(x, a.embed_c);
  if constexpr (MODE == kInTail) tail_compute(x, T, a.tail.moe != nullptr, H, a.eps, red);
  if constexpr (MODE != kInNormed) {
    // the residual store is issued after the last reduction, so no barrier
    // waits for it (the norm's round in a region of its own)
    const float r = vrms<256, true>(x, H, a.eps, red + 12);
    if (blockIdx.x == 0 && a.x_out != nullptr) vstore(x, (u32x4*)a.x_out, NCH);
    vscale_w(x, r, win);
  }
  vstore(x, xs, NCH);
  lds_barrier();
#pragma unroll
  for (int d = 1; d < NPF; ++d) load_row<32, IT>(rowptr(min(pw.p + 4 * d, pw.plast)), l, w[d]);
  int p = pw.p;
  // full batches: consume pair p+4d, refill it with pair p+4d+4*NPF (clamped)
  for (; p + 4 * NPF < pw.pend; p += 4 * NPF) {
#pragma unroll
    for (int d = 0; d < NPF; ++d) {
      const float acc = dot_row<32, IT>(w[d], xs, l);
      const int r = 2 * (p + 4 * d) + half;
      if (r < total && l == 0) a.out[r] = f2bf(acc);
      load_row<32, IT>(rowptr(min(p + 4 * d + 4 * NPF, pw.plast)), l, w[d]);
    }
  }
  // last batch: no refills
#pragma unroll
  for (int d = 0; d < NPF; ++d) {
    const float acc = dot_row<32, IT>(w[d], xs, l);
    const int r = 2 * (p + 4 * d) + half;
    if (p + 4 * d < pw.pend && r < total && l == 0) a.out[r] = f2bf(acc);
  }
}

// ------------------------------------------------------------------ oproj
// out[H] = ctx[K] . W[H, K]; S lanes per row (64/S rows per wave).  Each wave
// requests its first kOprojPrefetch row groups before ctx reaches LDS (ctx is
// loaded into registers first: loads complete in issue order, so the LDS
// store waits for ctx alone), then refills a group as it consumes one.
constexpr int kOprojPrefetch = 3;  // the 26B o_proj: 2,816 rows over 235 blocks is 3 rows per wave

template <int S, int IT>
__global__ __launch_bounds__(256) void oproj_kernel(const uint16_t* __restrict__ ctx, const uint16_t* __restrict__ W,
                                                    int rows, int groups_per_block, uint16_t* __restrict__ out) {
  constexpr int K = 8 * S * IT;
  constexpr int RPW = 64 / S;  // rows per wave step (a "group")
  constexpr int CPT = (K / 8 + 255) / 256;  // ctx chunks per thread
  constexpr int NPF = kOprojPrefetch;
  __shared__ u32x4 xs[K / 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), sub = lane % S;
  const int ngroups = (rows + RPW - 1) / RPW;
  const int g0 = blockIdx.x * groups_per_block;
  const int gend = min(g0 + groups_per_block, ngroups), glast = max(gend - 1, 0);
  auto rowp = [&](int grp) { return W + (size_t)min(grp * RPW + lane / S, rows - 1) * K; };
  u32x4 cv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) cv[j] = ld16((const u32x4*)ctx + min(tid + 256 * j, K / 8 - 1));
  int gi = g0 + wave;
  u32x4 w[NPF][IT];
#pragma unroll
  for (int d = 0; d < NPF; ++d) load_row<S, IT>(rowp(min(gi + 4 * d, glast)), sub, w[d]);
#pragma unroll
  for (int j = 0; j < CPT; ++j)
    if (tid + 256 * j < K / 8) xs[tid + 256 * j] = cv[j];
  __syncthreads();
  for (; gi + 4 * NPF < gend; gi += 4 * NPF) {
#pragma unroll
    for (int d = 0; d < NPF; ++d) {
      const float acc = dot_row<S, IT>(w[d], xs, sub);
      const int r = (gi + 4 * d) * RPW + lane / S;
      if (r < rows && sub == 0) out[r] = f2bf(acc);
      load_row<S, IT>(rowp(min(gi + 4 * d + 4 * NPF, glast)), sub, w[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < NPF; ++d) {
    const float acc = dot_row<S, IT>(w[d], xs, sub);
    const int r = (gi + 4 * d) * RPW + lane / S;
    if (gi + 4 * d < gend && r < rows && sub == 0) out[r] = f2bf(acc);
  }
}

// ------------------------------------------------------------------ ffn_in
struct FfnInArgs {
  const uint16_t *x, *o, *w_pa, *w_pf, *w_pf2;
  uint16_t *x1_out, *xe_out;
  const uint16_t *gate, *up;   // dense MLP [I, H]
  int I;
  uint16_t* act_mlp;           // [I]
  int dense_blocks;            // the last dense_blocks blocks do dense rows (router blocks first)
  int tasks_per_block;         // dense (gate, up) row pairs per dense block
  const uint16_t *r_scale, *r_proj;  // router (null: no MoE)
  int E;
  float r_c;                   // bf16(H^-0.5)
  float* scores;               // [E]
  const uint16_t* pes;         // per_expert_scale [E] (null: no selection)
  int K;                       // experts per token
  float* top_w;                // [K]
  int32_t* top_i;              // [K]
  unsigned int* counter;       // router-block arrivals (zero between launches)
  int xcd_local;               // router blocks on one XCD (see ffn_in_kernel)
  int H;
  float eps;
};

constexpr int kFfnInTasks = 3;  // dense (gate, up) row pairs per wave requested up front

template <int IT>
__global__ __launch_bounds__(256) void ffn_in_kernel(FfnInArgs a) {
  constexpr int H = IT * 256;
  constexpr int NCH = H / 8;
  __shared__ u32x4 xs[NCH];
  __shared__ double red[16];
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l = lane & 31, wave = wave_id();
  // The router and the expert selection are this kernel's longest chain, so
  // the router blocks come first in dispatch order.  With xcd_local they are
  // blocks 0, 8, 16, ... (one XCD: block b runs on the XCD of block b % 8),
  // so their scores reach the selecting block through that XCD's L2 (plain
  // stores and loads); otherwise blocks 0 .. rblocks-1, with device-scope
  // stores and loads.
  const int rblocks = (int)gridDim.x - a.dense_blocks;
  const int bid = (int)blockIdx.x;
  int rb, db;  // router block index (or -1), dense block index
  if (a.xcd_local) {
    const bool r = (bid & 7) == 0 && (bid >> 3) < rblocks;
    rb = r ? (bid >> 3) : -1;
    db = (bid < 8 * rblocks) ? bid - (bid >> 3) - 1 : bid - rblocks;
  } else {
    rb = bid < rblocks ? bid : -1;
    db = bid - rblocks;
  }
  const bool dense = rb < 0;
  // prologue operands first (see layer_in), then the weight rows.  Every
  // load is unconditional (a valid stand-in pointer where an operand is
  // absent): under a branch the compiler waits for the load inside it,
  // before the weight rows below are requested.  The per-expert scale the
  // selection multiplies in comes first: the selection is the kernel's tail.
  const float pes_t = bf2f(((a.pes != nullptr) ? a.pes : a.x)[min(tid, max(a.E, 1) - 1)]);
  Vec x, o, wpa, wf, rsc;
  vload(o, a.o, NCH);
  vload(x, a.x, NCH);
  vload(wpa, a.w_pa, NCH);
  vload(wf, dense ? a.w_pf : a.w_pf2, NCH);
  vload(rsc, (!dense && a.r_scale != nullptr) ? a.r_scale : a.w_pa, NCH);
  // dense: this block owns tasks (one (gate, up) row pair each) [t0, tend),
  // wave w takes t0+w, t0+w+4, ...; router blocks own 8 expert rows each.
  const int t0 = db * a.tasks_per_block;
  const int tend = min(t0 + a.tasks_per_block, a.I), tlast = max(tend - 1, 0);
  const int e = rb * 8 + wave * 2 + half;
  auto dense_row = [&](int f) { return (half ? a.up : a.gate) + (size_t)f * H; };
  // the wave's first task (router blocks: their one row) is requested
  // before the prologue, the other tasks (t0 + wave + 4j, j < kFfnInTasks)
  // after it, so the prologue does not wait behind requests stalled at issue
  u32x4 w[kFfnInTasks][IT];
  load_row<32, IT>(dense ? dense_row(min(t0 + wave, tlast)) : a.r_proj + (size_t)min(e, a.E - 1) * H, l, w[0]);
  // x1 = bf16(x + rms(o, post_attention_ln)); xm = rms(x1, pre_ff); xe = rms(x1, pre_ff_2)
  // the three norms' reduction rounds in regions of their own (red[0, 12))
  vscale_w(o, vrms<256, true>(o, H, a.eps, red), wpa);
  vadd(x, o);
  if (bid == 0) vstore(x, (u32x4*)a.x1_out, NCH);
  const float r1 = vrms<256, true>(x, H, a.eps, red + 4);
  if (dense) {
    vscale_w(x, r1, wf);
    vstore(x, xs, NCH);
  } else {
    Vec xe = x;
    vscale_w(xe, r1, wf);
    if (rb == 0) vstore(xe, (u32x4*)a.xe_out, NCH);
    // router input x2 = bf16(bf16(rms(xe) * scale) * bf16(H^-0.5)) (model.py:225-226)
    const float r2 = vrms<256, true>(xe, H, a.eps, red + 8);
#pragma unroll
    for (int j = 0; j < Vec::NC; ++j) {
      const int c = tid + 256 * j;
      if (c < NCH) {
        float f[8], g[8];
        unpack8(xe.c[j], f);
        unpack8(rsc.c[j], g);
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = rbf(rbf(rbf(f[q] * r2) * g[q]) * a.r_c);
        u32x4 v;
        v.x = pack2(f[0], f[1]); v.y = pack2(f[2], f[3]); v.z = pack2(f[4], f[5]); v.w = pack2(f[6], f[7]);
        xs[c] = v;
      }
    }
  }
  lds_barrier();
  if (dense) {
#pragma unroll
    for (int j = 1; j < kFfnInTasks; ++j) load_row<32, IT>(dense_row(min(t0 + wave + 4 * j, tlast)), l, w[j]);
#pragma unroll
    for (int j = 0; j < kFfnInTasks; ++j) {
      const int t = t0 + wave + 4 * j;
      const float acc = dot_row<32, IT>(w[j], xs, l);
      const float up = __shfl(acc, 32, kWave);
      if (t < tend && lane == 0) a.act_mlp[t] = f2bf(rbf(gelu_tanh(rbf(acc))) * rbf(up));
    }
    // tasks beyond kFfnInTasks per wave (small grids), one pair at a time
    for (int t = t0 + wave + 4 * kFfnInTasks; t < tend; t += 4) {
      u32x4 wr[IT];
      load_row<32, IT>(dense_row(t), l, wr);
      const float acc = dot_row<32, IT>(wr, xs, l);
      const float up = __shfl(acc, 32, kWave);
      if (lane == 0) a.act_mlp[t] = f2bf(rbf(gelu_tanh(rbf(acc))) * rbf(up));
    }
  } else {
    const u32x4* w0 = w[0];
    double d0 = 0.0, d1 = 0.0;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      if (i & 1) d1 = dot8_f64(w0[i], xs[l + 32 * i], d1);
      else d0 = dot8_f64(w0[i], xs[l + 32 * i], d0);
    }
    const double acc = group_sum_f64<32>(d0 + d1);
    if (e >= 0 && e < a.E && l == 0) {
      if (a.xcd_local) a.scores[e] = rbf(f32_of(acc));
      else __hip_atomic_store(a.scores + e, rbf(f32_of(acc)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.pes == nullptr) return;
    // the last router block to finish selects the experts (model.py:228-231)
    // once, so the expert kernel starts from the routing instead of the scores
    __shared__ SelectLds L;
    __shared__ int flag;
    if (!arrive_last(a.counter, (unsigned)rblocks, &flag)) return;
    const int t = threadIdx.x;
    float sv = -INFINITY;
    if (t < a.E)
      sv = a.xcd_local ? __hip_atomic_load(a.scores + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                       : __hip_atomic_load(a.scores + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_values_pes(sv, pes_t, a.E, a.K, L);
    if (t < a.K) {
      a.top_w[t] = L.topw[t];
      a.top_i[t] = L.topi[t];
    }
  }
}

// ------------------------------------------------------------------ ffn_out
// One wave per output row h (kOutRows rows per block): the dense down row
// (I values, 64 lanes) and the k selected experts' down rows (8 lanes per
// expert slot, FIT = F/64 chunks).
// 11 waves per block: the 26B layer's 2,816 rows are then one block on every
// one of the 256 CUs (4-row blocks left 192 CUs with 3 blocks and 64 with 2,
// and the kernel ended with the 3-block CUs).
constexpr int kOutThreads = 704;
constexpr int kOutRows = kOutThreads / 64;
struct FfnOutArgs {
  const uint16_t* act_mlp;  // [I]
  const uint16_t* down;     // [H, I]
  int I;
  uint16_t* mlp_out;        // [H]
  const uint16_t* act_moe;  // [k, F]
  const uint16_t* e_down;   // [E, H, F] (null: no MoE)
  const int32_t* top_i;     // [k]
  int E, K;
  int bf16_running;
  uint16_t* moe_out;        // [H]
  int H;
  // optional epilogue: the layer tail and the next norm, by the last block
  TailArgs tail;            // tail.mlp / tail.moe are mlp_out / moe_out
  const uint16_t* w_next;   // next layer's input_layernorm (or the final norm); null: no epilogue
  uint16_t* x_out;          // residual after this layer [H]
  uint16_t* xn_out;         // rms_norm(x_out, w_next) [H]
  unsigned int* counter;
  float eps;
};

template <int FIT>
__global__ __launch_bounds__(kOutThreads) void ffn_out_kernel(FfnOutArgs a) {
  constexpr int F = FIT * 64;
  constexpr int NT = kOutThreads;
  extern __shared__ u32x4 act_lds[];  // I/8 chunks of act_mlp, then K * F/8 of act_moe
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int h = blockIdx.x * kOutRows + wave;
  const int ich = a.I / 8;
  constexpr int DIT = 8;  // dense chunks per lane, at most (I <= 4096)
  const int dit = (ich + 63) / 64;  // of which this I needs
  const bool hv = h < a.H;
  const int hc = min(h, a.H - 1);
  const int g = lane >> 3, l8 = lane & 7;
  // small operands first (issue order = completion order for vmcnt): the
  // routed expert of this lane group and this thread's share of act_mlp
  const int ei = (a.e_down != nullptr) ? a.top_i[min(g, a.K - 1)] : -1;
  constexpr int ACT_PER = (4096 / 8 + NT - 1) / NT;  // act_mlp chunks per thread: I <= 4096
  u32x4 av[ACT_PER];
#pragma unroll
  for (int j = 0; j < ACT_PER; ++j) av[j] = ld16((const u32x4*)a.act_mlp + min(tid + NT * j, ich - 1));
  // the routed experts' activations (K * F/8 chunks, written by the previous
  // kernel) are staged in LDS once per block like act_mlp: loaded per wave
  // they took as many vector memory slots as the expert rows
  constexpr int MOE_PER = (8 * F / 8 + NT - 1) / NT;  // act_moe chunks per thread: K <= 8
  const int mch = (a.act_moe != nullptr) ? a.K * (F / 8) : 0;
  u32x4 avm[MOE_PER];
#pragma unroll
  for (int j = 0; j < MOE_PER; ++j)
    avm[j] = ld16((const u32x4*)(a.act_moe != nullptr ? a.act_moe : a.act_mlp) + min(tid + NT * j, max(mch, 1) - 1));
  // weight rows, unconditional with clamped addresses (the dense row: only
  // the chunks this I has)
  u32x4 wd[DIT];
  {
    const u32x4* drow = (const u32x4*)(a.down + (size_t)hc * a.I);
#pragma unroll
    for (int i = 0; i < DIT; ++i)
      if (i < dit) wd[i] = ld_stream(drow + min(lane + 64 * i, ich - 1));
  }
  const int e = (g < a.K && ei >= 0 && ei < a.E) ? ei : -1;
  u32x4 we[FIT];
  if (a.e_down != nullptr) {
    const u32x4* erow = (const u32x4*)(a.e_down + ((size_t)max(e, 0) * a.H + hc) * F);
#pragma unroll
    for (int i = 0; i < FIT; ++i) we[i] = ld_stream(erow + l8 + 8 * i);
  }
#pragma unroll
  for (int j = 0; j < ACT_PER; ++j)
    if (tid + NT * j < ich) act_lds[tid + NT * j] = av[j];
#pragma unroll
  for (int j = 0; j < MOE_PER; ++j)
    if (tid + NT * j < mch) act_lds[ich + tid + NT * j] = avm[j];
  lds_barrier();
  if (hv) {  // wave-uniform
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < DIT; ++i) {
      const int c = lane + 64 * i;
      if (c < ich) acc = dot8(wd[i], act_lds[c], acc);
    }
    acc = group_sum<64>(acc);
    if (lane == 0) coherent_store_bf16(a.mlp_out + h, f2bf(acc));
    if (a.e_down != nullptr) {
      float part = 0.0f;
      if (e >= 0) {
        const u32x4* am = act_lds + ich + g * (F / 8);  // this lane group's slot (e >= 0: g < K)
#pragma unroll
        for (int i = 0; i < FIT; ++i) part = dot8(we[i], am[l8 + 8 * i], part);
      }
      part = group_sum<8>(part);
      float run = 0.0f;
      for (int q = 0; q < a.K && q < 8; ++q) {
        const float pq = __shfl(part, 8 * q, kWave);
        if (a.bf16_running) run = (q == 0) ? rbf(pq) : rbf(run + rbf(pq));
        else run = (q == 0) ? pq : run + pq;
      }
      if (lane == 0) coherent_store_bf16(a.moe_out + h, f2bf(run));
    }
  }
  if (a.w_next == nullptr) return;
  // The last block to finish applies the layer tail (model.py:317-322) and
  // the next layer's input norm (model.py:298) once, so the next kernel
  // starts from the normalised vector instead of three dependent reductions.
  __shared__ int flag;
  __shared__ double red[4 * NT / 64];
  if (!arrive_last_grid(a.counter, &flag)) return;
  const int nch = a.H / 8;
  TailRegs<NT> T;
  VecT<NT> wn, x;
  vload_coherent(T.a, a.mlp_out, nch);
  if (a.e_down != nullptr) vload_coherent(T.b, a.moe_out, nch);
  vload(T.x1, a.tail.x1, nch);
  vload(T.w3, a.tail.w_pf, nch);
  if (a.e_down != nullptr) {
    vload(T.w1, a.tail.w_pf1, nch);
    vload(T.w2, a.tail.w_pf2, nch);
  }
  vload(wn, a.w_next, nch);
  T.ls = a.tail.ls[0];
  tail_compute(x, T, a.e_down != nullptr, a.H, a.eps, red);
  const float r = vrms<NT, true>(x, a.H, a.eps, red + 3 * NT / 64);
  vstore(x, (u32x4*)a.x_out, nch);
  vscale_w(x, r, wn);
  vstore(x, (u32x4*)a.xn_out, nch);
}

// ------------------------------------------------------------------ lm_head
struct LmArgs {
  TailArgs tail;
  const uint16_t* xn;       // already normalised input (NORMED variant)
  const uint16_t* w_norm;   // final norm
  const uint16_t* embed;    // [V, H]
  int V;
  float softcap;            // 0 = off
  float* logits;            // [V] f32
  float* blk_val;           // [nblocks]
  int32_t* blk_idx;
  int rows_per_block;
  int H;
  float eps;
};

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

template <int IT, bool NORMED>
__global__ __launch_bounds__(256) void lmhead_kernel(LmArgs a) {
  constexpr int H = IT * 256;
  constexpr int NCH = H / 8;
  __shared__ u32x4 xs[NCH];
  __shared__ double red[16];
  __shared__ float bvs[8];
  __shared__ int bis[8];
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l = lane & 31, wave = wave_id();
  const int r0 = blockIdx.x * a.rows_per_block;
  const int r1 = min(a.V, r0 + a.rows_per_block);
  // first row pair of this wave, loads issued before the prologue
  int r = r0 + wave * 2 + half;
  Vec x, wn0;
  TailRegs<256> T;
  if constexpr (NORMED) {
    vload(x, a.xn, NCH);
  } else {
    tail_load(T, a.tail, NCH);
    vload(wn0, a.w_norm, NCH);
  }
  asm volatile("" ::: "memory");
  u32x4 w[IT];
  load_row<32, IT>(a.embed + (size_t)min(r, a.V - 1) * H, l, w);
  if constexpr (!NORMED) {
    tail_compute(x, T, a.tail.moe != nullptr, H, a.eps, red);
    vscale_w(x, vrms<256, true>(x, H, a.eps, red + 12), wn0);
  }
  vstore(x, xs, NCH);
  __syncthreads();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const float cap = a.softcap;
  for (; r - half < r1; r += 8) {
    u32x4 wn[IT];
    load_row<32, IT>(a.embed + (size_t)min(r + 8, a.V - 1) * H, l, wn);  // next pair (clamped)
    const float acc = dot_row<32, IT>(w, xs, l);
    float v = rbf(acc);
    if (cap > 0.0f) v = tanhf(v / cap) * cap;
    if (r < r1 && l == 0) {
      a.logits[r] = v;
      better(bv, bi, v, r);
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = wn[i];
  }
  // lanes 0 and 32 hold their half's best
  if (l == 0) {
    bvs[wave * 2 + half] = bv;
    bis[wave * 2 + half] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = bvs[0];
    int i = bis[0];
    for (int q = 1; q < 8; ++q) better(v, i, bvs[q], bis[q]);
    a.blk_val[blockIdx.x] = v;
    a.blk_idx[blockIdx.x] = i;
  }
}

// One block: token = argmax over the per-block maxima (value desc, index asc).
// Writes tok[0]; when pos != null advances pos[0] and stores the token at
// hist[new pos] (hist_len entries, ignored past the end).
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ blk_val,
                                                     const int32_t* __restrict__ blk_idx, int n, int32_t* tok,
                                                     int32_t* pos, int32_t* hist, int hist_len) {
  __shared__ float vs[256];
  __shared__ int is[256];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = threadIdx.x; j < n; j += 256) better(bv, bi, blk_val[j], blk_idx[j]);
  vs[threadIdx.x] = bv;
  is[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      float v = vs[threadIdx.x];
      int i = is[threadIdx.x];
      better(v, i, vs[threadIdx.x + s], is[threadIdx.x + s]);
      vs[threadIdx.x] = v;
      is[threadIdx.x] = i;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int t = is[0];
    tok[0] = t;
    if (pos != nullptr) {
      const int p = pos[0] + 1;
      pos[0] = p;
      if (hist != nullptr && p >= 0 && p < hist_len) hist[p] = t;
    }
  }
}

// Teacher forcing through a prompt: pos += 1; tok = feed[pos]; hist[pos] = tok.
__global__ void advance_feed_kernel(const int32_t* __restrict__ feed, int feed_cap, int32_t* tok, int32_t* pos,
                                    int32_t* hist, int hist_len) {
  if (threadIdx.x != 0) return;
  const int p = pos[0] + 1;
  pos[0] = p;
  if (p >= 0 && p < feed_cap) {
    const int t = feed[p];
    tok[0] = t;
    if (hist != nullptr && p < hist_len) hist[p] = t;
  }
}

// Work units (row pairs, row groups or tasks) per block for the row walks:
// about gemv_blocks() blocks (one per CU by default; G4MI_GEMV_BLOCKS
// overrides it for tuning), 4 waves each, at least one unit per wave.
// The XCD-local router of ffn_in_kernel (on unless G4MI_FFN_IN_XCD=0).
static bool ffn_in_xcd_enabled() {
  const char* e = getenv("G4MI_FFN_IN_XCD");
  return e == nullptr || atoi(e) != 0;
}

static int gemv_blocks() {
  static const int n = [] {
    const char* e = getenv("G4MI_GEMV_BLOCKS");
    const int v = e ? atoi(e) : 0;
    return (v >= 16 && v <= 65536) ? v : 256;
  }();
  return n;
}
static int row_groups_per_block(int units) {
  const int nb = gemv_blocks();
  int per = (units + nb - 1) / nb;
  per = ((per + 3) / 4) * 4;
  return per < 4 ? 4 : per;
}

static float bf16_round_host(double v) {
  float f = (float)v;
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace g4mi

using namespace g4mi;

#define G4MI_IT16(M) M(1) M(2) M(3) M(4) M(5) M(6) M(7) M(8) M(9) M(10) M(11) M(12) M(13) M(14) M(15) M(16)

extern "C" {

int g4mi_layer_in(int32_t mode, const int32_t* tok, const uint16_t* embed, int64_t vocab, const uint16_t* x_in,
                  const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, const uint16_t* post_ff1_ln,
                  const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                  const uint16_t* input_ln, uint16_t* x_out, const uint16_t* wq, int64_t q_rows, const uint16_t* wk,
                  int64_t k_rows, const uint16_t* wv, int64_t v_rows, uint16_t* qkv_out, int64_t H, float eps,
                  void* stream) {
  G4MI_REQUIRE(mode >= 0 && mode <= 3, G4MI_EINVAL, "layer_in: bad mode %d", mode);
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "layer_in: H=%lld must be 256*i, i <= 16", (long long)H);
  G4MI_REQUIRE(qkv_out && wq && q_rows >= 1 && k_rows >= 0 && v_rows >= 0, G4MI_EINVAL, "layer_in: missing argument");
  G4MI_REQUIRE(mode == kInNormed || (input_ln && x_out), G4MI_EINVAL, "layer_in: missing input norm or x_out");
  G4MI_REQUIRE(mode != kInNormed || x_in, G4MI_EINVAL, "layer_in: normed mode needs x_in");
  G4MI_REQUIRE(mode != 0 || (tok && embed && vocab >= 1), G4MI_EINVAL, "layer_in: embed mode needs tok/embed");
  G4MI_REQUIRE(mode != 1 || (x1 && mlp_out && post_ff_ln && layer_scalar), G4MI_EINVAL,
               "layer_in: tail mode needs x1/mlp_out/post_ff_ln/layer_scalar");
  G4MI_REQUIRE(mode != 1 || moe_out == nullptr || (post_ff1_ln && post_ff2_ln), G4MI_EINVAL,
               "layer_in: tail mode with MoE needs post_feedforward_layernorm_1/2");
  G4MI_REQUIRE(mode != 2 || x_in, G4MI_EINVAL, "layer_in: plain mode needs x_in");
  G4MI_REQUIRE((k_rows == 0 || wk) && (v_rows == 0 || wv), G4MI_EINVAL, "layer_in: missing k/v weights");
  InArgs a;
  a.mode = mode; a.tok = tok; a.embed = embed; a.vocab = (int)vocab;
  a.embed_c = bf16_round_host((double)(float)sqrt((double)H));
  a.x_in = x_in;
  a.tail = TailArgs{x1, mlp_out, moe_out, post_ff1_ln, post_ff2_ln, post_ff_ln, layer_scalar};
  a.w_in = input_ln; a.x_out = x_out;
  a.W[0] = wq; a.W[1] = wk; a.W[2] = wv;
  a.rows[0] = (int)q_rows; a.rows[1] = (int)k_rows; a.rows[2] = (int)v_rows;
  a.out = qkv_out; a.H = (int)H; a.eps = eps;
  const int total = (int)(q_rows + k_rows + v_rows);
  const int npairs = (total + 1) / 2;
  // one block per CU: the pairs are not rounded up to a multiple of the 4
  // waves (the full 26B layer's 4,608 pairs are 18 per block on 256 CUs, not
  // 20 on 231; a CU streams its block's rows at its own rate, so the waves'
  // 5 or 4 pairs do not matter)
  a.pairs_per_block = max(1, (npairs + gemv_blocks() - 1) / gemv_blocks());
  dim3 grid((unsigned)((npairs + a.pairs_per_block - 1) / a.pairs_per_block));
  hipStream_t st = as_stream(stream);
  switch (H / 256) {
#define G4MI_C(I)                                                                                   \
  case I:                                                                                           \
    if (mode == kInEmbed) hipLaunchKernelGGL((layer_in_kernel<I, kInEmbed>), grid, dim3(256), 0, st, a); \
    else if (mode == kInTail) hipLaunchKernelGGL((layer_in_kernel<I, kInTail>), grid, dim3(256), 0, st, a); \
    else if (mode == kInPlain) hipLaunchKernelGGL((layer_in_kernel<I, kInPlain>), grid, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((layer_in_kernel<I, kInNormed>), grid, dim3(256), 0, st, a);          \
    break;
    G4MI_IT16(G4MI_C)
#undef G4MI_C
  }
  return check_launch("layer_in");
}

int g4mi_oproj(const uint16_t* ctx, const uint16_t* w, int64_t rows, int64_t K, uint16_t* out, void* stream) {
  G4MI_REQUIRE(ctx && w && out && rows >= 1, G4MI_EINVAL, "oproj: missing argument");
  hipStream_t st = as_stream(stream);
  if (K % 512 == 0 && K / 512 >= 1 && K / 512 <= 16) {
    const int ng = (int)rows, gpb = row_groups_per_block(ng);
    dim3 grid((unsigned)((ng + gpb - 1) / gpb));
    switch (K / 512) {
#define G4MI_C(I) case I: hipLaunchKernelGGL((oproj_kernel<64, I>), grid, dim3(256), 0, st, ctx, w, (int)rows, gpb, out); break;
      G4MI_IT16(G4MI_C)
#undef G4MI_C
    }
  } else if (K % 256 == 0 && K / 256 <= 16) {
    const int ng = (int)((rows + 1) / 2), gpb = row_groups_per_block(ng);
    dim3 grid((unsigned)((ng + gpb - 1) / gpb));
    switch (K / 256) {
#define G4MI_C(I) case I: hipLaunchKernelGGL((oproj_kernel<32, I>), grid, dim3(256), 0, st, ctx, w, (int)rows, gpb, out); break;
      G4MI_IT16(G4MI_C)
#undef G4MI_C
    }
  } else {
    G4MI_REQUIRE(false, G4MI_EUNSUPPORTED, "oproj: K=%lld must be 512*i or 256*i (i <= 16)", (long long)K);
  }
  return check_launch("oproj");
}

int64_t g4mi_ffn_in_workspace_bytes(void) { return 256; }

int g4mi_ffn_in(const uint16_t* x, const uint16_t* o, const uint16_t* post_attn_ln, const uint16_t* pre_ff_ln,
                const uint16_t* pre_ff2_ln, uint16_t* x1_out, uint16_t* xe_out, const uint16_t* gate,
                const uint16_t* up, int64_t I, uint16_t* act_mlp, const uint16_t* router_scale,
                const uint16_t* router_proj, int64_t E, float* scores, const uint16_t* per_expert_scale, int64_t k,
                float* top_w, int32_t* top_i, void* ws, int64_t ws_bytes, int64_t H, float eps, void* stream) {
  G4MI_REQUIRE(x && o && post_attn_ln && pre_ff_ln && x1_out && gate && up && act_mlp && I >= 1, G4MI_EINVAL,
               "ffn_in: missing argument");
  G4MI_REQUIRE(router_proj == nullptr || (router_scale && pre_ff2_ln && xe_out && scores && E >= 1 && E <= 65536),
               G4MI_EINVAL, "ffn_in: router needs scale, pre_ff_2 norm, xe_out and scores");
  G4MI_REQUIRE(per_expert_scale == nullptr || (router_proj && top_w && top_i && k >= 1 && k <= 32 && k <= E &&
                                               E <= 256 && ws && ws_bytes >= g4mi_ffn_in_workspace_bytes()),
               G4MI_EINVAL, "ffn_in: selection needs the router, top_w/top_i, 1 <= k <= 32, E <= 256, workspace");
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "ffn_in: H=%lld must be 256*i, i <= 16", (long long)H);
  FfnInArgs a;
  a.x = x; a.o = o; a.w_pa = post_attn_ln; a.w_pf = pre_ff_ln; a.w_pf2 = pre_ff2_ln;
  a.x1_out = x1_out; a.xe_out = xe_out; a.gate = gate; a.up = up; a.I = (int)I; a.act_mlp = act_mlp;
  // dense blocks fill the CUs the router blocks leave, with at most
  // 4 * kFfnInTasks tasks per block when that covers I
  const int rblocks_host = router_proj ? (int)((E + 7) / 8) : 0;
  const int dense_target = std::max(16, gemv_blocks() - rblocks_host);
  a.tasks_per_block = (int)std::max<int64_t>(1, (I + dense_target - 1) / dense_target);
  a.dense_blocks = (int)((I + a.tasks_per_block - 1) / a.tasks_per_block);
  a.r_scale = router_scale; a.r_proj = router_proj; a.E = router_proj ? (int)E : 0;
  a.r_c = bf16_round_host(1.0 / sqrt((double)H));
  a.scores = scores; a.H = (int)H; a.eps = eps;
  a.pes = per_expert_scale; a.K = (int)k; a.top_w = top_w; a.top_i = top_i; a.counter = (unsigned int*)ws;
  const int rblocks = router_proj ? (int)((E + 7) / 8) : 0;
  dim3 grid((unsigned)(a.dense_blocks + rblocks));
  a.xcd_local = rblocks > 0 && per_expert_scale != nullptr && a.dense_blocks >= 7 * rblocks && ffn_in_xcd_enabled() &&
                xcc_round_robin(as_stream(stream));
  hipStream_t st = as_stream(stream);
  switch (H / 256) {
#define G4MI_C(I) case I: hipLaunchKernelGGL(ffn_in_kernel<I>, grid, dim3(256), 0, st, a); break;
    G4MI_IT16(G4MI_C)
#undef G4MI_C
  }
  return check_launch("ffn_in");
}

int64_t g4mi_ffn_out_workspace_bytes(void) {
  // arrival counters of a grid of up to 4096 blocks (H <= 4096 rows, kOutRows per block)
  return 4 * kArriveStride * (1 + (4096 / kOutRows + kArriveGroup - 1) / kArriveGroup);
}

int g4mi_ffn_out(const uint16_t* act_mlp, const uint16_t* down, int64_t I, uint16_t* mlp_out,
                 const uint16_t* act_moe, const uint16_t* experts_down, const int32_t* top_i, int64_t E, int64_t k,
                 int64_t F, int32_t combine, uint16_t* moe_out, const uint16_t* x1, const uint16_t* post_ff1_ln,
                 const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                 const uint16_t* next_ln, uint16_t* x_out, uint16_t* xn_out, float eps, void* ws, int64_t ws_bytes,
                 int64_t H, void* stream) {
  G4MI_REQUIRE(act_mlp && down && mlp_out && H >= 1, G4MI_EINVAL, "ffn_out: missing argument");
  G4MI_REQUIRE(next_ln == nullptr || (x1 && post_ff_ln && layer_scalar && x_out && xn_out && ws &&
                                      ws_bytes >= g4mi_ffn_out_workspace_bytes()),
               G4MI_EINVAL, "ffn_out: the tail epilogue needs x1, post_ff norm, layer_scalar, x_out, xn_out, ws");
  G4MI_REQUIRE(next_ln == nullptr || experts_down == nullptr || (post_ff1_ln && post_ff2_ln), G4MI_EINVAL,
               "ffn_out: the tail epilogue with experts needs post_ff_1/post_ff_2 norms");
  G4MI_REQUIRE(next_ln == nullptr || (H % 8 == 0 && H <= 4096), G4MI_EUNSUPPORTED,
               "ffn_out: the tail epilogue needs H = 8*i <= 4096");
  G4MI_REQUIRE(I % 8 == 0 && I >= 8 && I <= 4096, G4MI_EUNSUPPORTED, "ffn_out: I=%lld must be 8*i <= 4096",
               (long long)I);
  G4MI_REQUIRE(experts_down == nullptr || (act_moe && top_i && moe_out && k >= 1 && k <= 8 && E >= 1), G4MI_EINVAL,
               "ffn_out: expert path needs act_moe/top_i/moe_out and 1 <= k <= 8");
  G4MI_REQUIRE(experts_down == nullptr || (F % 64 == 0 && F / 64 >= 1 && F / 64 <= 16), G4MI_EUNSUPPORTED,
               "ffn_out: F=%lld must be 64*i, i <= 16", (long long)F);
  G4MI_REQUIRE(combine == G4MI_COMBINE_BF16_RUNNING || combine == G4MI_COMBINE_F32, G4MI_EINVAL,
               "ffn_out: unknown combine mode %d", combine);
  FfnOutArgs a;
  a.act_mlp = act_mlp; a.down = down; a.I = (int)I; a.mlp_out = mlp_out;
  a.act_moe = act_moe; a.e_down = experts_down; a.top_i = top_i; a.E = (int)E; a.K = (int)k;
  a.bf16_running = combine == G4MI_COMBINE_BF16_RUNNING; a.moe_out = moe_out; a.H = (int)H;
  a.tail = TailArgs{x1, mlp_out, moe_out, post_ff1_ln, post_ff2_ln, post_ff_ln, layer_scalar};
  a.w_next = next_ln; a.x_out = x_out; a.xn_out = xn_out; a.counter = (unsigned int*)ws; a.eps = eps;
  dim3 grid((unsigned)((H + kOutRows - 1) / kOutRows));
  const size_t lds = (size_t)(I / 8 + (experts_down ? k * (F / 8) : 0)) * 16;
  hipStream_t st = as_stream(stream);
  const int fit = experts_down ? (int)(F / 64) : 1;
  switch (fit) {
#define G4MI_C(I) case I: hipLaunchKernelGGL(ffn_out_kernel<I>, grid, dim3(kOutThreads), lds, st, a); break;
    G4MI_IT16(G4MI_C)
#undef G4MI_C
  }
  return check_launch("ffn_out");
}

// lm_head rows per block: the vocabulary in about 3 * gemv_blocks() blocks,
// the number resident at once (3 per CU at 148 VGPRs), so no second, partial
// round of blocks trails the stream; a multiple of the 8 rows a block step takes
static int lm_rows_per_block(int64_t V) {
  const int64_t nb = 3 * (int64_t)gemv_blocks();
  const int64_t r = ((V + nb - 1) / nb + 7) / 8 * 8;
  return (int)std::max<int64_t>(8, r);
}

int64_t g4mi_lm_head_blocks(int64_t V) {
  const int r = lm_rows_per_block(V);
  return (V + r - 1) / r;
}

int g4mi_lm_head(const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, const uint16_t* post_ff1_ln,
                 const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln, const uint16_t* layer_scalar,
                 const uint16_t* final_norm, const uint16_t* embed, int64_t V, int64_t H, float softcap, float eps,
                 float* logits, float* blk_val, int32_t* blk_idx, void* stream) {
  G4MI_REQUIRE(x1 && mlp_out && post_ff_ln && layer_scalar && final_norm && embed && logits && blk_val && blk_idx,
               G4MI_EINVAL, "lm_head: missing argument");
  G4MI_REQUIRE(moe_out == nullptr || (post_ff1_ln && post_ff2_ln), G4MI_EINVAL,
               "lm_head: MoE tail needs post_feedforward_layernorm_1/2");
  G4MI_REQUIRE(V >= 1 && V <= (int64_t)1 << 30, G4MI_EINVAL, "lm_head: bad vocab");
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "lm_head: H=%lld must be 256*i, i <= 16", (long long)H);
  LmArgs a;
  a.tail = TailArgs{x1, mlp_out, moe_out, post_ff1_ln, post_ff2_ln, post_ff_ln, layer_scalar};
  a.w_norm = final_norm; a.embed = embed; a.V = (int)V; a.softcap = softcap; a.logits = logits;
  a.blk_val = blk_val; a.blk_idx = blk_idx; a.rows_per_block = lm_rows_per_block(V); a.H = (int)H; a.eps = eps;
  dim3 grid((unsigned)g4mi_lm_head_blocks(V));
  hipStream_t st = as_stream(stream);
  switch (H / 256) {
#define G4MI_C(I) case I: hipLaunchKernelGGL((lmhead_kernel<I, false>), grid, dim3(256), 0, st, a); break;
    G4MI_IT16(G4MI_C)
#undef G4MI_C
  }
  return check_launch("lm_head");
}

int g4mi_lm_head_normed(const uint16_t* xn, const uint16_t* embed, int64_t V, int64_t H, float softcap,
                        float* logits, float* blk_val, int32_t* blk_idx, void* stream) {
  G4MI_REQUIRE(xn && embed && logits && blk_val && blk_idx, G4MI_EINVAL, "lm_head_normed: missing argument");
  G4MI_REQUIRE(V >= 1 && V <= (int64_t)1 << 30, G4MI_EINVAL, "lm_head_normed: bad vocab");
  G4MI_REQUIRE(H % 256 == 0 && H / 256 >= 1 && H / 256 <= 16, G4MI_EUNSUPPORTED,
               "lm_head_normed: H=%lld must be 256*i, i <= 16", (long long)H);
  LmArgs a = {};
  a.xn = xn; a.embed = embed; a.V = (int)V; a.softcap = softcap; a.logits = logits;
  a.blk_val = blk_val; a.blk_idx = blk_idx; a.rows_per_block = lm_rows_per_block(V); a.H = (int)H;
  dim3 grid((unsigned)g4mi_lm_head_blocks(V));
  hipStream_t st = as_stream(stream);
  switch (H / 256) {
#define G4MI_C(I) case I: hipLaunchKernelGGL((lmhead_kernel<I, true>), grid, dim3(256), 0, st, a); break;
    G4MI_IT16(G4MI_C)
#undef G4MI_C
  }
  return check_launch("lm_head_normed");
}

int g4mi_argmax_finalize(const float* blk_val, const int32_t* blk_idx, int64_t n, int32_t* tok, int32_t* pos,
                         int32_t* hist, int64_t hist_len, void* stream) {
  G4MI_REQUIRE(blk_val && blk_idx && tok && n >= 1, G4MI_EINVAL, "argmax_finalize: missing argument");
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, as_stream(stream), blk_val, blk_idx, (int)n, tok, pos,
                     hist, (int)hist_len);
  return check_launch("argmax_finalize");
}

int g4mi_advance_feed(const int32_t* feed, int64_t feed_cap, int32_t* tok, int32_t* pos, int32_t* hist,
                      int64_t hist_len, void* stream) {
  G4MI_REQUIRE(feed && tok && pos && feed_cap >= 1 && feed_cap <= INT32_MAX, G4MI_EINVAL,
               "advance_feed: missing argument");
  hipLaunchKernelGGL(advance_feed_kernel, dim3(1), dim3(64), 0, as_stream(stream), feed, (int)feed_cap, tok, pos,
                     hist, (int)hist_len);
  return check_launch("advance_feed");
}

}  // extern "C"
