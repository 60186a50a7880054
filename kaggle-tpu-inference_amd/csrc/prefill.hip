// Batched prefill pieces: the dense-MoE prefill on MFMA (model.py:241-250)
// and the row-wise glue between the prefill GEMMs (model.py:297-322, 355-357).
//
// MoE prefill (K8).  The reference evaluates all E experts for every token
// and masks the result with the routing weights (w_full = 0 for experts a
// token did not select), so an unselected expert contributes act = bf16(x * 0)
// = 0 to the down contraction: exact zeros.  This path therefore runs only
// the selected (token, expert) pairs as grouped GEMMs, 16x fewer FLOPs at
// E = 128, k = 8, with the same rounding points:
//   1. moe_sort_kernel: tokens grouped by expert (counts, offsets, a gather
//      list, the per-slot routing weight) and 128- or 192-row GEMM tiles per
//      expert (one tile covers an expert's rows up to the tile height, so its
//      weights stream once);
//   2. gate/up GEMM over the gathered rows with the gated epilogue:
//      act = bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(w))   (model.py:246-247);
//   3. down GEMM, f32 output per (token, expert);
//   4. moe_combine_kernel: out[t] = bf16(sum over the token's slots in order)
//      -- one f32 sum over (expert, f) as the dense einsum (model.py:250).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "capi_util.h"
#include "common.h"
#include "rowvec.h"

namespace g4mi {

// gemm.hip: g4mi_gemm_bf16 with grouped tiles of up to tile_rows (128 or 192) rows
int gemm_bf16_tiles(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b, int64_t ldb,
                    int64_t b_group_stride, int64_t pair_offset, int64_t M, int64_t N, int64_t K,
                    const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles, int32_t epilogue, void* c,
                    int64_t ldc, const float* row_scale, int64_t k_slices, void* ws, int64_t ws_bytes, int tile_rows,
                    void* stream);

constexpr int kTileRows = 128;  // grouped GEMM tile height, the smaller of the two (gemm.hip's grouped tiles)
constexpr int kSortIpt = 16;    // routing items per thread per chunk in moe_sort_kernel
constexpr int kMaxExperts = 256;

// One block.  entries i = t*K + s (token t, slot s) of the routing.
//   sorted position p of entry i: offsets[e] + (rank among entries of expert e)
//   a_rows[p] = t, w_sorted[p] = top_w[i], slot_pos[i] = p (-1: invalid expert)
//   tiles: (e, m0, m1) for every tile_rows rows of every expert, ntiles[0] = count.
__global__ __launch_bounds__(1024) void moe_sort_kernel(const int32_t* __restrict__ top_i,
                                                        const float* __restrict__ top_w, int n, int K, int E,
                                                        int32_t* __restrict__ a_rows, float* __restrict__ w_sorted,
                                                        int32_t* __restrict__ slot_pos, int32_t* __restrict__ tiles,
                                                        int32_t* __restrict__ ntiles, int tile_rows) {
  __shared__ int cnt[kMaxExperts], off[kMaxExperts], cur[kMaxExperts], toff[kMaxExperts];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  const int total = n * K;
  // items in chunks of kSortIpt per thread: each chunk's loads are all in
  // flight before its LDS atomics (one memory round trip per chunk, not per
  // item); a single chunk (up to 16,384 items) stays in registers for the
  // scatter below
  const int stride = (int)blockDim.x;
  const bool one = total <= stride * kSortIpt;
  int ev[kSortIpt];
  float wv[kSortIpt];
  for (int i0 = 0; i0 < total; i0 += stride * kSortIpt) {
#pragma unroll
    for (int u = 0; u < kSortIpt; ++u) {
      const int i = i0 + u * stride + tid;
      ev[u] = (i < total) ? top_i[i] : -1;
      wv[u] = (i < total && one) ? top_w[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kSortIpt; ++u)
      if (ev[u] >= 0 && ev[u] < E) atomicAdd(&cnt[ev[u]], 1);
  }
  __syncthreads();
  // expert offsets and tile offsets: an exclusive scan over the experts in
  // one wave (lane l holds experts 4l .. 4l + 3, E <= 256)
  if (tid < 64) {
    int c[4], t[4], sc = 0, stl = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      c[q] = (e < E) ? cnt[e] : 0;
      t[q] = (c[q] + tile_rows - 1) / tile_rows;
      sc += c[q];
      stl += t[q];
    }
    int ic = sc, it = stl;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(ic, d, 64), z = __shfl_up(it, d, 64);
      if (tid >= d) {
        ic += y;
        it += z;
      }
    }
    int o = ic - sc, to = it - stl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      if (e < E) {
        off[e] = o;
        toff[e] = to;
        cur[e] = 0;
      }
      o += c[q];
      to += t[q];
    }
    if (tid == 63) ntiles[0] = it;
  }
  __syncthreads();
  for (int i0 = 0; i0 < total; i0 += stride * kSortIpt) {
    if (!one) {
#pragma unroll
      for (int u = 0; u < kSortIpt; ++u) {
        const int i = i0 + u * stride + tid;
        ev[u] = (i < total) ? top_i[i] : -1;
        wv[u] = (i < total) ? top_w[i] : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < kSortIpt; ++u) {
      const int i = i0 + u * stride + tid;
      if (i >= total) continue;
      const int e = ev[u];
      if (e >= 0 && e < E) {
        const int p = off[e] + atomicAdd(&cur[e], 1);
        a_rows[p] = i / K;
        w_sorted[p] = wv[u];
        slot_pos[i] = p;
      } else {
        slot_pos[i] = -1;
      }
    }
  }
  for (int e = tid; e < E; e += blockDim.x) {
    const int nt = (cnt[e] + tile_rows - 1) / tile_rows;
    for (int j = 0; j < nt; ++j) {
      int32_t* t = tiles + 3 * (toff[e] + j);
      t[0] = e;
      t[1] = off[e] + j * tile_rows;
      t[2] = min(off[e] + (j + 1) * tile_rows, off[e] + cnt[e]);
    }
  }
}

// The same sort for many entries, over several blocks in two launches (one
// block serialises its LDS atomics: 16,384 entries on 128 counters).  Block b
// of either launch owns entries [b * per, (b + 1) * per), per = kSortBlk *
// ipt.
//   moe_count_kernel: the block's per-expert counts -> hist[b][e];
//   moe_place_kernel: every block reads all counts, scans them (expert
//     offsets, this block's start within each expert, the tile offsets;
//     block 0 writes the tile list) and places its own entries, each at its
//     expert's offset + this block's start + its rank among the block's
//     entries of that expert.
// Rows of an expert may come in any order (each output row of the grouped
// GEMMs depends on its own row only, and the combine reads them through
// slot_pos), as in moe_sort_kernel, whose ranks come from LDS atomics too.
constexpr int kSortBlk = 1024;        // threads per block
constexpr int kSortMaxBlocks = 64;    // hist holds kSortMaxBlocks * kMaxExperts counts
constexpr int kSortIptMax = 16;       // entries per thread at most

__global__ __launch_bounds__(kSortBlk) void moe_count_kernel(const int32_t* __restrict__ top_i, int total, int ipt,
                                                             int E, int32_t* __restrict__ hist) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x, per = kSortBlk * ipt, i0 = (int)blockIdx.x * per;
  for (int e = tid; e < E; e += kSortBlk) cnt[e] = 0;
  __syncthreads();
  for (int u = 0; u < ipt; ++u) {
    const int i = i0 + u * kSortBlk + tid;
    const int e = (i < total) ? top_i[i] : -1;
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += kSortBlk) hist[(size_t)blockIdx.x * E + e] = cnt[e];
}

__global__ __launch_bounds__(kSortBlk) void moe_place_kernel(const int32_t* __restrict__ top_i,
                                                             const float* __restrict__ top_w, int total, int ipt,
                                                             int K, int E, const int32_t* __restrict__ hist,
                                                             int32_t* __restrict__ a_rows,
                                                             float* __restrict__ w_sorted,
                                                             int32_t* __restrict__ slot_pos,
                                                             int32_t* __restrict__ tiles,
                                                             int32_t* __restrict__ ntiles, int tile_rows) {
  __shared__ int cnt[kMaxExperts], off[kMaxExperts], cur[kMaxExperts], toff[kMaxExperts];
  __shared__ int hl[kSortMaxBlocks * kMaxExperts];
  const int tid = threadIdx.x, nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = kSortBlk * ipt, i0 = b * per;
  // this block's entries and every block's counts, all requested at once
  int ev[kSortIptMax];
  float wv[kSortIptMax];
#pragma unroll
  for (int u = 0; u < kSortIptMax; ++u) {
    const int i = i0 + u * kSortBlk + tid;
    ev[u] = (u < ipt && i < total) ? top_i[i] : -1;
    wv[u] = (u < ipt && i < total) ? top_w[i] : 0.0f;
  }
  for (int j = tid; j < nb * E; j += kSortBlk) hl[j] = hist[j];
  __syncthreads();
  // per expert: the total count, and the entries of the blocks before this one
  for (int e = tid; e < E; e += kSortBlk) {
    int t = 0, before = 0;
    for (int q = 0; q < nb; ++q) {
      const int c = hl[q * E + e];
      before += (q < b) ? c : 0;
      t += c;
    }
    cnt[e] = t;
    cur[e] = before;
  }
  __syncthreads();
  // expert offsets and tile offsets: an exclusive scan over the experts in
  // one wave (lane l holds experts 4l .. 4l + 3, E <= 256)
  if (tid < 64) {
    int c[4], t[4], sc = 0, stl = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      c[q] = (e < E) ? cnt[e] : 0;
      t[q] = (c[q] + tile_rows - 1) / tile_rows;
      sc += c[q];
      stl += t[q];
    }
    int ic = sc, it = stl;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(ic, d, 64), z = __shfl_up(it, d, 64);
      if (tid >= d) {
        ic += y;
        it += z;
      }
    }
    int o = ic - sc, to = it - stl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * tid + q;
      if (e < E) {
        off[e] = o;
        toff[e] = to;
      }
      o += c[q];
      to += t[q];
    }
    if (tid == 63 && b == 0) ntiles[0] = it;
  }
  __syncthreads();
  if (b == 0) {
    for (int e = tid; e < E; e += kSortBlk) {
      const int nt = (cnt[e] + tile_rows - 1) / tile_rows;
      for (int j = 0; j < nt; ++j) {
        int32_t* t = tiles + 3 * (toff[e] + j);
        t[0] = e;
        t[1] = off[e] + j * tile_rows;
        t[2] = min(off[e] + (j + 1) * tile_rows, off[e] + cnt[e]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kSortIptMax; ++u) {
    const int i = i0 + u * kSortBlk + tid;
    if (u >= ipt || i >= total) continue;
    const int e = ev[u];
    if (e >= 0 && e < E) {
      const int p = off[e] + atomicAdd(&cur[e], 1);
      a_rows[p] = i / K;
      w_sorted[p] = wv[u];
      slot_pos[i] = p;
    } else {
      slot_pos[i] = -1;
    }
  }
}

// out[t, h] = bf16(sum over s < K, in order, of part[slot_pos[t*K + s], h]) (f32),
// or with `running` the decode combine: a bf16 running sum of bf16(part) in
// slot order (model.py:289-293)
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ part,
                                                          const int32_t* __restrict__ slot_pos, int n, int K, int H,
                                                          int running, uint16_t* __restrict__ out) {
  // four consecutive h per thread (H % 4 == 0): every slot's float4 is
  // requested before the first is added
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (t >= n || h >= H) return;
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool first = true;
  for (int q0 = 0; q0 < K; q0 += 8) {
    float4 v[8];
    int pv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      pv[u] = (q0 + u < K) ? slot_pos[t * K + q0 + u] : -1;
      v[u] = *(const float4*)(part + (size_t)max(pv[u], 0) * H + h);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (pv[u] < 0) continue;
      const float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (running) {
          const float b = rbf(x[i]);
          s[i] = first ? b : rbf(s[i] + b);
        } else {
          s[i] += x[i];
        }
      }
      first = false;
    }
  }
  uint2 o;
  o.x = pack2(s[0], s[1]);
  o.y = pack2(s[2], s[3]);
  *(uint2*)(out + (size_t)t * H + h) = o;
}

// ------------------------------------------------------------------ grouped decode experts
// A decode step of n <= 16 tokens with their routing (model.py:262-294 per
// token): after moe_sort_kernel every expert's (token, slot) pairs form one
// tile, so each selected expert's rows stream from HBM once for all the
// tokens that chose it, as GEMV row walks (the union of the routed experts,
// not one read per pair).  The dot products use the decode kernels' lane
// layout and order, so act and the partials equal moe_gateup / moe_down's.
constexpr int kGrpPairs = 4;   // gate/up row pairs per wave
constexpr int kGrpDownRows = 2;  // down rows per 8-lane group

// act[p, f] = bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(w_sorted[p]))
// for the pairs p of tile blockIdx.x; wave w of block y takes row pairs
// f = (4y + w) * kGrpPairs + r (lanes 0-31 the gate row, 32-63 the up row).
template <int IT>
__global__ __launch_bounds__(256) void moe_gateup_grouped_kernel(const uint16_t* __restrict__ xn,
                                                                 const uint16_t* __restrict__ gate_up,
                                                                 const int32_t* __restrict__ a_rows,
                                                                 const float* __restrict__ w_sorted,
                                                                 const int32_t* __restrict__ tiles,
                                                                 const int32_t* __restrict__ ntiles, int F,
                                                                 uint16_t* __restrict__ act) {
  constexpr int H = IT * 256;
  const int tile = blockIdx.x;
  if (tile >= ntiles[0]) return;
  const int e = tiles[3 * tile], m0 = tiles[3 * tile + 1], m1 = tiles[3 * tile + 2];
  const int lane = threadIdx.x & 63, half = lane >> 5, l = lane & 31, wave = wave_id();
  const int fb = (blockIdx.y * 4 + wave) * kGrpPairs;
  u32x4 w[kGrpPairs][IT];
#pragma unroll
  for (int r = 0; r < kGrpPairs; ++r) {
    const u32x4* row = (const u32x4*)(gate_up + ((size_t)(e * 2 + half) * F + min(fb + r, F - 1)) * H);
#pragma unroll
    for (int i = 0; i < IT; ++i) w[r][i] = ld_stream(row + l + 32 * i);
  }
  for (int p = m0; p < m1; ++p) {
    const u32x4* xv = (const u32x4*)(xn + (size_t)a_rows[p] * H);
    u32x4 xr[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) xr[i] = ld16(xv + l + 32 * i);
    const float wt = rbf(w_sorted[p]);
#pragma unroll
    for (int r = 0; r < kGrpPairs; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < IT; ++i) acc = dot8(w[r][i], xr[i], acc);
      acc = group_sum<32>(acc);
      const float up = __shfl(acc, 32, kWave);
      if (lane == 0 && fb + r < F)
        act[(size_t)p * F + fb + r] = f2bf(rbf(rbf(rbf(gelu_tanh(rbf(acc))) * rbf(up)) * wt));
    }
  }
}

// part[p, h] = act[p] . down[e, h] (f32) for the pairs p of tile blockIdx.x;
// 8-lane group g of wave w in block y takes rows h = ((4y + w) * 8 + g) *
// kGrpDownRows + r.
template <int FIT>
__global__ __launch_bounds__(256) void moe_down_grouped_kernel(const uint16_t* __restrict__ act,
                                                               const uint16_t* __restrict__ down,
                                                               const int32_t* __restrict__ tiles,
                                                               const int32_t* __restrict__ ntiles, int H,
                                                               float* __restrict__ part) {
  constexpr int F = FIT * 64;
  const int tile = blockIdx.x;
  if (tile >= ntiles[0]) return;
  const int e = tiles[3 * tile], m0 = tiles[3 * tile + 1], m1 = tiles[3 * tile + 2];
  const int lane = threadIdx.x & 63, g = lane >> 3, l8 = lane & 7, wave = wave_id();
  const int hb = ((blockIdx.y * 4 + wave) * 8 + g) * kGrpDownRows;
  u32x4 wd[kGrpDownRows][FIT];
#pragma unroll
  for (int r = 0; r < kGrpDownRows; ++r) {
    const u32x4* row = (const u32x4*)(down + ((size_t)e * H + min(hb + r, H - 1)) * F);
#pragma unroll
    for (int i = 0; i < FIT; ++i) wd[r][i] = ld_stream(row + l8 + 8 * i);
  }
  for (int p = m0; p < m1; ++p) {
    const u32x4* av = (const u32x4*)(act + (size_t)p * F);
    u32x4 ar[FIT];
#pragma unroll
    for (int i = 0; i < FIT; ++i) ar[i] = ld16(av + l8 + 8 * i);
#pragma unroll
    for (int r = 0; r < kGrpDownRows; ++r) {
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < FIT; ++i) d = dot8(wd[r][i], ar[i], d);
      d = group_sum<8>(d);
      if (l8 == 0 && hb + r < H) part[(size_t)p * H + hb + r] = d;
    }
  }
}

// ------------------------------------------------------------------ row kernels
// One block per token row, the row held as a VecT<256> (H <= 4096).  The
// arithmetic is the decode kernels' prologue arithmetic (rowvec.h), so the
// prefill and the decode steps round identically.

// x[t] = bf16(embed[tok[t]] * bf16(sqrt(H))) (model.py:355-357); xn[t] =
// rms_norm(x[t], input_layernorm) (model.py:298).
__global__ __launch_bounds__(256) void rows_embed_kernel(const int32_t* __restrict__ tok,
                                                         const uint16_t* __restrict__ embed, int vocab, float c,
                                                         const uint16_t* __restrict__ w_in, int H, float eps,
                                                         uint16_t* __restrict__ x_out, uint16_t* __restrict__ xn_out) {
  __shared__ double red[8];
  const int t = blockIdx.x, nch = H / 8;
  int id = tok[t];
  id = (id < 0 || id >= vocab) ? 0 : id;
  Vec x, w;
  vload(x, embed + (size_t)id * H, nch);
  vload(w, w_in, nch);
  vmul(x, c);
  const float r = vrms(x, H, eps, red);
  vstore(x, (u32x4*)(x_out + (size_t)t * H), nch);
  vscale_w(x, r, w);
  vstore(x, (u32x4*)(xn_out + (size_t)t * H), nch);
}

// x1 = bf16(x + rms_norm(o, post_attention_layernorm)); xm = rms_norm(x1,
// pre_feedforward_layernorm); xe = rms_norm(x1, pre_feedforward_layernorm_2)
// (model.py:301-315; xe only with the MoE block).
__global__ __launch_bounds__(256) void rows_post_attn_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ o,
                                                             const uint16_t* __restrict__ w_pa,
                                                             const uint16_t* __restrict__ w_pf,
                                                             const uint16_t* __restrict__ w_pf2, int H, float eps,
                                                             uint16_t* __restrict__ x1_out,
                                                             uint16_t* __restrict__ xm_out,
                                                             uint16_t* __restrict__ xe_out) {
  __shared__ double red[8];
  const int t = blockIdx.x, nch = H / 8;
  const size_t ro = (size_t)t * H;
  Vec xv, ov, wpa, wf, wf2;
  vload(ov, o + ro, nch);
  vload(xv, x + ro, nch);
  vload(wpa, w_pa, nch);
  vload(wf, w_pf, nch);
  if (xe_out != nullptr) vload(wf2, w_pf2, nch);
  vscale_w(ov, vrms(ov, H, eps, red), wpa);
  vadd(xv, ov);
  vstore(xv, (u32x4*)(x1_out + ro), nch);
  const float r1 = vrms(xv, H, eps, red);
  Vec xm = xv;
  vscale_w(xm, r1, wf);
  vstore(xm, (u32x4*)(xm_out + ro), nch);
  if (xe_out != nullptr) {
    vscale_w(xv, r1, wf2);
    vstore(xv, (u32x4*)(xe_out + ro), nch);
  }
}

// x = the layer tail of (x1, mlp, moe) (model.py:312-322); xn =
// rms_norm(x, next input_layernorm) (model.py:298).
__global__ __launch_bounds__(256) void rows_tail_kernel(TailArgs ta, const uint16_t* __restrict__ w_next, int H,
                                                        float eps, uint16_t* __restrict__ x_out,
                                                        uint16_t* __restrict__ xn_out) {
  __shared__ double red[16];
  const int t = blockIdx.x, nch = H / 8;
  const size_t ro = (size_t)t * H;
  TailArgs tr = ta;
  tr.x1 += ro;
  tr.mlp += ro;
  if (tr.moe != nullptr) tr.moe += ro;
  TailRegs<256> T;
  Vec x, wn;
  tail_load(T, tr, nch);
  vload(wn, w_next, nch);
  tail_compute(x, T, tr.moe != nullptr, H, eps, red);
  const float r = vrms<256, true>(x, H, eps, red + 12);
  vstore(x, (u32x4*)(x_out + ro), nch);
  vscale_w(x, r, wn);
  vstore(x, (u32x4*)(xn_out + ro), nch);
}

// rows_tail_kernel with the MoE output combined here: moe[t, h] =
// bf16(sum over s < K, in order, of part[slot_pos[t*K + s], h]) (f32, as
// moe_combine_kernel), then the tail.  Every slot's part chunks of this
// thread are requested with the other operands, before the first add.
constexpr int kTailSlots = 8;  // slots summed per pass
__global__ __launch_bounds__(256) void rows_tail_combine_kernel(TailArgs ta, const float* __restrict__ part,
                                                                const int32_t* __restrict__ slot_pos, int K,
                                                                const uint16_t* __restrict__ w_next, int H, float eps,
                                                                uint16_t* __restrict__ x_out,
                                                                uint16_t* __restrict__ xn_out) {
  __shared__ double red[16];
  const int t = blockIdx.x, nch = H / 8;
  const size_t ro = (size_t)t * H;
  TailRegs<256> T;
  Vec x, wn;
  vload(T.a, ta.mlp + ro, nch);
  vload(T.x1, ta.x1 + ro, nch);
  vload(T.w3, ta.w_pf, nch);
  vload(T.w1, ta.w_pf1, nch);
  vload(T.w2, ta.w_pf2, nch);
  T.ls = ta.ls[0];
  vload(wn, w_next, nch);
  float s[Vec::NC][8];
#pragma unroll
  for (int j = 0; j < Vec::NC; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) s[j][i] = 0.0f;
  for (int q0 = 0; q0 < K; q0 += kTailSlots) {
    int pv[kTailSlots];
    float4 v[kTailSlots][Vec::NC][2];
#pragma unroll
    for (int u = 0; u < kTailSlots; ++u) {
      pv[u] = (q0 + u < K) ? slot_pos[(size_t)t * K + q0 + u] : -1;
#pragma unroll
      for (int j = 0; j < Vec::NC; ++j) {
        const int c = min((int)threadIdx.x + 256 * j, nch - 1);
        const float4* src = (const float4*)(part + (size_t)max(pv[u], 0) * H + 8 * c);
        v[u][j][0] = src[0];
        v[u][j][1] = src[1];
      }
    }
#pragma unroll
    for (int u = 0; u < kTailSlots; ++u) {
      if (pv[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < Vec::NC; ++j) {
        s[j][0] += v[u][j][0].x; s[j][1] += v[u][j][0].y; s[j][2] += v[u][j][0].z; s[j][3] += v[u][j][0].w;
        s[j][4] += v[u][j][1].x; s[j][5] += v[u][j][1].y; s[j][6] += v[u][j][1].z; s[j][7] += v[u][j][1].w;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < Vec::NC; ++j) {
    const int c = (int)threadIdx.x + 256 * j;
    u32x4 o;
    o.x = pack2(s[j][0], s[j][1]); o.y = pack2(s[j][2], s[j][3]);
    o.z = pack2(s[j][4], s[j][5]); o.w = pack2(s[j][6], s[j][7]);
    T.b.c[j] = (c < nch) ? o : u32x4{0u, 0u, 0u, 0u};
  }
  tail_compute(x, T, true, H, eps, red);
  const float r = vrms<256, true>(x, H, eps, red + 12);
  vstore(x, (u32x4*)(x_out + ro), nch);
  vscale_w(x, r, wn);
  vstore(x, (u32x4*)(xn_out + ro), nch);
}

static int64_t al256(int64_t x) { return ((x + 255) / 256) * 256; }

static float bf16_round_host(double v) {
  float f = (float)v;
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}

// Expert tile height: 192 rows while the experts average 96 to 176 rows (an
// expert's rows then mostly spill past 128 but fit 192, and every further
// tile of an expert streams its weights again), else 128.
// G4MI_MOE_TILE_ROWS = 128 or 192 overrides.
static int moe_prefill_tile_rows(int64_t pairs, int64_t E) {
  const char* e = getenv("G4MI_MOE_TILE_ROWS");
  if (e != nullptr && (atoi(e) == 128 || atoi(e) == 192)) return atoi(e);
  return (pairs >= 96 * E && pairs < 176 * E) ? 192 : 128;
}

struct MoePrefillWs {
  int32_t *a_rows, *slot_pos, *tiles, *ntiles, *hist;
  float *w_sorted, *part;
  uint16_t* act;
};

static MoePrefillWs moe_prefill_ws(void* ws, int64_t n, int64_t K, int64_t E, int64_t F, int64_t H) {
  const int64_t nk = n * K, max_tiles = (nk + kTileRows - 1) / kTileRows + E;
  char* p = (char*)ws;
  MoePrefillWs w;
  w.a_rows = (int32_t*)p; p += al256(nk * 4);
  w.slot_pos = (int32_t*)p; p += al256(nk * 4);
  w.tiles = (int32_t*)p; p += al256(max_tiles * 12);
  w.ntiles = (int32_t*)p; p += 256;
  w.w_sorted = (float*)p; p += al256(nk * 4);
  w.hist = (int32_t*)p; p += al256((int64_t)kSortMaxBlocks * kMaxExperts * 4);
  w.act = (uint16_t*)p; p += al256(nk * F * 2);
  w.part = (float*)p;
  return w;
}

// Groups the (token, slot) entries by expert and lists the expert tiles: one
// block up to kSortIpt entries per thread, else the two-launch form.
static void launch_moe_sort(const int32_t* top_i, const float* top_w, int n, int K, int E, const MoePrefillWs& w,
                            int tile_rows, hipStream_t st) {
  const int total = n * K;
  const int ipt = (total + kSortBlk * kSortMaxBlocks - 1) / (kSortBlk * kSortMaxBlocks);
  const char* one = getenv("G4MI_MOE_SORT_ONE_BLOCK");
  if (total <= 4 * kSortBlk || ipt > kSortIptMax || (one != nullptr && atoi(one) != 0)) {
    hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(1024), 0, st, top_i, top_w, n, K, E, w.a_rows, w.w_sorted,
                       w.slot_pos, w.tiles, w.ntiles, tile_rows);
    return;
  }
  const int nb = (total + kSortBlk * ipt - 1) / (kSortBlk * ipt);  // <= kSortMaxBlocks
  hipLaunchKernelGGL(moe_count_kernel, dim3((unsigned)nb), dim3(kSortBlk), 0, st, top_i, total, ipt, E, w.hist);
  hipLaunchKernelGGL(moe_place_kernel, dim3((unsigned)nb), dim3(kSortBlk), 0, st, top_i, top_w, total, ipt, K, E,
                     w.hist, w.a_rows, w.w_sorted, w.slot_pos, w.tiles, w.ntiles, tile_rows);
}

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int64_t g4mi_moe_prefill_workspace_bytes(int64_t n, int64_t K, int64_t E, int64_t F, int64_t H) {
  const int64_t nk = n * K, max_tiles = (nk + kTileRows - 1) / kTileRows + E;
  return 3 * al256(nk * 4) + al256(max_tiles * 12) + 256 + al256((int64_t)kSortMaxBlocks * kMaxExperts * 4) +
         al256(nk * F * 2) + al256(nk * H * 4);
}

int g4mi_moe_prefill(const uint16_t* xn, const float* top_w, const int32_t* top_i, const uint16_t* gate_up,
                     const uint16_t* down, int64_t n, int64_t H, int64_t F, int64_t E, int64_t K, uint16_t* out,
                     void* ws, int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(xn && top_w && top_i && gate_up && down && ws, G4MI_EINVAL, "moe_prefill: missing argument");
  G4MI_REQUIRE(n >= 1 && n <= 65535 && K >= 1 && K <= 32 && E >= 1 && E <= kMaxExperts, G4MI_EINVAL,
               "moe_prefill: bad n/K/E");
  G4MI_REQUIRE(H % 64 == 0 && F % 64 == 0, G4MI_EUNSUPPORTED, "moe_prefill: H and F must be multiples of 64");
  G4MI_REQUIRE(ws_bytes >= g4mi_moe_prefill_workspace_bytes(n, K, E, F, H), G4MI_EWORKSPACE,
               "moe_prefill: workspace too small");
  hipStream_t st = as_stream(stream);
  const MoePrefillWs w = moe_prefill_ws(ws, n, K, E, F, H);
  const int tile_rows = moe_prefill_tile_rows(n * K, E);
  const int64_t max_tiles = (n * K + tile_rows - 1) / tile_rows + E;
  launch_moe_sort(top_i, top_w, (int)n, (int)K, (int)E, w, tile_rows, st);
  int rc = check_launch("moe_prefill sort");
  if (rc) return rc;
  // gate/up: gathered token rows x the expert's (gate, up) rows -> act [n*K, F]
  rc = gemm_bf16_tiles(xn, H, w.a_rows, gate_up, H, 2 * F * H, F * H, n * K, F, H, w.tiles, w.ntiles, max_tiles,
                       2, w.act, F, w.w_sorted, 1, nullptr, 0, tile_rows, stream);
  if (rc) return rc;
  // down: act rows x the expert's down rows -> f32 partial [n*K, H]
  rc = gemm_bf16_tiles(w.act, F, nullptr, down, F, H * F, 0, n * K, H, F, w.tiles, w.ntiles, max_tiles, 1, w.part,
                       H, nullptr, 1, nullptr, 0, tile_rows, stream);
  if (rc) return rc;
  if (out == nullptr) return 0;  // the per-slot outputs stay in ws (g4mi_rows_tail_experts combines them)
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H / 4 + 255) / 256), (unsigned)n), dim3(256), 0, st, w.part,
                     w.slot_pos, (int)n, (int)K, (int)H, 0, out);
  return check_launch("moe_prefill combine");
}

int g4mi_moe_decode_grouped(const uint16_t* xn, const float* top_w, const int32_t* top_i, const uint16_t* gate_up,
                            const uint16_t* down, int64_t n, int64_t H, int64_t F, int64_t E, int64_t K,
                            int32_t combine, uint16_t* out, void* ws, int64_t ws_bytes, void* stream) {
  G4MI_REQUIRE(xn && top_w && top_i && gate_up && down && out && ws, G4MI_EINVAL,
               "moe_decode_grouped: missing argument");
  G4MI_REQUIRE(n >= 1 && n <= 16 && K >= 1 && K <= 32 && E >= 1 && E <= kMaxExperts, G4MI_EINVAL,
               "moe_decode_grouped: n=%lld (at most 16 tokens), K=%lld, E=%lld", (long long)n, (long long)K,
               (long long)E);
  G4MI_REQUIRE(H % 256 == 0 && H / 256 <= 16 && F % 64 == 0 && F / 64 >= 1 && F / 64 <= 16, G4MI_EUNSUPPORTED,
               "moe_decode_grouped: H=%lld must be 256*i (i <= 16), F=%lld 64*j (j <= 16)", (long long)H,
               (long long)F);
  G4MI_REQUIRE(combine == 0 || combine == 1, G4MI_EINVAL, "moe_decode_grouped: bad combine %d", combine);
  G4MI_REQUIRE(((uintptr_t)xn & 15u) == 0 && ((uintptr_t)gate_up & 15u) == 0 && ((uintptr_t)down & 15u) == 0,
               G4MI_EALIGN, "moe_decode_grouped: operands must be 16-byte aligned");
  G4MI_REQUIRE(ws_bytes >= g4mi_moe_prefill_workspace_bytes(n, K, E, F, H), G4MI_EWORKSPACE,
               "moe_decode_grouped: workspace too small (g4mi_moe_prefill_workspace_bytes)");
  hipStream_t st = as_stream(stream);
  const MoePrefillWs w = moe_prefill_ws(ws, n, K, E, F, H);
  // at most n <= 16 pairs per expert: one tile per selected expert
  const int tiles = (int)(n * K < E ? n * K : E);
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(1024), 0, st, top_i, top_w, (int)n, (int)K, (int)E, w.a_rows,
                     w.w_sorted, w.slot_pos, w.tiles, w.ntiles, kTileRows);
  const dim3 ggrid((unsigned)tiles, (unsigned)((F + 4 * kGrpPairs - 1) / (4 * kGrpPairs)));
  switch (H / 256) {
#define G4MI_GU(I)                                                                                             \
  case I:                                                                                                      \
    hipLaunchKernelGGL(moe_gateup_grouped_kernel<I>, ggrid, dim3(256), 0, st, xn, gate_up, w.a_rows, w.w_sorted, \
                       w.tiles, w.ntiles, (int)F, w.act);                                                     \
    break;
    G4MI_GU(1) G4MI_GU(2) G4MI_GU(3) G4MI_GU(4) G4MI_GU(5) G4MI_GU(6) G4MI_GU(7) G4MI_GU(8)
    G4MI_GU(9) G4MI_GU(10) G4MI_GU(11) G4MI_GU(12) G4MI_GU(13) G4MI_GU(14) G4MI_GU(15) G4MI_GU(16)
#undef G4MI_GU
  }
  const dim3 dgrid((unsigned)tiles, (unsigned)((H + 32 * kGrpDownRows - 1) / (32 * kGrpDownRows)));
  switch (F / 64) {
#define G4MI_DN(I)                                                                                              \
  case I:                                                                                                       \
    hipLaunchKernelGGL(moe_down_grouped_kernel<I>, dgrid, dim3(256), 0, st, w.act, down, w.tiles, w.ntiles,     \
                       (int)H, w.part);                                                                         \
    break;
    G4MI_DN(1) G4MI_DN(2) G4MI_DN(3) G4MI_DN(4) G4MI_DN(5) G4MI_DN(6) G4MI_DN(7) G4MI_DN(8)
    G4MI_DN(9) G4MI_DN(10) G4MI_DN(11) G4MI_DN(12) G4MI_DN(13) G4MI_DN(14) G4MI_DN(15) G4MI_DN(16)
#undef G4MI_DN
  }
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H / 4 + 255) / 256), (unsigned)n), dim3(256), 0, st, w.part,
                     w.slot_pos, (int)n, (int)K, (int)H, combine == 0 ? 1 : 0, out);
  return check_launch("moe_decode_grouped");
}

int g4mi_rows_embed(const int32_t* tok, int64_t n, const uint16_t* embed, int64_t vocab, const uint16_t* input_ln,
                    int64_t H, float eps, uint16_t* x_out, uint16_t* xn_out, void* stream) {
  G4MI_REQUIRE(tok && embed && input_ln && x_out && xn_out && vocab >= 1, G4MI_EINVAL, "rows_embed: missing argument");
  G4MI_REQUIRE(n >= 1 && n <= 2147483647 && H % 8 == 0 && H >= 8 && H <= 4096, G4MI_EUNSUPPORTED,
               "rows_embed: n=%lld H=%lld (H = 8*i <= 4096)", (long long)n, (long long)H);
  const float c = bf16_round_host((double)(float)sqrt((double)H));
  hipLaunchKernelGGL(rows_embed_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), tok, embed, (int)vocab,
                     c, input_ln, (int)H, eps, x_out, xn_out);
  return check_launch("rows_embed");
}

int g4mi_rows_post_attn(const uint16_t* x, const uint16_t* o, int64_t n, const uint16_t* post_attn_ln,
                        const uint16_t* pre_ff_ln, const uint16_t* pre_ff2_ln, int64_t H, float eps, uint16_t* x1_out,
                        uint16_t* xm_out, uint16_t* xe_out, void* stream) {
  G4MI_REQUIRE(x && o && post_attn_ln && pre_ff_ln && x1_out && xm_out, G4MI_EINVAL, "rows_post_attn: missing argument");
  G4MI_REQUIRE(xe_out == nullptr || pre_ff2_ln, G4MI_EINVAL, "rows_post_attn: xe needs pre_feedforward_layernorm_2");
  G4MI_REQUIRE(n >= 1 && n <= 2147483647 && H % 8 == 0 && H >= 8 && H <= 4096, G4MI_EUNSUPPORTED,
               "rows_post_attn: n=%lld H=%lld (H = 8*i <= 4096)", (long long)n, (long long)H);
  hipLaunchKernelGGL(rows_post_attn_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), x, o, post_attn_ln,
                     pre_ff_ln, pre_ff2_ln, (int)H, eps, x1_out, xm_out, xe_out);
  return check_launch("rows_post_attn");
}

int g4mi_rows_tail(const uint16_t* x1, const uint16_t* mlp_out, const uint16_t* moe_out, int64_t n,
                   const uint16_t* post_ff1_ln, const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln,
                   const uint16_t* layer_scalar, const uint16_t* next_ln, int64_t H, float eps, uint16_t* x_out,
                   uint16_t* xn_out, void* stream) {
  G4MI_REQUIRE(x1 && mlp_out && post_ff_ln && layer_scalar && next_ln && x_out && xn_out, G4MI_EINVAL,
               "rows_tail: missing argument");
  G4MI_REQUIRE(moe_out == nullptr || (post_ff1_ln && post_ff2_ln), G4MI_EINVAL,
               "rows_tail: the MoE tail needs post_feedforward_layernorm_1/2");
  G4MI_REQUIRE(n >= 1 && n <= 2147483647 && H % 8 == 0 && H >= 8 && H <= 4096, G4MI_EUNSUPPORTED,
               "rows_tail: n=%lld H=%lld (H = 8*i <= 4096)", (long long)n, (long long)H);
  const TailArgs ta{x1, mlp_out, moe_out, post_ff1_ln, post_ff2_ln, post_ff_ln, layer_scalar};
  hipLaunchKernelGGL(rows_tail_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), ta, next_ln, (int)H, eps,
                     x_out, xn_out);
  return check_launch("rows_tail");
}

int g4mi_rows_tail_experts(const uint16_t* x1, const uint16_t* mlp_out, int64_t n, int64_t K, int64_t E, int64_t F,
                           const uint16_t* post_ff1_ln, const uint16_t* post_ff2_ln, const uint16_t* post_ff_ln,
                           const uint16_t* layer_scalar, const uint16_t* next_ln, int64_t H, float eps,
                           uint16_t* x_out, uint16_t* xn_out, const void* moe_ws, int64_t moe_ws_bytes,
                           void* stream) {
  G4MI_REQUIRE(x1 && mlp_out && post_ff1_ln && post_ff2_ln && post_ff_ln && layer_scalar && next_ln && x_out &&
                   xn_out && moe_ws,
               G4MI_EINVAL, "rows_tail_experts: missing argument");
  G4MI_REQUIRE(n >= 1 && n <= 65535 && K >= 1 && K <= 32 && E >= 1 && E <= kMaxExperts, G4MI_EINVAL,
               "rows_tail_experts: bad n/K/E");
  G4MI_REQUIRE(H % 64 == 0 && H <= 4096 && F % 64 == 0, G4MI_EUNSUPPORTED,
               "rows_tail_experts: H=%lld F=%lld (multiples of 64, H <= 4096)", (long long)H, (long long)F);
  G4MI_REQUIRE(moe_ws_bytes >= g4mi_moe_prefill_workspace_bytes(n, K, E, F, H), G4MI_EWORKSPACE,
               "rows_tail_experts: workspace smaller than the moe_prefill one it reads");
  const MoePrefillWs w = moe_prefill_ws(const_cast<void*>(moe_ws), n, K, E, F, H);
  const TailArgs ta{x1, mlp_out, nullptr, post_ff1_ln, post_ff2_ln, post_ff_ln, layer_scalar};
  hipLaunchKernelGGL(rows_tail_combine_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), ta, w.part,
                     w.slot_pos, (int)K, next_ln, (int)H, eps, x_out, xn_out);
  return check_launch("rows_tail_experts");
}

}  // extern "C"
