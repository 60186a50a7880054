// Decode attention over a paged bf16 KV cache (model.py:197-213).
//
// Cache layout per layer: pages [num_pages, KV, PAGE, D] bf16 for K and for V
// (the reference keeps separate K and V even for k==v layers, model.py:201-206);
// a page table [B, max_pages] int32 maps position p of sequence b to page
// pt[b][p / PAGE], slot p % PAGE.  One (page, kv head) is PAGE*D contiguous
// values, so a split of consecutive positions streams contiguous memory.
//
// Two kernels per call, split-K over positions (grid: splits x KV heads x B):
//   qk: q = rope(rms_norm(q_raw, q_norm)) for the G query heads of a KV
//       head; the block whose split ends at `pos` also builds
//       k = rope(rms_norm(k_raw, k_norm)), v = rms_norm(v_raw) and appends
//       them to the cache; s = f32(bf16(q . k)) (scale 1.0) on MFMA,
//       optional softcap, causal/sliding range; per-split max and sum of exp.
//   pv: merges the split statistics, p = bf16(exp(s - m) / sum) -- the
//       reference rounds the normalised probabilities to bf16 before the
//       PV product (model.py:212) -- and accumulates p . V in f32.  Up to
//       kShortLen attended positions a block owns a kSliceD-wide slice of
//       the head dims over all positions and writes ctx = bf16(sum)
//       directly; longer ranges take split partials reduced in a fixed
//       order by the last split to finish.
// Masked positions contribute exp(-1e30 - m) = 0 in the reference, so only the
// attended range [lo, pos] is visited.
//
// Device-side positions and page indices are range-checked: an out-of-range
// position attends to nothing (ctx = 0, no cache write) and an out-of-range
// page entry is skipped, so bad inputs cannot address outside the buffers.
#include <cstdlib>
#include <mutex>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

constexpr int kChunkMin = 64;   // positions per split, at least
constexpr int kChunkMax = 256;  // positions per split, at most (LDS score buffer)

struct AttnDims {
  int B, NH, KV, G, D, page, max_pages, num_pages, window, n_split_max, lmax;
  float softcap, eps;
};

// Attended range of a sequence at position `pos`, cut into n_eff splits.
struct Range {
  int lo, len, chunk, n_eff;
};
__device__ __forceinline__ Range attn_range(const AttnDims& a, int pos) {
  Range r;
  if (pos < 0 || pos >= a.lmax || pos >= a.max_pages * a.page) {
    r.lo = 0; r.len = 0; r.chunk = kChunkMin; r.n_eff = 0;
    return r;
  }
  const int end = pos + 1;
  r.lo = (a.window > 0) ? max(0, end - a.window) : 0;
  r.len = end - r.lo;
  r.chunk = max((r.len + a.n_split_max - 1) / a.n_split_max, kChunkMin);
  r.n_eff = (r.len + r.chunk - 1) / r.chunk;
  return r;
}

// Element offset of (position p, kv head) in the page pool, or -1 when the
// page table entry is out of range.
__device__ __forceinline__ long long page_off(const AttnDims& a, const int32_t* pt_row, int p, int kv) {
  const int page = pt_row[p / a.page];
  if (page < 0 || page >= a.num_pages) return -1;
  return ((((long long)page * a.KV + kv) * a.page) + (p % a.page)) * (long long)a.D;
}

// The same through page-table entries staged in LDS (ptl[i] = entry of page
// first + i): no dependent global load per tile, so the next tile's rows can
// be requested while the current one is multiplied.
__device__ __forceinline__ long long page_off_lds(const AttnDims& a, const int* ptl, int first, int p, int kv) {
  const int page = ptl[p / a.page - first];
  if (page < 0 || page >= a.num_pages) return -1;
  return ((((long long)page * a.KV + kv) * a.page) + (p % a.page)) * (long long)a.D;
}

// A sequence's page-table row.  With DENSE the caller passed no table: the
// cache's sequence b owns pages [b * max_pages, (b + 1) * max_pages) in
// order, and an entry is computed instead of loaded (one dependent memory
// round trip less between a position and its K/V rows).
template <bool DENSE>
struct PtRow {
  const int32_t* row;  // unused when DENSE
  int base;            // b * max_pages when DENSE
  __device__ __forceinline__ int operator[](int i) const {
    if constexpr (DENSE) return base + i;
    else return row[i];
  }
};
template <bool DENSE>
__device__ __forceinline__ PtRow<DENSE> pt_row_of(const AttnDims& a, const int32_t* page_table, int b) {
  PtRow<DENSE> r;
  r.row = DENSE ? page_table : page_table + (size_t)b * a.max_pages;
  r.base = b * a.max_pages;
  return r;
}

// Requests the page-table entries of pages [first, first + 512) of one
// sequence (clamped to the row) into registers of an NT-thread block;
// stage_store() writes them to LDS before the block's next barrier.  A split
// spans at most kChunkMax + 1 pages.
template <int NT = 256>
struct PtStage {
  int v[512 / NT];
};
template <int NT = 256, typename PT>
__device__ __forceinline__ PtStage<NT> stage_load(const AttnDims& a, const PT& pt_row, int first) {
  PtStage<NT> s;
#pragma unroll
  for (int r = 0; r < 512 / NT; ++r) s.v[r] = pt_row[min(first + (int)threadIdx.x + NT * r, a.max_pages - 1)];
  return s;
}
template <int NT = 256>
__device__ __forceinline__ void stage_store(const PtStage<NT>& s, int* ptl) {
#pragma unroll
  for (int r = 0; r < 512 / NT; ++r) ptl[threadIdx.x + NT * r] = s.v[r];
}

// The maximum over the 64 lanes, in every lane: the DPP steps of group_sum
// inside each row of 16 lanes, then two ds_bpermute steps (max is exact, so
// any order gives the same bits).
__device__ __forceinline__ float wave_max_bfly(float m) {
  m = fmaxf(m, dpp_f<kDppXor1>(m));
  m = fmaxf(m, dpp_f<kDppXor2>(m));
  m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
  m = fmaxf(m, dpp_f<kDppMirror>(m));
  m = fmaxf(m, __shfl_xor(m, 16, kWave));
  m = fmaxf(m, __shfl_xor(m, 32, kWave));
  return m;
}

// Per-lane slice of one head: lane l owns the PL = D/64 consecutive values
// starting at l*PL, so the RoPE partner (d +- D/2) of a value sits in lane l^32.
template <int PL>
__device__ __forceinline__ void load_slice(const uint16_t* __restrict__ p, float* x) {
  if constexpr (PL == 8) {
    unpack8(ld16(p), x);
  } else if constexpr (PL == 4) {
    const uint2 v = *(const uint2*)p;
    x[0] = bf_lo(v.x); x[1] = bf_hi(v.x); x[2] = bf_lo(v.y); x[3] = bf_hi(v.y);
  } else if constexpr (PL == 2) {
    const uint32_t v = *(const uint32_t*)p;
    x[0] = bf_lo(v); x[1] = bf_hi(v);
  } else {
    x[0] = bf2f(*p);
  }
}

// rms_norm(x, w) (w may be null) and optional RoPE of one head held as
// per-lane slices (see load_slice); cs/sn are the lane's cos/sin values
// (the reference duplicates the table halves, model.py:66).  In place.
template <int D>
__device__ __forceinline__ void norm_rope_slice(float* x, const float* w, const float* cs, const float* sn, float eps,
                                                bool rope) {
  constexpr int PL = D / 64;
  const int lane = threadIdx.x & 63;
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < PL; ++i) ss = fma((double)x[i], (double)x[i], ss);
  const float r = rms_scale(group_sum_f64<64>(ss), D, eps);
#pragma unroll
  for (int i = 0; i < PL; ++i) x[i] = (w != nullptr) ? rbf(x[i] * r * w[i]) : rbf(x[i] * r);
  if (rope) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const float partner = __shfl_xor(x[i], 32, kWave);
      const float rot = (lane * PL + i < D / 2) ? -partner : partner;
      x[i] = rbf(rbf(x[i] * cs[i]) + rbf(rot * sn[i]));
    }
  }
}

// ------------------------------------------------------------------ scores
// grid (n_split_max, KV, B), 256 threads.  The G query heads of a KV head
// (zero-padded to 16 rows) times K^T on MFMA: v_mfma_f32_16x16x32_bf16 takes
// A = q rows [16 x 32 dims] and B = K^T [32 dims x 16 positions]; lane l holds
// A[l%16][8(l/16)..+7], B[8(l/16)..+7][l%16] (16 contiguous bytes of the K row
// of position l%16) and gets C[4(l/16)+i][l%16], i < 4.  Wave w takes the
// 16-position tiles w, w+4, ... of the split; the next tile's K loads are in
// flight while the current one is multiplied.  ONE: the launch guarantees
// at most kChunkMin positions per split (one tile per wave), so there is
// nothing to prefetch.  NW = 8 (long ranges): 8 waves, each owning tiles w
// and w + 8 of a split's 16 at most, all requested by the end of the q
// prologue (part of the first before it, see KS0), so a whole split's K rows
// are in flight at once.
template <int D, int G, bool ONE, int NW, bool DPT>
__global__ __launch_bounds__(NW * 64) void attn_qk_kernel(
    AttnDims a, const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
    const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const uint16_t* __restrict__ rope_cos, const uint16_t* __restrict__ rope_sin, uint16_t* __restrict__ k_pages,
    uint16_t* __restrict__ v_pages, const int32_t* __restrict__ page_table, const int32_t* __restrict__ pos_arr,
    int append, float* __restrict__ ws_scores, float* __restrict__ ws_stats) {
  constexpr int PL = D / 64;
  constexpr int NT = NW * 64;
  constexpr int GW = (G + NW - 1) / NW;
  constexpr int KS = D / 32;  // MFMA steps along the head dimension
  constexpr int TPW = (NW == 8 && !ONE) ? kChunkMax / 16 / NW : 1;  // tiles requested up front per wave
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  __shared__ __align__(16) uint16_t qa[16 * D];
  __shared__ __align__(16) uint16_t kn16[D];
  __shared__ float knew[D];
  __shared__ float vnew[D];
  __shared__ float sc[G][kChunkMax];
  __shared__ int ptl[512];
  const int split = blockIdx.x, kv = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int pos = pos_arr[b];
  const Range R = attn_range(a, pos);
  if (split >= R.n_eff) return;
  const int start = R.lo + split * R.chunk;
  const int end = min(R.lo + R.len, start + R.chunk);
  const int npos = end - start;
  const PtRow<DPT> pt_row = pt_row_of<DPT>(a, page_table, b);

  // Everything that needs only pos is requested first, in this order: the
  // split's page-table entries, this wave's first K tile's entry, and the
  // prologue rows (q heads, norms, cos/sin, the new K/V); then the first K
  // tile itself.  Its HBM latency overlaps the q prologue; later tiles find
  // their pages in LDS.  The loads are unconditional (clamped indices,
  // selected pointers), so each wait covers only what it needs.
  const int kg = lane >> 4, col = lane & 15;
  const int ntiles = (npos + 15) >> 4;
  const int first = start / a.page;
  const PtStage<NT> pts = stage_load<NT>(a, pt_row, first);
  auto load_tile = [&](int t, u32x4* bf, long long& off) {
    const int jc = min(t * 16 + col, npos - 1);
    off = page_off_lds(a, ptl, first, start + jc, kv);
    const uint16_t* kp = k_pages + max(off, 0ll) + 8 * kg;
#pragma unroll
    for (int s = 0; s < KS; ++s) bf[s] = ld16((const u32x4*)(kp + 32 * s));
  };
  int jc0[TPW], pe0[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    jc0[tt] = min(min(wave + NW * tt, ntiles - 1) * 16 + col, npos - 1);
    pe0[tt] = pt_row[(start + jc0[tt]) / a.page];
  }

  // Prologue: wave w owns q heads w, w+4 (G <= 8); with the append, waves 2
  // and 3 also own the new K and V rows.
  const int so = lane * PL;                 // this lane's slice offset
  const int jo = so % (D / 2);              // its cos/sin offset
  const bool mine = append && (end == pos + 1);
  float qx[GW][PL], qw[PL], cs[PL], sn[PL], kvx[PL], kw[PL];
#pragma unroll
  for (int u = 0; u < GW; ++u)
    load_slice<PL>(q_raw + ((size_t)b * a.NH + kv * G + min(wave + NW * u, G - 1)) * D + so, qx[u]);
  load_slice<PL>(q_norm + so, qw);
  load_slice<PL>(rope_cos + (size_t)pos * (D / 2) + jo, cs);
  load_slice<PL>(rope_sin + (size_t)pos * (D / 2) + jo, sn);
  {
    const uint16_t* kr = mine ? k_raw + ((size_t)b * a.KV + kv) * D : q_norm;
    const uint16_t* vr = (mine && v_raw != nullptr) ? v_raw + ((size_t)b * a.KV + kv) * D : kr;
    load_slice<PL>((wave == 2 ? kr : vr) + so, kvx);
    load_slice<PL>((mine ? k_norm : q_norm) + so, kw);
  }
  u32x4 bt[TPW][KS];
  long long ot[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const bool valid = pe0[tt] >= 0 && pe0[tt] < a.num_pages;
    ot[tt] = valid ? ((((long long)pe0[tt] * a.KV + kv) * a.page) + ((start + jc0[tt]) % a.page)) * (long long)D
                   : -1ll;
  }
  auto load_chunks = [&](int tt, int s0, int s1) {
    const uint16_t* kp = k_pages + max(ot[tt], 0ll) + 8 * kg;
#pragma unroll
    for (int s = s0; s < s1; ++s) bt[tt][s] = ld16((const u32x4*)(kp + 32 * s));
  };
  // On the 8-wave path only the first KS0 chunks of each wave's first tile
  // are requested before the prologue, the rest after it: a CU queues only so
  // many vector memory instructions, and a wave that requested its whole
  // tiles up front would stall at issue with the prologue behind them (8 of
  // the 16 chunks at head_dim 512: the full 32K layer 41.1 -> 40.2 us against
  // 4, no better with 16).
  constexpr int KS0 = (NW == 8 && KS > 8) ? 8 : KS;
  load_chunks(0, 0, KS0);
  // padding rows G..15 of the A operand are zero
  for (int c = tid; c < (16 - G) * D / 8; c += NT) ((u32x4*)(qa + G * D))[c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    const int g = wave + NW * u;
    if (g < G) {
      norm_rope_slice<D>(qx[u], qw, cs, sn, a.eps, true);
#pragma unroll
      for (int i = 0; i < PL; ++i) qa[g * D + so + i] = f2bf(qx[u][i]);
    }
  }
  if (mine && wave >= 2) {
    norm_rope_slice<D>(kvx, wave == 2 ? kw : nullptr, cs, sn, a.eps, wave == 2);
    float* dst = (wave == 2) ? knew : vnew;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      dst[so + i] = kvx[i];
      if (wave == 2) kn16[so + i] = f2bf(kvx[i]);
    }
  }
  stage_store<NT>(pts, ptl);
  lds_barrier();
  load_chunks(0, KS0, KS);
#pragma unroll
  for (int tt = 1; tt < TPW; ++tt) load_chunks(tt, 0, KS);
  if (mine) {
    const long long off = page_off_lds(a, ptl, first, pos, kv);
    if (off >= 0)
      for (int d = tid; d < D; d += NT) {
        k_pages[off + d] = f2bf(knew[d]);
        v_pages[off + d] = f2bf(vnew[d]);
      }
  }

  u32x4 af[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) af[s] = *(const u32x4*)(qa + col * D + 32 * s + 8 * kg);
  const float cap = a.softcap;
  // scores of tile t (K rows in bf) into sc
  auto score_tile = [&](int t, const u32x4* bf, long long off) {
    const int j = t * 16 + col;
    const bool isnew = mine && (start + j == pos);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 kb = bf[s];
      if (mine) kb = isnew ? *(const u32x4*)(kn16 + 32 * s + 8 * kg) : kb;
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[s]), __builtin_bit_cast(bf16x8, kb),
                                                    acc, 0, 0, 0);
    }
    const bool ok = (off >= 0) || isnew;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G && j < npos) {
        float sv = rbf(acc[i]);
        if (cap > 0.0f) sv = tanhf(sv / cap) * cap;
        sc[h][j] = ok ? sv : -INFINITY;
      }
    }
  };
  if constexpr (ONE) {
    if (wave < ntiles) score_tile(wave, bt[0], ot[0]);
  } else if constexpr (NW == 8) {
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
      if (wave + NW * tt < ntiles) score_tile(wave + NW * tt, bt[tt], ot[tt]);
  } else {
    u32x4 bcur[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) bcur[s] = bt[0][s];
    long long ocur = ot[0];
    for (int t = wave; t < ntiles; t += 4) {
      u32x4 bnext[KS];
      long long onext;
      // the next tile of this wave, or this tile again on the last pass (a
      // cache hit, so the barrier after the loop does not wait on HBM)
      load_tile(t + 4 < ntiles ? t + 4 : t, bnext, onext);
      score_tile(t, bcur, ocur);
#pragma unroll
      for (int s = 0; s < KS; ++s) bcur[s] = bnext[s];
      ocur = onext;
    }
  }
  lds_barrier();
  // the split's max and sum of exp per head: wave w owns heads w, w+NW, so
  // the heads reduce in parallel and no further barrier is needed
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    const int g = wave + NW * u;
    if (g < G) {
      float m = -INFINITY;
      for (int j = lane; j < npos; j += 64) m = fmaxf(m, sc[g][j]);
      m = wave_max_bfly(m);
      float* srow = ws_scores + ((size_t)b * a.NH + kv * G + g) * a.lmax + (start - R.lo);
      float l = 0.0f;
      for (int j = lane; j < npos; j += 64) {
        const float s = sc[g][j];
        l += (s == -INFINITY) ? 0.0f : expf(s - m);
        srow[j] = s;
      }
      l = group_sum<64>(l);
      if (lane == 0) {
        const int h = kv * G + g;
        ws_stats[((size_t)b * a.NH + h) * a.n_split_max + split] = m;
        ws_stats[((size_t)(a.B + b) * a.NH + h) * a.n_split_max + split] = l;
      }
    }
  }
}

// ------------------------------------------------------------------ pv + reduce
// grid (n_split_max, KV, B), 256 threads.  Wave w owns the values
// [w*D/4, (w+1)*D/4) of every head; LPV = D/32 lanes per position, the PPV
// positions of a step in consecutive lanes (their sum is a DPP reduction).
// The block's V loads are issued before the split statistics are merged.  Each
// split writes its f32 partial [G, D]; the last split of each group of
// kGroup to finish sums the group's partials in split order, and with more
// than one group the last group to finish sums the group sums in order, so
// ctx is deterministic (no float atomics).  The partials pass between blocks
// through coherent (device-scope) 16-byte stores and loads, see arrive_last().
constexpr int kGroup = 16;
constexpr int kMaxSplits = 256;
constexpr int kMaxGroups = kMaxSplits / kGroup;

// sum[r] = sum over i < n (n <= 16, in order) of the float4 at byte offset
// base + i*stride + 16*e4, e4 = threadIdx.x + 256*r < N4, read with coherent
// loads (the sources were written by other blocks of this kernel).  All loads
// of a half (8 sources) are issued before the first add, so a half costs one
// round trip.
template <int E4, int N4, int NT = 256>
__device__ __forceinline__ void ordered_sum(__amdgpu_buffer_rsrc_t rs, uint32_t base, uint32_t stride, int n,
                                            float4* sum) {
#pragma unroll
  for (int r = 0; r < E4; ++r) sum[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int h0 = 0; h0 < kGroup; h0 += 8) {
    if (h0 < n) {
      float4 v[8][E4];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < E4; ++r) {
          const int e4 = min((int)threadIdx.x + NT * r, N4 - 1);
          v[i][r] = coherent_load4(rs, base + (uint32_t)min(h0 + i, n - 1) * stride + 16u * (uint32_t)e4);
        }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < E4; ++r)
          if (h0 + i < n) {
            sum[r].x += v[i][r].x;
            sum[r].y += v[i][r].y;
            sum[r].z += v[i][r].z;
            sum[r].w += v[i][r].w;
          }
    }
  }
}

template <int E4, int N4, int NT = 256>
__device__ __forceinline__ void store_bf16x4(uint16_t* out, const float4* sum) {
#pragma unroll
  for (int r = 0; r < E4; ++r) {
    const int e4 = threadIdx.x + NT * r;
    if (e4 < N4) {
      uint2 w;
      w.x = pack2(sum[r].x, sum[r].y);
      w.y = pack2(sum[r].z, sum[r].w);
      ((uint2*)out)[e4] = w;
    }
  }
}

// Merged softmax statistics of the splits of every head of a KV head into
// mg/sg (LDS): wave w owns heads w, w+NW; lanes stride the splits.  The
// score and statistics pointers of the pv kernels are not __restrict__: with
// it the compiler may sink their loads past the V rows (and past an asm
// memory barrier) to where they are used, and the in-order vmcnt wait for
// them then waits for every V row in flight.
// load_split_stats requests every head's split statistics (unconditional
// loads from clamped indices; issue it before any load that waits on a
// page-table entry), reduce_split_stats merges them.  R.n_eff >= 1.
template <int G, int NW = 4>
struct SplitStats {
  float m[(G + NW - 1) / NW][kMaxSplits / 64], l[(G + NW - 1) / NW][kMaxSplits / 64];
};
template <int G, int NW = 4>
__device__ __forceinline__ SplitStats<G, NW> load_split_stats(const AttnDims& a, const Range& R, int kv, int b,
                                                              int wave, int lane, const float* ws_stats) {
  SplitStats<G, NW> st;
#pragma unroll
  for (int u = 0; u < (G + NW - 1) / NW; ++u) {
    const int h = kv * G + min(wave + NW * u, G - 1);
    const float* sm = ws_stats + ((size_t)b * a.NH + h) * a.n_split_max;
    const float* sl = ws_stats + ((size_t)(a.B + b) * a.NH + h) * a.n_split_max;
#pragma unroll
    for (int q = 0; q < kMaxSplits / 64; ++q) {
      const int ic = min(lane + 64 * q, R.n_eff - 1);
      st.m[u][q] = sm[ic];
      st.l[u][q] = sl[ic];
    }
  }
  return st;
}
template <int G, int NW = 4>
__device__ __forceinline__ void reduce_split_stats(SplitStats<G, NW>& st, const Range& R, int wave, int lane, float* mg,
                                                   float* sg) {
  constexpr int Q = kMaxSplits / 64;
#pragma unroll
  for (int u = 0; u < (G + NW - 1) / NW; ++u) {
    const int g = wave + NW * u;
    if (g < G) {
      float m = -INFINITY;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const bool in = lane + 64 * q < R.n_eff;
        st.m[u][q] = in ? st.m[u][q] : -INFINITY;
        st.l[u][q] = in ? st.l[u][q] : 0.0f;
        m = fmaxf(m, st.m[u][q]);
      }
      m = wave_max_bfly(m);
      float t = 0.0f;
#pragma unroll
      for (int q = 0; q < Q; ++q) t += (st.m[u][q] == -INFINITY) ? 0.0f : expf(st.m[u][q] - m) * st.l[u][q];
      t = group_sum<64>(t);
      if (lane == 0) {
        mg[g] = m;
        sg[g] = t;
      }
    }
  }
}

// Short ranges (len <= kShortLen): block x of a KV head owns head dims
// [x*kSliceD, (x+1)*kSliceD) of its G query heads over every attended
// position, so no partials cross blocks.  LPS lanes (8 dims each) cover a
// position's slice, a wave takes PPW positions per step and the block PPB.
// Each lane sums its positions in increasing order, then the lanes with the
// same dims (consecutive lanes) are combined by a DPP sum and the four waves
// in wave order.
constexpr int kShortLen = 512;
constexpr int kSliceD = 32;

template <int D, int G, int NW, typename PT>
__device__ __forceinline__ void pv_short(const AttnDims& a, const Range& R, int kv, int b,
                                         const uint16_t* __restrict__ v_pages, const PT& pt_row,
                                         const float* ws_scores, const float* ws_stats,
                                         uint16_t* __restrict__ ctx, float* pr, float* red, float* mg, float* sg) {
  constexpr int NT = NW * 64;
  constexpr int LPS = kSliceD / 8;
  constexpr int PPW = 64 / LPS;
  constexpr int PPB = NW * PPW;
  constexpr int NST = kShortLen / PPB;       // V steps per lane at most
  constexpr int SPT = G * kShortLen / NT;    // scores per thread at most
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int slot = lane % PPW, sub = lane / PPW;  // the positions of a step are consecutive lanes
  const int d0 = blockIdx.x * kSliceD + sub * 8;
  const int len = R.len;
  const int nst = (len + PPB - 1) / PPB;
  // Loads first, in this order: every step's page-table entry, the scores
  // and the split statistics (none waits on anything but pos), then this
  // block's V slice at every position (unconditional loads from clamped
  // positions), so the V rows cost one round trip after the entries and the
  // statistics merge runs while they are in flight.
  int pg[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) pg[st] = pt_row[(R.lo + min(st * PPB + wave * PPW + slot, len - 1)) / a.page];
  float sreg[SPT];
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const int idx = tid + NT * r, g = idx / kShortLen, j = idx % kShortLen;
    sreg[r] = ws_scores[((size_t)b * a.NH + kv * G + g) * a.lmax + min(j, len - 1)];
  }
  SplitStats<G, NW> sst = load_split_stats<G, NW>(a, R, kv, b, wave, lane, ws_stats);
  asm volatile("" ::: "memory");  // the loads above stay ahead of the V rows in issue order
  u32x4 vv[NST];
  bool ok[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    const int j = st * PPB + wave * PPW + slot;
    const int p = R.lo + min(j, len - 1);
    const bool valid = pg[st] >= 0 && pg[st] < a.num_pages;
    const long long off = ((((long long)(valid ? pg[st] : 0) * a.KV + kv) * a.page) + (p % a.page)) * (long long)a.D;
    vv[st] = ld16((const u32x4*)(v_pages + off + d0));
    ok[st] = (st < nst) && (j < len) && valid;
  }
  reduce_split_stats<G, NW>(sst, R, wave, lane, mg, sg);
  lds_barrier();
  // normalised probabilities, rounded to bf16 (model.py:212), zero past len
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const int idx = tid + NT * r, g = idx / kShortLen, j = idx % kShortLen;
    const float sv = sreg[r];
    if (j < len) pr[g * kShortLen + j] = (sv == -INFINITY) ? 0.0f : rbf(expf(sv - mg[g]) / sg[g]);
  }
  lds_barrier();
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    if (st < nst) {
      const int j = min(st * PPB + wave * PPW + slot, kShortLen - 1);
      float vf[8];
      unpack8(vv[st], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = ok[st] ? pr[g * kShortLen + j] : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(p, vf[i], acc[g][i]);
      }
    }
  }
  // the PPW positions of a wave step sit in consecutive lanes: a DPP sum
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = group_sum<PPW>(acc[g][i]);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) red[(wave * G + g) * kSliceD + sub * 8 + i] = acc[g][i];
  }
  lds_barrier();
  for (int e = tid; e < G * kSliceD; e += NT) {
    const int g = e / kSliceD, dd = e % kSliceD;
    float v = red[g * kSliceD + dd];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[(w * G + g) * kSliceD + dd];  // in wave order
    ctx[((size_t)b * a.NH + kv * G + g) * D + blockIdx.x * kSliceD + dd] = f2bf(v);
  }
}

// pv_long8: the long-range body for 8 waves (NW = 8).  Wave w owns the
// head dims [w*D/8, (w+1)*D/8): DW/8 lanes per position, PPV positions per
// wave step, at most kChunkMax / PPV steps per split.  The V row slices of
// the first 8 steps are requested before the split statistics are merged,
// those of the next kPvRing - 8 once the probabilities are in LDS; then the
// pairs of steps are dotted with the bf16 probabilities as in the 4-wave
// body, each consumed pair's registers refilled with the pair kPvRing steps
// ahead.  (A CU queues only so many vector memory instructions: a wave that
// requests more rows than that ahead of other work stalls at issue until
// the earlier requests drain, so the merge and the products would start
// only once most of the split had arrived.)
// Writes the wave's partial sums to v_out (per head, 8 dims per lane, summed
// over the PPV positions of a step).
constexpr int kPvRing = 12;

template <int D, int G, typename PT>
__device__ __forceinline__ void pv_long8(const AttnDims& a, const Range& R, int split, int kv, int b,
                                         const uint16_t* __restrict__ v_pages, const PT& pt_row,
                                         const float* ws_scores, const float* ws_stats,
                                         float* lds_f, float* mg, float* sg, int* ptl, float (*v_out)[8],
                                         int& dofs_out, int& slot_out) {
  constexpr int NW = 8, NT = 512;
  constexpr int DW = D / NW;                    // dims per wave
  constexpr int LPV = DW / 8;                   // lanes per position
  constexpr int PPV = 64 / LPV;                 // positions per wave step
  constexpr int MAXST = kChunkMax / PPV;        // steps per split at most
  constexpr int RB = kPvRing < MAXST ? kPvRing : MAXST;  // steps in flight
  constexpr int RB0 = RB < 8 ? RB : 8;                   // of which requested before the merge
  constexpr int RS = (G * kChunkMax + NT - 1) / NT;  // scores per thread
  static_assert(D % (NW * 8) == 0 && MAXST % 2 == 0 && RB % 2 == 0, "pv_long8 layout");
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int start = R.lo + split * R.chunk;
  const int end = min(R.lo + R.len, start + R.chunk);
  const int npos = end - start;
  const int slot = lane % PPV, sub = lane / PPV;
  const int dofs = wave * DW + sub * 8;
  // the split's scores, the split statistics, the page-table entries of the
  // first RB0 steps and of the whole split (staged in LDS for the later
  // steps), then the first RB0 steps' V rows
  float sreg[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int idx = tid + NT * r, g = min(idx / kChunkMax, G - 1), j = idx % kChunkMax;
    sreg[r] = ws_scores[((size_t)b * a.NH + kv * G + g) * a.lmax + (start - R.lo) + min(j, npos - 1)];
  }
  SplitStats<G, NW> sst = load_split_stats<G, NW>(a, R, kv, b, wave, lane, ws_stats);
  const int nsteps = (npos + PPV - 1) / PPV;
  const int first = start / a.page;
  int pg0[RB0];
#pragma unroll
  for (int st = 0; st < RB0; ++st) pg0[st] = pt_row[(start + min(st * PPV + slot, npos - 1)) / a.page];
  const PtStage<NT> pts = stage_load<NT>(a, pt_row, first);
  // keep the small loads above ahead of the V rows in issue order: vmcnt
  // waits are in order, and a statistics load moved after the rows would
  // wait for the rows
  asm volatile("" ::: "memory");
  bool ok[MAXST];
  // V slice of step st (clamped position; page 0 when the entry is invalid)
  auto vrow = [&](auto S) __attribute__((always_inline)) {
    constexpr int st = S;
    const int j = st * PPV + slot;
    const int p = start + min(j, npos - 1);
    int e;
    if constexpr (st < RB0) e = pg0[st];
    else e = ptl[p / a.page - first];
    const bool valid = e >= 0 && e < a.num_pages;
    ok[st] = (st < nsteps) && (j < npos) && valid;
    const long long off = ((((long long)(valid ? e : 0) * a.KV + kv) * a.page) + (p % a.page)) * (long long)a.D;
    return ld16((const u32x4*)(v_pages + off + dofs));
  };
  u32x4 vv[RB];
  static_for<RB0>([&](auto S) __attribute__((always_inline)) { vv[S] = vrow(S); });
  stage_store<NT>(pts, ptl);
  reduce_split_stats<G, NW>(sst, R, wave, lane, mg, sg);
  lds_barrier();
  // normalised probabilities, rounded to bf16 (model.py:212), as bf16 pairs:
  // the positions of wave steps 2q and 2q + 1 at lane slot `sl` share word
  // q * PPV + sl (zero past npos)
  uint16_t* pr16 = reinterpret_cast<uint16_t*>(lds_f);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int idx = tid + NT * r, g = idx / kChunkMax, j = idx % kChunkMax;
    if (idx < G * kChunkMax) {
      const float sv = sreg[r];
      const float pv = (j < npos && sv != -INFINITY) ? rbf(expf(sv - mg[g]) / sg[g]) : 0.0f;
      const int step = j / PPV, sl = j % PPV;
      pr16[g * kChunkMax + ((step >> 1) * PPV + sl) * 2 + (step & 1)] = f2bf(pv);
    }
  }
  lds_barrier();
  static_for<RB - RB0>([&](auto S) __attribute__((always_inline)) {
    vv[RB0 + S] = vrow(std::integral_constant<int, RB0 + S>{});
  });
  const uint32_t* pr32 = reinterpret_cast<const uint32_t*>(lds_f);
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
  static_for<MAXST / 2>([&](auto U) __attribute__((always_inline)) {
    constexpr int u = 2 * U;
    if (u < nsteps) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 va = ok[u] ? vv[u % RB] : z, vb = ok[u + 1] ? vv[(u + 1) % RB] : z;
      uint32_t vp[8];
      vp[0] = __builtin_amdgcn_perm(vb.x, va.x, 0x05040100u);
      vp[1] = __builtin_amdgcn_perm(vb.x, va.x, 0x07060302u);
      vp[2] = __builtin_amdgcn_perm(vb.y, va.y, 0x05040100u);
      vp[3] = __builtin_amdgcn_perm(vb.y, va.y, 0x07060302u);
      vp[4] = __builtin_amdgcn_perm(vb.z, va.z, 0x05040100u);
      vp[5] = __builtin_amdgcn_perm(vb.z, va.z, 0x07060302u);
      vp[6] = __builtin_amdgcn_perm(vb.w, va.w, 0x05040100u);
      vp[7] = __builtin_amdgcn_perm(vb.w, va.w, 0x07060302u);
      const int pi = (u >> 1) * PPV + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t pp = pr32[g * (kChunkMax / 2) + pi];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = dot2bf(vp[i], pp, acc[g][i]);
      }
    }
    if constexpr (u + RB < MAXST) {
      vv[u % RB] = vrow(std::integral_constant<int, u + RB>{});
      vv[(u + 1) % RB] = vrow(std::integral_constant<int, u + RB + 1>{});
    }
  });
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) v_out[g][i] = group_sum<PPV>(acc[g][i]);
  dofs_out = dofs;
  slot_out = slot;
}

template <int D, int G, int NW, bool DPT>
__global__ __launch_bounds__(NW * 64) void attn_pv_kernel(AttnDims a, const uint16_t* __restrict__ v_pages,
                                                      const int32_t* __restrict__ page_table,
                                                      const int32_t* __restrict__ pos_arr,
                                                      const float* ws_scores,
                                                      const float* ws_stats, float* ws_part,
                                                      float* ws_group, unsigned int* counters,
                                                      uint16_t* __restrict__ ctx) {
  constexpr int LPV = D / 32;
  constexpr int PPV = 64 / LPV;
  constexpr int UB = 8;                        // wave steps of V loads in flight
  constexpr int RS = G * kChunkMax / 256;      // scores per thread
  constexpr int NT = NW * 64;
  constexpr int E4 = (G * D / 4 + NT - 1) / NT;  // reduced float4s per thread
  constexpr int kLdsF = (G * kShortLen + NW * G * kSliceD > G * kChunkMax) ? G * kShortLen + NW * G * kSliceD
                                                                           : G * kChunkMax;
  __shared__ float lds_f[kLdsF];
  __shared__ float mg[G], sg[G];
  __shared__ int flag;
  __shared__ int ptl[512];
  const int split = blockIdx.x, kv = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int pos = pos_arr[b];
  const Range R = attn_range(a, pos);
  if (R.n_eff > 0 && R.len <= kShortLen) {  // grid.x >= D / kSliceD (see launch_attn)
    if (split < D / kSliceD)
      pv_short<D, G, NW>(a, R, kv, b, v_pages, pt_row_of<DPT>(a, page_table, b), ws_scores, ws_stats, ctx,
                         lds_f, lds_f + G * kShortLen, mg, sg);
    return;
  }
  if (split >= R.n_eff) {
    if (R.n_eff == 0 && split == 0)  // nothing attended: ctx = 0
      for (int e = tid; e < G * D; e += NT) ctx[(size_t)b * a.NH * D + (size_t)kv * G * D + e] = 0;
    return;
  }
  const size_t hd = (size_t)kv * G * D;  // offset of this KV head's group in [NH, D]
  const uint32_t sstride = (uint32_t)(a.NH * D * 4);  // bytes per split partial
  const __amdgpu_buffer_rsrc_t rpart = buffer_rsrc(ws_part, (uint32_t)(a.B * a.n_split_max) * sstride);
  const uint32_t pbase = (uint32_t)(((size_t)b * a.n_split_max + split) * sstride + hd * 4);
  if constexpr (NW == 8) {
    float v[G][8];
    int dofs, slot;
    pv_long8<D, G>(a, R, split, kv, b, v_pages, pt_row_of<DPT>(a, page_table, b), ws_scores, ws_stats, lds_f, mg,
                   sg, ptl, v, dofs, slot);
    // the partials are reduced by attn_reduce_kernel, the next launch
    if (slot == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t o = pbase + (uint32_t)(g * D + dofs) * 4;
        store4(rpart, o, make_float4(v[g][0], v[g][1], v[g][2], v[g][3]));
        store4(rpart, o + 16, make_float4(v[g][4], v[g][5], v[g][6], v[g][7]));
      }
    }
    return;
  } else {
  const int start = R.lo + split * R.chunk;
  const int end = min(R.lo + R.len, start + R.chunk);
  const int npos = end - start;
  const PtRow<DPT> pt_row = pt_row_of<DPT>(a, page_table, b);
  const int slot = lane % PPV, sub = lane / PPV;  // the positions of a step are consecutive lanes
  const int dofs = wave * (D / 4) + sub * 8;

  // this split's scores, the split statistics and the first batch of V rows
  // are all in flight before the first wait
  float sreg[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int idx = tid + 256 * r, g = idx / kChunkMax, j = idx % kChunkMax;
    sreg[r] = ws_scores[((size_t)b * a.NH + kv * G + g) * a.lmax + (start - R.lo) + min(j, npos - 1)];
  }
  const int nsteps = (npos + PPV - 1) / PPV;
  const int first = start / a.page;
  const PtStage pts = stage_load(a, pt_row, first);
  // the first batch through the page table in memory (every entry requested
  // before the first V row), later ones through LDS
  auto vload = [&](int st0, u32x4* vf, bool* okv, bool staged) {
    int pg[UB];
    if (!staged) {
#pragma unroll
      for (int u = 0; u < UB; ++u) pg[u] = pt_row[(start + min((st0 + u) * PPV + slot, npos - 1)) / a.page];
    }
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int j = (st0 + u) * PPV + slot;
      const int p = start + min(j, npos - 1);
      const int e = staged ? ptl[p / a.page - first] : pg[u];
      const bool valid = e >= 0 && e < a.num_pages;
      const long long off = ((((long long)(valid ? e : 0) * a.KV + kv) * a.page) + (p % a.page)) * (long long)a.D;
      vf[u] = ld16((const u32x4*)(v_pages + off + dofs));
      okv[u] = (j < npos) && valid;
    }
  };
  SplitStats<G> sst = load_split_stats<G>(a, R, kv, b, wave, lane, ws_stats);
  asm volatile("" ::: "memory");  // the loads above stay ahead of the V rows in issue order
  u32x4 vcur[UB];
  bool okcur[UB];
  vload(0, vcur, okcur, false);
  stage_store(pts, ptl);
  reduce_split_stats<G>(sst, R, wave, lane, mg, sg);
  lds_barrier();
  // normalised probabilities, rounded to bf16 as the reference does
  // (model.py:212), stored as bf16 pairs: the positions of wave steps 2q and
  // 2q + 1 at lane slot `sl` share word q * PPV + sl (zero past npos)
  uint16_t* pr16 = reinterpret_cast<uint16_t*>(lds_f);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int idx = tid + 256 * r, g = idx / kChunkMax, j = idx % kChunkMax;
    const float s = sreg[r];
    const float pv = (j < npos && s != -INFINITY) ? rbf(expf(s - mg[g]) / sg[g]) : 0.0f;
    const int step = j / PPV, sl = j % PPV;
    pr16[g * kChunkMax + ((step >> 1) * PPV + sl) * 2 + (step & 1)] = f2bf(pv);
  }
  lds_barrier();
  const uint32_t* pr32 = reinterpret_cast<const uint32_t*>(lds_f);
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
  for (int st0 = 0; st0 < nsteps; st0 += UB) {
    u32x4 vnext[UB];
    bool oknext[UB];
    if (st0 + UB < nsteps) vload(st0 + UB, vnext, oknext, true);
    // two wave steps at a time: each dim's values at the two positions form
    // one bf16 pair, dotted with the pair of probabilities (v_dot2c_f32_bf16;
    // the products are exact, the pair is added to acc with one rounding)
#pragma unroll
    for (int u = 0; u < UB; u += 2) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 va = okcur[u] ? vcur[u] : z, vb = okcur[u + 1] ? vcur[u + 1] : z;
      uint32_t vp[8];
      vp[0] = __builtin_amdgcn_perm(vb.x, va.x, 0x05040100u);
      vp[1] = __builtin_amdgcn_perm(vb.x, va.x, 0x07060302u);
      vp[2] = __builtin_amdgcn_perm(vb.y, va.y, 0x05040100u);
      vp[3] = __builtin_amdgcn_perm(vb.y, va.y, 0x07060302u);
      vp[4] = __builtin_amdgcn_perm(vb.z, va.z, 0x05040100u);
      vp[5] = __builtin_amdgcn_perm(vb.z, va.z, 0x07060302u);
      vp[6] = __builtin_amdgcn_perm(vb.w, va.w, 0x05040100u);
      vp[7] = __builtin_amdgcn_perm(vb.w, va.w, 0x07060302u);
      const int pi = ((st0 + u) >> 1) * PPV + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t pp = pr32[g * (kChunkMax / 2) + pi];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = dot2bf(vp[i], pp, acc[g][i]);
      }
    }
    if (st0 + UB < nsteps) {
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        vcur[u] = vnext[u];
        okcur[u] = oknext[u];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = group_sum<PPV>(acc[g][i]);
    if (slot == 0) {
      const uint32_t o = pbase + (uint32_t)(g * D + dofs) * 4;
      coherent_store4(rpart, o, make_float4(v[0], v[1], v[2], v[3]));
      coherent_store4(rpart, o + 16, make_float4(v[4], v[5], v[6], v[7]));
    }
  }
  }  // NW == 4

  // two-level ordered reduction of the partials
  const int grp = split / kGroup;
  const int ngroups = (R.n_eff + kGroup - 1) / kGroup;
  const int gsz = min(kGroup, R.n_eff - grp * kGroup);
  unsigned int* cnt = counters + ((size_t)b * a.KV + kv) * (kMaxGroups + 1);
  if (!arrive_last(cnt + 1 + grp, (unsigned)gsz, &flag)) return;
  float4 sum[E4];
  ordered_sum<E4, G * D / 4, NT>(rpart, (uint32_t)(((size_t)b * a.n_split_max + grp * kGroup) * sstride + hd * 4),
                             sstride, gsz, sum);
  uint16_t* out = ctx + (size_t)b * a.NH * D + hd;
  if (ngroups == 1) {
    store_bf16x4<E4, G * D / 4, NT>(out, sum);
    return;
  }
  const __amdgpu_buffer_rsrc_t rgrp = buffer_rsrc(ws_group, (uint32_t)(a.B * kMaxGroups) * sstride);
  const uint32_t gbase = (uint32_t)((size_t)b * kMaxGroups * sstride + hd * 4);
#pragma unroll
  for (int r = 0; r < E4; ++r) {
    const int e4 = threadIdx.x + NT * r;
    if (e4 < G * D / 4) coherent_store4(rgrp, gbase + (uint32_t)grp * sstride + 16u * (uint32_t)e4, sum[r]);
  }
  if (!arrive_last(cnt, (unsigned)ngroups, &flag)) return;
  ordered_sum<E4, G * D / 4, NT>(rgrp, gbase, sstride, ngroups, sum);
  store_bf16x4<E4, G * D / 4, NT>(out, sum);
}

// ------------------------------------------------------------------ split reduction (8-wave path)
// ctx[b, kv*G + g, :] = bf16(sum of the split partials of the 8-wave P.V
// launch), summed in the order of the in-kernel reduction of the 4-wave path
// (groups of kGroup consecutive splits, each in split order from +0, then
// the group sums in group order from +0).  Run as its own launch, every
// partial in flight at once: a chain of in-kernel arrivals costs a
// write-through, an atomic round trip and a read per level.  grid
// (ceil(G*D/4 / kRedCols), KV, B), 256 threads: thread (h, c) sums groups
// h, h + 8 of float4 column c.  Ranges the P.V launch finished itself
// (nothing attended, or at most kShortLen positions) are left alone.
constexpr int kRedCols = 32;   // float4 columns per block
constexpr int kRedRows = 8;    // groups summed side by side

template <int D, int G>
__global__ __launch_bounds__(256) void attn_reduce_kernel(AttnDims a, const int32_t* __restrict__ pos_arr,
                                                          const float* __restrict__ ws_part,
                                                          uint16_t* __restrict__ ctx) {
  constexpr int N4 = G * D / 4;  // float4 columns of one KV head's group of heads
  __shared__ float4 gs[kMaxGroups][kRedCols];
  const int kv = blockIdx.y, b = blockIdx.z;
  const Range R = attn_range(a, pos_arr[b]);
  if (R.n_eff == 0 || R.len <= kShortLen) return;
  const int c = threadIdx.x % kRedCols, h = threadIdx.x / kRedCols;
  const int col = min((int)blockIdx.x * kRedCols + c, N4 - 1);
  const int ngroups = (R.n_eff + kGroup - 1) / kGroup;
  const size_t stride4 = (size_t)a.NH * D / 4;  // float4s per split partial
  const float4* part = reinterpret_cast<const float4*>(ws_part) + (size_t)b * a.n_split_max * stride4 +
                       (size_t)kv * G * D / 4 + col;
#pragma unroll
  for (int m = 0; m < kMaxGroups / kRedRows; ++m) {
    const int g = h + kRedRows * m;
    if (g < ngroups) {
      const int n = min(kGroup, R.n_eff - g * kGroup);
      float4 v[kGroup];
#pragma unroll
      for (int i = 0; i < kGroup; ++i) v[i] = part[(size_t)(g * kGroup + min(i, n - 1)) * stride4];
      float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int i = 0; i < kGroup; ++i)
        if (i < n) {
          t.x += v[i].x; t.y += v[i].y; t.z += v[i].z; t.w += v[i].w;
        }
      gs[g][c] = t;
    }
  }
  __syncthreads();
  if (h == 0 && (int)blockIdx.x * kRedCols + c < N4) {
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int g = 0; g < ngroups; ++g) {
      const float4 u = gs[g][c];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    uint2 w;
    w.x = pack2(t.x, t.y);
    w.y = pack2(t.z, t.w);
    reinterpret_cast<uint2*>(ctx + (size_t)b * a.NH * D + (size_t)kv * G * D)[col] = w;
  }
}

// ------------------------------------------------------------------ one launch per layer, one XCD per KV head
// Batch 1, at most 8 KV heads (the sliding layers, 8 heads of 256 with 2
// query heads each: model.py:207-213 with the window mask of
// model.py:402-408; and the full k==v layers, 2 heads of 512 with 8 query
// heads each, while they span at most kLocalLen positions), every split at
// most kChunkMin positions and at most kLocalLen positions attended.  XCDs
// past the last KV head have nothing to do.  The 8 XCDs take a launch's blocks in
// turn (block b runs on XCD b % 8, checked on the host before the path is
// used), so the blocks b, b + 8, b + 16, ... share one XCD and its L2.  A
// block serves KV head kv = its XCD, and role r = b / 8:
//   r < n_split_max (scores): split r's scores, as attn_qk_kernel computes
//     them (q norm + RoPE, the append, MFMA scores, softcap, the split's max
//     and sum of exp), stored with plain stores (they stay in the XCD's L2);
//     then the block counts in on its head's counter;
//   r - n_split_max = x < D / kSliceD (P.V): requests the V rows of head
//     dims [x * kSliceD, +kSliceD) at every attended position at its start,
//     rebuilds the new V row of position pos from v_raw (the rows were
//     requested before the append), waits until all n_eff splits have
//     counted in (device-scope polls, a bounded wait), reads the head's
//     scores and statistics from the L2 and sums P.V in the order of
//     pv_short (each lane its positions in step order, a DPP sum over the
//     lanes of a step, then the waves in order), extended to kLocalLen
//     positions.
// The last P.V block of a head resets the head's counters for the next
// launch.
constexpr int kLocalLen = 1024;
constexpr int kLocalPage = 64;       // cache page size of this path (positions per page)
constexpr int kLocalSpin = 1 << 22;  // polls before a waiting block gives up (~0.1 s)

template <int D, int G, bool DPT>
__device__ __forceinline__ void attn_local_scores(
    const AttnDims& a, const Range& R, int kv, int split, int pos, const uint16_t* __restrict__ q_raw,
    const uint16_t* __restrict__ k_raw, const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, const uint16_t* __restrict__ rope_cos, const uint16_t* __restrict__ rope_sin,
    uint16_t* __restrict__ k_pages, uint16_t* __restrict__ v_pages, const int32_t* __restrict__ page_table,
    int append, float* ws_scores, float* ws_stats, unsigned int* cnt) {
  constexpr int PL = D / 64;
  constexpr int NT = 256;
  constexpr int KS = D / 32;
  constexpr int GW = (G + 3) / 4;  // query heads per wave: wave w takes heads w, w + 4
  static_assert(G <= 8, "at most 8 query heads per KV head");
  if (threadIdx.x >= NT) return;  // the fifth wave polls in the P.V role only
  __shared__ __align__(16) uint16_t qa[16 * D];
  __shared__ __align__(16) uint16_t kn16[D];
  __shared__ float knew[D];
  __shared__ float vnew[D];
  __shared__ float sc[G][kChunkMin];
  __shared__ int ptl[512];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int start = R.lo + split * R.chunk;
  const int end = min(R.lo + R.len, start + R.chunk);
  const int npos = end - start;
  const PtRow<DPT> pt_row = pt_row_of<DPT>(a, page_table, 0);
  const int kg = lane >> 4, col = lane & 15;
  constexpr int PG = kLocalPage;
  const int first = start / PG;
  const PtStage<NT> pts = stage_load<NT>(a, pt_row, first);
  const int jc0 = min(wave * 16 + col, npos - 1);
  const int pe0 = pt_row[(start + jc0) / PG];
  // prologue rows: wave w takes q heads w, w + 4; the split that ends at
  // pos appends the new K (wave 2) and V (wave 3)
  const int so = lane * PL, jo = so % (D / 2);
  const bool mine = append && (end == pos + 1);
  float qx[GW][PL], qw[PL], cs[PL], sn[PL], kvx[PL], kw[PL];
#pragma unroll
  for (int u = 0; u < GW; ++u) load_slice<PL>(q_raw + ((size_t)kv * G + min(wave + 4 * u, G - 1)) * D + so, qx[u]);
  load_slice<PL>(q_norm + so, qw);
  load_slice<PL>(rope_cos + (size_t)pos * (D / 2) + jo, cs);
  load_slice<PL>(rope_sin + (size_t)pos * (D / 2) + jo, sn);
  {
    const uint16_t* kr = mine ? k_raw + (size_t)kv * D : q_norm;
    const uint16_t* vr = (mine && v_raw != nullptr) ? v_raw + (size_t)kv * D : kr;
    load_slice<PL>((wave == 2 ? kr : vr) + so, kvx);
    load_slice<PL>((mine ? k_norm : q_norm) + so, kw);
  }
  // this wave's K tile (positions 16 w .. 16 w + 15 of the split)
  u32x4 bt[KS];
  const bool valid0 = pe0 >= 0 && pe0 < a.num_pages;
  const long long ot = valid0 ? ((((long long)pe0 * a.KV + kv) * PG) + ((start + jc0) % PG)) * (long long)D : -1ll;
  {
    const uint16_t* kp = k_pages + max(ot, 0ll) + 8 * kg;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) bt[s2] = ld16((const u32x4*)(kp + 32 * s2));
  }
  for (int c = tid; c < (16 - G) * D / 8; c += NT) ((u32x4*)(qa + G * D))[c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    const int g = wave + 4 * u;
    if (g < G) {
      norm_rope_slice<D>(qx[u], qw, cs, sn, a.eps, true);
#pragma unroll
      for (int i = 0; i < PL; ++i) qa[g * D + so + i] = f2bf(qx[u][i]);
    }
  }
  if (mine && wave >= 2) {
    norm_rope_slice<D>(kvx, wave == 2 ? kw : nullptr, cs, sn, a.eps, wave == 2);
    float* dst = (wave == 2) ? knew : vnew;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      dst[so + i] = kvx[i];
      if (wave == 2) kn16[so + i] = f2bf(kvx[i]);
    }
  }
  stage_store<NT>(pts, ptl);
  lds_barrier();
  if (mine) {
    const int pe = ptl[pos / PG - first];
    if (pe >= 0 && pe < a.num_pages) {
      const long long off = ((((long long)pe * a.KV + kv) * PG) + (pos % PG)) * (long long)D;
      for (int d = tid; d < D; d += NT) {
        k_pages[off + d] = f2bf(knew[d]);
        v_pages[off + d] = f2bf(vnew[d]);
      }
    }
  }
  u32x4 af[KS];
#pragma unroll
  for (int s2 = 0; s2 < KS; ++s2) af[s2] = *(const u32x4*)(qa + col * D + 32 * s2 + 8 * kg);
  const int ntiles = (npos + 15) >> 4;
  if (wave < ntiles) {
    const int j = wave * 16 + col;
    const bool isnew = mine && (start + j == pos);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) {
      u32x4 kb = bt[s2];
      if (mine) kb = isnew ? *(const u32x4*)(kn16 + 32 * s2 + 8 * kg) : kb;
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[s2]),
                                                    __builtin_bit_cast(bf16x8, kb), acc, 0, 0, 0);
    }
    const bool ok = (ot >= 0) || isnew;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kg + i;
      if (h < G && j < npos) {
        float sv = rbf(acc[i]);
        if (a.softcap > 0.0f) sv = tanhf(sv / a.softcap) * a.softcap;
        sc[h][j] = ok ? sv : -INFINITY;
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    const int g = wave + 4 * u;
    if (g < G) {
      float m = -INFINITY;
      for (int j = lane; j < npos; j += 64) m = fmaxf(m, sc[g][j]);
      m = wave_max_bfly(m);
      float* srow = ws_scores + ((size_t)kv * G + g) * a.lmax + (start - R.lo);
      float l = 0.0f;
      for (int j = lane; j < npos; j += 64) {
        const float s2 = sc[g][j];
        l += (s2 == -INFINITY) ? 0.0f : expf(s2 - m);
        srow[j] = s2;
      }
      l = group_sum<64>(l);
      if (lane == 0) {
        const int h = kv * G + g;
        ws_stats[(size_t)h * a.n_split_max + split] = m;
        ws_stats[((size_t)a.NH + h) * a.n_split_max + split] = l;
      }
    }
  }
  // the block's scores and statistics (and its cache append) have reached
  // the L2; then count in
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int G, bool DPT>
__device__ __forceinline__ void attn_local_pv(const AttnDims& a, const Range& R, int kv, int slice, int pos,
                                              const uint16_t* __restrict__ k_raw, const uint16_t* __restrict__ v_raw,
                                              const uint16_t* v_pages, const int32_t* __restrict__ page_table,
                                              int append, const float* ws_scores, const float* ws_stats,
                                              unsigned int* cnt, uint16_t* __restrict__ ctx) {
  constexpr int PL = D / 64;
  constexpr int NT = 256, NW = 4;
  constexpr int LPS = kSliceD / 8, PPW = 64 / LPS, PPB = NW * PPW;
  constexpr int NST = kLocalLen / PPB;     // V steps per lane at most
  constexpr int SPT = G * kLocalLen / NT;  // scores per thread at most
  __shared__ __align__(16) uint16_t vn16[D];
  __shared__ float pr[G * kLocalLen];
  __shared__ float red[NW * G * kSliceD];
  __shared__ float mg[G], sg[G];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int slot = lane % PPW, sub = lane / PPW;
  const int d0 = slice * kSliceD + sub * 8;
  const int len = R.len;
  const int nst = (len + PPB - 1) / PPB;
  constexpr int PG = kLocalPage;
  const PtRow<DPT> pt_row = pt_row_of<DPT>(a, page_table, 0);
  // the attended range spans at most kLocalLen / PG + 1 pages; with a page
  // table their entries are staged in LDS first (one round trip; a table
  // load per step, under the step's branch, waited for each before its V row)
  constexpr int NPG = kLocalLen / PG + 1;
  __shared__ int ptv[NPG];
  const int pfirst = R.lo / PG;
  // the new V row's raw values, then the V slice at every attended position
  float vx[PL], dummy[PL];
  if (append && wave < NW) load_slice<PL>((v_raw != nullptr ? v_raw : k_raw) + (size_t)kv * D + lane * PL, vx);
  if constexpr (!DPT) {
    if (tid < NPG) ptv[tid] = pt_row[min(pfirst + tid, a.max_pages - 1)];
    __syncthreads();
  }
  // V steps in chunks of CH (a block-uniform branch per chunk, none inside:
  // a chunk's LDS reads are then issued together); the rows of steps past
  // the range are not requested and read as zero
  constexpr int CH = 4;
  static_assert(NST % CH == 0, "whole chunks");
  u32x4 vv[NST];
  bool okv[NST];
  if (wave < NW) {
    int pgv[NST];  // every step's page, before the first V row is requested
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int p = R.lo + min(st * PPB + wave * PPW + slot, len - 1);
      if constexpr (DPT) pgv[st] = pt_row[p / PG];
      else pgv[st] = ptv[p / PG - pfirst];
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int j = st * PPB + wave * PPW + slot;
      okv[st] = false;
      vv[st] = u32x4{0u, 0u, 0u, 0u};
      if (st < nst) {  // block-uniform: no loads for the steps past the range
        const int p = R.lo + min(j, len - 1);
        const int pg = pgv[st];
        const bool valid = pg >= 0 && pg < a.num_pages;
        const long long off = ((((long long)(valid ? pg : 0) * a.KV + kv) * PG) + (p % PG)) * (long long)D;
        vv[st] = ld16((const u32x4*)(v_pages + off + d0));
        okv[st] = (j < len) && valid;
      }
    }
    // wave 1 rebuilds the new V row (it waits for the loads above)
    if (append && wave == 1) {
      norm_rope_slice<D>(vx, nullptr, dummy, dummy, a.eps, false);
#pragma unroll
      for (int i = 0; i < PL; ++i) vn16[lane * PL + i] = f2bf(vx[i]);
    }
  } else if (lane == 0) {
    // the fifth wave, with no loads of its own in flight (a wave's loads
    // return in order, so a poll behind the V rows would see the count
    // only after them), waits until every split of this head has counted in
    int it = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)R.n_eff &&
           ++it < kLocalSpin)
      __builtin_amdgcn_s_sleep(1);
  }
  __syncthreads();
  if (wave >= NW) return;
  float sreg[SPT];
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const int idx = tid + NT * r, g = idx / kLocalLen, j = idx % kLocalLen;
    sreg[r] = ws_scores[((size_t)kv * G + g) * a.lmax + min(j, len - 1)];
  }
  SplitStats<G, NW> sst = load_split_stats<G, NW>(a, R, kv, 0, wave, lane, ws_stats);
  // this block has passed the wait: count out (the last P.V block of the
  // head resets its counters at the end).  Issued after the score loads, so
  // waiting for them does not wait for the atomic's return; the returned
  // count is looked at only at the end of the block.
  unsigned prev = 0;
  if (tid == 3 * 64) prev = __hip_atomic_fetch_add(cnt + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  reduce_split_stats<G, NW>(sst, R, wave, lane, mg, sg);
  lds_barrier();
  float mr[G], sr[G];  // in registers: the probability loop's LDS stores would otherwise reload them
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mr[g] = mg[g];
    sr[g] = sg[g];
  }
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const int idx = tid + NT * r, g = idx / kLocalLen, j = idx % kLocalLen;
    const float sv = sreg[r];
    if (j < len) pr[g * kLocalLen + j] = (sv == -INFINITY) ? 0.0f : rbf(expf(sv - mr[g]) / sr[g]);
  }
  lds_barrier();
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
  const u32x4 vnew_slice = append ? *(const u32x4*)(vn16 + d0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int c0 = 0; c0 < NST; c0 += CH) {
    if (c0 < nst) {
      float pc[CH][G];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int j = min((c0 + u) * PPB + wave * PPW + slot, kLocalLen - 1);
#pragma unroll
        for (int g = 0; g < G; ++g) pc[u][g] = okv[c0 + u] ? pr[g * kLocalLen + j] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int j = (c0 + u) * PPB + wave * PPW + slot;
        const u32x4 v = (append && R.lo + j == pos) ? vnew_slice : vv[c0 + u];
        float vf[8];
        unpack8(v, vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(pc[u][g], vf[i], acc[g][i]);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = group_sum<PPW>(acc[g][i]);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) red[(wave * G + g) * kSliceD + sub * 8 + i] = acc[g][i];
  }
  lds_barrier();
  for (int e = tid; e < G * kSliceD; e += NT) {
    const int g = e / kSliceD, dd = e % kSliceD;
    float v = red[g * kSliceD + dd];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[(w * G + g) * kSliceD + dd];  // in wave order
    ctx[((size_t)kv * G + g) * D + slice * kSliceD + dd] = f2bf(v);
  }
  if (tid == 3 * 64 && prev == (unsigned)(D / kSliceD) - 1) {  // every P.V block of the head is past the wait
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(cnt + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// grid 8 * (n_split_max + D / kSliceD) blocks of 320 threads (the P.V
// role's fifth wave polls; the scores role uses four)
constexpr int kLocalThreads = 320;
template <int D, int G, bool DPT>
__global__ __launch_bounds__(kLocalThreads) void attn_local_kernel(
    AttnDims a, const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
    const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const uint16_t* __restrict__ rope_cos, const uint16_t* __restrict__ rope_sin, uint16_t* __restrict__ k_pages,
    uint16_t* v_pages, const int32_t* __restrict__ page_table, const int32_t* __restrict__ pos_arr, int append,
    float* ws_scores, float* ws_stats, unsigned int* counters, uint16_t* __restrict__ ctx) {
  const int kv = xcc_id();
  const int role = (int)blockIdx.x >> 3;
  if (kv >= a.KV) return;
  const int pos = pos_arr[0];
  const Range R = attn_range(a, pos);
  if (R.n_eff == 0) {  // nothing attended: ctx = 0
    if (role == 0)
      for (int e = threadIdx.x; e < G * D; e += kLocalThreads) ctx[(size_t)kv * G * D + e] = 0;
    return;
  }
  unsigned int* cnt = counters + (size_t)kv * (kMaxGroups + 1);
  if (role < a.n_split_max) {
    if (role < R.n_eff)
      attn_local_scores<D, G, DPT>(a, R, kv, role, pos, q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin,
                                   k_pages, v_pages, page_table, append, ws_scores, ws_stats, cnt);
  } else if (role - a.n_split_max < D / kSliceD) {
    attn_local_pv<D, G, DPT>(a, R, kv, role - a.n_split_max, pos, k_raw, v_raw, v_pages, page_table, append,
                             ws_scores, ws_stats, cnt, ctx);
  }
}


// ------------------------------------------------------------------ append
// k = rope(rms_norm(k_raw, k_norm)), v = rms_norm(v_raw) of T tokens of one
// sequence written at positions pos[t] (model.py:202-206).  grid (T, KV).
template <int D>
__global__ __launch_bounds__(128) void kv_append_kernel(AttnDims a, const uint16_t* __restrict__ k_raw,
                                                        const uint16_t* __restrict__ v_raw,
                                                        const uint16_t* __restrict__ k_norm,
                                                        const uint16_t* __restrict__ rope_cos,
                                                        const uint16_t* __restrict__ rope_sin,
                                                        uint16_t* __restrict__ k_pages, uint16_t* __restrict__ v_pages,
                                                        const int32_t* __restrict__ page_table,
                                                        const int32_t* __restrict__ pos_arr) {
  __shared__ float kn[D], vn[D];
  constexpr int PL = D / 64;
  const int t = blockIdx.x, kv = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pos = pos_arr[t];
  if (pos < 0 || pos >= a.lmax || pos >= a.max_pages * a.page) return;
  const int so = lane * PL, jo = so % (D / 2);
  const uint16_t* kr = k_raw + ((size_t)t * a.KV + kv) * D;
  const uint16_t* vr = (v_raw != nullptr) ? v_raw + ((size_t)t * a.KV + kv) * D : kr;
  float x[PL], w[PL], cs[PL], sn[PL];
  load_slice<PL>((wave == 0 ? kr : vr) + so, x);
  load_slice<PL>(k_norm + so, w);
  load_slice<PL>(rope_cos + (size_t)pos * (D / 2) + jo, cs);
  load_slice<PL>(rope_sin + (size_t)pos * (D / 2) + jo, sn);
  norm_rope_slice<D>(x, wave == 0 ? w : nullptr, cs, sn, a.eps, wave == 0);
  float* dst = (wave == 0) ? kn : vn;
#pragma unroll
  for (int i = 0; i < PL; ++i) dst[so + i] = x[i];
  __syncthreads();
  const long long off = page_off(a, page_table, pos, kv);
  if (off < 0) return;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    k_pages[off + d] = f2bf(kn[d]);
    v_pages[off + d] = f2bf(vn[d]);
  }
}

// ------------------------------------------------------------------ launch
struct AttnWs {
  float *scores, *stats, *part, *group;
  unsigned int* counters;
};

template <int D, int G, bool DPT>
static void launch_attn(const AttnDims& a, dim3 grid, hipStream_t st, const uint16_t* q_raw, const uint16_t* k_raw,
                        const uint16_t* v_raw, const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* cs,
                        const uint16_t* sn, uint16_t* kp, uint16_t* vp, const int32_t* pt, const int32_t* pos,
                        int append, const AttnWs& w, uint16_t* ctx) {
  // every split holds at most kChunkMin positions when the longest range
  // does: one K tile per wave, 4 waves.  Longer ranges (up to kChunkMax
  // positions per split) run 8 waves per block with every K tile and V row
  // of a split requested at once.
  const int span = (a.window > 0 && a.window < a.lmax) ? a.window : a.lmax;
  const dim3 pgrid(max(grid.x, (unsigned)(D / kSliceD)), grid.y, grid.z);  // short ranges use D / kSliceD blocks
  if (span <= kChunkMin * a.n_split_max) {
    hipLaunchKernelGGL((attn_qk_kernel<D, G, true, 4, DPT>), grid, dim3(256), 0, st, a, q_raw, k_raw, v_raw, q_norm,
                       k_norm, cs, sn, kp, vp, pt, pos, append, w.scores, w.stats);
    hipLaunchKernelGGL((attn_pv_kernel<D, G, 4, DPT>), pgrid, dim3(256), 0, st, a, vp, pt, pos, w.scores, w.stats,
                       w.part, w.group, w.counters, ctx);
  } else {
    hipLaunchKernelGGL((attn_qk_kernel<D, G, false, 8, DPT>), grid, dim3(512), 0, st, a, q_raw, k_raw, v_raw,
                       q_norm, k_norm, cs, sn, kp, vp, pt, pos, append, w.scores, w.stats);
    hipLaunchKernelGGL((attn_pv_kernel<D, G, 8, DPT>), pgrid, dim3(512), 0, st, a, vp, pt, pos, w.scores, w.stats,
                       w.part, w.group, w.counters, ctx);
    const dim3 rgrid((unsigned)((G * D / 4 + kRedCols - 1) / kRedCols), grid.y, grid.z);
    hipLaunchKernelGGL((attn_reduce_kernel<D, G>), rgrid, dim3(256), 0, st, a, pos, w.part, ctx);
  }
}

static int64_t al256(int64_t x) { return ((x + 255) / 256) * 256; }

static bool attn_local_enabled() {
  const char* e = getenv("G4MI_ATTN_LOCAL");
  return e == nullptr || atoi(e) != 0;
}

// Zeroes n words (the arrival counters of a call that brings no workspace of
// its own, see g4mi_decode_attention_noalloc).
__global__ __launch_bounds__(256) void zero_words_kernel(unsigned int* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

// ------------------------------------------------------------------ no-allocation scratch
// The workspace of g4mi_decode_attention_noalloc: a file-scope device array,
// one copy per GPU, held until the process ends.  Its device address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that address is handed to kernels.
constexpr int64_t kNoAllocScratchBytes = G4MI_NOALLOC_ATTENTION_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("decode_attention_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  G4MI_REQUIRE(dev >= 0 && dev < kMaxDevices, G4MI_EUNSUPPORTED, "decode_attention_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("decode_attention_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return e != hipSuccess ? (int)e : G4MI_EINVAL;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Argument checks and launches shared by the two decode attention entry
// points.  With clear_counters the workspace's arrival counters are zeroed
// first by a fill kernel on the same stream (a shared scratch may hold
// another call's data where this call's counters sit).
static int decode_attention_impl(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                 const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                                 const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                                 const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B,
                                 int64_t NH, int64_t KV, int64_t D, int64_t page_size, int64_t window, float softcap,
                                 float eps, int32_t append, int64_t lmax, int64_t n_split_max, uint16_t* ctx,
                                 void* ws, int64_t ws_bytes, bool clear_counters, void* stream);

}  // namespace g4mi

using namespace g4mi;

extern "C" {

// Workspace layout: the arrival counters first, so calls with the same B and
// NH find them at the same place whatever their head_dim, lmax and split
// count (the decode step shares one workspace between its sliding and full
// layers); then scores, split statistics, split partials, group partials.
int64_t g4mi_decode_attention_workspace_bytes(int64_t B, int64_t NH, int64_t D, int64_t lmax, int64_t n_split_max) {
  return al256(B * NH * (kMaxGroups + 1) * 4) + al256(B * NH * lmax * 4) + al256(2 * B * NH * n_split_max * 4) +
         al256(B * n_split_max * NH * D * 4) + al256(B * kMaxGroups * NH * D * 4);
}

int64_t g4mi_attention_min_splits(int64_t lmax) { return (lmax + kChunkMax - 1) / kChunkMax; }

int g4mi_decode_attention(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                          const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                          const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                          const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B, int64_t NH,
                          int64_t KV, int64_t D, int64_t page_size, int64_t window, float softcap, float eps,
                          int32_t append, int64_t lmax, int64_t n_split_max, uint16_t* ctx, void* ws,
                          int64_t ws_bytes, void* stream) {
  return decode_attention_impl(q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, num_pages,
                               page_table, max_pages, pos, B, NH, KV, D, page_size, window, softcap, eps, append,
                               lmax, n_split_max, ctx, ws, ws_bytes, false, stream);
}

int g4mi_decode_attention_noalloc(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                  const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                                  const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                                  const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B,
                                  int64_t NH, int64_t KV, int64_t D, int64_t page_size, int64_t window,
                                  float softcap, float eps, int32_t append, int64_t lmax, int64_t n_split_max,
                                  uint16_t* ctx, void* stream) {
  G4MI_REQUIRE(B >= 1 && NH >= 1 && D >= 1 && lmax >= 1 && n_split_max >= 1, G4MI_EINVAL,
               "decode_attention_noalloc: bad B/NH/D/lmax/n_split_max");
  G4MI_REQUIRE(B <= 65535 && NH <= 65535 && D <= 512 && lmax <= (1 << 20) && n_split_max <= 4096, G4MI_EINVAL,
               "decode_attention_noalloc: B/NH/D/lmax/n_split_max out of range");
  const int64_t need = g4mi_decode_attention_workspace_bytes(B, NH, D, lmax, n_split_max);
  G4MI_REQUIRE(need <= kNoAllocScratchBytes, G4MI_EWORKSPACE,
               "decode_attention_noalloc: this call needs %lld bytes of scratch, more than the %lld held per device",
               (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != 0) return rc;
  return decode_attention_impl(q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, num_pages,
                               page_table, max_pages, pos, B, NH, KV, D, page_size, window, softcap, eps, append,
                               lmax, n_split_max, ctx, ws, kNoAllocScratchBytes, true, stream);
}

}  // extern "C"

namespace g4mi {

static int decode_attention_impl(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                 const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope_cos,
                                 const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                                 const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t B,
                                 int64_t NH, int64_t KV, int64_t D, int64_t page_size, int64_t window, float softcap,
                                 float eps, int32_t append, int64_t lmax, int64_t n_split_max, uint16_t* ctx,
                                 void* ws, int64_t ws_bytes, bool clear_counters, void* stream) {
  G4MI_REQUIRE(q_raw && q_norm && rope_cos && rope_sin && k_pages && v_pages && pos && ctx && ws, G4MI_EINVAL,
               "decode_attention: null pointer argument");
  G4MI_REQUIRE(!append || (k_raw && k_norm), G4MI_EINVAL, "decode_attention: append needs k_raw and k_norm");
  G4MI_REQUIRE(B >= 1 && B <= 65535 && KV >= 1 && KV <= 65535 && NH >= KV && NH % KV == 0, G4MI_EINVAL,
               "decode_attention: bad B=%lld NH=%lld KV=%lld", (long long)B, (long long)NH, (long long)KV);
  const int64_t G = NH / KV;
  G4MI_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, G4MI_EUNSUPPORTED,
               "decode_attention: head_dim %lld not in {64,128,256,512}", (long long)D);
  G4MI_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, G4MI_EUNSUPPORTED,
               "decode_attention: %lld query heads per KV head not in {1,2,4,8}", (long long)G);
  G4MI_REQUIRE(page_size >= 1 && max_pages >= 1 && num_pages >= 1 && lmax >= 1, G4MI_EINVAL,
               "decode_attention: bad page_size/max_pages/num_pages/lmax");
  // no page table: sequence b owns pages [b * max_pages, (b + 1) * max_pages)
  const bool dense = page_table == nullptr;
  G4MI_REQUIRE(!dense || B * max_pages <= num_pages, G4MI_EINVAL,
               "decode_attention: without a page table the pool needs B * max_pages = %lld pages, has %lld",
               (long long)(B * max_pages), (long long)num_pages);
  G4MI_REQUIRE(window >= 0, G4MI_EINVAL, "decode_attention: negative window");
  const int64_t span = (window > 0 && window < lmax) ? window : lmax;  // most positions one query attends
  G4MI_REQUIRE(n_split_max >= g4mi_attention_min_splits(span) && n_split_max <= kMaxSplits, G4MI_EINVAL,
               "decode_attention: n_split_max %lld < %lld (a split holds at most %d positions)",
               (long long)n_split_max, (long long)g4mi_attention_min_splits(span), kChunkMax);
  G4MI_REQUIRE(B * n_split_max * NH * D * 4 < ((int64_t)1 << 31), G4MI_EUNSUPPORTED,
               "decode_attention: B * n_split_max * NH * D partials exceed 2 GiB");
  G4MI_REQUIRE(((uintptr_t)k_pages & 15u) == 0 && ((uintptr_t)v_pages & 15u) == 0, G4MI_EALIGN,
               "decode_attention: cache pages must be 16-byte aligned");
  G4MI_REQUIRE(ws_bytes >= g4mi_decode_attention_workspace_bytes(B, NH, D, lmax, n_split_max), G4MI_EWORKSPACE,
               "decode_attention: workspace too small");
  AttnDims a;
  a.B = (int)B; a.NH = (int)NH; a.KV = (int)KV; a.G = (int)G; a.D = (int)D; a.page = (int)page_size;
  a.max_pages = (int)max_pages; a.num_pages = (int)num_pages; a.window = (int)window;
  a.n_split_max = (int)n_split_max; a.lmax = (int)lmax; a.softcap = softcap; a.eps = eps;
  AttnWs w;
  w.counters = (unsigned int*)ws;
  w.scores = (float*)((char*)ws + al256(B * NH * (kMaxGroups + 1) * 4));
  w.stats = (float*)((char*)w.scores + al256(B * NH * lmax * 4));
  w.part = (float*)((char*)w.stats + al256(2 * B * NH * n_split_max * 4));
  w.group = (float*)((char*)w.part + al256(B * n_split_max * NH * D * 4));
  hipStream_t st = as_stream(stream);
  if (clear_counters) {
    const int64_t words = B * NH * (kMaxGroups + 1);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st, w.counters, words);
  }
  // batch 1 with one KV head per XCD and every split within one K tile per
  // wave: the one-launch attention (attn_local_kernel)
  if (B == 1 && KV <= 8 && page_size == kLocalPage && span <= kLocalLen && span <= (int64_t)kChunkMin * n_split_max &&
      ((KV == 8 && G <= 2 && D <= 256) || (KV <= 2 && G == 8 && D == 512)) &&
      attn_local_enabled() && xcc_round_robin(st)) {
    const dim3 lgrid((unsigned)(8 * (n_split_max + D / kSliceD)));
#define G4MI_LOC(DD, GG)                                                                                       \
    if (D == DD && G == GG) {                                                                                  \
      if (dense)                                                                                               \
        hipLaunchKernelGGL((attn_local_kernel<DD, GG, true>), lgrid, dim3(kLocalThreads), 0, st, a, q_raw, k_raw, v_raw,  \
                           q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table, pos, append,       \
                           w.scores, w.stats, w.counters, ctx);                                                 \
      else                                                                                                     \
        hipLaunchKernelGGL((attn_local_kernel<DD, GG, false>), lgrid, dim3(kLocalThreads), 0, st, a, q_raw, k_raw, v_raw, \
                           q_norm, k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table, pos, append,       \
                           w.scores, w.stats, w.counters, ctx);                                                 \
    }
    G4MI_LOC(64, 1) G4MI_LOC(64, 2) G4MI_LOC(128, 1) G4MI_LOC(128, 2) G4MI_LOC(256, 1) G4MI_LOC(256, 2)
    G4MI_LOC(512, 8)
#undef G4MI_LOC
    return check_launch("decode_attention");
  }
  dim3 grid((unsigned)n_split_max, (unsigned)KV, (unsigned)B);
#define G4MI_ATT(DD, GG)                                                                                      \
  if (D == DD && G == GG) {                                                                                   \
    if (dense)                                                                                                \
      launch_attn<DD, GG, true>(a, grid, st, q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin, k_pages, \
                                v_pages, page_table, pos, append, w, ctx);                                    \
    else                                                                                                      \
      launch_attn<DD, GG, false>(a, grid, st, q_raw, k_raw, v_raw, q_norm, k_norm, rope_cos, rope_sin,         \
                                 k_pages, v_pages, page_table, pos, append, w, ctx);                          \
  }
  G4MI_ATT(64, 1) G4MI_ATT(64, 2) G4MI_ATT(64, 4) G4MI_ATT(64, 8)
  G4MI_ATT(128, 1) G4MI_ATT(128, 2) G4MI_ATT(128, 4) G4MI_ATT(128, 8)
  G4MI_ATT(256, 1) G4MI_ATT(256, 2) G4MI_ATT(256, 4) G4MI_ATT(256, 8)
  G4MI_ATT(512, 1) G4MI_ATT(512, 2) G4MI_ATT(512, 4) G4MI_ATT(512, 8)
#undef G4MI_ATT
  return check_launch("decode_attention");
}

}  // namespace g4mi

extern "C" {

int g4mi_kv_append(const uint16_t* k_raw, const uint16_t* v_raw, const uint16_t* k_norm, const uint16_t* rope_cos,
                   const uint16_t* rope_sin, uint16_t* k_pages, uint16_t* v_pages, int64_t num_pages,
                   const int32_t* page_table, int64_t max_pages, const int32_t* pos, int64_t T, int64_t KV, int64_t D,
                   int64_t page_size, int64_t lmax, float eps, void* stream) {
  G4MI_REQUIRE(k_raw && k_norm && rope_cos && rope_sin && k_pages && v_pages && page_table && pos, G4MI_EINVAL,
               "kv_append: null pointer argument");
  G4MI_REQUIRE(T >= 1 && T <= 65535 && KV >= 1 && KV <= 65535, G4MI_EINVAL, "kv_append: bad T/KV");
  G4MI_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, G4MI_EUNSUPPORTED, "kv_append: bad head_dim");
  G4MI_REQUIRE(page_size >= 1 && max_pages >= 1 && num_pages >= 1 && lmax >= 1, G4MI_EINVAL,
               "kv_append: bad page geometry");
  AttnDims a = {};
  a.KV = (int)KV; a.D = (int)D; a.page = (int)page_size; a.max_pages = (int)max_pages;
  a.num_pages = (int)num_pages; a.lmax = (int)lmax; a.eps = eps;
  hipStream_t st = as_stream(stream);
  switch (D) {
#define G4MI_APP(DD)                                                                                          \
  case DD:                                                                                                    \
    hipLaunchKernelGGL(kv_append_kernel<DD>, dim3((unsigned)T, (unsigned)KV), dim3(128), 0, st, a, k_raw, v_raw, \
                       k_norm, rope_cos, rope_sin, k_pages, v_pages, page_table, pos);                        \
    break;
    G4MI_APP(64) G4MI_APP(128) G4MI_APP(256) G4MI_APP(512)
#undef G4MI_APP
  }
  return check_launch("kv_append");
}

}  // extern "C"
