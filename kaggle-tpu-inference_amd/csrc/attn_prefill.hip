// Causal prefill attention on MFMA (model.py:195-215 at T > 1).
//
// The prompt's query rows attend the paged K/V cache (written beforehand by
// kv_append): query row t sits at position p0 + t and attends keys
// [lo, p0 + t], lo = max(0, p0 + t + 1 - W) on sliding layers, else 0.
// The reference's rounding points are kept: s = f32(bf16(q . k)) with scale
// 1.0, optional softcap, an f32 softmax over the row, probabilities rounded to
// bf16 after normalisation, ctx = bf16(sum_j p_j v_j) with f32 accumulation
// (model.py:207-213).  So the kernel makes two passes over the keys of a query
// block: pass 1 computes each row's max m and sum l of exp(s - m) (online
// over key blocks); pass 2 recomputes the scores, forms p = bf16(exp(s - m) /
// l) -- exactly the bf16 operand the reference's PV product takes -- and
// accumulates P . V on MFMA.
//
// Block: 16 * NW query rows = 16 * NW / G positions x the G query heads of
// one KV head (the K/V tiles are shared by the group), NW waves of 16 rows:
// 8 waves up to head_dim 256 (each staged K/V tile then serves 128 rows: the
// kernel is bound by the K/V rows each CU loads from the caches), 4 at 512
// (a wave holds 16 x 512 accumulators and the Q fragments: one wave per SIMD
// fits).  Key blocks of
// KB keys (one page slice) are staged in LDS: K as [key][D] (the B operand of
// Q.K^T reads 16-byte rows), V transposed to [D][key] (the B operand of P.V).
// The next key block's K/V rows are requested into registers while the
// current one is multiplied (LDS-only barriers, so they stay in flight), and
// the block's page-table entries are staged in LDS once, so no step waits on
// a page-table load.
// v_mfma_f32_16x16x32_bf16: lane l holds A[l%16][8(l/16)..+7],
// B[l%16][8(l/16)..+7] and receives C[4(l/16)+i][l%16].
#include <math.h>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

// waves (of 16 query rows) per block
template <int D>
constexpr int pf_waves() {
  return D >= 512 ? 4 : 8;
}
constexpr int kPfPtl = 256;  // page-table entries of a block staged in LDS (later pages are loaded directly)

struct PfAttnArgs {
  const uint16_t* q;        // [T, NH, D] normalised + rotated
  const uint16_t* k_pages;  // [num_pages, KV, PAGE, D]
  const uint16_t* v_pages;
  const int32_t* pt;        // page table row [max_pages]
  uint16_t* ctx;            // [T, NH, D]
  int T, NH, KV, page, num_pages, max_pages, p0, window;
  float softcap;
  int nqb;   // query blocks per KV head
  int xmap;  // block order: 0 plain, 1 KV divides 8, 2 KV a multiple of 8
};

// Block order.  The launch is a 1-D grid whose blocks the dispatcher hands to
// the 8 XCDs in turn (block b to the XCD of b % 8), and each XCD has its own
// L2.  The query blocks of one KV head read the same K/V rows, so they are
// kept on the XCDs of that head: with KV dividing 8, XCD x serves head
// x % KV and every (8 / KV)-th query block of it (long and short blocks
// alike, so the XCDs finish together); with KV a multiple of 8, XCD x serves
// heads x, x + 8, ...; other head counts take the plain order (block b: head
// b / nqb).  Within a head the query blocks go longest first.  Returns false
// for the padding blocks of the first order.
__device__ __forceinline__ bool pf_block(const PfAttnArgs& a, int& kv, int& qb) {
  const int b = (int)blockIdx.x, x = b & 7, slot = b >> 3;
  int j;
  if (a.xmap == 1) {
    kv = x % a.KV;
    j = x / a.KV + (8 / a.KV) * slot;
  } else if (a.xmap == 2) {
    const int per = a.KV / 8;
    kv = x + 8 * (slot % per);
    j = slot / per;
  } else {
    kv = b / a.nqb;
    j = b % a.nqb;
  }
  qb = a.nqb - 1 - j;
  return j < a.nqb;
}

// ---------------------------------------------------------------- q norm + RoPE
// q = rope(rms_norm(q_raw, q_norm)) in place for T rows of NH heads at
// positions p0 + t (model.py:198-199); grid (T, ceil(NH/4)), wave per head.
// Lane l owns the D/64 consecutive values at l*D/64; the RoPE partner
// (d +- D/2) sits in lane l^32.
template <int D>
__global__ __launch_bounds__(256) void q_norm_rope_kernel(uint16_t* __restrict__ q, const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ cs_tab,
                                                          const uint16_t* __restrict__ sn_tab, int NH, int p0,
                                                          float eps) {
  constexpr int PL = D / 64;
  const int t = blockIdx.x, lane = threadIdx.x & 63;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (h >= NH) return;
  const int so = lane * PL, jo = so % (D / 2);
  const int pos = p0 + t;
  uint16_t* row = q + ((size_t)t * NH + h) * D + so;
  float x[PL], ww[PL], cs[PL], sn[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    x[i] = bf2f(row[i]);
    ww[i] = bf2f(w[so + i]);
    cs[i] = bf2f(cs_tab[(size_t)pos * (D / 2) + jo + i]);
    sn[i] = bf2f(sn_tab[(size_t)pos * (D / 2) + jo + i]);
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < PL; ++i) ss = fma((double)x[i], (double)x[i], ss);
  const float r = rms_scale(group_sum_f64<64>(ss), D, eps);
#pragma unroll
  for (int i = 0; i < PL; ++i) x[i] = rbf(x[i] * r * ww[i]);
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const float partner = __shfl_xor(x[i], 32, kWave);
    const float rot = (so + i < D / 2) ? -partner : partner;
    row[i] = f2bf(rbf(rbf(x[i] * cs[i]) + rbf(rot * sn[i])));
  }
}

// ---------------------------------------------------------------- attention
// max / sum over the 16 lanes of a DPP row (the 16 key columns of a tile row).
// The max is one v_max_f32 with a DPP operand per round (fmaxf on a DPP move
// would add a move and two canonicalising maxes; the scores hold no NaN); the
// s_nop gives the two wait states a DPP read of a just-written VGPR needs.
template <int CTRL>
__device__ __forceinline__ float dpp_max_f(float v) {
  float r;
  if constexpr (CTRL == kDppXor1)
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
  else if constexpr (CTRL == kDppXor2)
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
  else if constexpr (CTRL == kDppHalfMirror)
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
  else
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
  return r;
}
__device__ __forceinline__ float row16_max(float v) {
  v = dpp_max_f<kDppXor1>(v);
  v = dpp_max_f<kDppXor2>(v);
  v = dpp_max_f<kDppHalfMirror>(v);
  v = dpp_max_f<kDppMirror>(v);
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return v;
}

// p = bf16(e / l) from the reciprocal rl = rcp(l): e * rl lies within 3.5 f32
// ulps of the rounded quotient (rcp within 1 ulp, the product's rounding), so
// it rounds to the same bf16 unless it sits within 8 ulps of a bf16 rounding
// midpoint (low 16 bits 0x7ff8..0x8008); those take the IEEE division.
__device__ __forceinline__ bool near_bf16_midpoint(float x) {
  return ((__float_as_uint(x) - 0x7ff8u) & 0xffffu) <= 16u;
}

template <int D, int G, bool CAP>
__global__ __launch_bounds__(64 * pf_waves<D>()) void attn_prefill_kernel(PfAttnArgs a) {
  constexpr int NW = pf_waves<D>();
  constexpr int NTH = 64 * NW;              // threads
  constexpr int ROWS = 16 * NW;             // query rows per block
  constexpr int KB = (D >= 512) ? 32 : 64;  // keys per block step (divides the page)
  constexpr int QP = ROWS / G;              // positions per block
  constexpr int KS = D / 32;                // MFMA k-steps over D (scores)
  constexpr int NT = KB / 16;               // key tiles per step
  constexpr int DT = D / 16;                // output d tiles
  constexpr int LDK = D + 8;                // K row stride in LDS (elements)
  constexpr int LDV = KB + 8;               // V^T row stride
  constexpr int LDP = KB + 8;               // P row stride
  // From head_dim 256 the K/V tiles are double-buffered (the next step's rows
  // go to the other buffer while this one is read: one barrier per step; 157
  // KB of LDS at 256, 151 KB at 512, where one block per CU runs anyway).
  constexpr int NBUF = (D >= 256) ? 2 : 1;
  __shared__ __align__(16) uint16_t kt[NBUF][KB * LDK];
  __shared__ __align__(16) uint16_t vt[NBUF][D * LDV];
  __shared__ __align__(16) uint16_t pt[ROWS * LDP];
  __shared__ int ptl[kPfPtl];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  int kv, qb;
  if (!pf_block(a, kv, qb)) return;
  const int t0 = qb * QP;
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  // this lane's rows in the C layout: r = 16*wave + 4*(lane/16) + i
  int rpos[4];
  bool rvalid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * (lane >> 4) + i;
    const int t = t0 + r / G;
    rvalid[i] = t < a.T;
    rpos[i] = a.p0 + min(t, a.T - 1);
  }
  // A fragments of Q: row 16*wave + fr (position t0 + row/G, head kv*G + row%G)
  u32x4 qf[KS];
  {
    const int r = 16 * wave + fr;
    const int t = min(t0 + r / G, a.T - 1);
    const uint16_t* qrow = a.q + ((size_t)t * a.NH + kv * G + r % G) * D + fk;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = ld16((const u32x4*)(qrow + 32 * s));
  }
  // key range of the block
  const int pos_first = a.p0 + t0, pos_last = a.p0 + min(t0 + QP, a.T) - 1;
  const int k_lo = (a.window > 0) ? max(0, pos_first + 1 - a.window) : 0;
  const int kb0 = k_lo / KB, kb1 = pos_last / KB;
  const float cap = a.softcap;
  // key block kb is interior when every row of the block attends all its keys
  // (no mask, no -inf score); the others (the diagonal, the window's start)
  // take the masked steps
  const int lo_max = (a.window > 0) ? max(0, pos_last + 1 - a.window) : 0;
  auto interior = [&](int kb) { return kb * KB >= lo_max && kb * KB + KB - 1 <= pos_first; };
  using Edge = std::true_type;
  using Inner = std::false_type;

  // the block's page-table entries, staged once (a barrier follows before use)
  const int first_pg = (kb0 * KB) / a.page;
  for (int i = tid; i < kPfPtl; i += NTH) ptl[i] = a.pt[min(first_pg + i, a.max_pages - 1)];
  auto page_of = [&](int kb) {
    const int idx = (kb * KB) / a.page - first_pg;
    return (idx < kPfPtl) ? ptl[idx] : a.pt[min(first_pg + idx, a.max_pages - 1)];
  };
  // K (and V) rows of key block kb into registers (fetch), then into LDS
  // (put); invalid pages read as zero.  The loads are unconditional (page 0
  // stands in for an invalid entry) and the zero is selected afterwards.
  constexpr int CPT = KB * D / 8 / NTH;  // 16-byte chunks per thread and tile
  static_assert(CPT >= 1 && CPT * NTH * 8 == KB * D, "tile chunks");
  struct Tile {
    u32x4 k[CPT], v[CPT];
    bool ok;
  };
  auto fetch = [&](int kb, bool with_v, Tile& T) {
    const int k0 = kb * KB;
    const int pg = page_of(kb);
    T.ok = pg >= 0 && pg < a.num_pages;
    const size_t base = (((size_t)(T.ok ? pg : 0) * a.KV + kv) * a.page + (k0 % a.page)) * D;
#pragma unroll
    for (int i = 0; i < CPT; ++i) T.k[i] = ld16((const u32x4*)(a.k_pages + base) + tid + NTH * i);
    if (with_v) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = tid + NTH * i, j = c % KB, d0 = (c / KB) * 8;
        T.v[i] = ld16((const u32x4*)(a.v_pages + base + (size_t)j * D + d0));
      }
    }
  };
  auto put = [&](const Tile& T, bool with_v, int buf) {
    uint16_t* kw = kt[buf];
    uint16_t* vw = vt[buf];
    const u32x4 z = {0u, 0u, 0u, 0u};
    // K: lanes walk a key row (conflict-free 16-byte stores)
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NTH * i, j = c / (D / 8), d0 = (c % (D / 8)) * 8;
      *(u32x4*)(kw + j * LDK + d0) = T.ok ? T.k[i] : z;
    }
    // V transposed: lanes walk the keys of one 8-value column group, so the
    // 2-byte LDS stores of a wave land in consecutive halfwords
    if (with_v) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = tid + NTH * i, j = c % KB, d0 = (c / KB) * 8;
        const u32x4 v4 = T.ok ? T.v[i] : z;
        const uint32_t w[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vw[(d0 + 2 * e) * LDV + j] = (uint16_t)(w[e] & 0xffffu);
          vw[(d0 + 2 * e + 1) * LDV + j] = (uint16_t)(w[e] >> 16);
        }
      }
    }
  };
  // scores of this wave's 16 rows x KB keys: s[n][i] = row 4(l/16)+i, key k0 + 16n + l%16
  auto scores = [&](int kb, float (*s)[4], auto edge, int buf) {
    const int k0 = kb * KB;
    const uint16_t* kr = kt[buf];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const u32x4 b = *(const u32x4*)(kr + (16 * n + fr) * LDK + 32 * st + fk);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qf[st]),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
      }
      const int j = k0 + 16 * n + fr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sv = rbf(acc[i]);
        if constexpr (CAP) sv = tanhf(sv / cap) * cap;
        if constexpr (decltype(edge)::value) {
          const int lo = (a.window > 0) ? max(0, rpos[i] + 1 - a.window) : 0;
          s[n][i] = (j >= lo && j <= rpos[i]) ? sv : -INFINITY;
        } else {
          s[n][i] = sv;
        }
      }
    }
  };

  // Pass 1 (row max and sum of exp), then pass 2 (p = bf16(exp(s - m) / l),
  // O += P . V), each step's K/V rows requested one step ahead (pass 2's
  // first tile during pass 1's last step).  Step q < n is pass 1 over key
  // block kb0 + q, step n + q pass 2 over the same block.  (Two tiles in
  // flight at head_dim 512 spilled registers and ran slower: 459 against
  // 441 us per full layer of a 2,048-token prompt.)
  const int n = kb1 - kb0 + 1;
  auto target = [&](int q, Tile& T) {  // request step q's rows (no-op past the last step)
    if (q < 2 * n) fetch(kb0 + (q < n ? q : q - n), q >= n, T);
  };
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }
  // Step g (pass 1: g = q, pass 2: g = n + q) reads buffer g % NBUF.  With
  // two buffers, step g stores step g + 1's rows (requested one step earlier)
  // into the other buffer, requests step g + 2's, and ends at the barrier
  // that makes them visible (and frees buffer g % 2 for step g + 2); with one,
  // the step stores its own rows between two barriers.
  auto stage = [&](int g, Tile& T) {
    if constexpr (NBUF == 2) {
      if (g + 1 < 2 * n) put(T, g + 1 >= n, (g + 1) & 1);
      target(g + 2, T);
    } else {
      lds_barrier();
      put(T, g >= n, 0);
      target(g + 1, T);
      lds_barrier();
    }
  };
  auto end_step = [&]() {
    if constexpr (NBUF == 2) lds_barrier();
  };
  auto step1 = [&](int q, Tile& T, auto edge) {
    stage(q, T);
    float s[NT][4];
    scores(kb0 + q, s, edge, q % NBUF);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float bm = s[0][i];
#pragma unroll
      for (int n = 1; n < NT; ++n) bm = fmaxf(bm, s[n][i]);
      bm = row16_max(bm);
      const float mn = fmaxf(m[i], bm);
      float e = 0.0f;
      if constexpr (decltype(edge)::value) {
        if (mn != -INFINITY) {
#pragma unroll
          for (int n = 0; n < NT; ++n) e += (s[n][i] == -INFINITY) ? 0.0f : exp_nonpos(s[n][i] - mn);
        }
      } else {
#pragma unroll
        for (int n = 0; n < NT; ++n) e += exp_nonpos(s[n][i] - mn);
      }
      e = row16_sum(e);
      // rescale the sum when the max moved (exp(0) = 1 leaves it as it is)
      if (m[i] == -INFINITY)
        l[i] = e;
      else if (m[i] != mn)
        l[i] = l[i] * exp_nonpos(m[i] - mn) + e;
      else
        l[i] += e;
      m[i] = mn;
    }
    end_step();
  };
  Tile tile;
  lds_barrier();  // ptl
  target(0, tile);
  if constexpr (NBUF == 2) {
    put(tile, false, 0);  // step 0 is a pass-1 step (n >= 1)
    target(1, tile);
    lds_barrier();
  }
  {
    int q = 0;
    for (; q < n && !interior(kb0 + q); ++q) step1(q, tile, Edge{});
    for (; q < n && interior(kb0 + q); ++q) step1(q, tile, Inner{});
    for (; q < n; ++q) step1(q, tile, Edge{});
  }

  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint16_t* pw = pt + 16 * wave * LDP;  // this wave's 16 rows of P
  float rl[4];                          // 1 / l (0 for a row without keys)
#pragma unroll
  for (int i = 0; i < 4; ++i) rl[i] = (l[i] > 0.0f) ? __builtin_amdgcn_rcpf(l[i]) : 0.0f;
  auto step2 = [&](int q, Tile& T, auto edge) {
    const int g = n + q, buf = g % NBUF;
    stage(g, T);
    float s[NT][4];
    scores(kb0 + q, s, edge, buf);
    // p = bf16(exp(s - m) / l), 0 for a masked key or a row without keys
#pragma unroll
    for (int nn = 0; nn < NT; ++nn)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float e;
        if constexpr (decltype(edge)::value)
          e = (s[nn][i] == -INFINITY) ? 0.0f : exp_nonpos(s[nn][i] - m[i]);
        else
          e = exp_nonpos(s[nn][i] - m[i]);
        float p = e * rl[i];
        if (near_bf16_midpoint(p)) p = e / l[i];
        pw[(4 * (lane >> 4) + i) * LDP + 16 * nn + fr] = f2bf(p);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int st = 0; st < KB / 32; ++st) {
      const u32x4 pa = *(const u32x4*)(pw + fr * LDP + 32 * st + fk);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const u32x4 vb = *(const u32x4*)(vt[buf] + (16 * dt + fr) * LDV + 32 * st + fk);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, pa),
                                                        __builtin_bit_cast(bf16x8, vb), o[dt], 0, 0, 0);
      }
    }
    end_step();
  };
  {
    int q = 0;
    for (; q < n && !interior(kb0 + q); ++q) step2(q, tile, Edge{});
    for (; q < n && interior(kb0 + q); ++q) step2(q, tile, Inner{});
    for (; q < n; ++q) step2(q, tile, Edge{});
  }

  // ---- ctx = bf16(O): row 4(l/16)+i of the wave, d = 16*dt + l%16
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!rvalid[i]) continue;
    const int r = 16 * wave + 4 * (lane >> 4) + i;
    uint16_t* out = a.ctx + ((size_t)(t0 + r / G) * a.NH + kv * G + r % G) * D + fr;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) out[16 * dt] = f2bf(o[dt][i]);
  }
}

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int g4mi_q_norm_rope(uint16_t* q, const uint16_t* q_norm, const uint16_t* rope_cos, const uint16_t* rope_sin,
                     int64_t T, int64_t NH, int64_t D, int64_t p0, int64_t rope_len, float eps, void* stream) {
  G4MI_REQUIRE(q && q_norm && rope_cos && rope_sin, G4MI_EINVAL, "q_norm_rope: missing argument");
  G4MI_REQUIRE(T >= 1 && T <= 2147483647 && NH >= 1 && NH <= 65535 * 4 && p0 >= 0 && p0 + T <= rope_len, G4MI_EINVAL,
               "q_norm_rope: T=%lld NH=%lld p0=%lld outside the rope table (%lld positions)", (long long)T,
               (long long)NH, (long long)p0, (long long)rope_len);
  dim3 grid((unsigned)T, (unsigned)((NH + 3) / 4));
  hipStream_t st = as_stream(stream);
  switch (D) {
    case 64: hipLaunchKernelGGL(q_norm_rope_kernel<64>, grid, dim3(256), 0, st, q, q_norm, rope_cos, rope_sin, (int)NH, (int)p0, eps); break;
    case 128: hipLaunchKernelGGL(q_norm_rope_kernel<128>, grid, dim3(256), 0, st, q, q_norm, rope_cos, rope_sin, (int)NH, (int)p0, eps); break;
    case 256: hipLaunchKernelGGL(q_norm_rope_kernel<256>, grid, dim3(256), 0, st, q, q_norm, rope_cos, rope_sin, (int)NH, (int)p0, eps); break;
    case 512: hipLaunchKernelGGL(q_norm_rope_kernel<512>, grid, dim3(256), 0, st, q, q_norm, rope_cos, rope_sin, (int)NH, (int)p0, eps); break;
    default: G4MI_REQUIRE(false, G4MI_EUNSUPPORTED, "q_norm_rope: head_dim %lld not in {64,128,256,512}", (long long)D);
  }
  return check_launch("q_norm_rope");
}

int g4mi_prefill_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages, int64_t num_pages,
                           const int32_t* page_table, int64_t max_pages, int64_t page_size, int64_t T, int64_t p0,
                           int64_t NH, int64_t KV, int64_t D, int64_t window, float softcap, uint16_t* ctx,
                           void* stream) {
  G4MI_REQUIRE(q && k_pages && v_pages && page_table && ctx, G4MI_EINVAL, "prefill_attention: missing argument");
  G4MI_REQUIRE(KV >= 1 && KV <= 65535 && NH >= KV && NH % KV == 0, G4MI_EINVAL,
               "prefill_attention: bad NH=%lld KV=%lld", (long long)NH, (long long)KV);
  const int64_t G = NH / KV;
  G4MI_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, G4MI_EUNSUPPORTED,
               "prefill_attention: head_dim %lld not in {64,128,256,512}", (long long)D);
  G4MI_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, G4MI_EUNSUPPORTED,
               "prefill_attention: %lld query heads per KV head not in {1,2,4,8}", (long long)G);
  G4MI_REQUIRE(page_size % 64 == 0 && page_size >= 64, G4MI_EUNSUPPORTED,
               "prefill_attention: page size %lld must be a multiple of 64", (long long)page_size);
  G4MI_REQUIRE(T >= 1 && p0 >= 0 && p0 + T <= max_pages * page_size, G4MI_EINVAL,
               "prefill_attention: positions [%lld, %lld) beyond the page table", (long long)p0, (long long)(p0 + T));
  G4MI_REQUIRE(((uintptr_t)q & 15u) == 0 && ((uintptr_t)k_pages & 15u) == 0 && ((uintptr_t)v_pages & 15u) == 0,
               G4MI_EALIGN, "prefill_attention: q and the pages must be 16-byte aligned");
  PfAttnArgs a;
  a.q = q; a.k_pages = k_pages; a.v_pages = v_pages; a.pt = page_table; a.ctx = ctx;
  a.T = (int)T; a.NH = (int)NH; a.KV = (int)KV; a.page = (int)page_size; a.num_pages = (int)num_pages;
  a.max_pages = (int)max_pages; a.p0 = (int)p0; a.window = (int)window; a.softcap = softcap;
  hipStream_t st = as_stream(stream);
  // 1-D grid in the order of pf_block
  auto grid_of = [&](int64_t qp) -> int64_t {
    const int64_t nqb = (T + qp - 1) / qp;
    a.nqb = (int)nqb;
    if (8 % KV == 0) {
      a.xmap = 1;
      const int64_t per = 8 / KV;
      return KV * ((nqb + per - 1) / per * per);
    }
    a.xmap = (KV % 8 == 0) ? 2 : 0;
    return KV * nqb;
  };
#define G4MI_PF(DD, GG)                                                                                      \
  if (D == DD && G == GG) {                                                                                  \
    const int64_t nb = grid_of(16 * pf_waves<DD>() / GG);                                                    \
    G4MI_REQUIRE(nb <= 2147483647, G4MI_EINVAL, "prefill_attention: %lld blocks", (long long)nb);            \
    if (softcap > 0.0f)                                                                                      \
      hipLaunchKernelGGL((attn_prefill_kernel<DD, GG, true>), dim3((unsigned)nb), dim3(64 * pf_waves<DD>()), \
                         0, st, a);                                                                          \
    else                                                                                                     \
      hipLaunchKernelGGL((attn_prefill_kernel<DD, GG, false>), dim3((unsigned)nb), dim3(64 * pf_waves<DD>()),\
                         0, st, a);                                                                          \
  }
  G4MI_PF(64, 1) G4MI_PF(64, 2) G4MI_PF(64, 4) G4MI_PF(64, 8)
  G4MI_PF(128, 1) G4MI_PF(128, 2) G4MI_PF(128, 4) G4MI_PF(128, 8)
  G4MI_PF(256, 1) G4MI_PF(256, 2) G4MI_PF(256, 4) G4MI_PF(256, 8)
  G4MI_PF(512, 1) G4MI_PF(512, 2) G4MI_PF(512, 4) G4MI_PF(512, 8)
#undef G4MI_PF
  return check_launch("prefill_attention");
}

}  // extern "C"
